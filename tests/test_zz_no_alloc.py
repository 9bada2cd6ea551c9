"""limn_hip_matmul_noalloc against limn_hip_matmul, through the C ABI, on the GPU.

The no-allocation entry point keeps the split-k slices in a static device array instead of a
caller workspace; its results must equal the workspace entry point's bit for bit (same kernels,
same slice order). Two calls in a row, the second smaller, so the second reads the array after
the first left its own slices in it; both shapes split k, so the array is really used.
"""

from __future__ import annotations


import numpy as np
import pytest

from limn_amd.dtypes import bf16_bits
from limn_amd.hip import runtime

pytestmark = pytest.mark.gpu

BF16 = 3
SCRATCH_BYTES = 128 << 20


def _matmul_pair(dev, M: int, N: int, K: int, seed: int, epilogue: int) -> tuple[np.ndarray, np.ndarray]:
    lib = dev.lib
    need = int(lib.limn_hip_matmul_workspace(BF16, 1, M, N, K))
    assert 0 < need <= SCRATCH_BYTES, need  # the shape splits k and fits the static array
    rng = np.random.default_rng(seed)
    a_host = bf16_bits(rng.standard_normal((M, K), dtype=np.float32) * 0.125)
    b_host = bf16_bits(rng.standard_normal((K, N), dtype=np.float32) * 0.125)
    a, b = dev._alloc(a_host.nbytes), dev._alloc(b_host.nbytes)
    dev.copyin(a, a_host)
    dev.copyin(b, b_host)
    c_ref, c_new, ws = dev._alloc(M * N * 2), dev._alloc(M * N * 2), dev._alloc(need)
    strides = (1, M, N, K, M * K, K, 1, K * N, N, 1, M * N, N, 1)
    print(f"no_alloc: M={M} N={N} K={K} epilogue={epilogue}, workspace {need} bytes", flush=True)
    runtime.check_limn(lib.limn_hip_matmul(a.ptr, b.ptr, c_ref.ptr, BF16, *strides, epilogue, ws.ptr, need, None))
    runtime.check_limn(lib.limn_hip_matmul_noalloc(a.ptr, b.ptr, c_new.ptr, BF16, *strides, epilogue, None))
    dev.finish()
    return dev.copyout(c_ref), dev.copyout(c_new)


def test_noalloc_matches_the_workspace_entry_point(hipdev):
    for (M, N, K, seed, epilogue) in ((512, 512, 8192, 1, 0), (256, 256, 4096, 2, 1)):
        want, got = _matmul_pair(hipdev, M, N, K, seed, epilogue)
        assert want.any()
        np.testing.assert_array_equal(got, want)
