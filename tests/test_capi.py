"""The C ABI without a GPU: the library loads, exports every function include/limn_hip.h declares,
routes shapes to the right kernel family, and refuses invalid calls before touching a device."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from limn_amd.hip import runtime

HEADER = Path(__file__).resolve().parent.parent / "include" / "limn_hip.h"


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(limn_hip_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_entry_points():
    names = declared()
    for name in ("limn_hip_sdpa_fwd", "limn_hip_sdpa_bwd_q", "limn_hip_sdpa_bwd_kv", "limn_hip_last_error"):
        assert name in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(runtime.LIBRARY))
    missing = [name for name in declared() if not hasattr(lib, name)]
    assert not missing, f"liblimn_hip.so lacks {missing}"


def test_abi_version():
    assert runtime.kernels().limn_hip_abi_version() == runtime.ABI_VERSION == 3


def test_sdpa_path_routing():
    lib = runtime.kernels()
    bf16, f16, f32, f64 = 3, 2, 1, 0
    assert lib.limn_hip_sdpa_path(bf16, 128, 128) == 1
    assert lib.limn_hip_sdpa_path(f16, 64, 64) == 1
    assert lib.limn_hip_sdpa_path(bf16, 64, 128) == 0  # hd != hd_v: general kernels
    assert lib.limn_hip_sdpa_path(f32, 64, 64) == 0
    assert lib.limn_hip_sdpa_path(f64, 16, 24) == 0
    assert lib.limn_hip_sdpa_path(f32, 300, 64) == -1
    assert lib.limn_hip_sdpa_path(7, 64, 64) == -1


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation first


def _fwd(**kw):
    args = dict(dtype=1, batch=2, t_q=8, t_k=8, hd=16, hd_v=16, causal=0, scale=0.25)
    args.update(kw)
    lib = runtime.kernels()
    return lib.limn_hip_sdpa_fwd(FAKE, FAKE, FAKE, None, FAKE, FAKE, args["dtype"], args["batch"], args["t_q"],
                                 args["t_k"], args["hd"], args["hd_v"], args["causal"], args["scale"], None)


@pytest.mark.parametrize(
    "kw,code,message",
    [
        (dict(causal=1, t_k=9), 1, "square keys"),
        (dict(batch=0), 1, "positive"),
        (dict(hd=0), 1, "positive"),
        (dict(scale=float("inf")), 1, "finite"),
        (dict(dtype=5), 2, "float dtype"),
        (dict(hd=300), 2, "head dims"),
    ],
)
def test_invalid_calls_are_refused_with_a_reason(kw, code, message):
    assert _fwd(**kw) == code
    assert message in runtime.kernels().limn_hip_last_error().decode()


def test_status_codes_map_to_limns_exceptions():
    _fwd(causal=1, t_k=9)
    with pytest.raises(ValueError, match="square keys"):
        runtime.check_limn(1)
    with pytest.raises(NotImplementedError):
        runtime.check_limn(2)
    with pytest.raises(RuntimeError):
        runtime.check_limn(3)


def test_null_buffers_are_refused():
    lib = runtime.kernels()
    rc = lib.limn_hip_sdpa_bwd_q(FAKE, FAKE, FAKE, None, FAKE, FAKE, None, FAKE, 1, 1, 4, 4, 8, 8, 0, 0.5, None)
    assert rc == 1 and "null" in lib.limn_hip_last_error().decode()


def test_every_split_fits_the_static_scratch():
    """limn_hip_matmul_noalloc keeps split-k slices in a static array of LIMN_HIP_SCRATCH_BYTES.
    The planner splits only while output tiles x slices stay under two waves of 256 workgroups,
    so no contraction needs more; swept over batch, M, N (multiples of 64) and k."""
    lib = runtime.kernels()
    text = HEADER.read_text()
    limit = int(re.search(r"#define LIMN_HIP_SCRATCH_BYTES \((\d+)ll << (\d+)\)", text).group(1)) << 20
    assert limit == 128 << 20
    worst = 0
    for batch in (1, 2, 3, 8):
        for m in range(64, 4097, 192):
            for n in range(64, 4097, 320):
                for k in (1024, 5376, 1 << 14, 1 << 20):
                    worst = max(worst, lib.limn_hip_matmul_workspace(3, batch, m, n, k))
    assert 0 < worst <= limit
