"""Checks of the reference's GPU device tests restated on the hip device.

- grad of grad through attention (reference tests/test_attention.py:192-210): under create_graph
  the backward must be the composed form (a CUSTOM node has no derivative of its own), and the
  second gradients match torch's math backend;
- a split reduce gives the same bits twice (reference tests/test_backend_cuda.py:146-150);
- the buffer pool recycles dropped buffers and trim() empties it (:158-167).
"""

from __future__ import annotations

from functools import reduce
from operator import add

import numpy as np
import pytest

from limn_amd.seam import Op, Tensor, grad, topological, use_device

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_grad_of_grad_through_attention_matches_torch(hipdev, causal):
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    use_device(hipdev)
    rng = np.random.default_rng(11)
    qd, kd, vd = (rng.uniform(-2, 2, (2, 3, 16, 8)).astype(np.float32) for _ in range(3))
    q, k, v = (Tensor(d, requires_grad=True) for d in (qd, kd, vd))
    loss = (q.attention(k, v, causal=causal) ** 2).sum()
    first = grad(loss, [q, k, v], create_graph=True)
    names = {n.arg.name for g in first for n in topological([g.node]) if n.op is Op.CUSTOM}
    assert names == {"sdpa"}, f"the differentiable backward is composed, not {names - {'sdpa'}}"
    second = grad(reduce(add, (g.sum() for g in first)), [q, k, v])
    tq, tk, tv = (torch.tensor(d, requires_grad=True) for d in (qd, kd, vd))
    with sdpa_kernel(SDPBackend.MATH):
        tloss = (F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal) ** 2).sum()
        tfirst = torch.autograd.grad(tloss, (tq, tk, tv), create_graph=True)
        tsecond = torch.autograd.grad(reduce(add, (t.sum() for t in tfirst)), (tq, tk, tv))
    for got, want in zip(first, tfirst):
        np.testing.assert_allclose(got.numpy(), want.detach().numpy(), rtol=1e-3, atol=1e-3)
    for got, want in zip(second, tsecond):
        np.testing.assert_allclose(got.numpy(), want.detach().numpy(), rtol=1e-3, atol=1e-3)


def test_a_split_reduce_gives_the_same_bits_twice(hipdev):
    use_device(hipdev)
    x = np.random.default_rng(7).uniform(-2, 2, 1 << 20).astype(np.float32)
    total = Tensor(x).sum()
    once = hipdev.copyout(hipdev.execute([total.node])[0])
    twice = hipdev.copyout(hipdev.execute([total.node])[0])
    np.testing.assert_array_equal(once, twice)
    np.testing.assert_allclose(once.view(np.float32)[0], float(x.astype(np.float64).sum()), rtol=1e-4)


def test_the_pool_recycles_dropped_buffers(hipdev):
    first = hipdev._alloc(1024)
    ptr = first.ptr
    del first
    second = hipdev._alloc(1024)
    assert second.ptr == ptr
    del second
    hipdev.trim()
    assert not any(hipdev.pool.values())
    assert hipdev._alloc(1024).ptr != 0
