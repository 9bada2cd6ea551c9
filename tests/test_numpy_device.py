"""Pins of the numpy oracle (oracle/numpy_device.py) against things it did not compute itself.

- The graph corpus (tests/graphs.py, the reference's tests/conftest.py:76-93 set) against torch on
  the CPU: the same expressions spelled in torch, float64 (to 1e-12) and float32 (to 1e-5).
- The reference's known answers for what one dtype must get right (reference
  tests/test_dtypes.py:207-238): half-width sums total in float32, narrow ints wrap at their width.
- The transaction rule (reference tests/test_device.py:11-44): reads in an assign's batch see the
  pre-assign bytes, an assign whose value is a buffer another assign overwrites takes the old
  value, and a result cached before an assign is not reused after it.
- capture on a compiled device (the C device) returning each replay's own tensor: 8.0 and 12.0
  (reference tests/test_jit.py:75-78).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from graphs import GRAPHS
from limn_amd.seam import Tensor, bfloat16, capture, float16, float32, float64, int8, int16, realize
from limn_amd.seam import device as limn_device
from oracle import c_device
from oracle.numpy_device import NumpyDevice


@pytest.fixture(autouse=True)
def on_numpy():
    limn_device.active_device = NumpyDevice()


def _pad(t, before_after):
    (r0, r1), (c0, c1) = before_after
    return torch.nn.functional.pad(t, (c0, c1, r0, r1))


TORCH = {
    "elementwise": lambda a, b: (a + b) * 2.0 - a,
    "relu": lambda a, b: torch.relu(a * b) + 1.0,
    "unary math": lambda a, b: torch.sqrt(torch.exp(torch.log(a * a + 1.0))),
    "divide": lambda a, b: a / (b * b + 0.5),
    "where": lambda a, b: torch.where(a < b, a, b),
    "cast round trip": lambda a, b: (a * 4.0).to(torch.int32).to(torch.float32) + 0.5,
    "sum an axis": lambda a, b: (a + b).sum(dim=1),
    "sum everything": lambda a, b: (a * b).sum(),
    "max keepdim": lambda a, b: (a * b).amax(dim=0, keepdim=True),
    "mean": lambda a, b: (a + b).mean(dim=1),
    "matmul": lambda a, b: a @ b.T,
    "softmax": lambda a, b: torch.softmax(a + b, dim=1),
    "log softmax": lambda a, b: torch.log_softmax(a * b, dim=0),
    "padded reduce": lambda a, b: _pad(a, ((1, 1), (0, 2))).sum(dim=1),
    "movement then reduce": lambda a, b: (a.T * 2.0).sum(dim=0),
    "reduce then elementwise": lambda a, b: torch.relu(a.sum(dim=1, keepdim=True) * b),
}


def test_every_corpus_graph_has_a_torch_spelling():
    assert set(TORCH) == set(GRAPHS)


@pytest.mark.parametrize("name", sorted(GRAPHS))
@pytest.mark.parametrize("width", ["float64", "float32"])
def test_corpus_matches_torch(name, width):
    rng = np.random.default_rng(sorted(GRAPHS).index(name))
    np_dtype, limn_dtype, tol = (np.float64, float64, 1e-12) if width == "float64" else (np.float32, float32, 1e-5)
    a, b = (rng.standard_normal((6, 5)).astype(np_dtype) for _ in range(2))
    got = GRAPHS[name](Tensor(a, dtype=limn_dtype), Tensor(b, dtype=limn_dtype)).numpy()
    want = TORCH[name](torch.from_numpy(a), torch.from_numpy(b)).numpy()
    if name == "cast round trip":  # an int cast ends in float32 on both sides whatever the input width
        want = want.astype(np.float32)
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=tol, atol=tol)


def test_a_planted_mistake_is_caught():
    """The comparison above is not vacuous: a wrong spelling (log softmax over the other axis)
    differs from torch by far more than the tolerance."""
    rng = np.random.default_rng(0)
    a, b = (rng.standard_normal((6, 5)) for _ in range(2))
    got = (Tensor(a, dtype=float64) * Tensor(b, dtype=float64)).log_softmax(axis=1).numpy()
    want = TORCH["log softmax"](torch.from_numpy(a), torch.from_numpy(b)).numpy()
    assert np.max(np.abs(got - want)) > 1e-3


def test_a_float16_sum_totals_in_float32():
    data = np.concatenate([np.array([2048.0], dtype=np.float16), np.ones(4096, dtype=np.float16)])
    assert float(Tensor(data, dtype=float16).sum().numpy()) == pytest.approx(2048.0 + 4096.0, rel=1e-3)


def test_a_bfloat16_sum_totals_in_float32():
    data = np.concatenate([np.array([256.0], dtype=np.float32), np.full(4096, 0.5, dtype=np.float32)])
    assert float(Tensor(data, dtype=bfloat16).sum().numpy()) == pytest.approx(256.0 + 2048.0, rel=1e-2)


def test_narrow_sums_wrap_at_their_width():
    assert Tensor(np.ones(300, np.int8), dtype=int8).sum().item() == 44  # 300 mod 256
    assert Tensor(np.full(5000, 100, np.int16), dtype=int16).sum().item() == np.array(500000).astype(np.int16).item()


def test_narrow_arithmetic_wraps_like_numpy():
    rng = np.random.default_rng(1)
    x, y = (rng.integers(-128, 128, (5, 7)).astype(np.int8) for _ in range(2))
    got = (Tensor(x, dtype=int8) * Tensor(y, dtype=int8) + 100).numpy()
    np.testing.assert_array_equal(got, x * y + np.int8(100))


def test_reads_in_an_assign_batch_see_pre_assign_bytes():
    t = Tensor(np.ones((2, 2), dtype=np.float32))
    before = t * 10.0
    t.assign(t + 100.0)
    bufs = limn_device.active_device.execute([before.node, t.node])
    got_before, got_after = (b.view(np.float32).reshape(2, 2) for b in bufs)
    np.testing.assert_array_equal(got_before, np.full((2, 2), 10.0, np.float32))
    np.testing.assert_array_equal(got_after, np.full((2, 2), 101.0, np.float32))


def test_an_assign_of_a_buffer_another_assign_overwrites_takes_the_old_value():
    a = Tensor(np.array([1.0], dtype=np.float32))
    b = Tensor(np.array([0.0], dtype=np.float32))
    a_before = a.detach()
    a.assign(a_before * 0.0 + 7.0)
    b.assign(a_before)
    realize(a, b)
    assert (a.item(), b.item()) == (7.0, 1.0)


def test_a_result_cached_before_an_assign_is_not_reused_after_it():
    t = Tensor(np.ones((2, 2), dtype=np.float32))
    doubled = t * 2.0
    np.testing.assert_array_equal((doubled + 1.0).numpy(), np.full((2, 2), 3.0, np.float32))
    t.assign(t + 10.0).realize()
    np.testing.assert_array_equal((doubled + 1.0).numpy(), np.full((2, 2), 23.0, np.float32))


@pytest.mark.skipif(c_device.compiler() is None, reason="no host C compiler")
def test_each_replay_returns_its_own_tensor():
    limn_device.active_device = c_device.CDevice()

    def step(x):
        return (x + 1.0).sum().realize()

    fn = capture(step)
    fn(Tensor(np.zeros(4, np.float32)))
    fn(Tensor(np.zeros(4, np.float32)))
    third = fn(Tensor(np.full(4, 1.0, dtype=np.float32)))
    fourth = fn(Tensor(np.full(4, 2.0, dtype=np.float32)))
    assert third is not fourth
    assert (third.item(), fourth.item()) == (8.0, 12.0)


def test_a_bfloat16_scatter_rounds_every_add():
    """np.add.at into limn's bfloat16 table (reference limn/device.py:155-157) adds in float32 and
    rounds to bfloat16 after every add: at 256 the bf16 spacing is 2, so each 0.5 rounds away and
    the row stays 256, where a float32 total rounded once would give 258."""
    from limn_amd.seam import scatter_rows

    values = np.array([[256.0], [0.5], [0.5], [0.5], [0.5], [3.0]], dtype=np.float32)
    idx = np.array([0, 0, 0, 0, 0, 1], dtype=np.int32)
    got = scatter_rows(Tensor(values, dtype=bfloat16), Tensor(idx), (2, 1)).numpy()
    np.testing.assert_array_equal(got, np.array([[256.0], [3.0]], np.float32))
    halves = scatter_rows(Tensor(values, dtype=float16), Tensor(idx), (2, 1)).numpy()  # spacing 0.25 at 256
    np.testing.assert_array_equal(halves, np.array([[258.0], [3.0]], np.float16))
