"""The CPU baseline (oracle/c_device.py, a restatement of reference limn/backend_c.py) against the
numpy oracle, as the reference's tests/test_backend_c.py runs its C device: the graph corpus,
int wrap, NaN-propagating max, gathers and scatters, the assign transaction, the dtypes it
declines, the mask split's bit-identity, and attention taking the composed path (it has no
CUSTOM kernels). CPU only: it needs a host C compiler, not a GPU."""

from __future__ import annotations

import numpy as np
import pytest

from graphs import GRAPHS, check
from limn_amd.seam import bfloat16, float16, float32, float64, grad, int16, int32, int8, lower_all, Op, Opcode, scatter_rows, Tensor, topological
from limn_amd.seam import device as limn_device
from oracle import c_device
from oracle import sdpa as ref

pytestmark = pytest.mark.skipif(c_device.compiler() is None, reason="no host C compiler")

rng = np.random.default_rng(11)


def randf(*shape: int) -> np.ndarray:
    return rng.uniform(-2, 2, shape).astype(np.float32)


@pytest.fixture(autouse=True)
def on_numpy():
    limn_device.set_device("numpy")
    yield


@pytest.fixture
def cdev():
    return c_device.CDevice()


@pytest.mark.parametrize("name", list(GRAPHS))
def test_corpus(cdev, name):
    check(cdev, GRAPHS[name](Tensor(randf(6, 5)), Tensor(randf(6, 5))))


@pytest.mark.parametrize("name", ["elementwise", "softmax", "sum an axis", "matmul"])
def test_corpus_float64(cdev, name):
    a, b = Tensor(randf(5, 7), dtype=float64), Tensor(randf(5, 7), dtype=float64)
    check(cdev, GRAPHS[name](a, b), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dtype", [int32, int16, int8], ids=str)
def test_int_dtypes_wrap_exactly(cdev, dtype):
    a = Tensor(rng.integers(-100, 100, size=(20, 30)), dtype=dtype)
    b = Tensor(rng.integers(-100, 100, size=(20, 30)), dtype=dtype)
    check(cdev, (a * b + a).sum(axis=1), exact=True)
    check(cdev, (a < b).where(a, b * b), exact=True)


def test_int8_sum_of_300_ones_wraps_to_44(cdev):
    check(cdev, Tensor(np.ones(300, dtype=np.int8), dtype=int8).sum(), exact=True)


def test_int32_overflow_wraps_like_numpy(cdev):
    big = Tensor(np.full(4, 2**31 - 1, dtype=np.int32), dtype=int32)
    check(cdev, big + big, exact=True)


def test_max_propagates_nan(cdev):
    x = randf(4, 6)
    x[1, 3] = np.nan
    check(cdev, Tensor(x).max(axis=1))


def test_gather_rows(cdev):
    table = Tensor(randf(10, 4))
    idx = Tensor(rng.integers(0, 10, size=(6, 3)).astype(np.int32))
    check(cdev, table[idx] * 2.0, exact=True)


def test_scatter_matches_np_add_at_bit_for_bit(cdev):
    """One thread adds the rows in the loop's order, which is np.add.at's order."""
    values = Tensor(randf(512, 8))
    idx = Tensor(rng.integers(0, 4, size=512).astype(np.int32))
    check(cdev, scatter_rows(values, idx, (4, 8)), exact=True)


def test_gather_backward_scatters(cdev):
    table = Tensor(randf(10, 4), requires_grad=True)
    idx = Tensor(rng.integers(0, 10, size=(6, 3)).astype(np.int32))
    (g,) = grad((table[idx] * Tensor(randf(6, 3, 4))).sum(), [table])
    check(cdev, g)


def test_assign_is_deferred_until_every_sink_is_computed(cdev):
    limn_device.active_device = cdev
    w = Tensor(np.ones(4, dtype=np.float32))
    read = w * 2.0
    w.assign(w + 1.0)
    bufs = cdev.execute([read.node, w.node])
    np.testing.assert_array_equal(cdev.copyout(bufs[0]).view(np.float32), np.full(4, 2.0, np.float32))
    np.testing.assert_array_equal(cdev.copyout(bufs[1]).view(np.float32), np.full(4, 2.0, np.float32))


@pytest.mark.parametrize("dtype", [float16, bfloat16], ids=str)
def test_half_widths_are_declined(cdev, dtype):
    """Reference limn/backend_c.py:189-208: a half width anywhere in a nest is refused at plan time."""
    x = Tensor(randf(4, 4), dtype=dtype)
    with pytest.raises(NotImplementedError, match="no"):
        cdev.execute([(x * 2.0).node])


def test_a_half_intermediate_is_declined(cdev):
    x = Tensor(randf(4, 4))
    with pytest.raises(NotImplementedError):
        cdev.execute([((x * 2.0).cast(float16).cast(float32) + 1.0).node])


def padded_graph():
    a, b = Tensor(randf(7, 9)), Tensor(randf(9, 7))
    return (a.pad(((2, 1), (3, 4))) * 1.5 + b.transpose().pad(((2, 1), (3, 4)))).sum(axis=1)


def test_split_masked_cuts_the_innermost_loop():
    """The padded innermost loop becomes three pieces (before, inside, after the pad) and the
    pieces outside read literal zeros, with no range check left on that variable."""
    t = padded_graph()
    nests = lower_all([t.node])
    plain = c_device.emit_c(nests, split=False)
    cut = c_device.emit_c(nests, split=True)
    assert cut.count("for (") > plain.count("for (")
    split_instrs = c_device.split_masked(nests[0].instrs)
    innermost = [i for i in split_instrs if i.opcode is Opcode.LOOP]
    var = innermost[-1].dest
    for instr in split_instrs:
        if instr.opcode is Opcode.LOAD:
            assert all(bvar != var for bvar, *_ in instr.arg[2].bounds)


def test_split_masked_is_bit_identical():
    want = c_device.CDevice(split=False)
    got = c_device.CDevice(split=True)
    t = padded_graph()
    a = want.copyout(want.execute([t.node])[0])
    b = got.copyout(got.execute([t.node])[0])
    np.testing.assert_array_equal(a, b)
    check(got, t)


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attention_takes_the_composed_path(cdev, causal):
    """No CUSTOM kernels: the forward and backward are ordinary nests, with (t, t) intermediates,
    and they agree with the oracle's textbook attention (reference limn/tensor.py:559-560)."""
    limn_device.active_device = cdev  # the seam asks the active device for CUSTOM kernels
    shape = (2, 40, 8)
    host = [randf(*shape) for _ in range(3)]
    q, k, v = (Tensor(x, requires_grad=True) for x in host)
    out = q.attention(k, v, causal=causal)
    gq, gk, gv = grad(out.sum(), [q, k, v])
    nodes = topological([out.node, gq.node, gk.node, gv.node])
    assert not [n for n in nodes if n.op is Op.CUSTOM]
    assert [n for n in nodes if n.shape[-2:] == (40, 40)]
    got = [t.numpy() for t in (out, gq, gk, gv)]
    q64, k64, v64 = (x.astype(np.float64) for x in host)
    want = ref.plain(q64, k64, v64, causal=causal, scale=8**-0.5)
    np.testing.assert_allclose(got[0], want, rtol=1e-5, atol=1e-5)
    lse = ref.plain_lse(q64, k64, causal=causal, scale=8**-0.5)
    do = np.ones_like(want)
    delta = (do * want).sum(axis=-1, keepdims=True)
    np.testing.assert_allclose(got[1], ref.sdpa_backward_q(q64, k64, v64, do, lse, delta, causal=causal, scale=8**-0.5, dtype="float64"), rtol=1e-4, atol=1e-5)
    dk, dv = ref.sdpa_backward_kv(q64, k64, v64, do, lse, delta, causal=causal, scale=8**-0.5, dtype="float64")
    np.testing.assert_allclose(got[2], dk, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(got[3], dv, rtol=1e-4, atol=1e-5)
