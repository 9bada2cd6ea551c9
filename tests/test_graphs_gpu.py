"""The hip device's compiled-device contract on the MI355X (reference
tests/test_compiled_devices.py, test_backend_cuda.py, test_dtypes.py and test_attention.py's GPU
cases): the graph corpus, every reduce form, gathers and scatters, dtypes, the assign
transaction, plan reuse, and attention through the Tensor API, each diffed against the numpy
oracle on the same graph. Tensors are created under the numpy device (host buffers) and the hip
device uploads them per batch, as the reference's GPU tests do."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import storage_values
from graphs import GRAPHS, check
from limn_amd.seam import bfloat16, float16, float32, float64, grad, int16, int32, int8, Op, Tensor, topological
from limn_amd.seam import device as limn_device

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(7)


def randf(*shape: int) -> np.ndarray:
    return rng.uniform(-2, 2, shape).astype(np.float32)


@pytest.fixture(autouse=True)
def on_numpy():
    limn_device.set_device("numpy")
    yield


@pytest.mark.parametrize("name", list(GRAPHS))
def test_corpus(hipdev, name):
    a, b = Tensor(randf(5, 7)), Tensor(randf(5, 7))
    check(hipdev, GRAPHS[name](a, b))


@pytest.mark.parametrize("name", ["softmax", "sum an axis", "log softmax", "movement then reduce", "matmul"])
def test_corpus_at_size(hipdev, name):
    a, b = Tensor(randf(300, 300)), Tensor(randf(300, 300))
    check(hipdev, GRAPHS[name](a, b), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize(
    "shape,axis",
    [((3, 10), 1), ((9000, 70), 1), ((700, 3000), 1), ((64, 9000), 1), ((4, 300000), 1), ((3000, 40), 0), ((40, 3000), 0), ((2, 3, 4000, 5), (1, 2)), ((5000, 64), 1), ((777, 72), 1)],
    ids=["tiny", "thread-per-cell", "wave-per-cell", "workgroup-per-cell", "split", "accum-columns", "accum-few-columns", "two-axes", "lanes-per-cell", "ragged-lanes-per-cell"],
)
def test_every_reduce_form(hipdev, shape, axis):
    x = Tensor(rng.standard_normal(shape).astype(np.float32))
    check(hipdev, x.sum(axis=axis), rtol=1e-4, atol=1e-3)
    check(hipdev, x.max(axis=axis), exact=True)


def test_short_bf16_rows_reduce_in_lane_groups(hipdev):
    """Rows of 64 bf16 (the attention delta's shape): 8 lanes per row, 8 rows per wave."""
    a = Tensor(randf(2, 4, 300, 64), dtype=bfloat16)
    b = Tensor(randf(2, 4, 300, 64), dtype=bfloat16)
    check(hipdev, (a.cast(float32) * b.cast(float32)).sum(axis=-1, keepdim=True), rtol=1e-4, atol=1e-4)
    check(hipdev, a.max(axis=-1), exact=True)


@pytest.mark.parametrize("dtype", [float32, bfloat16], ids=str)
def test_concatenation_by_pads_loads_whole_runs(hipdev, dtype):
    """Three tensors stacked along a new leading dim by pad-and-add (how a gradient of a split
    is formed): each load is masked by the leading dim only."""
    parts = [Tensor(randf(1, 6, 40), dtype=dtype) for _ in range(3)]
    stacked = parts[0].pad(((0, 2), (0, 0), (0, 0))) + parts[1].pad(((1, 1), (0, 0), (0, 0))) + parts[2].pad(((2, 0), (0, 0), (0, 0)))
    check(hipdev, stacked, exact=True)


@pytest.mark.parametrize("shape,dtype", [((256, 96), bfloat16), ((4000, 36), float32), ((500, 37), float32), ((3, 700, 24), float32)],
                         ids=["bf16-runs-of-8", "f32-runs-of-4", "odd-width", "two-reduce-axes"])
def test_column_reduces_take_runs_of_cells(hipdev, shape, dtype):
    """Sums and maxes down the columns (a bias gradient's shape): a lane takes 16 bytes of
    consecutive columns when the width allows."""
    x = Tensor(randf(*shape), dtype=dtype)
    axes = tuple(range(len(shape) - 1))
    check(hipdev, x.cast(float32).sum(axis=axes), worst=1e-5)
    check(hipdev, x.max(axis=axes), exact=True)


def test_max_propagates_nan(hipdev):
    data = rng.standard_normal((4, 5000)).astype(np.float32)
    data[1, 4321] = np.nan
    data[3, 0] = np.nan
    got = Tensor(data).max(axis=1)
    check(hipdev, got, exact=True)


def test_reduce_to_a_scalar(hipdev):
    x = Tensor(rng.standard_normal((1000, 1000)).astype(np.float32))
    check(hipdev, x.sum(), rtol=1e-4, atol=1e-2)
    check(hipdev, (x * x).mean(), rtol=1e-4, atol=1e-4)


def test_grid_stride_covers_everything(hipdev):
    n = 2 * 4096 * 256 + 3
    x = Tensor(np.arange(n, dtype=np.float32))
    check(hipdev, x * 2.0 + 1.0, exact=True)


def test_gather_rows(hipdev):
    table = Tensor(randf(50, 16))
    idx = Tensor(rng.integers(0, 50, size=(7, 9)).astype(np.int32))
    check(hipdev, table[idx], exact=True)


def order_sensitive(*shape: int, seed: int = 0) -> np.ndarray:
    """Values whose float sum tends to depend on the order of the adds: large terms that cancel
    among small ones, so a reordering moves the small ones' rounding."""
    r = np.random.default_rng(seed)
    big = r.choice(np.array([3e7, -3e7, 1e8, -1e8], np.float32), size=shape)
    small = r.uniform(-4, 4, shape).astype(np.float32)
    return np.where(r.random(shape) < 0.3, big, small).astype(np.float32)


def test_scatter_with_repeats(hipdev):
    """512 values land on one row (reference tests/test_backend_cuda.py:125-131 allows 1e-4 for
    its atomics); here the total is np.add.at's, bit for bit. The values are drawn until adding
    them in reverse gives other bits, so that an unordered sum would fail."""
    from limn_amd.seam import scatter_rows

    idx = np.zeros(512, dtype=np.int32)
    for seed in range(100):
        values = order_sensitive(512, 8, seed=seed)
        forward, backward = np.zeros((4, 8), np.float32), np.zeros((4, 8), np.float32)
        np.add.at(forward, idx, values)
        np.add.at(backward, idx[::-1], values[::-1])
        if np.any(forward != backward):
            break
    else:
        raise AssertionError("no order-sensitive draw in 100 seeds")
    check(hipdev, scatter_rows(Tensor(values), Tensor(idx), (4, 8)), bitwise=True)


@pytest.mark.parametrize(
    "occurrences,rows,cols",
    [((7, 9), 10, 16), ((3000,), 5, 100), ((70000,), 300, 3), ((300000,), 40, 2), ((32, 512), 256, 512), ((5,), 3, 1), ((4,), 1000, 8)],
    ids=["small", "ragged-columns", "tiles-of-4096", "more-tiles-than-a-wave", "gpt-token-table", "one-column", "mostly-empty-rows"],
)
def test_float_scatter_is_occurrence_ordered(hipdev, occurrences, rows, cols):
    """Float SCATTER equals np.add.at bit for bit (the oracle's rule, reference
    limn/device.py:153-158): each row adds its values in occurrence order onto 0. Negative
    indices count from the end as numpy's do; some rows get nothing and stay 0."""
    from limn_amd.seam import scatter_rows

    values = order_sensitive(*occurrences, cols)
    idx = rng.integers(-rows, rows, size=occurrences).astype(np.int32)
    check(hipdev, scatter_rows(Tensor(values), Tensor(idx), (rows, cols)), bitwise=True)


def test_float64_scatter_and_computed_values_are_ordered(hipdev):
    """A float64 table, and values computed in the nest (a product then a sum, which must not be
    fused into one rounding)."""
    from limn_amd.seam import scatter_rows

    idx = Tensor(rng.integers(0, 7, size=(400,)).astype(np.int32))
    v64 = Tensor(order_sensitive(400, 6).astype(np.float64) * 1.1, dtype=float64)
    check(hipdev, scatter_rows(v64, idx, (7, 6)), bitwise=True)
    v = Tensor(order_sensitive(400, 6))
    check(hipdev, scatter_rows(v * 3.3 + 0.7, idx, (7, 6)), bitwise=True)


def test_scatter_grid_covers_more_rows_than_one_launch(hipdev):
    """A table of more (row, column block) items than the accumulating launch has workgroups."""
    from limn_amd.seam import scatter_rows

    rows = (1 << 20) + 77
    idx = Tensor(rng.integers(0, rows, size=(5000,)).astype(np.int32))
    values = Tensor(order_sensitive(5000, 1))
    check(hipdev, scatter_rows(values, idx, (rows, 1)), bitwise=True)


def launch_free_calls(hipdev, sinks) -> int:
    """How many of the plan's calls launch nothing (their nest runs inside its readers)."""
    hipdev.record = []
    hipdev.execute(sinks)
    plan = hipdev.record[0].plan
    hipdev.record = None
    return sum(1 for call in plan.calls if getattr(call.fn, "launches_nothing", False))


def test_softmax_layernorm_with_inlined_row_statistics(hipdev):
    """Without row programs the six per-row and scalar kernels of softmax -> LayerNorm run inside
    their readers (four launches stay); with them the ten kernels run inside the last one's
    launch. Both match the oracle."""
    from limn_amd.hip.device import HipDevice

    data = randf(300, 257)

    def chain() -> Tensor:
        y = Tensor(data).softmax(-1)
        c = y - y.mean(axis=-1, keepdim=True)
        return c / ((c * c).mean(axis=-1, keepdim=True) + 1e-5).sqrt()

    plain = HipDevice()
    plain.row_programs = False
    assert launch_free_calls(plain, [chain().node]) == 6
    check(plain, chain(), rtol=1e-4, atol=1e-5)
    assert launch_free_calls(hipdev, [chain().node]) == 10
    check(hipdev, chain(), rtol=1e-4, atol=1e-5)


def test_inlined_producer_read_through_a_pad_and_a_gather_index(hipdev):
    """An inlined producer read through a masked view (zero outside, nothing evaluated there)
    and one that computes gather indices."""
    x = Tensor(randf(8, 5))
    s = x.max(axis=1, keepdim=True) * 2.0
    padded = s.pad(((1, 1), (0, 0))) * Tensor(randf(10, 16))
    check(hipdev, padded, exact=True)
    idx = Tensor(rng.integers(0, 7, size=(6,)).astype(np.int32))
    shifted = Tensor(randf(9, 3)).gather_rows(idx + Tensor(np.ones(6, np.int32)))
    check(hipdev, shifted * 1.5, exact=True)


def test_scatter_int32_is_exact(hipdev):
    from limn_amd.seam import scatter_rows

    values = Tensor(rng.integers(-1000, 1000, size=(300, 5)).astype(np.int32))
    idx = Tensor(rng.integers(0, 6, size=300).astype(np.int32))
    check(hipdev, scatter_rows(values, idx, (6, 5)), exact=True)


@pytest.mark.parametrize("dtype", [bfloat16, float16], ids=["bfloat16", "float16"])
def test_half_width_scatter_rounds_each_add(hipdev, dtype):
    """A half-width table at the GPT's token-table shape (16384 occurrences into 256 rows of 512):
    np.add.at into a half array rounds the running total after every add, so the kernel's bits
    must equal the oracle's, which would not hold for a float32 total rounded once."""
    from limn_amd.seam import scatter_rows

    values = Tensor(order_sensitive(32, 512, 512), dtype=dtype)
    idx = Tensor(rng.integers(-256, 256, size=(32, 512)).astype(np.int32))
    check(hipdev, scatter_rows(values, idx, (256, 512)), bitwise=True)


def test_scatter_refuses_narrow_ints(hipdev):
    from limn_amd.seam import scatter_rows

    values = Tensor(rng.integers(-5, 5, size=(8, 4)).astype(np.int8), dtype=int8)
    idx = Tensor(np.zeros(8, dtype=np.int32))
    with pytest.raises(NotImplementedError):
        hipdev.execute([scatter_rows(values, idx, (2, 4)).node])


def test_gather_backward_scatters(hipdev):
    table = Tensor(randf(10, 4), requires_grad=True)
    idx = Tensor(rng.integers(0, 10, size=(6, 3)).astype(np.int32))
    (g,) = grad((table[idx] * Tensor(randf(6, 3, 4))).sum(), [table])
    check(hipdev, g, bitwise=True)


@pytest.mark.parametrize("dtype,tol", [(float64, 1e-12), (float16, 2e-3), (bfloat16, 1e-2)], ids=str)
def test_float_dtypes(hipdev, dtype, tol):
    """Half widths: the oracle rounds every node to its dtype while a kernel keeps fused
    intermediates in float, so sums over K products get an atol that grows with K."""
    a, b = Tensor(randf(9, 17), dtype=dtype), Tensor(randf(9, 17), dtype=dtype)
    for name in ("elementwise", "softmax", "max keepdim"):
        check(hipdev, GRAPHS[name](a, b), rtol=tol, atol=tol * 2)
    for name in ("sum an axis", "matmul"):
        check(hipdev, GRAPHS[name](a, b), rtol=tol, atol=tol * 16)


def test_half_sums_total_in_float32(hipdev):
    """1024 halves of 1 + tiny: a float16 running total would stall (reference
    tests/test_dtypes.py:207-216); the kernel totals in float32 and rounds once."""
    x = Tensor(np.full((2, 4096), 1.0, dtype=np.float32), dtype=float16)
    check(hipdev, x.sum(axis=1), exact=True)


@pytest.mark.parametrize("dtype", [int32, int16, int8], ids=str)
def test_int_dtypes_wrap_exactly(hipdev, dtype):
    a = Tensor(rng.integers(-100, 100, size=(20, 30)), dtype=dtype)
    b = Tensor(rng.integers(-100, 100, size=(20, 30)), dtype=dtype)
    check(hipdev, (a * b + a).sum(axis=1), exact=True)
    check(hipdev, (a < b).where(a, b * b), exact=True)


def test_int8_sum_of_300_ones_wraps_to_44(hipdev):
    x = Tensor(np.ones(300, dtype=np.int8), dtype=int8)
    got = x.sum()
    check(hipdev, got, exact=True)
    limn_device.set_device("numpy")
    assert got.item() == 44


def test_bf16_nan_store(hipdev):
    x = Tensor(np.array([1.0, np.nan, -2.0], dtype=np.float32), dtype=bfloat16)
    got = hipdev.execute([(x * 1.0).node])[0]
    vals = hipdev.copyout(got).view(np.uint16)
    assert np.isnan((vals.astype(np.uint32) << 16).view(np.float32)[1])


def test_assign_is_deferred_until_every_sink_is_computed(hipdev):
    """Both sinks read `w` before the assign commits (reference tests/test_compiled_devices.py:73-98)."""
    limn_device.active_device = hipdev
    w = Tensor(np.ones(4, dtype=np.float32))
    read = w * 2.0
    w.assign(w + 1.0)
    bufs = hipdev.execute([read.node, w.node])
    got_read = hipdev.copyout(bufs[0]).view(np.float32)
    np.testing.assert_array_equal(got_read, np.full(4, 2.0, np.float32))
    np.testing.assert_array_equal(hipdev.copyout(bufs[1]).view(np.float32), np.full(4, 2.0, np.float32))


def test_commits_of_a_batch_run_as_one_copy(hipdev):
    """Device-target commits are queued and copied in finish(): sizes that leave byte tails, a
    copy longer than one 64 KiB chunk, several dtypes in one batch, and a target committed twice
    (the later value wins)."""
    sizes = [1, 7, 16, 33, 65536, 65536 * 3 + 5, 1 << 20]
    targets, values, want = [], [], []
    for n in sizes:
        t, v = hipdev.alloc(n), hipdev.alloc(n)
        data = rng.integers(0, 256, size=n, dtype=np.uint8)
        hipdev.copyin(v, data)
        targets.append(t)
        values.append(v)
        want.append(data)
    for t, v in zip(targets, values):
        hipdev.commit(t, v)
    again = hipdev.alloc(sizes[3])
    later = rng.integers(0, 256, size=sizes[3], dtype=np.uint8)
    hipdev.copyin(again, later)
    hipdev.commit(targets[3], again)
    want[3] = later
    hipdev.finish()
    for t, w in zip(targets, want):
        np.testing.assert_array_equal(hipdev.copyout(t), w)


TRANSPOSED = {
    "bf16-cast-add": (lambda g, m: m * 0.9 + g.transpose().cast(float32) * 0.1, (300, 200), bfloat16),
    "batched-f32": (lambda g, m: g.transpose() * m, (3, 70, 130), float32),
    "outer-dims-swapped": (lambda g, m: g.permute(2, 1, 0) + m, (60, 3, 130), float32),
    "padded": (lambda g, m: g.transpose().pad(((1, 2), (0, 3))), (97, 180), float32),
    "optimizer-shape": (lambda g, m: m * 0.999 + (g.transpose().cast(float32) * g.transpose().cast(float32)) * 0.001, (1536, 512), bfloat16),
    "int32": (lambda g, m: g.transpose() * 3, (130, 129), int32),
}


@pytest.mark.parametrize("name", list(TRANSPOSED))
def test_reads_across_the_output_rows_go_by_tiles(hipdev, name):
    """Elementwise nests whose loads are contiguous along another variable than the output's
    (a gradient realized transposed, as an optimizer reads it): the plan stages those loads
    through LDS tiles (checked on the emitter's plan), and the values are numpy's: the copies
    bit for bit, the arithmetic to float32 rounding."""
    from limn_amd.hip import emit
    from limn_amd.seam import lower_all, schedule

    spell, out_shape, dtype = TRANSPOSED[name]
    src_shape = tuple(reversed(out_shape)) if name == "outer-dims-swapped" else out_shape[:-2] + out_shape[:-3:-1]
    if dtype is int32:
        g = Tensor(rng.integers(-1000, 1000, src_shape).astype(np.int32))
    else:
        g = Tensor(randf(*src_shape), dtype=dtype)
    m = Tensor(randf(*out_shape))
    y = spell(g, m)
    nodes = [y.node]
    order = topological(nodes)
    nests = lower_all(nodes, order, schedule(nodes, order))
    assert any(emit.plan_nest(n).notes.get("transposed") for n in nests)
    exact = name in ("padded", "int32")
    check(hipdev, y, bitwise=exact, rtol=1e-6, atol=1e-6)


def test_transposed_gradients_in_merged_optimizer_launches(hipdev):
    """Moments and parameters of several matrices whose gradients arrive transposed: the
    transposing members share merged launches (their LDS tiles from one pool), and every
    committed value matches numpy."""
    limn_device.active_device = hipdev
    shapes = [(200, 300), (96, 64), (512, 129)]
    ps = [Tensor(randf(*sh)) for sh in shapes]
    ms = [Tensor(randf(*sh)) for sh in shapes]
    g_raw = [randf(*sh[::-1]) for sh in shapes]
    gs = [Tensor(g, dtype=bfloat16) for g in g_raw]
    p_old, m_old = ([t.numpy().copy() for t in ts] for ts in (ps, ms))
    g_np = [storage_values(g, bfloat16) for g in g_raw]
    sinks = []
    for p, m, g in zip(ps, ms, gs):
        m_new = m * 0.9 + g.transpose().cast(float32) * 0.1
        m.assign(m_new)
        p.assign(p - m_new * 0.01)
        sinks += [m.node, p.node]
    bufs = hipdev.execute(sinks)
    for k in range(len(shapes)):
        want_m = m_old[k] * np.float32(0.9) + g_np[k].T * np.float32(0.1)
        got_m = hipdev.copyout(bufs[2 * k]).view(np.float32).reshape(shapes[k])
        got_p = hipdev.copyout(bufs[2 * k + 1]).view(np.float32).reshape(shapes[k])
        np.testing.assert_allclose(got_m, want_m, rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(got_p, p_old[k] - want_m * np.float32(0.01), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("batch,m,k,n,dtype", [(1, 64, 96, 256, bfloat16), (8, 64, 96, 256, bfloat16),
                                               (3, 50, 70, 36, bfloat16), (4, 64, 128, 192, float16)],
                         ids=["unbatched", "batched", "ragged", "float16"])
def test_matmul_forward_and_backward_in_limns_spelling(hipdev, batch, m, k, n, dtype):
    """x @ w.T for x (batch, m, k) and a weight w (n, k) shared over the batch, spelled as limn
    spells matmul: both operands broadcast to (batch, m, n, k), then a sum over k (reference
    limn/tensor.py:486-496, 806-812). The output and both gradients match the oracle's. For a
    batch above 1 the weight's gradient is a batched contraction and a sum over the batch, which
    the device runs as one contraction with the batch folded into k (checked on the recorded
    plan): it rounds to bfloat16 once where the oracle rounds every batch entry's product first,
    so the bound there is on the worst error over the largest magnitude. A ragged shape (rows not
    a multiple of 8) runs the products as ordinary reduces instead."""
    xd = rng.standard_normal((batch, m, k)).astype(np.float32)
    wd = rng.standard_normal((n, k)).astype(np.float32)
    x = Tensor(xd, dtype=dtype, requires_grad=True)
    w = Tensor(wd, dtype=dtype, requires_grad=True)
    y = x @ w.transpose()
    loss = (y.cast(float32) * Tensor(randf(batch, m, n))).sum()
    gx, gw = grad(loss, [x, w])
    check(hipdev, y, worst=1e-2)  # one bfloat16 rounding of sums taken in another order
    check(hipdev, gx, worst=1e-2)
    hipdev.record = []
    try:
        hipdev.execute([gw.node])
        plan = hipdev.record[0].plan
    finally:
        hipdev.record = None
    folded = [call.fn.folded for call in plan.calls if hasattr(call.fn, "folded")]
    if batch > 1 and m % 8 == 0:  # the MFMA contraction takes k in multiples of 8
        assert len(folded) == 1 and folded[0].batch == 1 and folded[0].K == batch * m
    check(hipdev, gw, worst=1e-2)


def test_optimizer_style_updates_in_merged_launches(hipdev):
    """Moments then parameters for several parameters, the way an optimizer step writes them:
    the device launches each group of independent updates as one kernel (checked through the
    recorded plan), and every committed value matches numpy."""
    limn_device.active_device = hipdev
    shapes = [(64,), (300, 7), (1000,), (48, 48)]
    ps = [Tensor(randf(*sh)) for sh in shapes]
    ms = [Tensor(randf(*sh)) for sh in shapes]
    gs = [Tensor(randf(*sh)) for sh in shapes]
    p_old, m_old, g_np = ([t.numpy().copy() for t in ts] for ts in (ps, ms, gs))
    sinks = []
    for p, m, g in zip(ps, ms, gs):
        m_new = m * 0.9 + g * 0.1
        m.assign(m_new)
        p.assign(p - m_new * 0.01)
        sinks += [m.node, p.node]
    hipdev.record = []
    bufs = hipdev.execute(sinks)
    plan = hipdev.record[0].plan
    hipdev.record = None
    assert sum(1 for call in plan.calls if getattr(call.fn, "launches_nothing", False)) >= 3
    for k in range(len(shapes)):
        want_m = m_old[k] * np.float32(0.9) + g_np[k] * np.float32(0.1)
        got_m = hipdev.copyout(bufs[2 * k]).view(np.float32).reshape(shapes[k])
        got_p = hipdev.copyout(bufs[2 * k + 1]).view(np.float32).reshape(shapes[k])
        np.testing.assert_allclose(got_m, want_m, rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(got_p, p_old[k] - want_m * np.float32(0.01), rtol=1e-6, atol=1e-6)


def test_independent_reduces_of_every_form_in_one_launch(hipdev):
    """Four independent row reductions, one of each single-launch form (a thread, a lane group, a
    wave and a workgroup per cell), share one merged launch and match the oracle."""
    xs = [Tensor(randf(100, 30)), Tensor(randf(200, 64)), Tensor(randf(50, 1000)), Tensor(randf(8, 5000))]
    sums = [x.sum(axis=1) for x in xs]
    assert launch_free_calls(hipdev, [t.node for t in sums]) == 3
    for t in sums:
        check(hipdev, t, rtol=1e-4, atol=1e-4)


def test_assigns_commit_after_every_call(hipdev):
    """A training-style batch: three tensors assigned from expressions that read all three; every
    read sees the old values (reference tests/test_compiled_devices.py:73-98), and the commits land
    through the batched copy."""
    limn_device.active_device = hipdev
    a = Tensor(np.arange(1000, dtype=np.float32))
    b = Tensor(np.arange(1000, dtype=np.float32) * 2.0, dtype=bfloat16)
    c = Tensor(np.full(70001, 3.0, dtype=np.float32))
    from limn_amd.dtypes import bf16_bits, bf16_values

    a_old = np.arange(1000, dtype=np.float32)
    b_old = bf16_values(bf16_bits(np.arange(1000, dtype=np.float32) * 2.0)).astype(np.float32)  # b is stored as bf16
    na, nb, nc = a + b.cast(float32), b * 2.0, c + a.sum()
    a.assign(na)
    b.assign(nb)
    c.assign(nc)
    got = [hipdev.copyout(buf) for buf in hipdev.execute([a.node, b.node, c.node])]
    from limn_amd.dtypes import from_storage

    np.testing.assert_allclose(got[0].view(np.float32), a_old + b_old)
    np.testing.assert_allclose(from_storage(got[1], bfloat16, (1000,)).astype(np.float32), b_old * 2.0, rtol=1e-2)
    np.testing.assert_allclose(got[2].view(np.float32), np.full(70001, 3.0 + a_old.sum(), np.float32), rtol=1e-5)


def test_one_plan_for_a_repeated_graph(hipdev):
    before = len(hipdev.plans)
    for _ in range(3):
        a, b = Tensor(randf(6, 6)), Tensor(randf(6, 6))
        hipdev.execute([((a + b) * 3.0).node])
    assert len(hipdev.plans) == before + 1


def test_a_changed_const_is_a_new_plan(hipdev):
    a = Tensor(randf(6, 6))
    before = len(hipdev.plans)
    hipdev.execute([(a * 3.0).node])
    hipdev.execute([(a * 4.0).node])
    assert len(hipdev.plans) == before + 2


# ---- attention through the Tensor API (the CUSTOM seam) ----


def _attention_grads(q_shape, k_shape, v_shape, causal, dtype=float32, live=None):
    data = [rng.standard_normal(s).astype(np.float32) for s in (q_shape, k_shape, v_shape)]
    out_shape = np.broadcast_shapes(q_shape[:-2], k_shape[:-2], v_shape[:-2]) + (q_shape[-2], v_shape[-1])
    w = rng.standard_normal(out_shape).astype(np.float32)
    q, k, v = (Tensor(d, dtype=dtype, requires_grad=True) for d in data)
    mask = None
    if live is not None:
        mask = Tensor(np.broadcast_to(np.arange(k_shape[-2]) < live, k_shape[:-1]).astype(np.float32))
    out = q.attention(k, v, causal=causal, key_mask=mask)
    return out, grad((out * Tensor(w, dtype=dtype)).sum(), [q, k, v])


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype,tol", [(float32, 1e-4), (float16, 4e-3), (bfloat16, 3e-2)], ids=str)
def test_attention_backward_through_the_tensor_api(hipdev, causal, dtype, tol):
    out, grads = _attention_grads((2, 3, 64, 16), (2, 3, 64, 16), (2, 3, 64, 24), causal, dtype)
    check(hipdev, out, rtol=tol, atol=tol)
    for g in grads:
        check(hipdev, g, rtol=tol, atol=tol)


def test_attention_backward_graph_is_custom(hipdev):
    out, grads = _attention_grads((2, 48, 8), (2, 48, 8), (2, 48, 12), True)
    nodes = topological([g.node for g in grads])
    names = {n.arg.name for n in nodes if n.op is Op.CUSTOM}
    assert names == {"sdpa", "sdpa_bwd_q", "sdpa_bwd_kv"}
    assert not [n for n in nodes if n.shape[-2:] == (48, 48)]


@pytest.mark.parametrize("shapes", [((1, 3, 16, 8), (4, 3, 16, 8), (4, 1, 16, 12)), ((40, 8), (72, 8), (72, 12))], ids=["broadcast", "rectangular"])
def test_attention_broadcast_and_rectangular(hipdev, shapes):
    out, grads = _attention_grads(*shapes, causal=False)
    check(hipdev, out)
    for g in grads:
        check(hipdev, g, rtol=1e-4, atol=1e-4)


def test_attention_key_mask_through_the_api(hipdev):
    out, grads = _attention_grads((2, 100, 16), (2, 100, 16), (2, 100, 16), True, live=66)
    check(hipdev, out)
    for g in grads:
        check(hipdev, g, rtol=1e-4, atol=1e-4)


def test_two_attentions_on_one_input(hipdev):
    q, k, v = (Tensor(randf(2, 3, 32, 8)) for _ in range(3))
    check(hipdev, q.attention(k, v, causal=True) + q.attention(k, v, causal=True))


def test_mfma_attention_through_the_api(hipdev):
    out, grads = _attention_grads((2, 4, 256, 64), (2, 4, 256, 64), (2, 4, 256, 64), True, bfloat16)
    check(hipdev, out, rtol=1e-2, atol=1e-2)
    for g in grads:
        check(hipdev, g, rtol=3e-2, atol=3e-2)


def test_config2_full_size(hipdev):
    """BASELINE config 2 at full size: x f32 (8192, 8192) from default_rng(2), row softmax then
    LayerNorm (gamma 1, beta 0, eps 1e-5). Rows are independent, so 16 sampled rows are diffed
    against the oracle run on just those rows; every row must be finite with mean ~ 0."""
    N = 8192
    x_host = np.random.default_rng(2).standard_normal((N, N), dtype=np.float32)

    def chain(x):
        w, b = Tensor.ones((N,)), Tensor.zeros((N,))
        y = x.softmax(-1)
        c = y - y.mean(axis=-1, keepdim=True)
        var = (c * c).mean(axis=-1, keepdim=True)
        return c / (var + 1e-5).sqrt() * w + b

    limn_device.active_device = hipdev
    out = chain(Tensor(x_host)).numpy()
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out.mean(axis=1), 0.0, atol=1e-6)
    rows = np.random.default_rng(0).choice(N, size=16, replace=False)
    limn_device.set_device("numpy")
    want = chain(Tensor(x_host[rows])).numpy()
    np.testing.assert_allclose(out[rows], want, rtol=1e-5, atol=1e-5)


# ---- dense contractions on matrix cores ----


def _plans(dev, t):
    """The emitter's plan for each nest of t's graph (which kernel family each nest got)."""
    from limn_amd.seam import lower_all
    from limn_amd.hip.emit import plan_nest

    return [plan_nest(n) for n in lower_all([t.node])]


@pytest.mark.parametrize(
    "a_shape,b_shape,ta,tb",
    [
        ((64, 32), (32, 48), False, False),
        ((100, 40), (40, 72), False, False),
        ((136, 208), (208, 264), False, False),
        ((40, 24), (40, 56), True, False),
        ((24, 64), (56, 64), False, True),
        ((64, 24), (56, 64), True, True),
        ((3, 33, 16), (3, 16, 40), False, False),
        ((4, 17, 32), (32, 24), False, False),
    ],
    ids=["square", "ragged", "multi-stage", "a-transposed", "b-transposed", "both-transposed", "batched", "broadcast"],
)
@pytest.mark.parametrize("dtype", [bfloat16, float16], ids=str)
def test_contraction_on_mfma(hipdev, a_shape, b_shape, ta, tb, dtype):
    a_data = rng.standard_normal(a_shape).astype(np.float32)
    b_data = rng.standard_normal(b_shape).astype(np.float32)
    a, b = Tensor(a_data, dtype=dtype), Tensor(b_data, dtype=dtype)
    if ta:
        a = a.transpose()
    if tb:
        b = b.transpose()
    out = a @ b
    assert any(p.contraction is not None for p in _plans(hipdev, out)), "the contraction did not reach the MFMA kernel"
    from limn_amd.dtypes import from_storage, to_storage

    got = from_storage(hipdev.copyout(hipdev.execute([out.node])[0]), dtype, out.shape).astype(np.float64)
    # the exact answer on the stored operand values (products are exact in f32; one rounding at
    # the store): the kernel may differ by accumulation order and that final rounding
    av = from_storage(to_storage(a_data, dtype).view(np.uint8), dtype, a_shape).astype(np.float64)
    bv = from_storage(to_storage(b_data, dtype).view(np.uint8), dtype, b_shape).astype(np.float64)
    av = np.swapaxes(av, -1, -2) if ta else av
    bv = np.swapaxes(bv, -1, -2) if tb else bv
    exact = av @ bv
    ulp = 2.0**-8 if dtype is bfloat16 else 2.0**-11
    np.testing.assert_allclose(got, exact, rtol=2 * ulp, atol=1e-3)
    # and the numpy oracle, which rounds every half-width product before summing: its error
    # grows like sqrt(K) rounding steps
    k = a.shape[-1]
    check(hipdev, out, rtol=2e-2, atol=4 * ulp * np.sqrt(k) * 2)


def test_contraction_falls_back_when_unaligned(hipdev):
    """K = 13 leaves 16-byte rows misaligned: the general reduce kernels take it."""
    a, b = Tensor(randf(20, 13), dtype=bfloat16), Tensor(randf(13, 9), dtype=bfloat16)
    out = a @ b
    assert all(p.contraction is None for p in _plans(hipdev, out))
    check(hipdev, out, rtol=2e-2, atol=5e-2)


def test_config3_full_size(hipdev):
    """bf16 A(4096x4096) @ B(4096x4096), f32 accumulate, relu, bf16 store.
    A, B ~ N(0, 0.125^2) from default_rng(3) (variance 1/sqrt(4096)). Checked against the f32
    closed form np.matmul on the same bf16 values, then relu and round to bf16."""
    from limn_amd.dtypes import bf16_bits, bf16_values

    n = 4096
    r = np.random.default_rng(3)
    a_vals = bf16_values(bf16_bits((r.standard_normal((n, n), dtype=np.float32) * 0.125)))
    b_vals = bf16_values(bf16_bits((r.standard_normal((n, n), dtype=np.float32) * 0.125)))
    limn_device.active_device = hipdev
    out = (Tensor(a_vals, dtype=bfloat16) @ Tensor(b_vals, dtype=bfloat16)).relu()
    assert any(p.contraction is not None for p in _plans(hipdev, out))
    got = out.numpy()
    want = bf16_values(bf16_bits(np.maximum(a_vals @ b_vals, 0.0)))
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("m,n,k", [(200, 72, 1024), (256, 128, 4096), (96, 40, 200)], ids=["dma", "split-k", "k-tail"])
def test_relu_epilogue_matches_the_separate_relu_bit_for_bit(hipdev, m, n, k):
    """(A @ B).relu() as one MFMA launch with a relu epilogue (the relu nest is the sum's only
    reader) against the same graph with the sum also a sink, which keeps the relu nest separate:
    rounding commutes with relu, so the bits agree. And both against the float64 closed form."""
    from limn_amd.dtypes import bf16_bits, bf16_values

    a_vals = bf16_values(bf16_bits(rng.standard_normal((m, k)).astype(np.float32)))
    b_vals = bf16_values(bf16_bits(rng.standard_normal((k, n)).astype(np.float32)))
    a, b = Tensor(a_vals, dtype=bfloat16), Tensor(b_vals, dtype=bfloat16)
    mm = a @ b
    relu = mm.relu()
    fused = hipdev.copyout(hipdev.execute([relu.node])[0]).view(np.uint16)
    total, separate = hipdev.execute([mm.node, relu.node])
    separate = hipdev.copyout(separate).view(np.uint16)
    np.testing.assert_array_equal(fused, separate)
    got = bf16_values(fused.reshape(m, n)).astype(np.float64)
    exact = np.maximum(a_vals.astype(np.float64) @ b_vals.astype(np.float64), 0.0)
    np.testing.assert_allclose(got, exact, rtol=2**-7, atol=1e-2 * np.sqrt(k / 1024))
    assert (got >= 0).all()


@pytest.mark.parametrize(
    "m,n,k,residual,dtype",
    [
        (200, 72, 1024, False, bfloat16),
        (200, 72, 1024, True, float16),
        (256, 128, 4096, True, bfloat16),
        (96, 40, 200, True, bfloat16),
        (300, 264, 512, False, bfloat16),
        (4160, 4096, 64, True, bfloat16),
        (200, 72, 1024, "cast", bfloat16),
        (256, 128, 4096, "cast", float16),
        (96, 40, 200, "cast", bfloat16),
    ],
    ids=["dma", "dma-f16-residual", "split-k", "k-tail", "ragged", "256-tile", "cast-bias", "cast-bias-split-k-f16",
         "cast-bias-k-tail"],
)
def test_bias_epilogue_matches_the_separate_add_bit_for_bit(hipdev, m, n, k, residual, dtype):
    """`a @ b + bias` and `res + (a @ b + bias)` as one launch of limn_hip_matmul_add (the add
    nest is the sum's only reader) against the same graph with the sum also a sink, which keeps
    the add nest separate: the sum rounded once, the terms added in float, one more rounding, so
    the bits agree. Every store path: the staged 16-byte rows, row tails, the register-staged
    kernel's element stores (k = 200) and the split-k fold; "cast": the bias a float32 vector cast
    to the operand type, which the epilogue rounds itself. And against the float64 closed form."""
    from limn_amd.dtypes import from_storage, to_storage
    from limn_amd.hip import emit
    from limn_amd.seam import lower_all, realized, schedule

    def vals(shape):
        x = rng.standard_normal(shape).astype(np.float32)
        return from_storage(to_storage(x, dtype).view(np.uint8), dtype, shape).astype(np.float64)

    a_v, b_v, bias_v, res_v = vals((m, k)), vals((k, n)), vals((n,)), vals((m, n))
    a, b = Tensor(a_v.astype(np.float32), dtype=dtype), Tensor(b_v.astype(np.float32), dtype=dtype)
    bias, res = Tensor(bias_v.astype(np.float32), dtype=dtype), Tensor(res_v.astype(np.float32), dtype=dtype)
    if residual == "cast":
        bias_f32 = rng.standard_normal(n).astype(np.float32)
        bias_v = from_storage(to_storage(bias_f32, dtype).view(np.uint8), dtype, (n,)).astype(np.float64)
        bias = Tensor(bias_f32, dtype=float32).cast(dtype)
        residual = False
    mm = a @ b
    out = res + (mm + bias) if residual else mm + bias
    nodes = [out.node]
    order = topological(nodes)
    nests = lower_all(nodes, order, schedule(nodes, order))
    _, addends, _ = emit.epilogue_pairs(nests, [emit.plan_nest(x) for x in nests], {realized(x) for x in nodes})
    assert addends, "the add did not become the contraction's epilogue"
    fused = hipdev.copyout(hipdev.execute([out.node])[0]).view(np.uint16)
    _, separate = hipdev.execute([mm.node, out.node])
    np.testing.assert_array_equal(fused, hipdev.copyout(separate).view(np.uint16))
    got = from_storage(fused.view(np.uint8), dtype, (m, n)).astype(np.float64)
    exact = a_v @ b_v + bias_v + (res_v if residual else 0.0)
    np.testing.assert_allclose(got, exact, rtol=2**-6, atol=2e-2 * np.sqrt(k / 1024) + 2e-2)


def test_weight_gradient_is_one_split_k_contraction(hipdev):
    """A weight gradient sums over batch and rows together (K = 8 * 512 = 4096) into a 256 x 128
    output. limn's matmul spelling makes it a product per batch entry and a sum over the batch;
    the device runs the two as one contraction with the batch folded into k, split in k (the
    output is two 128-tiles), its slices added in order. Checked against the float64 closed form
    on the same bf16 values and the float32 total rounded once at the store."""
    from limn_amd.dtypes import bf16_bits, bf16_values
    from limn_amd.hip import emit, runtime
    from limn_amd.seam import lower_all, realized

    B, T, C, O = 8, 512, 128, 256
    x_vals = bf16_values(bf16_bits(rng.standard_normal((B, T, C)).astype(np.float32)))
    dy_vals = bf16_values(bf16_bits(rng.standard_normal((B, T, O)).astype(np.float32)))
    limn_device.active_device = hipdev
    x, dy = Tensor(x_vals, dtype=bfloat16), Tensor(dy_vals, dtype=bfloat16)
    w = Tensor(np.zeros((O, C), np.float32), requires_grad=True)
    (gw,) = grad((x @ w.cast(bfloat16).transpose() * dy).sum(), [w])
    prog = emit.plan_program(lower_all([gw.node]), {realized(gw.node)}, set())
    cons = [p.contraction for p in prog.plans if p.contraction is not None] + list(prog.folds.values())
    wgrad = [c for c in cons if c.K == B * T]
    assert wgrad, f"no contraction over batch and rows: {[(c.M, c.N, c.K) for c in cons]}"
    c = wgrad[0]
    assert runtime.kernels().limn_hip_matmul_workspace(3, c.batch, c.M, c.N, c.K) > 0, "this shape should split k"
    got = gw.numpy().astype(np.float64)
    exact = np.einsum("bto,btc->oc", dy_vals.astype(np.float64), x_vals.astype(np.float64))
    np.testing.assert_allclose(got, exact, rtol=2**-7, atol=1e-2)


def test_split_k_without_workspace_runs_unsplit(hipdev):
    """The C ABI with no workspace for a shape that wants one: the same contraction, unsplit."""
    from limn_amd.dtypes import bf16_bits, bf16_values
    from limn_amd.hip import runtime

    M, N, K = 256, 128, 4096  # c[m, n] = sum_k a[m, k] b[k, n], a m-contiguous, b n-contiguous
    a_vals = bf16_values(bf16_bits(rng.standard_normal((K, M)).astype(np.float32)))
    b_vals = bf16_values(bf16_bits(rng.standard_normal((K, N)).astype(np.float32)))
    lib = runtime.kernels()
    ws_bytes = lib.limn_hip_matmul_workspace(3, 1, M, N, K)
    assert ws_bytes > 0
    a, b = hipdev.alloc(a_vals.size * 2), hipdev.alloc(b_vals.size * 2)
    hipdev.copyin(a, bf16_bits(a_vals))
    hipdev.copyin(b, bf16_bits(b_vals))
    outs = []
    for ws in (None, hipdev.alloc(ws_bytes)):
        c = hipdev.alloc(M * N * 2)
        runtime.check_limn(lib.limn_hip_matmul(a.ptr, b.ptr, c.ptr, 3, 1, M, N, K, 0, 1, M, 0, N, 1, 0, N, 1, 0,
                                               None if ws is None else ws.ptr, 0 if ws is None else ws_bytes, None))
        hipdev.finish()
        outs.append(bf16_values(hipdev.copyout(c).view(np.uint16).reshape(M, N)).astype(np.float64))
    exact = a_vals.astype(np.float64).T @ b_vals.astype(np.float64)
    for got in outs:
        np.testing.assert_allclose(got, exact, rtol=2**-7, atol=1e-2)


@pytest.mark.parametrize("a_kcontig", [True, False], ids=["a-k", "a-m"])
@pytest.mark.parametrize("b_kcontig", [True, False], ids=["b-k", "b-n"])
@pytest.mark.parametrize(
    "M,N,K,relu",
    [
        (256, 128, 4104, False),
        (200, 72, 1000, True),
        (520, 264, 72, False),
        (256, 128, 4096, False),
        (200, 72, 1024, True),
        (520, 264, 128, False),
        (4096, 4096, 64, True),
    ],
    ids=str,
)
def test_matmul_layouts_through_the_c_abi(hipdev, a_kcontig, b_kcontig, M, N, K, relu):
    """Every operand orientation through both kernels: k that ends mid-stage (4104 = 64 * 64 + 8,
    1000, 72) takes the register-staged kernel, k a multiple of 64 the DMA kernel; tiles that
    overhang m and n, 128- and 256-tiles, split (with a workspace) and unsplit, and the relu
    epilogue. Against the float64 product of the same bf16 values, rounded once."""
    from limn_amd.dtypes import bf16_bits, bf16_values
    from limn_amd.hip import runtime

    a_vals = bf16_values(bf16_bits(rng.standard_normal((M, K)).astype(np.float32)))
    b_vals = bf16_values(bf16_bits(rng.standard_normal((K, N)).astype(np.float32)))
    a_store = a_vals if a_kcontig else np.ascontiguousarray(a_vals.T)
    b_store = np.ascontiguousarray(b_vals.T) if b_kcontig else b_vals
    a_m, a_k = (K, 1) if a_kcontig else (1, M)
    b_k, b_n = (1, K) if b_kcontig else (N, 1)
    lib = runtime.kernels()
    a, b = hipdev.alloc(a_store.size * 2), hipdev.alloc(b_store.size * 2)
    hipdev.copyin(a, bf16_bits(a_store))
    hipdev.copyin(b, bf16_bits(b_store))
    ws_bytes = lib.limn_hip_matmul_workspace(3, 1, M, N, K)
    exact = a_vals.astype(np.float64) @ b_vals.astype(np.float64)
    if relu:
        exact = np.maximum(exact, 0.0)
    for ws in ([None, hipdev.alloc(ws_bytes)] if ws_bytes else [None]):
        c = hipdev.alloc(M * N * 2)
        runtime.check_limn(lib.limn_hip_matmul(a.ptr, b.ptr, c.ptr, 3, 1, M, N, K, 0, a_m, a_k, 0, b_k, b_n, 0, N, 1,
                                               1 if relu else 0, None if ws is None else ws.ptr,
                                               0 if ws is None else ws_bytes, None))
        hipdev.finish()
        got = bf16_values(hipdev.copyout(c).view(np.uint16).reshape(M, N)).astype(np.float64)
        np.testing.assert_allclose(got, exact, rtol=2**-7, atol=1e-2 * np.sqrt(K / 1024))


@pytest.mark.parametrize(
    "M,N,K,b_kcontig,layout",
    [
        (4160, 4096, 64, True, "rows"),
        (4160, 4096, 64, True, "rows+4"),
        (4160, 4096, 64, True, "rows+1"),
        (4160, 4100, 64, True, "rows"),
        (4160, 4096, 64, False, "columns"),
        (200, 72, 1024, False, "columns"),
        (304, 262, 8192, True, "rows"),
        (304, 264, 8192, False, "rows+4"),
    ],
    ids=str,
)
def test_matmul_output_layouts_through_the_c_abi(hipdev, M, N, K, b_kcontig, layout):
    """The store paths of the staged epilogue: 16-byte row stores ("rows", a 256-tile at 4160 x
    4096), 8-byte ones (an output 8 bytes past a 16-byte boundary, or rows of 4100), element
    stores (an odd element offset, a transposed output), row tails (N = 4100, 262), and the
    float32 partials of a split k with N % 4 != 0. Cells outside the output must stay as they
    were. Against the float64 product of the same bf16 values, rounded once."""
    from limn_amd.dtypes import bf16_bits, bf16_values
    from limn_amd.hip import runtime

    a_vals = bf16_values(bf16_bits(rng.standard_normal((M, K)).astype(np.float32)))
    b_vals = bf16_values(bf16_bits(rng.standard_normal((K, N)).astype(np.float32)))
    b_store = np.ascontiguousarray(b_vals.T) if b_kcontig else b_vals
    b_k, b_n = (1, K) if b_kcontig else (N, 1)
    lib = runtime.kernels()
    a, b = hipdev.alloc(a_vals.size * 2), hipdev.alloc(b_store.size * 2)
    hipdev.copyin(a, bf16_bits(a_vals))
    hipdev.copyin(b, bf16_bits(b_store))
    ws_bytes = lib.limn_hip_matmul_workspace(3, 1, M, N, K)
    ws = hipdev.alloc(ws_bytes) if ws_bytes else None
    offset = {"rows": 0, "rows+4": 4, "rows+1": 1, "columns": 0}[layout]
    c_m, c_n = (1, M) if layout == "columns" else (N, 1)
    sentinel = np.full(M * N + 16, 0x7FC1, np.uint16)  # a NaN no product rounds to
    c = hipdev.alloc(sentinel.size * 2)
    hipdev.copyin(c, sentinel)
    runtime.check_limn(lib.limn_hip_matmul(a.ptr, b.ptr, c.ptr + 2 * offset, 3, 1, M, N, K, 0, K, 1, 0, b_k, b_n, 0, c_m,
                                           c_n, 0, None if ws is None else ws.ptr, ws_bytes, None))
    hipdev.finish()
    raw = hipdev.copyout(c).view(np.uint16)
    assert (raw[:offset] == 0x7FC1).all() and (raw[offset + M * N:] == 0x7FC1).all(), "a store left the output"
    cells = raw[offset:offset + M * N]
    got = bf16_values(cells.reshape(N, M).T if layout == "columns" else cells.reshape(M, N)).astype(np.float64)
    exact = a_vals.astype(np.float64) @ b_vals.astype(np.float64)
    np.testing.assert_allclose(got, exact, rtol=2**-7, atol=1e-2 * np.sqrt(K / 1024))


@pytest.mark.parametrize("shape,dtype", [((8, 512, 96), float32), ((4, 300, 1536), bfloat16), ((2, 64, 200), float32)], ids=str)
def test_column_reduce_over_batch_and_rows(hipdev, shape, dtype):
    """A bias gradient's shape: (b, t, c) summed over b and t. 64 cells per workgroup, rows
    split into parts; a partial last tile (c % 64) and a single-part case (few rows) included."""
    x = Tensor(rng.standard_normal(shape).astype(np.float32), dtype=dtype)
    tol = 1e-5 if dtype is float32 else 2e-2
    # a column of N(0, 1) can total ~1 while its partial sums reach ~sqrt(rows): the error is
    # bounded relative to the largest total, not to each
    check(hipdev, x.sum(axis=(0, 1)), worst=tol)
    check(hipdev, (x * x).sum(axis=(0, 1), keepdim=True), worst=tol)


def test_column_max_keeps_nan(hipdev):
    x = rng.standard_normal((16, 128, 70)).astype(np.float32)
    x[3, 17, 5] = np.nan
    x[9, 100, 69] = np.nan
    check(hipdev, Tensor(x).max(axis=(0, 1)))


# row programs: a chain of row reductions and their readers in one launch (emit.row_chains)


def _softmax_layernorm(x: Tensor) -> Tensor:
    y = x.softmax(-1)
    c = y - y.mean(axis=-1, keepdim=True)
    return c / ((c * c).mean(axis=-1, keepdim=True) + 1e-5).sqrt()


def _layernorm(dtype, shape):
    from limn_amd.seam import nn

    def build(x):
        t = Tensor(x, dtype=dtype)
        return nn.LayerNorm(shape[-1])(t)

    return build


ROW_CASES = {
    # a workgroup per row (5000-wide rows), 70 rows
    "softmax_layernorm_wide": ((70, 5000), lambda x: _softmax_layernorm(Tensor(x))),
    # odd width: one value per vector chunk, a wave per row
    "softmax_layernorm_odd": ((33, 777), lambda x: _softmax_layernorm(Tensor(x))),
    "layernorm_bf16": ((100, 512), _layernorm(bfloat16, (100, 512))),
    # 16 lanes a row, four rows a wave; 103 rows leave a wave with rows past the end
    "layernorm_bf16_ragged": ((103, 512), _layernorm(bfloat16, (103, 512))),
    "layernorm_f16_3d": ((4, 50, 256), _layernorm(float16, (4, 50, 256))),
    # 160 chunks: four a lane over a whole wave
    "softmax_layernorm_640": ((45, 640), lambda x: _softmax_layernorm(Tensor(x))),
}


@pytest.mark.parametrize("case", sorted(ROW_CASES))
def test_row_programs_give_the_bits_of_separate_launches(hipdev, case):
    """The fused row program stores exactly what the same nests launched one by one store
    (same strided loops, vector widths and fold orders), and agrees with the numpy oracle."""
    from limn_amd.dtypes import from_storage
    from limn_amd.hip.device import HipDevice

    shape, build = ROW_CASES[case]
    x = randf(*shape)
    plain = HipDevice()
    plain.row_programs = False
    outs = []
    for dev in (hipdev, plain):
        t = build(x)
        outs.append(from_storage(dev.copyout(dev.execute([t.node])[0]), t.dtype, t.shape))
    got, want = (np.ascontiguousarray(o).reshape(-1) for o in outs)
    assert got.dtype == want.dtype and got.shape == want.shape
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), case
    half = case.startswith("layernorm")  # half-width x: every intermediate rounds to it
    check(hipdev, build(x), rtol=2e-2 if half else 1e-4, atol=2e-2 if half else 1e-4)
