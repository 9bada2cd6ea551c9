"""The hip device's plan-time decisions that need no GPU: which nests are dense contractions, and
when a relu nest may run as its contraction's epilogue (reference limn/tensor.py:365-366 spells
relu; the scheduler cuts after the SUM, limn/schedule.py:46-141, so the fusion is the device's to
make and only when nothing else reads the sum). The library is loaded for its layout check only;
no kernel runs."""

from __future__ import annotations

import math

import numpy as np
import pytest

from limn_amd.seam import bfloat16, float32, grad, lower_all, Op, realized, schedule, Tensor, topological
from limn_amd.seam import device as limn_device

emit = pytest.importorskip("limn_amd.hip.emit")

rng = np.random.default_rng(5)


@pytest.fixture(autouse=True)
def on_numpy():
    limn_device.set_device("numpy")
    yield


def lowered(sinks: list[Tensor]):
    nodes = [t.node for t in sinks]
    order = topological(nodes)
    nests = lower_all(nodes, order, schedule(nodes, order))
    kept = {realized(s) for s in nodes} | {realized(src) for n in order if n.op is Op.CUSTOM for src in n.srcs}
    return nests, kept


def operands(m: int = 64, k: int = 64, n: int = 48):
    a = Tensor(rng.standard_normal((m, k)).astype(np.float32), dtype=bfloat16)
    b = Tensor(rng.standard_normal((k, n)).astype(np.float32), dtype=bfloat16)
    return a, b


def pairs_of(sinks: list[Tensor]) -> dict[int, int]:
    nests, kept = lowered(sinks)
    return emit.epilogue_pairs(nests, [emit.plan_nest(n) for n in nests], kept)[0]


def addends_of(sinks: list[Tensor]) -> dict[int, tuple]:
    nests, kept = lowered(sinks)
    return emit.epilogue_pairs(nests, [emit.plan_nest(n) for n in nests], kept)[1]


def test_relu_nest_is_recognised():
    a, b = operands()
    nests, _ = lowered([(a @ b).relu()])
    assert [emit.is_relu(n) for n in nests] == [False, True]


@pytest.mark.parametrize(
    "spell",
    [lambda x: x * 2.0, lambda x: (x < 0).where(x, x * 0.0), lambda x: (x > 1).where(x, x * 0.0), lambda x: x.exp()],
    ids=["scale", "negative part", "threshold 1", "exp"],
)
def test_other_elementwise_nests_are_not_relu(spell):
    a, b = operands()
    nests, _ = lowered([spell(a @ b)])
    assert not emit.is_relu(nests[-1])


def test_relu_of_a_contraction_becomes_its_epilogue():
    a, b = operands()
    assert pairs_of([(a @ b).relu()]) == {0: 1}


def test_no_fusion_when_the_sum_is_also_a_sink():
    a, b = operands()
    mm = a @ b
    assert pairs_of([mm, mm.relu()]) == {}


def test_no_fusion_when_another_nest_reads_the_sum():
    a, b = operands()
    mm = a @ b
    assert pairs_of([mm.relu() + mm.exp()]) == {}


def test_no_fusion_when_a_custom_call_reads_the_sum():
    a, b = operands(64, 64, 64)
    mm = (a @ b).reshape(1, 64, 64)
    out = mm.relu().reshape(1, 64, 64).attention(mm, mm)
    nests, kept = lowered([out])
    plans = [emit.plan_nest(n) for n in nests]
    assert any(p.contraction is not None for p in plans)
    assert emit.epilogue_pairs(nests, plans, kept) == ({}, {}, {})


def test_no_fusion_without_a_record_of_readers():
    a, b = operands()
    nests, _ = lowered([(a @ b).relu()])
    assert emit.epilogue_pairs(nests, [emit.plan_nest(n) for n in nests], None) == ({}, {}, {})


def bias_operands(m: int = 64, k: int = 64, n: int = 48):
    a, b = operands(m, k, n)
    bias = Tensor(rng.standard_normal(n).astype(np.float32), dtype=bfloat16)
    res = Tensor(rng.standard_normal((m, n)).astype(np.float32), dtype=bfloat16)
    return a, b, bias, res


def test_bias_add_of_a_contraction_becomes_its_epilogue():
    """A Linear layer's `x @ w + b`: the add reads the sum at the cell it stores and the bias along
    the last axis, so it runs in the contraction's store (limn_hip_matmul_add)."""
    a, b, bias, _ = bias_operands()
    assert pairs_of([a @ b + bias]) == {0: 1}
    assert addends_of([a @ b + bias]) == {1: (1, None, None)}
    assert addends_of([bias + a @ b]) == {1: (0, None, None)}


def test_a_cast_bias_is_rounded_by_the_epilogue():
    """A bf16 bias cast from a float32 parameter (as the GPT's Linear layers make it): the cast
    nest, read only by the fused add, is absorbed (the epilogue rounds the float32 vector
    itself) and launches nothing; a cast something else also reads stays a nest."""
    a, b = operands()
    w = Tensor(rng.standard_normal(48).astype(np.float32), dtype=float32)
    nests, kept = lowered([a @ b + w.cast(bfloat16)])
    plans = [emit.plan_nest(n) for n in nests]
    pairs, addends, _ = emit.epilogue_pairs(nests, plans, kept)
    ((j, (bias, res, cast)),) = addends.items()
    assert cast is not None and nests[cast].kernel.target is nests[j].kernel.inputs[bias]
    prog = emit.plan_program(nests, kept, set())
    assert prog.role(cast) == "inlined" and not prog.plans[cast].launches
    wb = w.cast(bfloat16)
    nests, kept = lowered([a @ b + wb, wb * 2.0])
    _, addends, _ = emit.epilogue_pairs(nests, [emit.plan_nest(n) for n in nests], kept)
    assert [t[2] for t in addends.values()] == [None]


def test_residual_and_bias_add_becomes_the_epilogue():
    """The residual stream's `x + (h @ w + b)`: both terms join the store, the bias first."""
    a, b, bias, res = bias_operands()
    (terms,) = addends_of([res + (a @ b + bias)]).values()
    assert terms[1] is not None and terms[0] != terms[1]


@pytest.mark.parametrize(
    "spell",
    [
        lambda mm, bias, res: (res + mm) + bias,  # another association: another rounding
        lambda mm, bias, res: mm + res,  # no bias
        lambda mm, bias, res: mm * bias,  # not an add
        lambda mm, bias, res: mm + bias.reshape(1, 48).cast(float32).cast(bfloat16) + bias,  # three terms
        lambda mm, bias, res: (mm + bias).cast(float32),  # stored at another width
    ],
    ids=["residual-first", "residual-only", "scale", "two-biases", "wider"],
)
def test_other_adds_are_not_epilogues(spell):
    a, b, bias, res = bias_operands()
    assert addends_of([spell(a @ b, bias, res)]) == {}


def test_a_bias_along_the_rows_is_not_an_epilogue():
    """bias[m] (a column vector) is not the n-vector the epilogue adds."""
    a, b, _, _ = bias_operands()
    col = Tensor(rng.standard_normal((64, 1)).astype(np.float32), dtype=bfloat16)
    assert addends_of([a @ b + col]) == {}


def test_float32_sum_is_not_a_contraction():
    a = Tensor(rng.standard_normal((64, 64)).astype(np.float32), dtype=float32)
    nests, _ = lowered([(a @ a).relu()])
    assert all(emit.plan_nest(n).contraction is None for n in nests)


def inlined_of(sinks: list[Tensor], kept_override=None) -> tuple[list, set[int]]:
    nests, kept = lowered(sinks)
    plans = [emit.plan_nest(n) for n in nests]
    pairs = emit.epilogue_pairs(nests, plans, kept)[0]
    return nests, emit.inline_producers(nests, plans, kept if kept_override is None else kept_override(kept), pairs)


def softmax_layernorm(n: int = 64) -> Tensor:
    x = Tensor(rng.standard_normal((n, n)).astype(np.float32))
    y = x.softmax(-1)
    c = y - y.mean(axis=-1, keepdim=True)
    return c / ((c * c).mean(axis=-1, keepdim=True) + 1e-5).sqrt()


def test_broadcast_producers_of_softmax_layernorm_are_inlined():
    """The scheduler's 11 kernels (reference limn/schedule.py:46-141): the six per-row and scalar
    ones (NEG max, 1/sum, 1/n twice, NEG mean, 1/sqrt(var + eps)) run inside their readers."""
    nests, chosen = inlined_of([softmax_layernorm()])
    assert len(nests) == 11
    assert sorted(math.prod(nests[j].kernel.target.shape) for j in chosen) == [1, 1, 64, 64, 64, 64]
    assert all(emit.plan_nest(nests[j]).notes.get("elementwise") for j in chosen)


def test_a_kept_producer_is_not_inlined():
    x = Tensor(rng.standard_normal((8, 8)).astype(np.float32))
    neg = -x.max(axis=1, keepdim=True)
    out = (x + neg).exp()
    nests, chosen = inlined_of([out, neg])
    assert not any(nests[j].kernel.target is realized(neg.node) for j in chosen)
    nests, chosen = inlined_of([out])
    assert any(nests[j].kernel.target is realized(neg.node) for j in chosen)


def test_a_producer_read_by_a_contraction_runs():
    """The MFMA kernel reads its operands from memory, so a computed operand must be stored."""
    a, b = operands(64, 64, 64)
    scaled = a * 2.0
    nests, chosen = inlined_of([scaled @ b])
    plans = [emit.plan_nest(n) for n in nests]
    producer = [j for j, n in enumerate(nests) if n.kernel.target is realized(scaled.node)]
    assert len(producer) == 1 and any(p.contraction is not None for p in plans)
    assert chosen == set()


def test_a_gathered_table_is_not_inlined():
    table = Tensor(rng.standard_normal((16, 4)).astype(np.float32)) * 3.0
    idx = Tensor(rng.integers(0, 16, size=(5,)).astype(np.int32))
    _, chosen = inlined_of([table.gather_rows(idx)])
    assert chosen == set()


def test_nothing_is_inlined_without_a_record_of_readers():
    nests, _ = lowered([softmax_layernorm()])
    plans = [emit.plan_nest(n) for n in nests]
    assert emit.inline_producers(nests, plans, None, {}) == set()


def test_a_reader_of_an_inlined_producer_takes_its_inputs_as_parameters():
    nests, chosen = inlined_of([softmax_layernorm()])
    inl = emit.InlineSet(nests, chosen)
    last = nests[-1]
    plan = emit.plan_nest(last, inl)
    header = plan.source.split("{", 1)[0]
    for j, m in inl.extras(last):
        assert f"p{j}_in{m}" in header
    # every load of an inlined producer's output became an evaluation of its body
    inlined_inputs = {f"in{k}" for k, n in enumerate(last.kernel.inputs) if n in inl.by_target}
    assert inlined_inputs and not any(f"{name}[" in plan.source for name in inlined_inputs)


def test_short_rows_take_a_group_of_lanes_per_cell():
    """A 64-element bf16 row is 8 runs of 8: 8 lanes fold it, 8 rows per wave."""
    a = Tensor(rng.standard_normal((8, 300, 64)).astype(np.float32), dtype=bfloat16)
    nests, _ = lowered([a.cast(float32).sum(axis=-1)])
    plan = emit.plan_nest(nests[-1])
    assert plan.notes["group"] == 8 and plan.notes["vec"] == 8
    assert "__shfl_xor(acc, 4)" in plan.source and "__shfl_xor(acc, 8)" not in plan.source


def test_a_load_masked_by_an_outer_dim_reads_whole_runs():
    parts = [Tensor(rng.standard_normal((1, 6, 40)).astype(np.float32), dtype=bfloat16) for _ in range(3)]
    stacked = parts[0].pad(((0, 2), (0, 0), (0, 0))) + parts[1].pad(((1, 1), (0, 0), (0, 0))) + parts[2].pad(((2, 0), (0, 0), (0, 0)))
    nests, _ = lowered([stacked])
    source = emit.plan_nest(nests[-1]).source
    assert source.count("_ok ?") == 6 and source.count("_raw = ") == 3 and "out_p[j_] = " in source
    # a pad along the stride-1 dim keeps the per-element form for the load
    inner = Tensor(rng.standard_normal((6, 40)).astype(np.float32)).pad(((0, 0), (4, 4)))
    nests, _ = lowered([inner * 2.0])
    source = emit.plan_nest(nests[-1]).source
    assert "_raw" not in source and "in0[" in source


def runs_of(sinks: list[Tensor]):
    nodes = [t.node for t in sinks]
    order = topological(nodes)
    nests = lower_all(nodes, order, schedule(nodes, order))
    custom = {realized(src) for n in order if n.op is Op.CUSTOM for src in n.srcs}
    kept = {realized(s) for s in nodes} | custom
    plans = [emit.plan_nest(n) for n in nests]
    pairs = emit.epilogue_pairs(nests, plans, kept)[0]
    inl = emit.InlineSet(nests, emit.inline_producers(nests, plans, kept, pairs))
    return nests, emit.merge_runs(nests, plans, custom, inl, pairs)[0]


def test_independent_small_updates_share_a_launch():
    """Moment updates of several parameters (as an optimizer step writes them): each reads only
    old state and the gradient, so they form one group; an update that reads a new moment
    starts a new group."""
    params = [Tensor(rng.standard_normal((64,)).astype(np.float32)) for _ in range(3)]
    grads = [Tensor(rng.standard_normal((64,)).astype(np.float32)) for _ in range(3)]
    m = [p * 0.9 + g * 0.1 for p, g in zip(params, grads)]
    nests, runs = runs_of(m)
    assert [len(r) for r in runs] == [3]
    newer = m[0] * 2.0 + 1.0  # reads a group member's output
    nests, runs = runs_of(m + [newer])
    members = {nests[c].kernel.target for r in runs for c in r}
    assert realized(m[0].node) in members and all(
        not (set(nests[c].kernel.inputs) & {nests[d].kernel.target for d in r}) for r in runs for c in r
    )


def test_an_optimizer_step_groups_across_parameters():
    """Each parameter's moments read only old state and the gradient; its update reads the new
    moments. The moments of every parameter share a group and the updates a later one, which
    launches after the moments' group (as a run of consecutive nests, a launch per parameter)."""
    n = 6
    params = [Tensor(rng.standard_normal((64,)).astype(np.float32)) for _ in range(n)]
    grads = [Tensor(rng.standard_normal((64,)).astype(np.float32)) for _ in range(n)]
    moms = [Tensor(rng.standard_normal((64,)).astype(np.float32)) for _ in range(n)]
    sinks = []
    for p, g, m in zip(params, grads, moms):
        m_new = m * 0.9 + g * 0.1
        sinks += [m_new, p - m_new * 0.01]
    nodes = [t.node for t in sinks]
    order = topological(nodes)
    nests = lower_all(nodes, order, schedule(nodes, order))
    kept = {realized(s) for s in nodes}
    prog = emit.plan_program(nests, kept, set())
    runs = {key: run for key, (run, _) in prog.merged.items()}
    assert len(runs) == 2
    made = {nests[c].kernel.target: key for key, run in runs.items() for c in run}
    first, second = runs
    assert all(made.get(src) != second for c in runs[first] for src in nests[c].kernel.inputs)
    assert any(made.get(src) == first for c in runs[second] for src in nests[c].kernel.inputs)
    assert prog.launcher_of(first) < prog.launcher_of(second) or (
        prog.launcher_of(first) == prog.launcher_of(second) and list(prog.launches_from(prog.launcher_of(first))) == [first, second])
    # every nest of the plan is a member of one of the two groups, launched by two runners
    assert sorted(c for run in runs.values() for c in run) == list(range(len(nests)))
    assert sum(len(prog.launches_from(k)) for k in range(len(nests))) == 2


def test_nothing_merges_without_a_record_of_custom_inputs():
    params = [Tensor(rng.standard_normal((64,)).astype(np.float32)) for _ in range(2)]
    nests, _ = lowered([p * 2.0 for p in params])
    plans = [emit.plan_nest(n) for n in nests]
    assert emit.merge_runs(nests, plans, None, emit.InlineSet(nests, set()), {}) == ([], [])


def test_merged_kernel_binds_each_members_buffers():
    params = [Tensor(rng.standard_normal((64,)).astype(np.float32)) for _ in range(2)]
    sinks = [p * 2.0 for p in params]
    nests, runs = runs_of(sinks)
    plans = [emit.plan_nest(n) for n in nests]
    source, grid = emit.merged_source("merged", nests, plans, runs[0])
    assert grid == sum(plans[c].launches[0].grid for c in runs[0])
    assert "s0_in0" in source and "s1_out" in source and source.count("const i64 bid_") == 2


def test_a_read_across_the_output_rows_is_planned_by_tiles():
    """A gradient realized transposed, read by an optimizer's update: the load is contiguous
    along the output's row variable, so the nest goes by LDS tiles; a nest reading along the
    output's rows keeps the plain plan. Both compile (hipRTC needs no GPU)."""
    from limn_amd.hip import runtime

    g = Tensor(rng.standard_normal((200, 300)).astype(np.float32), dtype=bfloat16)
    m = Tensor(rng.standard_normal((300, 200)).astype(np.float32))
    nests, _ = lowered([m * 0.9 + g.transpose().cast(float32) * 0.1])
    tiled = emit.plan_nest(nests[0])
    assert tiled.notes.get("transposed") == "i0" and tiled.launches[0].grid == 4 * 5
    assert "__syncthreads" in tiled.source and "xt_" in tiled.source
    runtime.compile_source(emit.PRELUDE + tiled.source, [tiled.launches[0].name])
    nests, _ = lowered([m * 0.9 + g.transpose().transpose().transpose().cast(float32)])
    assert emit.plan_nest(nests[0]).notes.get("transposed") == "i0"
    nests, _ = lowered([m * 2.0 + 1.0])
    assert "transposed" not in emit.plan_nest(nests[0]).notes


def test_small_or_narrow_transposes_keep_the_plain_plan():
    """Below TRANSPOSE_MIN_CELLS cells, or with a side under 16, a tile would be mostly empty."""
    small = Tensor(rng.standard_normal((20, 30)).astype(np.float32))
    narrow = Tensor(rng.standard_normal((8, 4000)).astype(np.float32))
    for t in (small, narrow):
        nests, _ = lowered([t.transpose() * 2.0])
        assert "transposed" not in emit.plan_nest(nests[0]).notes


def test_transposing_members_of_a_merged_launch_share_one_lds_pool():
    """Moment updates of three matrices whose gradients arrive transposed merge into one launch;
    each member's tile becomes a pointer into the kernel's one LDS array, sized for the largest
    member, and the merged kernel compiles."""
    from limn_amd.hip import runtime

    shapes = [(200, 300), (96, 640), (512, 129)]
    moms = [Tensor(rng.standard_normal(sh).astype(np.float32)) for sh in shapes]
    grads = [Tensor(rng.standard_normal(sh[::-1]).astype(np.float32), dtype=bfloat16) for sh in shapes]
    nests, runs = runs_of([m * 0.9 + g.transpose().cast(float32) * 0.1 for m, g in zip(moms, grads)])
    assert [len(r) for r in runs] == [3]
    plans = [emit.plan_nest(n) for n in nests]
    assert all(plans[c].notes.get("transposed") for c in runs[0])
    source, grid = emit.merged_source("merged", nests, plans, runs[0])
    assert source.count("__shared__") == 1 and source.count("(mshared_ + 0)") == 3
    assert f"char mshared_[{64 * 65 * 2}]" in source
    runtime.compile_source(emit.PRELUDE + source, ["merged"])


def test_limn_spelled_weight_gradient_folds_the_batch_into_k():
    """limn's matmul broadcasts both operands to (batch, m, n, k) and sums k (reference
    limn/tensor.py:486-496). The gradient of a weight shared over the batch is then a batched
    contraction, a product per batch entry, and a sum over the batch: the emitter runs the two as
    one contraction with the batch folded into k, launched by the sum's runner (the batched
    products are never stored), and the optimizer-side read of that gradient, transposed, goes
    by tiles."""
    x = Tensor(rng.standard_normal((8, 64, 96)).astype(np.float32), dtype=bfloat16, requires_grad=True)
    w = Tensor(rng.standard_normal((256, 96)).astype(np.float32), dtype=bfloat16, requires_grad=True)
    y = x @ w.transpose()
    loss = (y.cast(float32) * Tensor(rng.standard_normal((8, 64, 256)).astype(np.float32))).sum()
    gx, gw = grad(loss, [x, w])
    update = Tensor(np.zeros((256, 96), np.float32)) * 0.9 + gw.cast(float32) * 0.1
    nests, kept = lowered([gx, update])
    prog = emit.plan_program(nests, kept, set())
    assert len(prog.folds) == 1
    (k, folded), = prog.folds.items()
    batched = next(c for c, j in prog.pairs.items() if j == k)
    assert prog.plans[batched].contraction.batch == 8
    assert folded.batch == 1 and folded.K == 8 * 64 and {folded.M, folded.N} == {96, 256}
    assert prog.role(batched) == "stash" and prog.role(k) == "epilogue"
    assert prog.plans[k].notes.get("batch folded into k")
    assert any(p.notes.get("transposed") for p in prog.plans)


def test_a_large_sink_streams_its_stores():
    """An output of STREAM_BYTES or more that no later nest reads is written non-temporally; a
    read-again output and a small sink keep plain stores."""
    n = 4096  # 4096 x 4096 float32 = 64 MiB
    x = Tensor(np.zeros((n, n), np.float32))
    doubled = x * 2.0
    out = (doubled + 1.0).relu()
    small = (Tensor(np.zeros((8, 8), np.float32)) * 3.0)
    nests, kept = lowered([out, doubled, small])
    streamed = emit.streamed_outputs(nests, kept, set())
    names = {nests[k].kernel.target for k in streamed}
    assert names == {realized(out.node)}
    prog = emit.plan_program(nests, kept, set())
    sources = {nests[k].kernel.target: prog.plans[k].source for k in range(len(nests))}
    assert "__builtin_nontemporal_store" in sources[realized(out.node)]
    assert "__builtin_nontemporal_store" not in sources[realized(doubled.node)]
    assert "__builtin_nontemporal_store" not in sources[realized(small.node)]
    assert emit.streamed_outputs(nests, None, None) == set()


# ---- row programs ----


def test_softmax_layernorm_is_one_row_program():
    """The five launching nests of a row softmax then LayerNorm (max, sum of exp, mean, sum of
    squares, the final pass) run as one row program; a workgroup per row at 4096-wide rows, a
    wave per row at 2048, a group of 32 lanes per row (two rows a wave) at 512."""
    for n, group in ((4096, emit.THREADS), (2048, 64), (512, 32)):
        nests, kept = lowered([softmax_layernorm(n)])
        prog = emit.plan_program(nests, kept, set())
        assert len(prog.names) == 1 and "_rows_" in prog.names[0]
        (run, _), = prog.merged.values()
        assert [nests[c].kernel.ast.op for c in run][:4] == [Op.MAX, Op.SUM, Op.SUM, Op.SUM] and len(run) == 5
        members = [emit.row_member(nests[c], prog.plans[c]) for c in run]
        assert [m.kind for m in members] == ["reduce"] * 4 + ["cells"]
        assert {m.group for m in members if m.kind == "reduce"} == {group}
        assert "rv0_" in prog.source  # later members read the row max from a register
        assert emit.plan_program(nests, kept, set(), rows=False).names != prog.names


def test_a_bfloat16_layernorm_is_one_row_program():
    from limn_amd.seam import nn
    x = Tensor(rng.standard_normal((64, 512)).astype(np.float32), dtype=bfloat16)
    nests, kept = lowered([nn.LayerNorm(512)(x)])
    prog = emit.plan_program(nests, kept, set())
    assert len(prog.names) == 1 and "_rows_" in prog.names[0]
    assert "f2b(rv0_)" in prog.source  # the mean is read back rounded as its bf16 store rounds it


def test_a_read_of_another_row_ends_the_row_program():
    """A nest reading the row statistics along its columns (a transposed broadcast) cannot be a
    member: the program ends before it and it launches on its own."""
    n = 512
    x = Tensor(rng.standard_normal((n, n)).astype(np.float32))
    s = x.max(axis=-1, keepdim=True)
    y = (x - s).exp().sum(axis=-1, keepdim=True)
    z = x * y.reshape(1, n)
    nests, kept = lowered([z])
    prog = emit.plan_program(nests, kept, set())
    runs = [run for run, _ in prog.merged.values()]
    target = realized(z.node)
    assert all(nests[c].kernel.target is not target for run in runs for c in run)
    assert any(len(run) == 2 for run in runs)  # max and sum still share a row program


def test_row_program_members_read_a_shared_input_through_one_pointer():
    """Members of a row program that read the same buffer (a LayerNorm backward's members all
    read dy and gamma) bind it from the first member's parameter, so the compiler sees one
    pointer and shares the loads and the arithmetic on them; every member keeps its own
    parameter in the signature, so the launch's arguments do not change."""
    from limn_amd.seam import grad, nn
    x = Tensor(rng.standard_normal((64, 512)).astype(np.float32), dtype=bfloat16, requires_grad=True)
    ln = nn.LayerNorm(512)
    (gx,) = grad((ln(x).cast(float32) * Tensor(rng.standard_normal((64, 512)).astype(np.float32))).sum(), [x])
    nests, kept = lowered([gx])
    prog = emit.plan_program(nests, kept, set())
    rows = [(run, launch) for run, launch in prog.merged.values() if "_rows_" in launch.name]
    assert rows
    shared = 0
    for run, launch in rows:
        src = prog.source[prog.source.index(f"void {launch.name}("):]
        end = src.find('extern "C"')
        src = src if end < 0 else src[:end]
        signature = src[: src.index(") {")]
        first: dict = {}
        for c_s, c in enumerate(run):
            for k, node in enumerate(nests[c].kernel.inputs):
                assert f"s{c_s}_in{k}" in signature  # the parameter stays
                if node in first and first[node][0] != c_s:
                    shared += 1
                    assert f"__builtin_assume_aligned(s{c_s}_in{k}, 16)" not in src, (launch.name, c_s, k)
                first.setdefault(node, (c_s, k))
    assert shared > 0, "no member of the program shares an input"


def test_a_row_program_never_caches_an_inlined_producer():
    """A small producer evaluated where it is read (a materialized x * 2 + a broadcast row, as the
    GPT's embedding sum) feeding a LayerNorm: its output buffer is never written, so the row
    program evaluates it in place instead of loading the row into registers from that buffer."""
    from limn_amd.seam import nn
    x = Tensor(rng.standard_normal((64, 128)).astype(np.float32))
    pos = Tensor(rng.standard_normal((128,)).astype(np.float32))
    from limn_amd.gpt import materialized
    nests, kept = lowered([nn.LayerNorm(128)(materialized(x * 2.0 + pos))])
    prog = emit.plan_program(nests, kept, set())
    rows = [(run, launch) for run, launch in prog.merged.values() if "_rows_" in launch.name]
    assert rows, "the LayerNorm runs as a row program"
    run, launch = rows[0]
    inlined = {nests[j].kernel.target for j in prog.inlined.producers}
    assert any(n in inlined for c in run for n in nests[c].kernel.inputs)
    src = prog.source[prog.source.index(f"void {launch.name}("):]
    for c_s, c in enumerate(run):
        for k, node in enumerate(nests[c].kernel.inputs):
            if node in inlined:  # no register row is filled from the producer's buffer
                assert f"__builtin_assume_aligned(s{c_s}_in{k}, 16) + row_" not in src
