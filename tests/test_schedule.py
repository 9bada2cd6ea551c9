"""The scheduler and loop-nest IR the device is handed, pinned to the reference's own figures.

- The printed IR of a 4x5 @ 5x3 matmul equals the dump in the reference's README.md:172-195
  (tests/golden/ir_dump_matmul.txt), byte for byte.
- A training step through fused attention holds 30 MiB of intermediates at any context length,
  the composed form 229 MiB at T=256 and 3.1 GiB at T=4096: the figures of the reference's
  README.md:126-129, computed as its examples/bench_attention.py:64-70 computes them (the bytes
  every scheduled kernel writes), 6 heads of 32, 8192 tokens, float32.
- Where the graph is cut and how each nest is ordered: the properties the reference's
  tests/test_schedule.py:144-331 asserts, restated.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

from limn_amd.seam import Op, Opcode, Tensor, Valid, codegen, grad, int32, lower_all, realized, schedule, schedule_module, tensor
from limn_amd.seam import device as limn_device
from oracle.numpy_device import NumpyDevice

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(autouse=True)
def on_numpy():
    limn_device.active_device = NumpyDevice()


def randf(*shape: int) -> np.ndarray:
    return np.random.default_rng(sum(shape)).standard_normal(shape).astype(np.float32)


def nbytes(node) -> int:
    return node.dtype.itemsize * math.prod(node.shape)


# ---- golden figures ----


def test_matmul_ir_matches_the_readme_dump():
    text = codegen.ir(Tensor.randn((4, 5)) @ Tensor.randn((5, 3)))
    assert text.rstrip("\n") == (GOLDEN / "ir_dump_matmul.txt").read_text().rstrip("\n")


@pytest.mark.parametrize("t", [256, 1024, 4096])
def test_attention_training_working_set(t):
    heads, hd, tokens = 6, 32, 8192

    def held(fused: bool) -> float:
        shape = (max(1, tokens // t), heads, t, hd)
        args = [Tensor(np.zeros(shape, np.float32), requires_grad=True) for _ in range(3)]
        q, k, v = args
        out = q.attention(k, v, causal=True) if fused else tensor.composed_attention(q, k, v, causal=True, scale=hd**-0.5)
        grads = grad((out * out).sum(), args)
        return sum(nbytes(kernel.target) for kernel in schedule([g.node for g in grads])) / 2**20

    assert round(held(True)) == 30
    if t == 256:
        assert round(held(False)) == 229
    if t == 4096:
        assert round(held(False) / 1024, 1) == 3.1


# ---- cuts ----


def test_an_elementwise_chain_is_one_kernel_with_literal_constants():
    a, b = Tensor(randf(2, 3)), Tensor(randf(2, 3))
    kernels = schedule([((a + b) * 2.0).relu().node])
    assert len(kernels) == 1 and set(kernels[0].inputs) == {a.node, b.node}


def test_a_value_used_twice_in_a_nest_is_computed_once():
    a, b = Tensor(randf(2, 3)), Tensor(randf(2, 3))
    p = a * b
    (nest,) = lower_all([(p + p).node])
    assert [i.arg for i in nest.instrs if i.opcode is Opcode.ARITH].count(Op.MUL) == 1


def test_a_reduce_ends_its_kernel_with_the_elementwise_work_fused_in():
    a, b = Tensor(randf(2, 3)), Tensor(randf(2, 3))
    (kernel,) = schedule([(a + b).sum(axis=1, keepdim=True).node])
    assert kernel.ast.op is Op.SUM and kernel.body[-1].op is Op.SUM and any(n.op is Op.ADD for n in kernel.body)


def test_a_matmul_is_one_reduce_nest_over_the_whole_space():
    a, b = Tensor(randf(4, 5)), Tensor(randf(5, 3))
    m = a @ b
    (nest,) = lower_all([m.node])
    assert nest.kernel.ast.op is Op.SUM and nest.space == (4, 3, 5)
    assert nest.kernel.inputs == (a.node, b.node)
    assert realized(m.node) is nest.kernel.target


def test_a_view_of_a_computed_value_is_a_cut():
    a, b = Tensor(randf(2, 3)), Tensor(randf(2, 3))
    kernels = schedule([((a + b).reshape(6) * 2.0).node])
    assert [k.ast.op for k in kernels] == [Op.ADD, Op.MUL] and kernels[1].inputs == (kernels[0].ast,)


def test_a_copy_to_row_major_is_its_own_kernel():
    a = Tensor(randf(3, 4))
    kernels = schedule([a.transpose().reshape(12).node])
    assert [k.ast.op for k in kernels] == [Op.CONTIGUOUS] and kernels[0].inputs == (a.node,)


def test_a_reshape_of_realized_bytes_schedules_nothing():
    a = Tensor(randf(2, 3))
    r = a.reshape(6)
    assert schedule_module.is_alias(r.node) and realized(r.node) is a.node and schedule([r.node]) == []


def test_a_trailing_reshape_aliases_the_reduce_buffer():
    a, b = Tensor(randf(2, 3)), Tensor(randf(2, 3))
    s = (a + b).sum(axis=1)
    (kernel,) = schedule([s.node])
    assert kernel.ast.op is Op.SUM and realized(s.node) is kernel.target


def test_a_dense_slab_reshape_fuses_into_its_reader():
    a = Tensor(randf(8, 4))
    out = a.shrink(((2, 6), (0, 4))).reshape(16) * 2.0
    assert [k.ast.op for k in schedule([out.node])] == [Op.MUL]
    np.testing.assert_allclose(out.numpy(), a.numpy()[2:6].reshape(16) * 2.0, atol=1e-6)


def test_a_view_that_moves_bytes_still_copies():
    a = Tensor(randf(3, 4))
    for moved in (a.transpose(), a.pad(((1, 0), (0, 0))), a.shrink(((0, 2), (0, 4)))):
        assert not schedule_module.is_alias(moved.node)
        assert [k.ast.op for k in schedule([moved.node])] == [Op.VIEW]


def test_an_assign_writes_the_buffer_it_reads():
    p = Tensor(np.zeros((2, 2), np.float32))
    home = p.node
    p.assign(p * 2.0 + 1.0)
    (kernel,) = schedule([p.node])
    assert kernel.ast.op is Op.ASSIGN and kernel.target is home and home in kernel.inputs
    assert realized(p.node) is home


def test_constants_get_no_buffer():
    a = Tensor(randf(2, 3))
    kernels = schedule([(a * 2.0 + 1.0).relu().node])
    assert all(k.target.op is not Op.CONST and all(n.op is not Op.CONST for n in k.inputs) for k in kernels)


def test_kernels_come_after_everything_they_read():
    x, w = Tensor(randf(4, 5), requires_grad=True), Tensor(randf(5, 3), requires_grad=True)
    loss = (x @ w).relu().sum()
    loss.backward()
    kernels = schedule([loss.node, x.grad.node, w.grad.node])
    assert len(kernels) > 3
    written = set()
    for k in kernels:
        assert all(n.op is Op.BUFFER or n in written for n in k.inputs)
        written.add(k.target)


def test_a_shared_reduce_is_scheduled_once():
    a, b = Tensor(randf(2, 3)), Tensor(randf(2, 3))
    s = (a + b).sum(axis=1, keepdim=True)
    kernels = schedule([(s * 2.0).node, (s * 3.0).node])
    assert [k.ast.op for k in kernels].count(Op.SUM) == 1


# ---- loop order and reduce forms ----


def loop_vars(instrs) -> list[list[str]]:
    """Each top-level nest's loop variables, outermost first; the loops must balance."""
    groups, open_ = [], []
    for i in instrs:
        if i.opcode is Opcode.LOOP:
            if not open_:
                groups.append([])
            groups[-1].append(i.dest)
            open_.append(i.dest)
        elif i.opcode is Opcode.ENDLOOP:
            assert open_.pop() == i.arg
    assert not open_
    return groups


def test_a_folding_reduce_starts_its_output_at_the_identity():
    a = Tensor(randf(2, 3))
    for reduced, identity in ((a.sum(axis=0), 0.0), (a.max(axis=0), float("-inf"))):
        (nest,) = lower_all([reduced.node])
        stored = {i.srcs[0] for i in nest.instrs if i.opcode is Opcode.STORE}
        assert [i.arg for i in nest.instrs if i.opcode is Opcode.CONST and i.dest in stored] == [(identity, Valid())]
    ints = Tensor(np.array([[1, 2], [3, 4]], np.int32))
    (nest,) = lower_all([ints.max(axis=0).node])
    stored = {i.srcs[0] for i in nest.instrs if i.opcode is Opcode.STORE}
    inits = [i for i in nest.instrs if i.opcode is Opcode.CONST and i.dest in stored]
    assert [i.arg for i in inits] == [(-(2**31), Valid())] and inits[0].dtype == int32


def test_a_last_axis_reduce_keeps_a_register_total():
    a = Tensor(randf(4, 5))
    for reduced, identity in ((a.sum(axis=1), 0.0), (a.max(axis=1), float("-inf"))):
        (nest,) = lower_all([reduced.node])
        assert loop_vars(nest.instrs) == [["i0", "r1"]]
        assert [i.opcode for i in nest.instrs if i.opcode in (Opcode.ACC, Opcode.ACCUM)] == [Opcode.ACC]
        assert [i.arg for i in nest.instrs if i.opcode is Opcode.ACC] == [identity]


def test_a_matmul_moves_its_reduce_axis_outward():
    (nest,) = lower_all([(Tensor(randf(4, 5)) @ Tensor(randf(5, 3))).node])
    assert loop_vars(nest.instrs) == [["i0", "i1"], ["i0", "r2", "i1"]]
    assert [i.opcode for i in nest.instrs if i.opcode in (Opcode.ACC, Opcode.ACCUM)] == [Opcode.ACCUM]


def test_an_elementwise_nest_keeps_shape_order():
    (nest,) = lower_all([(Tensor(randf(2, 3, 4)) * Tensor(randf(2, 3, 4)) + 1.0).node])
    assert loop_vars(nest.instrs) == [["i0", "i1", "i2"]]


def test_the_rendering_names_accumulators_and_shared_buffers():
    assert "ACC     acc = 0.0 : float32" in codegen.ir(Tensor(randf(4, 5)).sum(axis=1))
    assert "UPDATE  acc = ADD acc," in codegen.ir(Tensor(randf(4, 5)).sum(axis=1))
    assert "ACCUM   out[i0*3 + i1] = ADD out[i0*3 + i1], " in codegen.ir(Tensor(randf(4, 5)) @ Tensor(randf(5, 3)))
    chained = codegen.ir((Tensor(randf(2, 3)) + Tensor(randf(2, 3))).reshape(6) * 2.0)
    assert "out = buf2" in chained and "in0 = buf2" in chained


def test_the_sink_line_follows_an_assign_to_its_buffer():
    p = Tensor(np.zeros((2, 2), np.float32))
    p.assign(p * 2.0 + 1.0)
    text = codegen.ir(p)
    assert "out = buf0  float32[2, 2]" in text and text.rstrip().endswith("sink 0 = buf0  float32[2, 2]")
