"""Loop-nest IR: each scheduled kernel lowered to loops over an iteration space and a flat list
of instructions, with views turned into explicit affine index arithmetic and range checks.

This is the IR a limn compiled device receives through `runners()`; it restates reference
`limn/codegen.py:45-348` and `:479-513` with the same opcodes, operand conventions and loop
order decisions, because the HIP emitter (limn_amd/hip/emit.py) is written against exactly
this contract:

- the space is the output shape, or the pre-reduce shape for SUM/MAX, or the values' shape for
  SCATTER; loop variables are named `i<d>` (kept dims) and `r<d>` (reduced dims);
- a reduce whose axis stays innermost keeps a register total (ACC ... UPDATE ... STORE);
  one whose axis is moved outward folds into the output buffer in place (STORE identity, then
  ACCUM per element), visiting each cell's elements in ascending reduce order;
- `loop_order` moves innermost the dim that is stride-1 in the most buffers, if it strictly
  beats the default innermost dim;
- a masked read yields 0; a VIEW that is masked everywhere lowers to the constant 0.
"""

from __future__ import annotations

import itertools
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from enum import Enum, auto
from typing import TYPE_CHECKING, Any, NamedTuple

from .ops import FLOATS, INTS, DType, Node, Op
from .schedule import Kernel, addressed, realized, schedule
from .view import View, canonical_strides

if TYPE_CHECKING:
    from .tensor import Tensor

ARITH_OPS = (Op.NEG, Op.EXP, Op.LOG, Op.SQRT, Op.RECIP, Op.ADD, Op.MUL, Op.CMPLT, Op.WHERE)


class Reduce(NamedTuple):
    fold: Op
    identity: dict[DType, float | int]


REDUCES = {
    Op.SUM: Reduce(Op.ADD, {**{d: 0.0 for d in FLOATS}, **{d: 0 for d in INTS}}),
    Op.MAX: Reduce(Op.MAX, {**{d: float("-inf") for d in FLOATS}, **{d: -(1 << (8 * d.itemsize - 1)) for d in INTS}}),
}


@dataclass(frozen=True)
class Index:
    """const + sum(coeff * var) over loop variables (or a computed row name, for GATHER/SCATTER)."""

    const: int
    terms: tuple[tuple[str, int], ...] = ()

    def render(self) -> str:
        if not self.terms:
            return str(self.const)
        parts = [var if c == 1 else f"{var}*{c}" for var, c in self.terms]
        text = " + ".join(parts)
        if self.const > 0:
            text += f" + {self.const}"
        elif self.const < 0:
            text += f" - {-self.const}"
        return text

    def at(self, loops: Mapping[str, int]) -> int:
        return self.const + sum(c * loops[var] for var, c in self.terms)


@dataclass(frozen=True)
class Valid:
    """A conjunction of lo <= var < hi checks; each bound also records its dim's size so that a
    side covering the whole dim renders as nothing."""

    bounds: tuple[tuple[str, int, int, int], ...] = ()

    @property
    def never(self) -> bool:
        return any(lo >= hi for _, lo, hi, _ in self.bounds)

    def render(self) -> str:
        checks: list[str] = []
        for var, lo, hi, size in self.bounds:
            if lo > 0:
                checks.append(f"{var} >= {lo}")
            if hi < size:
                checks.append(f"{var} < {hi}")
        return " && ".join(checks)

    def at(self, loops: Mapping[str, int]) -> bool:
        return all(lo <= loops[var] < hi for var, lo, hi, _ in self.bounds)


def index_of(view: View, loop_vars: Sequence[str]) -> tuple[Index, Valid]:
    """A view read at one loop variable per dim."""
    assert len(view.shape) == len(loop_vars), f"view {view.shape} does not match loops {tuple(loop_vars)}"
    terms = tuple((var, s) for var, s in zip(loop_vars, view.strides) if s != 0)
    if view.mask is None:
        return Index(view.offset, terms), Valid()
    checks = tuple(
        (var, lo, hi, n) for var, (lo, hi), n in zip(loop_vars, view.mask, view.shape) if not (lo == 0 and hi == n)
    )
    return Index(view.offset, terms), Valid(checks)


def contiguous_index(shape: tuple[int, ...], loop_vars: Sequence[str]) -> Index:
    assert len(shape) == len(loop_vars), f"shape {shape} does not match loops {tuple(loop_vars)}"
    return Index(0, tuple((var, s) for var, s in zip(loop_vars, canonical_strides(shape)) if s != 0))


class Opcode(Enum):
    LOOP = auto()
    ENDLOOP = auto()
    CONST = auto()
    LOAD = auto()
    ARITH = auto()
    CAST = auto()
    ACC = auto()
    UPDATE = auto()
    STORE = auto()
    ACCUM = auto()
    GATHER = auto()
    SCATTER = auto()


@dataclass(frozen=True)
class Instr:
    opcode: Opcode
    dest: str = ""
    dtype: DType | None = None
    srcs: tuple[str, ...] = ()
    arg: Any = None

    @property
    def value_type(self) -> DType:
        assert self.dtype is not None, f"{self.opcode.name} defines no typed value"
        return self.dtype


@dataclass(frozen=True)
class LoopNest:
    name: str
    kernel: Kernel
    space: tuple[int, ...]
    instrs: tuple[Instr, ...]


def accesses(kernel: Kernel, ndim: int) -> list[tuple[int, ...]]:
    """One stride vector per buffer a reduce kernel touches: the output (row-major), each VIEW's
    own strides, and each input read directly (row-major)."""
    indexed = {a for node in kernel.body if (a := addressed(node)) is not None}
    out = [canonical_strides(kernel.target.shape)]
    out += [node.arg.strides for node in kernel.body if node.op is Op.VIEW and node.srcs[0].op is not Op.CONST]
    out += [canonical_strides(node.shape) for node in kernel.inputs if node not in indexed]
    bad = sorted({len(s) for s in out} - {ndim})
    assert not bad, f"a {ndim}-dim nest reads {bad}-dim buffers"
    return out


def loop_order(kernel: Kernel, ndim: int, axes: tuple[int, ...]) -> tuple[int, ...]:
    """Nesting of dims, outermost first: kept dims then reduce axes, unless some kept dim is
    stride-1 in strictly more buffers than the default innermost dim, which then goes last."""
    if not axes:
        return tuple(range(ndim))
    default = tuple(d for d in range(ndim) if d not in axes) + tuple(axes)
    strides = accesses(kernel, ndim)
    score = [sum(s[d] == 1 for s in strides) for d in range(ndim)]
    best = max(range(ndim), key=lambda d: (score[d], -d))
    if best in axes or score[best] <= score[default[-1]]:
        return default
    return tuple(d for d in default if d != best) + (best,)


def lower(kernel: Kernel, name: str) -> LoopNest:
    """One scheduled kernel as a loop nest."""
    root = kernel.ast
    axes: tuple[int, ...] = tuple(root.arg) if root.op in REDUCES else ()
    if root.op is Op.SCATTER:
        space = root.srcs[1].shape
    elif axes:
        space = root.srcs[0].shape
    else:
        space = root.shape
    loop_vars = tuple(("r" if d in axes else "i") + str(d) for d in range(len(space)))
    buffers = {node: f"in{k}" for k, node in enumerate(kernel.inputs)}
    instrs: list[Instr] = []
    memo: dict[tuple[int, tuple[str, ...]], str] = {}
    fresh = (f"v{k}" for k in itertools.count())

    def emit(opcode: Opcode, dtype: DType, srcs: tuple[str, ...] = (), arg: Any = None) -> str:
        dest = next(fresh)
        instrs.append(Instr(opcode, dest, dtype, srcs, arg))
        return dest

    def value(node: Node, at: tuple[str, ...]) -> str:
        key = (id(node), at)
        if key not in memo:
            if node in buffers:
                memo[key] = emit(Opcode.LOAD, node.dtype, arg=(buffers[node], contiguous_index(node.shape, at), Valid()))
            else:
                memo[key] = compute(node, at)
        return memo[key]

    def compute(node: Node, at: tuple[str, ...]) -> str:
        if node.op is Op.CONST:
            return emit(Opcode.CONST, node.dtype, arg=(node.arg, Valid()))
        if node.op is Op.VIEW:
            src = node.srcs[0]
            index, valid = index_of(node.arg, at)
            if valid.never:
                return emit(Opcode.CONST, node.dtype, arg=(0, Valid()))
            if src.op is Op.CONST:
                return emit(Opcode.CONST, node.dtype, arg=(src.arg, valid))
            return emit(Opcode.LOAD, node.dtype, arg=(buffers[src], index, valid))
        if node.op is Op.CAST:
            return emit(Opcode.CAST, node.dtype, srcs=(value(node.srcs[0], at),))
        if node.op in ARITH_OPS:
            return emit(Opcode.ARITH, node.dtype, srcs=tuple(value(s, at) for s in node.srcs), arg=node.op)
        raise NotImplementedError(f"codegen has no rule for {node.op} inside a kernel")

    def row_index(table_shape: tuple[int, ...], rows: Node) -> Index:
        row = value(rows, loop_vars[: len(rows.shape)])
        return contiguous_index(table_shape, (row, loop_vars[-1]))

    def open_(dims: Sequence[int]) -> None:
        instrs.extend(Instr(Opcode.LOOP, loop_vars[d], arg=space[d]) for d in dims)

    def close(dims: Sequence[int]) -> None:
        instrs.extend(Instr(Opcode.ENDLOOP, arg=loop_vars[d]) for d in reversed(dims))

    order = loop_order(kernel, len(space), axes)
    outer = tuple(d for d in order if d not in axes)

    if axes and order[-1] not in axes:
        out_index = contiguous_index(kernel.target.shape, loop_vars)
        reduce = REDUCES[root.op]
        open_(outer)
        start = emit(Opcode.CONST, root.dtype, arg=(reduce.identity[root.dtype], Valid()))
        instrs.append(Instr(Opcode.STORE, dtype=root.dtype, srcs=(start,), arg=("out", out_index)))
        close(outer)
        open_(order)
        item = value(root.srcs[0], loop_vars)
        instrs.append(Instr(Opcode.ACCUM, dtype=root.dtype, srcs=(item,), arg=("out", out_index, reduce.fold)))
        close(order)
        return LoopNest(name, kernel, tuple(space), tuple(instrs))

    open_(outer)
    if axes:
        reduce = REDUCES[root.op]
        instrs.append(Instr(Opcode.ACC, "acc", root.dtype, arg=reduce.identity[root.dtype]))
        open_(axes)
        item = value(root.srcs[0], loop_vars)
        instrs.append(Instr(Opcode.UPDATE, "acc", root.dtype, (item,), reduce.fold))
        close(axes)
        result = "acc"
    elif root.op in (Op.ASSIGN, Op.SCATTER):
        result = value(root.srcs[1], loop_vars)
    elif root.op is Op.CONTIGUOUS:
        result = value(root.srcs[0], loop_vars)
    elif root.op is Op.GATHER:
        table = root.srcs[0]
        result = emit(Opcode.GATHER, root.dtype, arg=(buffers[table], row_index(table.shape, root.srcs[1])))
    else:
        result = value(root, loop_vars)

    if root.op is Op.SCATTER:
        instrs.append(Instr(Opcode.SCATTER, dtype=root.dtype, srcs=(result,), arg=("out", row_index(root.shape, root.srcs[0]))))
    else:
        out_index = contiguous_index(kernel.target.shape, loop_vars)
        instrs.append(Instr(Opcode.STORE, dtype=root.dtype, srcs=(result,), arg=("out", out_index)))
    close(outer)
    return LoopNest(name, kernel, tuple(space), tuple(instrs))


def lower_all(sinks: list[Node], order: list[Node] | None = None, kernels: list[Kernel] | None = None) -> list[LoopNest]:
    """Every non-CUSTOM kernel of the schedule as a nest, named k0, k1, ... in schedule order."""
    if kernels is None:
        kernels = schedule(sinks, order)
    plain = [k for k in kernels if k.ast.op is not Op.CUSTOM]
    return [lower(k, f"k{n}") for n, k in enumerate(plain)]


def loop_range(instr: Instr) -> tuple[int, int]:
    return instr.arg if isinstance(instr.arg, tuple) else (0, instr.arg)


def _guard(valid: Valid) -> str:
    return f" if {valid.render()} else 0" if valid.bounds else ""


def render_instr(instr: Instr) -> str:
    op = instr.opcode
    if op is Opcode.LOOP:
        lo, hi = loop_range(instr)
        return f"LOOP    {instr.dest} < {hi}" if lo == 0 else f"LOOP    {lo} <= {instr.dest} < {hi}"
    if op is Opcode.ENDLOOP:
        return f"ENDLOOP {instr.arg}"
    if op is Opcode.ACC:
        return f"ACC     {instr.dest} = {instr.arg} : {instr.dtype}"
    if op is Opcode.CONST:
        v, valid = instr.arg
        return f"CONST   {instr.dest} = {v}{_guard(valid)} : {instr.dtype}"
    if op is Opcode.LOAD:
        buf, index, valid = instr.arg
        return f"LOAD    {instr.dest} = {buf}[{index.render()}]{_guard(valid)} : {instr.dtype}"
    if op is Opcode.ARITH:
        return f"ARITH   {instr.dest} = {instr.arg.name} {', '.join(instr.srcs)} : {instr.dtype}"
    if op is Opcode.CAST:
        return f"CAST    {instr.dest} = {instr.srcs[0]} : {instr.dtype}"
    if op is Opcode.UPDATE:
        return f"UPDATE  {instr.dest} = {instr.arg.name} {instr.dest}, {instr.srcs[0]}"
    if op is Opcode.STORE:
        buf, index = instr.arg
        return f"STORE   {buf}[{index.render()}] = {instr.srcs[0]}"
    if op is Opcode.ACCUM:
        buf, index, fold = instr.arg
        cell = f"{buf}[{index.render()}]"
        return f"ACCUM   {cell} = {fold.name} {cell}, {instr.srcs[0]}"
    if op is Opcode.GATHER:
        buf, index = instr.arg
        return f"GATHER  {instr.dest} = {buf}[{index.render()}] : {instr.dtype}"
    buf, index = instr.arg
    return f"SCATTER {buf}[{index.render()}] += {instr.srcs[0]}"


def render(nests: Sequence[LoopNest], sinks: Sequence[Node] = ()) -> str:
    """The schedule as text, buffers numbered across nests by first use (reference
    `limn/codegen.py:479-506`; its README prints the same layout)."""
    ids: dict[Node, str] = {}

    def buf(node: Node) -> str:
        return ids.setdefault(node, f"buf{len(ids)}")

    lines: list[str] = []
    for nest in nests:
        k = nest.kernel
        lines.append(f"{nest.name}  {k.ast.op.name}  loop{list(nest.space)}")
        lines += [f"    in{n} = {buf(node)}  {node.dtype}{list(node.shape)}" for n, node in enumerate(k.inputs)]
        lines.append(f"    out = {buf(k.target)}  {k.target.dtype}{list(k.target.shape)}")
        depth = 1
        for instr in nest.instrs:
            if instr.opcode is Opcode.ENDLOOP:
                depth -= 1
            lines.append("  " * depth + render_instr(instr))
            if instr.opcode is Opcode.LOOP:
                depth += 1
        lines.append("")
    lines += [f"sink {n} = {buf(realized(s))}  {s.dtype}{list(s.shape)}" for n, s in enumerate(sinks)]
    return "\n".join(lines)


def ir(*tensors: Tensor) -> str:
    sinks = [t.node for t in tensors]
    return render(lower_all(sinks), sinks)
