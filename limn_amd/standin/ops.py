"""The graph contract a limn device consumes: dtypes, the closed op set, nodes, CUSTOM kernels.

This restates limn's IR types (reference `limn/ops.py:18-154`) under the same names, meanings
and defaults, so a device written against this module is a device written against limn:

- seven dtypes; two of them (float16, bfloat16) are storage widths that compute widened;
- nineteen primitive ops plus CUSTOM; every user-facing op composes from these;
- a Node hashes by identity, so a BUFFER node keeps its identity while its bytes change;
- a CUSTOM kernel with several outputs is one node per output, told apart by `Custom.index`.

Nothing here computes or allocates.
"""

from __future__ import annotations

import operator
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from enum import Enum, auto
from typing import Any, TypeVar


@dataclass(frozen=True)
class DType:
    name: str
    itemsize: int

    def __repr__(self) -> str:
        return self.name


float64 = DType("float64", 8)
float32 = DType("float32", 4)
float16 = DType("float16", 2)
bfloat16 = DType("bfloat16", 2)
int32 = DType("int32", 4)
int16 = DType("int16", 2)
int8 = DType("int8", 1)
DTYPES = (float64, float32, float16, bfloat16, int32, int16, int8)
FLOATS = (float64, float32, float16, bfloat16)
INTS = (int32, int16, int8)
HALF_FLOATS = (float16, bfloat16)


def promote(a: DType, b: DType) -> DType:
    """Result dtype of a binary op (reference `limn/ops.py:40-50`).

    Same family: the wider wins, except that float16 meeting bfloat16 lands on float32 (neither
    holds the other's values). Int meeting float: the float side, at float32 or wider.
    """
    if a == b:
        return a
    a_float, b_float = a in FLOATS, b in FLOATS
    if a_float == b_float:
        if a in HALF_FLOATS and b in HALF_FLOATS:
            return float32
        return a if a.itemsize >= b.itemsize else b
    fl = a if a_float else b
    return fl if fl.itemsize >= float32.itemsize else float32


def accumulate_in(dtype: DType) -> DType:
    """Width of a reduce's running total (reference `limn/ops.py:53-62`): float32 for the two
    half widths, the dtype itself otherwise (ints wrap modulo 2**width either way)."""
    return float32 if dtype in HALF_FLOATS else dtype


class Op(Enum):
    BUFFER = auto()
    CONST = auto()
    VIEW = auto()
    NEG = auto()
    EXP = auto()
    LOG = auto()
    SQRT = auto()
    RECIP = auto()
    CAST = auto()
    ADD = auto()
    MUL = auto()
    CMPLT = auto()
    WHERE = auto()
    SUM = auto()
    MAX = auto()
    GATHER = auto()
    SCATTER = auto()
    CONTIGUOUS = auto()
    ASSIGN = auto()
    CUSTOM = auto()


@dataclass(eq=False)
class Node:
    """One value in the graph. `arg` is op-specific: the device buffer (BUFFER), the scalar
    (CONST), a View (VIEW), a DType (CAST), reduce axes (SUM/MAX), a Custom (CUSTOM)."""

    op: Op
    srcs: tuple[Node, ...]
    dtype: DType
    shape: tuple[int, ...]
    arg: Any = None

    def __repr__(self) -> str:
        return f"Node({self.op.name}, shape={self.shape}, dtype={self.dtype})"


@dataclass(frozen=True)
class Custom:
    """A CUSTOM node's arg (reference `limn/ops.py:108-127`): the kernel's name, its params, the
    (dtype, shape) of every output it writes, and which output this node stands for."""

    name: str
    params: tuple
    outs: tuple[tuple[DType, tuple[int, ...]], ...]
    index: int = 0


def custom(name: str, srcs: tuple[Node, ...], params: tuple, outs: Sequence[tuple[DType, tuple[int, ...]]]) -> tuple[Node, ...]:
    """One CUSTOM node per output, in output order (reference `limn/ops.py:130-136`)."""
    specs = tuple((dtype, tuple(shape)) for dtype, shape in outs)
    return tuple(Node(Op.CUSTOM, tuple(srcs), dtype, shape, Custom(name, params, specs, k)) for k, (dtype, shape) in enumerate(specs))


T = TypeVar("T")


def topological(sinks: Sequence[T], srcs: Callable[[T], Sequence[T]] = operator.attrgetter("srcs")) -> list[T]:
    """Every node reachable from `sinks`, each after all of its sources, sinks' order kept
    (reference `limn/ops.py:139-154`). Iterative post-order with an explicit stack."""
    order: list[T] = []
    done: set[int] = set()
    entered: set[int] = set()
    for sink in sinks:
        if id(sink) in done:
            continue
        stack: list[tuple[T, int]] = [(sink, 0)]
        entered.add(id(sink))
        while stack:
            node, k = stack[-1]
            children = srcs(node)
            if k < len(children):
                stack[-1] = (node, k + 1)
                child = children[k]
                if id(child) not in entered:
                    entered.add(id(child))
                    stack.append((child, 0))
            else:
                stack.pop()
                done.add(id(node))
                order.append(node)
    return order
