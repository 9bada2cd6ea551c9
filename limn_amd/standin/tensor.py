"""Stand-in for limn's Tensor frontend: lazy graph building, broadcasting, composed ops and
reverse-mode gradients, enough to drive the hip device where limn itself cannot be imported.

Caller contract kept from limn (reference `limn/tensor.py`), because it decides which graphs
reach a device and what the tests compare:

- methods only build Nodes; `realize()` hands the sinks to the active device in one batch and
  turns every computed sink (and every ASSIGN) into the BUFFER it now is;
- broadcasting lifts a tensor with size-1 dims (a reshape view) and expands it; a python scalar
  is a CONST of the tensor's dtype; unequal dtypes meet at `promote`;
- subtraction is `a + (-b)`, division `a * b.reciprocal()` at the wider float, a mean the sum
  times the reciprocal of a float count, softmax a detached-max shift (reference
  `limn/tensor.py:295-300, 401-405, 501-507`): these spellings fix the scheduler's cuts;
- attention emits CUSTOM "sdpa" when the device registers it, and its backward "sdpa_bwd_q"
  and "sdpa_bwd_kv" over a delta row-sum (reference `limn/tensor.py:509-575, 679-746`).

Design of this stand-in:

- A tensor made by an op that needs a gradient carries a `Derivation`: a rule, the input
  tensors and whatever the rule keeps (shapes, axes). Rules are named module functions
  `rule(g, out, d) -> one cotangent per input`; `out` is handed in by the backward pass, so no
  rule holds a reference to the tensor that holds it.
- The backward pass counts, for every tensor that needs a gradient, how many consumers feed it,
  and finalises a tensor's cotangent once all of them have (Kahn's order over the reversed
  graph); `grad()` and `Tensor.backward()` read the finished cotangents.
- `matmul` lifts each operand to full rank once and expands it once, so an operand broadcast
  over batch and rows (a weight) gets its gradient as one sum over all of them: one contraction.

numpy has no bfloat16 here, so `numpy()` of a bfloat16 tensor gives the float32 values it holds.
"""

from __future__ import annotations

import math
import operator
from collections import deque
from collections.abc import Callable, Iterator, Sequence
from contextlib import contextmanager
from dataclasses import dataclass
from typing import Any

import numpy as np

from . import device
from .ops import DTYPES, FLOATS, DType, Node, Op, accumulate_in, bfloat16, custom, float16, float32, float64, int32, promote, topological
from .schedule import CUT_OPS, realized
from .view import View

SDPA, SDPA_BWD_Q, SDPA_BWD_KV = "sdpa", "sdpa_bwd_q", "sdpa_bwd_kv"


class _Mode:
    """Process-wide frontend state: whether ops record derivations, and the draw generator."""

    recording = True
    rng = np.random.default_rng(0)


def set_seed(seed: int) -> None:
    _Mode.rng = np.random.default_rng(seed)


@contextmanager
def no_grad() -> Iterator[None]:
    """Ops built inside record no derivations (optimizer updates, evaluation)."""
    outer = _Mode.recording
    _Mode.recording = False
    try:
        yield
    finally:
        _Mode.recording = outer


Rule = Callable[["Tensor", "Tensor", "Derivation"], "tuple[Tensor | None, ...]"]


@dataclass(frozen=True, slots=True)
class Derivation:
    rule: Rule
    inputs: tuple["Tensor", ...]
    keep: Any = None


class Tensor:
    __slots__ = ("node", "requires_grad", "grad", "derivation", "__weakref__")

    def __init__(self, data: Any, dtype: DType | None = None, requires_grad: bool = False):
        host = np.asarray(data)
        if dtype is None:
            dtype = int32 if host.dtype.kind in "biu" else float32
        if dtype not in DTYPES:
            raise ValueError(f"unsupported dtype {dtype}; limn has {[str(d) for d in DTYPES]}")
        if host.size == 0:
            raise ValueError(f"zero-size tensors are not supported (shape {host.shape})")
        if requires_grad and dtype not in FLOATS:
            raise ValueError(f"requires_grad needs a float dtype, got {dtype}")
        stored = device.to_numpy_storage(host, dtype)
        dev = device.active()
        buf = dev.alloc(stored.nbytes)
        dev.copyin(buf, stored)
        self.node = Node(Op.BUFFER, (), dtype, tuple(host.shape), buf)
        self.requires_grad = requires_grad
        self.grad: Tensor | None = None
        self.derivation: Derivation | None = None

    @classmethod
    def _made(cls, node: Node, inputs: tuple[Tensor, ...] = (), rule: Rule | None = None, keep: Any = None) -> Tensor:
        """A tensor over `node`; it needs a gradient when recording and some input needs one."""
        t = cls.__new__(cls)
        t.node, t.grad = node, None
        t.requires_grad = _Mode.recording and rule is not None and any(x.requires_grad for x in inputs)
        t.derivation = Derivation(rule, inputs, keep) if t.requires_grad else None
        return t

    @staticmethod
    def from_node(node: Node, parents: tuple[Tensor, ...] = (), grad_fn: Callable | None = None) -> Tensor:
        """limn's extension point: wrap a node whose gradient `grad_fn(g)` maps to one cotangent
        per parent."""
        return Tensor._made(node, tuple(parents), _closure_rule if grad_fn is not None else None, grad_fn)

    @staticmethod
    def const(value: float | int, dtype: DType) -> Tensor:
        return Tensor._made(Node(Op.CONST, (), dtype, (), value))

    # ---- creation: host values loaded as buffers ----

    @staticmethod
    def full(shape: Sequence[int], value: float | int, dtype: DType = float32, requires_grad: bool = False) -> Tensor:
        return Tensor(np.full(tuple(shape), value), dtype=dtype, requires_grad=requires_grad)

    @staticmethod
    def zeros(shape: Sequence[int], dtype: DType = float32, requires_grad: bool = False) -> Tensor:
        return Tensor.full(shape, 0, dtype, requires_grad)

    @staticmethod
    def ones(shape: Sequence[int], dtype: DType = float32, requires_grad: bool = False) -> Tensor:
        return Tensor.full(shape, 1, dtype, requires_grad)

    @staticmethod
    def arange(n: int, dtype: DType = int32) -> Tensor:
        return Tensor(np.arange(n), dtype=dtype)

    @staticmethod
    def randn(shape: Sequence[int], std: float = 1.0, requires_grad: bool = False, dtype: DType = float32) -> Tensor:
        return Tensor(_Mode.rng.standard_normal(tuple(shape)) * std, dtype=dtype, requires_grad=requires_grad)

    @staticmethod
    def uniform(shape: Sequence[int], low: float, high: float, requires_grad: bool = False, dtype: DType = float32) -> Tensor:
        return Tensor(_Mode.rng.uniform(low, high, tuple(shape)), dtype=dtype, requires_grad=requires_grad)

    # ---- properties ----

    shape = property(lambda self: self.node.shape)
    dtype = property(lambda self: self.node.dtype)
    ndim = property(lambda self: len(self.node.shape))
    numel = property(lambda self: math.prod(self.node.shape))

    def __repr__(self) -> str:
        return f"Tensor({self.shape}, {self.dtype}, {self.node.op.name}{', grad' if self.requires_grad else ''})"

    # ---- bytes ----

    def realize(self) -> Tensor:
        realize(self)
        return self

    def numpy(self) -> np.ndarray:
        (buf,) = realize(self)
        return device.from_numpy_storage(device.active().copyout(buf), self.dtype, self.shape)

    def item(self) -> float | int:
        return self.numpy().item()

    def detach(self) -> Tensor:
        return Tensor._made(self.node)

    def assign(self, value: Tensor) -> Tensor:
        """Overwrite this buffer with `value` when the batch commits (after every sink computed)."""
        if self.node.op is not Op.BUFFER:
            raise ValueError(f"assign target must be a realized buffer, this tensor is {self.node.op.name}")
        if (value.shape, value.dtype) != (self.shape, self.dtype):
            raise ValueError(f"assign mismatch: target {self.shape} {self.dtype}, value {value.shape} {value.dtype}")
        self.node = Node(Op.ASSIGN, (self.node, value.node), self.dtype, self.shape)
        return self

    # ---- movement: one VIEW over the base node, the movements composed ----

    def view(self) -> View:
        return self.node.arg if self.node.op is Op.VIEW else View.contiguous(self.shape)

    def _moved(self, layout: View, rule: Rule, keep: Any) -> Tensor:
        base = self.node.srcs[0] if self.node.op is Op.VIEW else self.node
        return Tensor._made(Node(Op.VIEW, (base,), self.dtype, layout.shape, layout), (self,), rule, keep)

    def reshape(self, *shape: int) -> Tensor:
        want = _fill_shape(_dims(shape), self.numel)
        layout = self.view().reshape(want)
        if layout is not None:
            return self._moved(layout, _vjp_reshape, self.shape)
        copy = Node(Op.CONTIGUOUS, (self.node,), self.dtype, self.shape)  # no view reaches it: copy first
        return Tensor._made(Node(Op.VIEW, (copy,), self.dtype, want, View.contiguous(want)), (self,), _vjp_reshape, self.shape)

    def permute(self, *order: int) -> Tensor:
        axes = tuple(_axis(d, self.ndim) for d in _dims(order))
        return self._moved(self.view().permute(axes), _vjp_permute, axes)

    def transpose(self, dim0: int = -2, dim1: int = -1) -> Tensor:
        order = list(range(self.ndim))
        a, b = _axis(dim0, self.ndim), _axis(dim1, self.ndim)
        order[a], order[b] = b, a
        return self.permute(*order)

    def expand(self, *shape: int) -> Tensor:
        sizes = _dims(shape)
        if len(sizes) != self.ndim:
            raise ValueError(f"expand: {sizes} has {len(sizes)} dims, tensor {self.shape} has {self.ndim}")
        target = tuple(old if new == -1 else new for old, new in zip(self.shape, sizes))
        grown = tuple(d for d in range(self.ndim) if target[d] != self.shape[d])
        return self._moved(self.view().expand(target), _vjp_expand, grown)

    def pad(self, padding: Sequence[tuple[int, int]]) -> Tensor:
        widths = tuple((int(lo), int(hi)) for lo, hi in padding)
        return self._moved(self.view().pad(widths), _vjp_pad, tuple((lo, lo + n) for n, (lo, _) in zip(self.shape, widths)))

    def shrink(self, bounds: Sequence[tuple[int, int]]) -> Tensor:
        box = tuple((int(lo), int(hi)) for lo, hi in bounds)
        return self._moved(self.view().shrink(box), _vjp_shrink, tuple((lo, n - hi) for n, (lo, hi) in zip(self.shape, box)))

    def flatten(self) -> Tensor:
        return self.reshape(-1)

    # ---- elementwise ----

    def cast(self, dtype: DType) -> Tensor:
        """Float to float keeps the gradient (at the source's width); a cast touching an int
        ends it."""
        if dtype == self.dtype:
            return self
        if dtype not in DTYPES:
            raise ValueError(f"cast: unsupported dtype {dtype}")
        node = Node(Op.CAST, (self.node,), dtype, self.shape, dtype)
        if self.dtype in FLOATS and dtype in FLOATS:
            return Tensor._made(node, (self,), _vjp_cast, self.dtype)
        return Tensor._made(node)

    def float(self) -> Tensor:
        return self.cast(float32)

    def int(self) -> Tensor:
        return self.cast(int32)

    def half(self) -> Tensor:
        return self.cast(float16)

    def bfloat16(self) -> Tensor:
        return self.cast(bfloat16)

    def double(self) -> Tensor:
        return self.cast(float64)

    def _unary(self, op: Op, rule: Rule) -> Tensor:
        if op is not Op.NEG and self.dtype not in FLOATS:
            raise ValueError(f"{op.name} requires a float dtype, got {self.dtype}")
        return Tensor._made(Node(op, (self.node,), self.dtype, self.shape), (self,), rule)

    def __neg__(self) -> Tensor:
        return self._unary(Op.NEG, _vjp_neg)

    def exp(self) -> Tensor:
        return self._unary(Op.EXP, _vjp_exp)

    def log(self) -> Tensor:
        return self._unary(Op.LOG, _vjp_log)

    def sqrt(self) -> Tensor:
        return self._unary(Op.SQRT, _vjp_sqrt)

    def reciprocal(self) -> Tensor:
        return self._unary(Op.RECIP, _vjp_recip)

    def _binary(self, other: Tensor | float | int, op: Op, rule: Rule | None) -> Tensor:
        a, b = _meet(self, other, op.name)
        return Tensor._made(Node(op, (a.node, b.node), a.dtype, a.shape), (a, b), rule)

    def __add__(self, other: Tensor | float | int) -> Tensor:
        return self._binary(other, Op.ADD, _vjp_add)

    def __mul__(self, other: Tensor | float | int) -> Tensor:
        return self._binary(other, Op.MUL, _vjp_mul)

    def __sub__(self, other: Tensor | float | int) -> Tensor:
        return self + -_tensor(other, self)

    def __truediv__(self, other: Tensor | float | int) -> Tensor:
        den = _tensor(other, self)
        common = promote(self.dtype, den.dtype)
        common = common if common in FLOATS else float32  # ints divide as floats: a reciprocal needs one
        return self.cast(common) * den.cast(common).reciprocal()

    __radd__ = __add__
    __rmul__ = __mul__

    def __rsub__(self, other: float | int) -> Tensor:
        return -self + other

    def __rtruediv__(self, other: float | int) -> Tensor:
        return _tensor(other, self) / self

    def __pow__(self, exponent: int | float) -> Tensor:
        if exponent == 0.5:
            return self.sqrt()
        if exponent >= 1 and float(exponent).is_integer():
            out = self
            for _ in range(int(exponent) - 1):
                out = out * self
            return out
        raise ValueError(f"pow supports positive integer exponents and 0.5, got {exponent}; limn has no POW primitive")

    def __lt__(self, other: Tensor | float | int) -> Tensor:
        return self._binary(other, Op.CMPLT, None)  # 0/1 in the operands' dtype, no gradient

    def __gt__(self, other: Tensor | float | int) -> Tensor:
        return _tensor(other, self) < self

    def __le__(self, other: Tensor | float | int) -> Tensor:
        return 1 - (self > other)

    def __ge__(self, other: Tensor | float | int) -> Tensor:
        return _tensor(other, self) <= self

    def eq(self, other: Tensor | float | int) -> Tensor:
        return 1 - (self < other) - (self > other)

    def where(self, if_true: Tensor | float | int, if_false: Tensor | float | int) -> Tensor:
        """Pick `if_true` where self is nonzero; the condition takes no gradient."""
        a, b = _tensor(if_true, self), _tensor(if_false, self)
        if a.dtype != b.dtype:
            common = promote(a.dtype, b.dtype)
            a, b = a.cast(common), b.cast(common)
        shape = _broadcast_shape(_broadcast_shape(a.shape, b.shape, "WHERE"), self.shape, "WHERE")
        a, b = _broadcast(a, shape, "WHERE"), _broadcast(b, shape, "WHERE")
        cond = _broadcast(self.detach(), shape, "WHERE")
        return Tensor._made(Node(Op.WHERE, (cond.node, a.node, b.node), a.dtype, shape), (a, b), _vjp_where, cond)

    def maximum(self, other: Tensor | float | int) -> Tensor:
        other = _tensor(other, self)
        return (self < other).where(other, self)

    def minimum(self, other: Tensor | float | int) -> Tensor:
        other = _tensor(other, self)
        return (other < self).where(other, self)

    def relu(self) -> Tensor:
        return (self > 0).where(self, Tensor.const(0, self.dtype))

    # ---- reduces: the primitive keeps reduced dims at size 1 ----

    def _reduce(self, op: Op, axis: int | Sequence[int] | None, keepdim: bool, rule: Rule) -> Tensor:
        axes = _axes(axis, self.ndim)
        if not axes:
            return self
        kept = tuple(1 if d in axes else n for d, n in enumerate(self.shape))
        out = Tensor._made(Node(op, (self.node,), self.dtype, kept, axes), (self,), rule, axes)
        return out if keepdim else out.reshape(*(n for d, n in enumerate(self.shape) if d not in axes))

    def sum(self, axis: int | Sequence[int] | None = None, keepdim: bool = False) -> Tensor:
        return self._reduce(Op.SUM, axis, keepdim, _vjp_sum)

    def max(self, axis: int | Sequence[int] | None = None, keepdim: bool = False) -> Tensor:
        return self._reduce(Op.MAX, axis, keepdim, _vjp_max)

    def mean(self, axis: int | Sequence[int] | None = None, keepdim: bool = False) -> Tensor:
        count = math.prod(self.shape[d] for d in _axes(axis, self.ndim))
        return self.sum(axis, keepdim) / float(count)

    # ---- indexing ----

    def __getitem__(self, index: Any) -> Tensor:
        """Integers, step-1 slices, one Ellipsis and None, as numpy reads them; a lone int32
        Tensor gathers rows."""
        if isinstance(index, Tensor):
            return self.gather_rows(index)
        keys = list(index) if isinstance(index, tuple) else [index]
        if any(isinstance(k, Tensor) for k in keys):
            raise ValueError(f"index {index}: a Tensor index selects rows and cannot be combined with others")
        if sum(k is Ellipsis for k in keys) > 1:
            raise ValueError(f"index {index}: at most one Ellipsis")
        used = sum(k is not None and k is not Ellipsis for k in keys)
        if used > self.ndim:
            raise IndexError(f"index {index}: too many indices, {used} for {self.ndim} dims")
        at = keys.index(Ellipsis) if Ellipsis in keys else len(keys)
        keys = keys[:at] + [slice(None)] * (self.ndim - used) + keys[at + 1 :]
        box: list[tuple[int, int]] = []
        out_shape: list[int] = []
        for key in keys:
            if key is None:
                out_shape.append(1)
                continue
            dim, size = len(box), self.shape[len(box)]
            if isinstance(key, slice):
                lo, hi, step = key.indices(size)
                if step != 1:
                    raise ValueError(f"index {index}: only step-1 slices are supported")
                if lo >= hi:
                    raise ValueError(f"index {index}: empty slice on dim {dim}, limn has no zero-size tensors")
                box.append((lo, hi))
                out_shape.append(hi - lo)
            elif isinstance(key, bool) or not hasattr(key, "__index__"):
                raise ValueError(f"index {index}: {type(key).__name__} is not a valid index")
            else:
                pos = operator.index(key)
                row = pos + size if pos < 0 else pos
                if not 0 <= row < size:
                    raise IndexError(f"index {index}: {pos} is out of range for dim {dim} of size {size}")
                box.append((row, row + 1))
        return self.shrink(box).reshape(*out_shape)

    def __iter__(self) -> Iterator[Tensor]:
        if self.ndim == 0:
            raise TypeError("iteration over a 0-d tensor")
        return (self[i] for i in range(self.shape[0]))

    def gather_rows(self, indices: Tensor) -> Tensor:
        """Rows of this 2D table at int32 indices: (V, D) at (...) is (..., D)."""
        if self.ndim != 2:
            raise ValueError(f"gather_rows needs a 2D table, got {self.shape}")
        if indices.dtype != int32:
            raise ValueError(f"gather_rows needs int32 indices, got {indices.dtype}")
        node = Node(Op.GATHER, (self.node, indices.node), self.dtype, indices.shape + self.shape[1:])
        return Tensor._made(node, (self,), _vjp_gather, (indices, self.shape))

    # ---- composed ----

    def matmul(self, other: Tensor) -> Tensor:
        """The product as limn spells it (reference limn/tensor.py:486-496): each operand
        broadcast to the batch shape, then reshaped and expanded over the other's rows, then one
        sum over k. Its backward follows the same views back: an operand that was broadcast over
        the batch (a weight under a batched activation) gets a batched contraction over the rows
        (one product per batch, at the operand's dtype) and then a sum over the batch."""
        if self.ndim < 2 or other.ndim < 2:
            raise ValueError(f"matmul needs 2D+ tensors, got {self.shape} @ {other.shape}")
        (m, k), (k2, n) = self.shape[-2:], other.shape[-2:]
        if k != k2:
            raise ValueError(f"matmul: inner dims differ, {self.shape} @ {other.shape}")
        batch = _broadcast_shape(self.shape[:-2], other.shape[:-2], "matmul")
        a = _broadcast(self, batch + (m, k), "matmul").reshape(*batch, m, 1, k).expand(*batch, m, n, k)
        b = _broadcast(other, batch + (k, n), "matmul").transpose(-2, -1).reshape(*batch, 1, n, k).expand(*batch, m, n, k)
        return (a * b).sum(axis=-1)

    __matmul__ = matmul

    def softmax(self, axis: int = -1) -> Tensor:
        e = (self - self.max(axis, keepdim=True).detach()).exp()
        return e / e.sum(axis, keepdim=True)

    def log_softmax(self, axis: int = -1) -> Tensor:
        shifted = self - self.max(axis, keepdim=True).detach()
        return shifted - shifted.exp().sum(axis, keepdim=True).log()

    def attention(self, k: Tensor, v: Tensor, *, causal: bool = False, key_mask: Tensor | None = None) -> Tensor:
        """softmax(q k^T / sqrt(hd)) v over the keys; one CUSTOM kernel where the device has one.

        q's head dim is k's, k's key count is v's, leading dims broadcast; causal wants square
        keys; `key_mask` is one flag per key, (..., t_k), zero hiding that key from every row.
        """
        q = self
        if min(q.ndim, k.ndim, v.ndim) < 2:
            raise ValueError(f"attention needs 2D+ tensors, got {q.shape}, {k.shape}, {v.shape}")
        if q.shape[-1] != k.shape[-1]:
            raise ValueError(f"attention: head dims differ, {q.shape[-1]} and {k.shape[-1]}")
        if k.shape[-2] != v.shape[-2]:
            raise ValueError(f"attention: key counts differ, {k.shape[-2]} and {v.shape[-2]}")
        if causal and q.shape[-2] != k.shape[-2]:
            raise ValueError(f"causal attention needs square keys, got {q.shape[-2]} queries and {k.shape[-2]} keys")
        if not all(t.dtype in FLOATS for t in (q, k, v)):
            raise ValueError(f"attention needs float dtypes, got {q.dtype}, {k.dtype}, {v.dtype}")
        if key_mask is not None and key_mask.shape[-1:] != k.shape[-2:-1]:
            raise ValueError(f"attention: a key mask ends in one flag per key, {k.shape[-2]}, got {key_mask.shape}")
        width = promote(promote(q.dtype, k.dtype), v.dtype)
        lead = _broadcast_shape(_broadcast_shape(q.shape[:-2], k.shape[:-2], "attention"), v.shape[:-2], "attention")
        q, k, v = (_broadcast(t.cast(width), lead + t.shape[-2:], "attention") for t in (q, k, v))
        if key_mask is not None:
            key_mask = _broadcast(key_mask.cast(width), lead + k.shape[-2:-1], "attention")
        scale = q.shape[-1] ** -0.5
        if not device.active().has_custom(SDPA):
            return composed_attention(q, k, v, causal=causal, scale=scale, key_mask=key_mask)
        q, k, v = _contiguous(q), _contiguous(k), _contiguous(v)
        mask = None if key_mask is None else _contiguous(key_mask)
        srcs = (q.node, k.node, v.node) + (() if mask is None else (mask.node,))
        t_q = q.shape[-2]
        outs = ((width, lead + (t_q, v.shape[-1])), (accumulate_in(width), lead + (t_q, 1)))
        o_node, lse_node = custom(SDPA, srcs, (causal, scale), outs)
        return Tensor._made(o_node, (q, k, v), _vjp_attention, (Tensor._made(lse_node), mask, causal, scale))

    # ---- gradients ----

    def backward(self, create_graph: bool = False) -> None:
        """Add d self / d leaf into `.grad` of every leaf (a tensor with no derivation) reached."""
        for t, g in _cotangents(self, create_graph):
            if t.derivation is None:
                t.grad = g if t.grad is None else t.grad + g


# ---- the backward pass ----


def _cotangents(output: Tensor, create_graph: bool) -> list[tuple[Tensor, Tensor]]:
    """(tensor, d output / d tensor) for every tensor on a path from the output to a leaf.

    A tensor's cotangent is final once every consumer on such a path has added its share, so
    each tensor first counts its consumers; a queue then releases tensors as their counts
    reach zero, the output first. Rules run under no_grad unless create_graph asks for
    differentiable cotangents.
    """
    if output.numel != 1:
        raise ValueError(f"gradients need a scalar, got shape {output.shape}")
    if output.dtype not in FLOATS or not output.requires_grad:
        raise ValueError("gradients need a float tensor with requires_grad=True")
    waiting: dict[int, int] = {id(output): 0}
    stack = [output]
    while stack:
        t = stack.pop()
        for x in t.derivation.inputs if t.derivation is not None else ():
            if not x.requires_grad:
                continue
            if id(x) not in waiting:
                waiting[id(x)] = 0
                stack.append(x)
            waiting[id(x)] += 1
    pending: dict[int, Tensor] = {id(output): Tensor.const(1.0, output.dtype).reshape(*output.shape)}
    ready = deque([output])
    finished: list[tuple[Tensor, Tensor]] = []
    outer = _Mode.recording
    _Mode.recording = create_graph
    try:
        while ready:
            t = ready.popleft()
            g = pending.pop(id(t), None)  # None: every consumer passed no gradient
            d = t.derivation
            if g is not None:
                finished.append((t, g))
            if d is None:
                continue
            shares = d.rule(g, t, d) if g is not None else (None,) * len(d.inputs)
            for x, gx in zip(d.inputs, shares, strict=True):
                if not x.requires_grad:
                    continue
                if gx is not None:
                    pending[id(x)] = gx if id(x) not in pending else pending[id(x)] + gx
                waiting[id(x)] -= 1
                if waiting[id(x)] == 0:
                    ready.append(x)
    finally:
        _Mode.recording = outer
    return finished


def grad(output: Tensor, inputs: Sequence[Tensor], create_graph: bool = False) -> list[Tensor]:
    """d output / d input for each input, as lazy tensors; no `.grad` is touched. An input the
    output does not depend on raises."""
    found = {id(t): g for t, g in _cotangents(output, create_graph)}
    missing = [i for i, t in enumerate(inputs) if id(t) not in found]
    if missing:
        raise ValueError(f"grad: output does not depend on inputs[{missing[0]}]")
    return [found[id(t)] for t in inputs]


# ---- derivative rules: rule(g, out, d) -> one cotangent (or None) per input ----


def _closure_rule(g: Tensor, out: Tensor, d: Derivation) -> tuple:
    return tuple(d.keep(g))


def _vjp_reshape(g, out, d):
    return (g.reshape(*d.keep),)


def _vjp_permute(g, out, d):
    return (g.permute(*(d.keep.index(i) for i in range(len(d.keep)))),)


def _vjp_expand(g, out, d):
    return (g.sum(axis=d.keep, keepdim=True),)


def _vjp_pad(g, out, d):
    return (g.shrink(d.keep),)


def _vjp_shrink(g, out, d):
    return (g.pad(d.keep),)


def _vjp_cast(g, out, d):
    return (g.cast(d.keep),)


def _vjp_neg(g, out, d):
    return (-g,)


def _vjp_exp(g, out, d):
    return (g * out,)


def _vjp_log(g, out, d):
    return (g * d.inputs[0].reciprocal(),)


def _vjp_sqrt(g, out, d):
    return (g * (out * 2.0).reciprocal(),)


def _vjp_recip(g, out, d):
    return (-g * out * out,)


def _vjp_add(g, out, d):
    return g, g


def _vjp_mul(g, out, d):
    a, b = d.inputs
    return g * b, g * a


def _vjp_where(g, out, d):
    none = Tensor.const(0, g.dtype)
    return d.keep.where(g, none), d.keep.where(none, g)


def _vjp_sum(g, out, d):
    return (_broadcast(g, d.inputs[0].shape, "SUM"),)


def _vjp_max(g, out, d):
    """Ties share the gradient evenly, as torch.amax does."""
    (x,) = d.inputs
    hit = x.eq(_broadcast(out.detach(), x.shape, "MAX"))
    return (_broadcast(g, x.shape, "MAX") * (hit / hit.sum(axis=d.keep, keepdim=True)),)


def _vjp_gather(g, out, d):
    indices, table = d.keep
    return (scatter_rows(g, indices, table),)


def _vjp_scatter(g, out, d):
    return (g.gather_rows(d.keep),)


def _vjp_contiguous(g, out, d):
    return (g,)


def _vjp_attention(g: Tensor, out: Tensor, d: Derivation) -> tuple[Tensor, Tensor, Tensor]:
    """Two more CUSTOM kernels over the saved L and a delta row-sum; the composed form where the
    device lacks either kernel, or when the gradient must itself be differentiable (a CUSTOM
    node has no derivative of its own)."""
    q, k, v = d.inputs
    lse, mask, causal, scale = d.keep
    dev = device.active()
    if _Mode.recording or not (dev.has_custom(SDPA_BWD_Q) and dev.has_custom(SDPA_BWD_KV)):
        p = _attention_probs(q, k, causal=causal, scale=scale, key_mask=mask)
        dp = g @ v.transpose(-2, -1)
        ds = p * (dp - (dp * p).sum(axis=-1, keepdim=True)) * scale
        return ds @ k, ds.transpose(-2, -1) @ q, p.transpose(-2, -1) @ g
    do = _contiguous(g)
    stat = lse.dtype
    delta = _contiguous((do.cast(stat) * Tensor._made(out.node).cast(stat)).sum(axis=-1, keepdim=True))
    srcs = tuple(t.node for t in (q, k, v, do, lse, delta)) + (() if mask is None else (mask.node,))
    (dq,) = custom(SDPA_BWD_Q, srcs, (causal, scale), ((q.dtype, q.shape),))
    dk, dv = custom(SDPA_BWD_KV, srcs, (causal, scale), ((k.dtype, k.shape), (v.dtype, v.shape)))
    return Tensor._made(dq), Tensor._made(dk), Tensor._made(dv)


# ---- batches ----


def realize(*tensors: Tensor) -> list:
    """Run every given tensor's graph in one device batch; afterwards each computed sink and
    each ASSIGN that ran is the BUFFER holding its bytes (a sink that only aliases a buffer
    keeps its VIEW)."""
    sinks = [t.node for t in tensors]
    bufs = device.active().execute(sinks)
    for node in topological(sinks):
        if node.op is Op.ASSIGN:  # committed: the node now is the buffer it wrote
            node.op, node.arg, node.srcs = Op.BUFFER, node.srcs[0].arg, ()
    for node, buf in zip(sinks, bufs):
        if realized(node).op is not Op.BUFFER:
            node.op, node.arg, node.srcs = Op.BUFFER, buf, ()
    return bufs


def scatter_rows(values: Tensor, indices: Tensor, shape: tuple[int, ...]) -> Tensor:
    """`values`' rows summed into a zeroed table of `shape` at `indices` (gather_rows' gradient)."""
    if values.shape != indices.shape + tuple(shape[1:]):
        raise ValueError(f"scatter_rows: values {values.shape} do not match indices {indices.shape} into {shape}")
    node = Node(Op.SCATTER, (indices.node, values.node), values.dtype, tuple(shape))
    return Tensor._made(node, (values,), _vjp_scatter, indices)


# ---- attention from primitives ----


def composed_attention(q: Tensor, k: Tensor, v: Tensor, *, causal: bool, scale: float, key_mask: Tensor | None = None) -> Tensor:
    return _attention_probs(q, k, causal=causal, scale=scale, key_mask=key_mask) @ v


def _attention_probs(q: Tensor, k: Tensor, *, causal: bool, scale: float, key_mask: Tensor | None = None) -> Tensor:
    """Softmax of the scaled scores with hidden entries at -1e9 (exp of which is exactly 0)."""
    scores = (q @ k.transpose(-2, -1)) * scale
    if causal:
        t_q, t_k = q.shape[-2], k.shape[-2]
        below = Tensor.arange(t_k).reshape(1, t_k) <= Tensor.arange(t_q).reshape(t_q, 1)
        scores = below.where(scores, -1e9)
    if key_mask is not None:
        scores = key_mask.reshape(*key_mask.shape[:-1], 1, key_mask.shape[-1]).where(scores, -1e9)
    return scores.softmax(-1)


def _contiguous(t: Tensor) -> Tensor:
    """t as row-major bytes: itself when it already is a buffer or a cut, else a CONTIGUOUS copy."""
    if t.node.op is Op.BUFFER or t.node.op in CUT_OPS:
        return t
    return Tensor._made(Node(Op.CONTIGUOUS, (t.node,), t.dtype, t.shape), (t,), _vjp_contiguous)


# ---- shapes and broadcasting ----


def _dims(args: Sequence) -> tuple[int, ...]:
    """f(2, 3) and f((2, 3)) alike."""
    if len(args) == 1 and isinstance(args[0], (tuple, list)):
        args = args[0]
    return tuple(int(a) for a in args)


def _fill_shape(shape: tuple[int, ...], numel: int) -> tuple[int, ...]:
    free = [d for d, n in enumerate(shape) if n == -1]
    if len(free) > 1:
        raise ValueError(f"reshape: more than one -1 in {shape}")
    if free:
        known = math.prod(n for n in shape if n != -1)
        shape = tuple(numel // known if n == -1 else n for n in shape)
    if any(n < 1 for n in shape) or math.prod(shape) != numel:
        raise ValueError(f"reshape: cannot view {numel} elements as {shape}")
    return shape


def _axis(axis: int, ndim: int) -> int:
    if not -ndim <= axis < ndim:
        raise ValueError(f"axis {axis} out of range for {ndim} dims")
    return axis % ndim


def _axes(axis: int | Sequence[int] | None, ndim: int) -> tuple[int, ...]:
    if axis is None:
        return tuple(range(ndim))
    picked = sorted(_axis(a, ndim) for a in ((axis,) if isinstance(axis, int) else axis))
    if len(set(picked)) != len(picked):
        raise ValueError(f"duplicate axes in {axis}")
    return tuple(picked)


def _tensor(x: Tensor | float | int, like: Tensor) -> Tensor:
    """A python scalar as a CONST: the tensor's dtype, except a float meeting an int tensor."""
    if isinstance(x, Tensor):
        return x
    return Tensor.const(x, like.dtype if like.dtype in FLOATS or isinstance(x, int) else float32)


def _broadcast_shape(a: tuple[int, ...], b: tuple[int, ...], what: str) -> tuple[int, ...]:
    n = max(len(a), len(b))
    a2, b2 = (1,) * (n - len(a)) + tuple(a), (1,) * (n - len(b)) + tuple(b)
    if any(x != y and 1 not in (x, y) for x, y in zip(a2, b2)):
        raise ValueError(f"{what}: cannot broadcast {a} with {b}")
    return tuple(max(x, y) for x, y in zip(a2, b2))


def _broadcast(t: Tensor, shape: tuple[int, ...], what: str) -> Tensor:
    """t viewed at `shape`: size-1 dims prepended by a reshape, then one expand."""
    if t.shape == shape:
        return t
    if _broadcast_shape(t.shape, shape, what) != shape:
        raise ValueError(f"{what}: cannot broadcast {t.shape} to {shape}")
    if t.ndim != len(shape):
        t = t.reshape(*((1,) * (len(shape) - t.ndim) + t.shape))
    return t.expand(*shape)


def _meet(a: Tensor, b: Tensor | float | int, what: str) -> tuple[Tensor, Tensor]:
    """Both operands of a binary op at one dtype and one shape."""
    b = _tensor(b, a)
    if a.dtype != b.dtype:
        common = promote(a.dtype, b.dtype)
        a, b = a.cast(common), b.cast(common)
    shape = _broadcast_shape(a.shape, b.shape, what)
    return _broadcast(a, shape, what), _broadcast(b, shape, what)
