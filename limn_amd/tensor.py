"""Tensor: limn's lazy user API (reference `limn/tensor.py`), restated as the caller that builds the
graphs the hip device runs.

Every method builds Nodes; nothing computes until `realize()`/`numpy()` hands the sinks to the
active device. Autograd is a record of parent Tensors and a closure per op that maps the output
gradient to parent gradients (themselves lazy Tensors), walked in reverse topological order.
Composed ops (matmul, softmax, division, ...) differentiate through their pieces.

Semantics kept from the reference, since they decide the graphs a device receives:
broadcasting through reshape+expand views, dtype promotion (`ops.promote`), reduces keeping
dims, `matmul` as expand-multiply-sum, softmax with a detached max, and the attention seam:
`attention()` emits CUSTOM "sdpa" when the device registers it (else the composed form), and
its backward emits "sdpa_bwd_q" and "sdpa_bwd_kv" with a fused delta row-sum
(reference `limn/tensor.py:509-575, 679-746`).

One deviation: numpy has no bfloat16 here (ml_dtypes is not part of this stack), so `numpy()`
of a bfloat16 tensor returns the float32 values it holds exactly.
"""

from __future__ import annotations

import math
import operator
from collections.abc import Callable, Iterator, Sequence
from contextlib import contextmanager, nullcontext
from typing import Any

import numpy as np

from limn_amd import device
from limn_amd.dtypes import from_storage, to_storage
from limn_amd.ops import (
    DTYPES,
    FLOATS,
    DType,
    Node,
    Op,
    accumulate_in,
    bfloat16,
    custom,
    float16,
    float32,
    float64,
    int32,
    promote,
    topological,
)
from limn_amd.schedule import CUT_OPS, realized
from limn_amd.view import View

SDPA, SDPA_BWD_Q, SDPA_BWD_KV = "sdpa", "sdpa_bwd_q", "sdpa_bwd_kv"

grad_enabled: bool = True
rng: np.random.Generator = np.random.default_rng(0)

BackwardFn = Callable[["Tensor"], "tuple[Tensor | None, ...]"]


def set_seed(seed: int) -> None:
    global rng
    rng = np.random.default_rng(seed)


@contextmanager
def no_grad() -> Iterator[None]:
    global grad_enabled
    saved, grad_enabled = grad_enabled, False
    try:
        yield
    finally:
        grad_enabled = saved


class Tensor:
    def __init__(self, data: Any, dtype: DType | None = None, requires_grad: bool = False):
        array = np.asarray(data)
        if dtype is None:
            dtype = int32 if array.dtype.kind in "iub" else float32
        if dtype not in DTYPES:
            raise ValueError(f"unsupported dtype {dtype}; limn has {[str(d) for d in DTYPES]}")
        if array.size == 0:
            raise ValueError(f"zero-size tensors are not supported (shape {array.shape})")
        if requires_grad and dtype not in FLOATS:
            raise ValueError(f"requires_grad needs a float dtype, got {dtype}")
        host = to_storage(array, dtype)
        dev = device.active()
        buf = dev.alloc(host.nbytes)
        dev.copyin(buf, host)
        self.node: Node = Node(Op.BUFFER, (), dtype, tuple(array.shape), buf)
        self.requires_grad = requires_grad
        self.grad: Tensor | None = None
        self.parents: tuple[Tensor, ...] = ()
        self.grad_fn: BackwardFn | None = None

    @staticmethod
    def from_node(node: Node, parents: tuple[Tensor, ...] = (), grad_fn: BackwardFn | None = None) -> Tensor:
        t = Tensor.__new__(Tensor)
        t.node = node
        t.requires_grad = grad_enabled and any(p.requires_grad for p in parents)
        t.grad = None
        t.parents = parents if t.requires_grad else ()
        t.grad_fn = grad_fn if t.requires_grad else None
        return t

    @staticmethod
    def const(value: float | int, dtype: DType) -> Tensor:
        return Tensor.from_node(Node(Op.CONST, (), dtype, (), value))

    # ---- creation ----

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
        return Tensor(rng.standard_normal(tuple(shape)) * std, dtype=dtype, requires_grad=requires_grad)

    @staticmethod
    def uniform(shape: Sequence[int], low: float, high: float, requires_grad: bool = False, dtype: DType = float32) -> Tensor:
        return Tensor(rng.uniform(low, high, tuple(shape)), dtype=dtype, requires_grad=requires_grad)

    # ---- properties ----

    @property
    def shape(self) -> tuple[int, ...]:
        return self.node.shape

    @property
    def dtype(self) -> DType:
        return self.node.dtype

    @property
    def ndim(self) -> int:
        return len(self.node.shape)

    @property
    def numel(self) -> int:
        return math.prod(self.node.shape)

    def __repr__(self) -> str:
        return f"Tensor(shape={self.shape}, dtype={self.dtype}, op={self.node.op.name}, requires_grad={self.requires_grad})"

    # ---- realization ----

    def realize(self) -> Tensor:
        realize(self)
        return self

    def numpy(self) -> np.ndarray:
        buf = realize(self)[0]
        return from_storage(device.active().copyout(buf), self.dtype, self.shape)

    def item(self) -> float | int:
        return self.numpy().item()

    def detach(self) -> Tensor:
        return Tensor.from_node(self.node)

    def assign(self, value: Tensor) -> Tensor:
        if self.node.op is not Op.BUFFER:
            raise ValueError(f"assign target must be a realized buffer, this tensor is {self.node.op.name}")
        if value.shape != self.shape or value.dtype != self.dtype:
            raise ValueError(f"assign mismatch: target {self.shape} {self.dtype}, value {value.shape} {value.dtype}")
        self.node = Node(Op.ASSIGN, (self.node, value.node), self.dtype, self.shape)
        return self

    # ---- movement ----

    def view(self) -> View:
        return self.node.arg if self.node.op is Op.VIEW else View.contiguous(self.shape)

    def moved(self, new_view: View, grad_fn: BackwardFn) -> Tensor:
        base = self.node.srcs[0] if self.node.op is Op.VIEW else self.node
        return Tensor.from_node(Node(Op.VIEW, (base,), self.dtype, new_view.shape, new_view), (self,), grad_fn)

    def reshape(self, *shape: int) -> Tensor:
        new_shape = resolve_shape(as_ints(shape), self.numel)
        if math.prod(new_shape) != self.numel:
            raise ValueError(f"reshape: cannot view {self.shape} as {new_shape}")
        old = self.shape

        def backward(g: Tensor) -> tuple[Tensor]:
            return (g.reshape(*old),)

        v = self.view().reshape(new_shape)
        if v is not None:
            return self.moved(v, backward)
        copy = Node(Op.CONTIGUOUS, (self.node,), self.dtype, self.shape)
        return Tensor.from_node(Node(Op.VIEW, (copy,), self.dtype, new_shape, View.contiguous(new_shape)), (self,), backward)

    def permute(self, *order: int) -> Tensor:
        axes = tuple(wrap_axis(d, self.ndim) for d in as_ints(order))
        inverse = tuple(axes.index(d) for d in range(self.ndim))
        return self.moved(self.view().permute(axes), lambda g: (g.permute(*inverse),))

    def transpose(self, dim0: int = -2, dim1: int = -1) -> Tensor:
        order = list(range(self.ndim))
        a, b = wrap_axis(dim0, self.ndim), wrap_axis(dim1, self.ndim)
        order[a], order[b] = order[b], order[a]
        return self.permute(*order)

    def expand(self, *shape: int) -> Tensor:
        sizes = as_ints(shape)
        if len(sizes) != self.ndim:
            raise ValueError(f"expand: {sizes} has {len(sizes)} dims, tensor {self.shape} has {self.ndim}")
        target = tuple(old if new == -1 else new for old, new in zip(self.shape, sizes))
        grown = tuple(d for d, (old, new) in enumerate(zip(self.shape, target)) if old != new)
        return self.moved(self.view().expand(target), lambda g: (g.sum(axis=grown, keepdim=True),))

    def pad(self, padding: Sequence[tuple[int, int]]) -> Tensor:
        pads = tuple((int(b), int(a)) for b, a in padding)
        bounds = tuple((b, b + n) for n, (b, _) in zip(self.shape, pads))
        return self.moved(self.view().pad(pads), lambda g: (g.shrink(bounds),))

    def shrink(self, bounds: Sequence[tuple[int, int]]) -> Tensor:
        cuts = tuple((int(lo), int(hi)) for lo, hi in bounds)
        padding = tuple((lo, n - hi) for n, (lo, hi) in zip(self.shape, cuts))
        return self.moved(self.view().shrink(cuts), lambda g: (g.pad(padding),))

    def flatten(self) -> Tensor:
        return self.reshape(-1)

    # ---- elementwise ----

    def cast(self, dtype: DType) -> Tensor:
        if dtype == self.dtype:
            return self
        if dtype not in DTYPES:
            raise ValueError(f"cast: unsupported dtype {dtype}")
        node = Node(Op.CAST, (self.node,), dtype, self.shape, dtype)
        if self.dtype not in FLOATS or dtype not in FLOATS:
            return Tensor.from_node(node)
        source = self.dtype
        return Tensor.from_node(node, (self,), lambda g: (g.cast(source),))

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

    def unary(self, op: Op, grad_fn: BackwardFn) -> Tensor:
        if op in (Op.EXP, Op.LOG, Op.SQRT, Op.RECIP) and self.dtype not in FLOATS:
            raise ValueError(f"{op.name} requires a float dtype, got {self.dtype}")
        return Tensor.from_node(Node(op, (self.node,), self.dtype, self.shape), (self,), grad_fn)

    def __neg__(self) -> Tensor:
        return self.unary(Op.NEG, lambda g: (-g,))

    def exp(self) -> Tensor:
        out = self.unary(Op.EXP, lambda g: (g * out,))
        return out

    def log(self) -> Tensor:
        return self.unary(Op.LOG, lambda g: (g * self.reciprocal(),))

    def sqrt(self) -> Tensor:
        out = self.unary(Op.SQRT, lambda g: (g * (out * 2.0).reciprocal(),))
        return out

    def reciprocal(self) -> Tensor:
        out = self.unary(Op.RECIP, lambda g: (-g * out * out,))
        return out

    def binary(self, other: Tensor | float | int, op: Op, make_grad: Callable[[Tensor, Tensor], BackwardFn]) -> Tensor:
        a, b = broadcast_pair(self, other, op.name)
        return Tensor.from_node(Node(op, (a.node, b.node), a.dtype, a.shape), (a, b), make_grad(a, b))

    def __add__(self, other: Tensor | float | int) -> Tensor:
        return self.binary(other, Op.ADD, lambda a, b: lambda g: (g, g))

    def __mul__(self, other: Tensor | float | int) -> Tensor:
        return self.binary(other, Op.MUL, lambda a, b: lambda g: (g * b, g * a))

    def __sub__(self, other: Tensor | float | int) -> Tensor:
        return self + (-as_tensor(other, self))

    def __truediv__(self, other: Tensor | float | int) -> Tensor:
        other = as_tensor(other, self)
        wide = promote(self.dtype, other.dtype)
        if wide not in FLOATS:
            wide = float32
        return self.cast(wide) * other.cast(wide).reciprocal()

    def __radd__(self, other: float | int) -> Tensor:
        return self + other

    def __rmul__(self, other: float | int) -> Tensor:
        return self * other

    def __rsub__(self, other: float | int) -> Tensor:
        return -self + other

    def __rtruediv__(self, other: float | int) -> Tensor:
        return as_tensor(other, self) / self

    def __pow__(self, exponent: int | float) -> Tensor:
        if exponent == 0.5:
            return self.sqrt()
        if float(exponent).is_integer() and exponent >= 1:
            out = self
            for _ in range(int(exponent) - 1):
                out = out * self
            return out
        raise ValueError(f"pow supports positive integer exponents and 0.5, got {exponent}; limn has no POW primitive")

    def __lt__(self, other: Tensor | float | int) -> Tensor:
        a, b = broadcast_pair(self, other, "CMPLT")
        return Tensor.from_node(Node(Op.CMPLT, (a.node, b.node), a.dtype, a.shape))

    def __gt__(self, other: Tensor | float | int) -> Tensor:
        return as_tensor(other, self) < self

    def __le__(self, other: Tensor | float | int) -> Tensor:
        return 1 - (self > other)

    def __ge__(self, other: Tensor | float | int) -> Tensor:
        return as_tensor(other, self) <= self

    def eq(self, other: Tensor | float | int) -> Tensor:
        return 1 - (self < other) - (self > other)

    def where(self, if_true: Tensor | float | int, if_false: Tensor | float | int) -> Tensor:
        x, y = as_tensor(if_true, self), as_tensor(if_false, self)
        if x.dtype != y.dtype:
            wide = promote(x.dtype, y.dtype)
            x, y = x.cast(wide), y.cast(wide)
        shape = broadcast_shape(broadcast_shape(x.shape, y.shape, "WHERE"), self.shape, "WHERE")
        x, y = broadcast_to(x, shape, "WHERE"), broadcast_to(y, shape, "WHERE")
        cond = broadcast_to(self.detach(), shape, "WHERE")
        node = Node(Op.WHERE, (cond.node, x.node, y.node), x.dtype, shape)

        def backward(g: Tensor) -> tuple[Tensor, Tensor]:
            return cond.where(g, zero(g)), cond.where(zero(g), g)

        return Tensor.from_node(node, (x, y), backward)

    def maximum(self, other: Tensor | float | int) -> Tensor:
        other = as_tensor(other, self)
        return (self < other).where(other, self)

    def minimum(self, other: Tensor | float | int) -> Tensor:
        other = as_tensor(other, self)
        return (other < self).where(other, self)

    def relu(self) -> Tensor:
        return (self > 0).where(self, zero(self))

    # ---- reduces ----

    def reduce(self, op: Op, axis, keepdim: bool, make_grad: Callable[[Tensor], BackwardFn]) -> Tensor:
        axes = canon_axes(axis, self.ndim)
        if not axes:
            return self
        kept_shape = tuple(1 if d in axes else n for d, n in enumerate(self.shape))
        kept = Tensor.from_node(Node(op, (self.node,), self.dtype, kept_shape, axes), (self,))
        if kept.requires_grad:
            kept.grad_fn = make_grad(kept)
        if keepdim:
            return kept
        return kept.reshape(*(n for d, n in enumerate(self.shape) if d not in axes))

    def sum(self, axis=None, keepdim: bool = False) -> Tensor:
        return self.reduce(Op.SUM, axis, keepdim, lambda kept: lambda g: (broadcast_to(g, self.shape, "SUM"),))

    def max(self, axis=None, keepdim: bool = False) -> Tensor:
        axes = canon_axes(axis, self.ndim)

        def make_grad(kept: Tensor) -> BackwardFn:
            def backward(g: Tensor) -> tuple[Tensor]:
                hit = self.eq(broadcast_to(kept.detach(), self.shape, "MAX"))
                share = hit / hit.sum(axis=axes, keepdim=True)
                return (broadcast_to(g, self.shape, "MAX") * share,)

            return backward

        return self.reduce(Op.MAX, axis, keepdim, make_grad)

    def mean(self, axis=None, keepdim: bool = False) -> Tensor:
        axes = canon_axes(axis, self.ndim)
        count = math.prod(self.shape[d] for d in axes) if axes else 1
        return self.sum(axis, keepdim) / float(count)

    # ---- indexing ----

    def __getitem__(self, index) -> Tensor:
        keys = list(index) if isinstance(index, tuple) else [index]
        if len(keys) == 1 and isinstance(keys[0], Tensor):
            return self.gather_rows(keys[0])
        if any(isinstance(k, Tensor) for k in keys):
            raise ValueError(f"index {index}: a Tensor index selects rows and cannot be combined with others")
        ellipses = [d for d, k in enumerate(keys) if k is Ellipsis]
        if len(ellipses) > 1:
            raise ValueError(f"index {index}: at most one Ellipsis")
        used = sum(k is not None and k is not Ellipsis for k in keys)
        if used > self.ndim:
            raise IndexError(f"index {index}: too many indices, {used} for {self.ndim} dims")
        at = ellipses[0] if ellipses else len(keys)
        keys[at : at + 1] = [slice(None)] * (self.ndim - used)
        bounds: list[tuple[int, int]] = []
        shape: list[int] = []
        for key in keys:
            if key is None:
                shape.append(1)
                continue
            dim = len(bounds)
            size = self.shape[dim]
            if isinstance(key, slice):
                start, stop, step = key.indices(size)
                if step != 1:
                    raise ValueError(f"index {index}: only step-1 slices are supported")
                if start >= stop:
                    raise ValueError(f"index {index}: empty slice on dim {dim}, limn has no zero-size tensors")
                bounds.append((start, stop))
                shape.append(stop - start)
                continue
            if isinstance(key, bool):
                raise ValueError(f"index {index}: a bool index is a numpy mask, which limn does not have")
            try:
                pos = operator.index(key)
            except TypeError:
                raise ValueError(f"index {index}: {type(key).__name__} is not a valid index") from None
            start = pos + size if pos < 0 else pos
            if not 0 <= start < size:
                raise IndexError(f"index {index}: {pos} is out of range for dim {dim} of size {size}")
            bounds.append((start, start + 1))
        return self.shrink(bounds).reshape(*shape)

    def __iter__(self) -> Iterator[Tensor]:
        if self.ndim == 0:
            raise TypeError("iteration over a 0-d tensor")
        return (self[i] for i in range(self.shape[0]))

    def gather_rows(self, indices: Tensor) -> Tensor:
        if self.ndim != 2:
            raise ValueError(f"gather_rows needs a 2D table, got {self.shape}")
        if indices.dtype != int32:
            raise ValueError(f"gather_rows needs int32 indices, got {indices.dtype}")
        node = Node(Op.GATHER, (self.node, indices.node), self.dtype, indices.shape + self.shape[1:])
        table = self.shape
        return Tensor.from_node(node, (self,), lambda g: (scatter_rows(g, indices, table),))

    # ---- composed ----

    def matmul(self, other: Tensor) -> Tensor:
        a, b = self, other
        if a.ndim < 2 or b.ndim < 2:
            raise ValueError(f"matmul needs 2D+ tensors, got {a.shape} @ {b.shape}")
        if a.shape[-1] != b.shape[-2]:
            raise ValueError(f"matmul: inner dims differ, {a.shape} @ {b.shape}")
        batch = broadcast_shape(a.shape[:-2], b.shape[:-2], "matmul")
        m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
        # each operand is lifted to full rank with size-1 dims and expanded once, so its gradient
        # is one sum over every broadcast axis (a weight's over batch and rows together: one
        # contraction) rather than a sum per axis
        lead_a = (1,) * (len(batch) - len(a.shape[:-2])) + a.shape[:-2]
        lead_b = (1,) * (len(batch) - len(b.shape[:-2])) + b.shape[:-2]
        a = a.reshape(*lead_a, m, 1, k).expand(*batch, m, n, k)
        b = b.transpose(-2, -1).reshape(*lead_b, 1, n, k).expand(*batch, m, n, k)
        return (a * b).sum(axis=-1)

    def __matmul__(self, other: Tensor) -> Tensor:
        return self.matmul(other)

    def softmax(self, axis: int = -1) -> Tensor:
        e = (self - self.max(axis, keepdim=True).detach()).exp()
        return e / e.sum(axis, keepdim=True)

    def log_softmax(self, axis: int = -1) -> Tensor:
        shifted = self - self.max(axis, keepdim=True).detach()
        return shifted - shifted.exp().sum(axis, keepdim=True).log()

    def attention(self, k: Tensor, v: Tensor, *, causal: bool = False, key_mask: Tensor | None = None) -> Tensor:
        """softmax(q k^T / sqrt(hd)) v over keys, fused where the device registers "sdpa"."""
        q = self
        if q.ndim < 2 or k.ndim < 2 or v.ndim < 2:
            raise ValueError(f"attention needs 2D+ tensors, got {q.shape}, {k.shape}, {v.shape}")
        if q.shape[-1] != k.shape[-1]:
            raise ValueError(f"attention: head dims differ, {q.shape[-1]} and {k.shape[-1]}")
        if k.shape[-2] != v.shape[-2]:
            raise ValueError(f"attention: key counts differ, {k.shape[-2]} and {v.shape[-2]}")
        if causal and q.shape[-2] != k.shape[-2]:
            raise ValueError(f"causal attention needs square keys, got {q.shape[-2]} queries and {k.shape[-2]} keys")
        if q.dtype not in FLOATS or k.dtype not in FLOATS or v.dtype not in FLOATS:
            raise ValueError(f"attention needs float dtypes, got {q.dtype}, {k.dtype}, {v.dtype}")
        if key_mask is not None and key_mask.shape[-1:] != k.shape[-2:-1]:
            raise ValueError(f"attention: a key mask ends in one flag per key, {k.shape[-2]}, got {key_mask.shape}")
        wide = promote(promote(q.dtype, k.dtype), v.dtype)
        q, k, v = q.cast(wide), k.cast(wide), v.cast(wide)
        batch = broadcast_shape(broadcast_shape(q.shape[:-2], k.shape[:-2], "attention"), v.shape[:-2], "attention")
        q = broadcast_to(q, batch + q.shape[-2:], "attention")
        k = broadcast_to(k, batch + k.shape[-2:], "attention")
        v = broadcast_to(v, batch + v.shape[-2:], "attention")
        if key_mask is not None:
            key_mask = broadcast_to(key_mask.cast(wide), batch + k.shape[-2:-1], "attention")
        scale = q.shape[-1] ** -0.5
        if not device.active().has_custom(SDPA):
            return composed_attention(q, k, v, causal=causal, scale=scale, key_mask=key_mask)
        q, k, v = _contiguous(q), _contiguous(k), _contiguous(v)
        mask = None if key_mask is None else _contiguous(key_mask)
        srcs = (q.node, k.node, v.node) + ((mask.node,) if mask is not None else ())
        outs = ((wide, batch + (q.shape[-2], v.shape[-1])), (accumulate_in(wide), batch + (q.shape[-2], 1)))
        node, lse = custom(SDPA, srcs, (causal, scale), outs)
        out = Tensor.from_node(node, (q, k, v))
        if out.requires_grad:
            saved = (Tensor.from_node(node), Tensor.from_node(lse))
            out.grad_fn = _attention_backward(*saved, q, k, v, mask, causal=causal, scale=scale)
        return out

    # ---- autograd ----

    def backward(self, create_graph: bool = False) -> None:
        for t, g in gradients(self, create_graph):
            if t.grad_fn is None:
                t.grad = g if t.grad is None else t.grad + g


def gradients(output: Tensor, create_graph: bool) -> list[tuple[Tensor, Tensor]]:
    if output.numel != 1:
        raise ValueError(f"gradients need a scalar, got shape {output.shape}")
    if output.dtype not in FLOATS or not output.requires_grad:
        raise ValueError("gradients need a float tensor with requires_grad=True")
    order = topological([output], lambda t: [p for p in t.parents if p.requires_grad])
    pending: dict[int, Tensor] = {id(output): Tensor.const(1.0, output.dtype).reshape(*output.shape)}
    done: list[tuple[Tensor, Tensor]] = []
    with nullcontext() if create_graph else no_grad():
        for t in reversed(order):
            g = pending.pop(id(t), None)
            if g is None:
                continue
            done.append((t, g))
            if t.grad_fn is None:
                continue
            for parent, pg in zip(t.parents, t.grad_fn(g)):
                if pg is None or not parent.requires_grad:
                    continue
                prior = pending.get(id(parent))
                pending[id(parent)] = pg if prior is None else prior + pg
    return done


def grad(output: Tensor, inputs: Sequence[Tensor], create_graph: bool = False) -> list[Tensor]:
    found = {id(t): g for t, g in gradients(output, create_graph)}
    for i, t in enumerate(inputs):
        if id(t) not in found:
            raise ValueError(f"grad: output does not depend on inputs[{i}]")
    return [found[id(t)] for t in inputs]


def realize(*tensors: Tensor) -> list:
    """Execute all given tensors' graphs in one batch; sinks and committed ASSIGNs become BUFFERs."""
    sinks = [t.node for t in tensors]
    buffers = device.active().execute(sinks)
    for node in topological(sinks):
        if node.op is Op.ASSIGN:
            node.op, node.srcs, node.arg = Op.BUFFER, (), node.srcs[0].arg
    for node, buf in zip(sinks, buffers):
        if realized(node).op is not Op.BUFFER:
            node.op, node.srcs, node.arg = Op.BUFFER, (), buf
    return buffers


def scatter_rows(values: Tensor, indices: Tensor, shape: tuple[int, ...]) -> Tensor:
    if values.shape != indices.shape + tuple(shape[1:]):
        raise ValueError(f"scatter_rows: values {values.shape} do not match indices {indices.shape} into {shape}")
    node = Node(Op.SCATTER, (indices.node, values.node), values.dtype, tuple(shape))
    return Tensor.from_node(node, (values,), lambda g: (g.gather_rows(indices),))


def composed_attention(q: Tensor, k: Tensor, v: Tensor, *, causal: bool, scale: float, key_mask: Tensor | None = None) -> Tensor:
    return _attention_probs(q, k, causal=causal, scale=scale, key_mask=key_mask) @ v


def _attention_backward(out: Tensor, lse: Tensor, q: Tensor, k: Tensor, v: Tensor, mask: Tensor | None, *, causal: bool, scale: float) -> BackwardFn:
    """Fused backward through sdpa_bwd_q / sdpa_bwd_kv, or the composed form when the gradient is
    itself being differentiated or the device lacks either kernel."""

    def backward(g: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        dev = device.active()
        if grad_enabled or not (dev.has_custom(SDPA_BWD_Q) and dev.has_custom(SDPA_BWD_KV)):
            p = _attention_probs(q, k, causal=causal, scale=scale, key_mask=mask)
            dp = g @ v.transpose(-2, -1)
            ds = p * (dp - (dp * p).sum(axis=-1, keepdim=True)) * scale
            return ds @ k, ds.transpose(-2, -1) @ q, p.transpose(-2, -1) @ g
        do = _contiguous(g)
        stat = lse.dtype
        delta = (do.cast(stat) * out.cast(stat)).sum(axis=-1, keepdim=True)
        held = (q, k, v, do, lse, _contiguous(delta)) + ((mask,) if mask is not None else ())
        srcs = tuple(t.node for t in held)
        (dq,) = custom(SDPA_BWD_Q, srcs, (causal, scale), ((q.dtype, q.shape),))
        dk, dv = custom(SDPA_BWD_KV, srcs, (causal, scale), ((k.dtype, k.shape), (v.dtype, v.shape)))
        return Tensor.from_node(dq), Tensor.from_node(dk), Tensor.from_node(dv)

    return backward


def _attention_probs(q: Tensor, k: Tensor, *, causal: bool, scale: float, key_mask: Tensor | None = None) -> Tensor:
    scores = (q @ k.transpose(-2, -1)) * scale
    if causal:
        scores = _causal_mask(q.shape[-2], k.shape[-2]).where(scores, -1e9)
    if key_mask is not None:
        scores = key_mask.reshape(*key_mask.shape[:-1], 1, key_mask.shape[-1]).where(scores, -1e9)
    return scores.softmax(-1)


def _causal_mask(t_q: int, t_k: int) -> Tensor:
    return Tensor.arange(t_k).reshape(1, t_k) <= Tensor.arange(t_q).reshape(t_q, 1)


def _contiguous(t: Tensor) -> Tensor:
    if t.node.op is Op.BUFFER or t.node.op in CUT_OPS:
        return t
    return Tensor.from_node(Node(Op.CONTIGUOUS, (t.node,), t.dtype, t.shape), (t,), lambda g: (g,))


def as_ints(shape) -> tuple[int, ...]:
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        return tuple(int(s) for s in shape[0])
    return tuple(int(s) for s in shape)


def resolve_shape(shape: tuple[int, ...], numel: int) -> tuple[int, ...]:
    if shape.count(-1) > 1:
        raise ValueError(f"reshape: more than one -1 in {shape}")
    if -1 in shape:
        rest = math.prod(s for s in shape if s != -1)
        shape = tuple(numel // rest if s == -1 else s for s in shape)
    if any(s < 1 for s in shape):
        raise ValueError(f"reshape: invalid shape {shape}")
    return shape


def wrap_axis(axis: int, ndim: int) -> int:
    if not -ndim <= axis < ndim:
        raise ValueError(f"axis {axis} out of range for {ndim} dims")
    return axis % ndim


def canon_axes(axis, ndim: int) -> tuple[int, ...]:
    if axis is None:
        return tuple(range(ndim))
    axes = (axis,) if isinstance(axis, int) else tuple(axis)
    wrapped = tuple(sorted(wrap_axis(a, ndim) for a in axes))
    if len(set(wrapped)) != len(wrapped):
        raise ValueError(f"duplicate axes in {axes}")
    return wrapped


def as_tensor(x: Tensor | float | int, like: Tensor) -> Tensor:
    if isinstance(x, Tensor):
        return x
    dtype = like.dtype if like.dtype in FLOATS or isinstance(x, int) else float32
    return Tensor.const(x, dtype)


def zero(like: Tensor) -> Tensor:
    return Tensor.const(0, like.dtype)


def broadcast_shape(s1: tuple[int, ...], s2: tuple[int, ...], opname: str) -> tuple[int, ...]:
    n = max(len(s1), len(s2))
    a = (1,) * (n - len(s1)) + tuple(s1)
    b = (1,) * (n - len(s2)) + tuple(s2)
    for x, y in zip(a, b):
        if x != y and 1 not in (x, y):
            raise ValueError(f"{opname}: cannot broadcast {s1} with {s2}")
    return tuple(max(x, y) for x, y in zip(a, b))


def broadcast_to(t: Tensor, shape: tuple[int, ...], opname: str) -> Tensor:
    shape = tuple(shape)
    if t.shape == shape:
        return t
    if broadcast_shape(t.shape, shape, opname) != shape:
        raise ValueError(f"{opname}: cannot broadcast {t.shape} to {shape}")
    lifted = t.reshape(*((1,) * (len(shape) - t.ndim) + t.shape)) if t.ndim != len(shape) else t
    return lifted.expand(*shape)


def broadcast_pair(a: Tensor, b: Tensor | float | int, opname: str) -> tuple[Tensor, Tensor]:
    b = as_tensor(b, a)
    if a.dtype != b.dtype:
        wide = promote(a.dtype, b.dtype)
        a, b = a.cast(wide), b.cast(wide)
    shape = broadcast_shape(a.shape, b.shape, opname)
    return broadcast_to(a, shape, opname), broadcast_to(b, shape, opname)
