"""limn's numpy reference interpreter, restated (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Follows reference limn/device.py:63-175 node for node: one numpy call per node, memoized per
node identity, BUFFER reads see live bytes, ASSIGNs are deferred until every value of the batch
is computed (the transaction rule), SUM totals at `accumulate_in` width, SCATTER is np.add.at
into zeros (occurrence order), every result is cast to its node's dtype.

bfloat16 has no numpy dtype here (the reference uses ml_dtypes); a bfloat16 value is carried as
the float32 it holds, and every bfloat16 node's result is rounded to nearest even
(oracle/bf16.py) where the reference's `astype(bfloat16)` rounds. Buffers are flat uint8 arrays
holding the storage bytes (bfloat16 as its 16-bit patterns).

VIEW reads gather through `materialize` (reference limn/view.py:129-143). CUSTOM "sdpa*" nodes
run oracle/sdpa.py.

Pinned by tests/test_numpy_device.py: the reference tests' known answers (half sums total in
float32, int8 wraps, the assign transaction, capture's 8.0/12.0) and torch on the GRAPHS corpus.
"""

from __future__ import annotations

import weakref

import numpy as np

from limn_amd.dtypes import STORAGE, bf16_bits
from limn_amd.seam import DType, HostDevice, Node, Op, accumulate_in, bfloat16, float16, float32, float64, int8, int16, int32, view
from oracle import bf16
from oracle import sdpa as attention

COMPUTE = {
    float64: np.float64,
    float32: np.float32,
    float16: np.float16,
    bfloat16: np.float32,
    int32: np.int32,
    int16: np.int16,
    int8: np.int8,
}


def cast(values: np.ndarray, dtype: DType) -> np.ndarray:
    """Values at `dtype`'s width: astype for numpy dtypes, round-to-nearest-even for bfloat16."""
    out = np.asarray(values)
    if dtype == bfloat16:
        return bf16.rne(out.astype(np.float32))
    if out.dtype.kind == "f" and np.dtype(COMPUTE[dtype]).kind in "iu":
        with np.errstate(invalid="ignore"):
            return out.astype(COMPUTE[dtype])
    return out.astype(COMPUTE[dtype], copy=False)


def materialize(view: "view.View", flat: np.ndarray) -> np.ndarray:
    """Gather a view out of a flat array (reference limn/view.py:129-143): offset + sum(i*stride),
    masked positions read 0."""
    idx = np.full(view.shape, view.offset, dtype=np.int64)
    ok = np.ones(view.shape, dtype=bool)
    for d, (n, s) in enumerate(zip(view.shape, view.strides)):
        ax = np.arange(n).reshape((1,) * d + (n,) + (1,) * (len(view.shape) - d - 1))
        idx = idx + ax * s
        if view.mask is not None:
            lo, hi = view.mask[d]
            ok = ok & (ax >= lo) & (ax < hi)
    if view.mask is None:
        return flat[idx]
    return np.where(ok, flat[np.clip(idx, 0, flat.size - 1)], np.zeros((), dtype=flat.dtype))


def scatter_rounding_each_add(table: np.ndarray, indices: np.ndarray, values: np.ndarray) -> None:
    """np.add.at into a bfloat16 table (reference limn/device.py:155-157, a table of the node's
    own dtype): occurrences in order, each add done in float32 and rounded to bfloat16 at once,
    as ml_dtypes' add does. `table` holds bfloat16 values as float32."""
    rows = table.shape[0]
    flat_idx = np.asarray(indices).reshape(-1)
    flat_val = np.asarray(values, dtype=np.float32).reshape(flat_idx.size, *table.shape[1:])
    for j, r in enumerate(flat_idx):
        r = int(r) + rows if r < 0 else int(r)
        table[r] = bf16.rne(table[r] + flat_val[j])


def read_buffer(buf: np.ndarray, dtype: DType, shape) -> np.ndarray:
    raw = buf.view(STORAGE[dtype]).reshape(shape)
    return bf16.widen(raw) if dtype == bfloat16 else raw


def to_bytes(values: np.ndarray, dtype: DType) -> np.ndarray:
    if dtype == bfloat16:
        return bf16_bits(np.asarray(values, dtype=np.float32)).view(np.uint8).reshape(-1)
    return np.ascontiguousarray(np.asarray(values).astype(STORAGE[dtype])).view(np.uint8).reshape(-1)


def _sdpa_kernel(name: str, srcs: list[np.ndarray], node: Node) -> tuple[np.ndarray, ...]:
    causal, scale = node.arg.params
    dtype = node.srcs[0].dtype.name
    if name == "sdpa":
        mask = srcs[3] if len(srcs) == 4 else None
        return attention.sdpa(*srcs[:3], mask, causal=causal, scale=scale, dtype=dtype)
    mask = srcs[6] if len(srcs) == 7 else None
    if name == "sdpa_bwd_q":
        return (attention.sdpa_backward_q(*srcs[:6], mask, causal=causal, scale=scale, dtype=dtype),)
    return attention.sdpa_backward_kv(*srcs[:6], mask, causal=causal, scale=scale, dtype=dtype)


class NumpyDevice(HostDevice):
    def __init__(self) -> None:
        self.cache: weakref.WeakKeyDictionary = weakref.WeakKeyDictionary()
        self.custom = {"sdpa": _sdpa_kernel, "sdpa_bwd_q": _sdpa_kernel, "sdpa_bwd_kv": _sdpa_kernel}

    def has_custom(self, name: str) -> bool:
        return name in self.custom

    def execute(self, sinks: list[Node]) -> list:
        from limn_amd.seam import topological

        values = {node: self.compute(node) for node in topological(sinks)}
        assigns = [node for node in values if node.op is Op.ASSIGN]
        writes = [(node.srcs[0].arg, to_bytes(values[node], node.dtype)) for node in assigns]
        for buf, data in writes:
            buf[:] = data
        if assigns:
            self.cache.clear()
        out = []
        for sink in sinks:
            if sink.op is Op.BUFFER:
                out.append(sink.arg)
            elif sink.op is Op.ASSIGN:
                out.append(sink.srcs[0].arg)
            else:
                out.append(to_bytes(values[sink], sink.dtype).copy())
        return out

    def compute(self, node: Node) -> np.ndarray:
        if node.op is Op.BUFFER:
            return read_buffer(node.arg, node.dtype, node.shape)
        hit = self.cache.get(node)
        if hit is not None:
            return hit
        srcs = [self.compute(s) for s in node.srcs]
        op = node.op
        with np.errstate(all="ignore"):
            if op is Op.CONST:
                result = cast(np.full((), node.arg), node.dtype) if node.dtype == bfloat16 else np.full((), node.arg, dtype=COMPUTE[node.dtype])
            elif op is Op.VIEW:
                result = materialize(node.arg, srcs[0].reshape(-1))
            elif op is Op.NEG:
                result = -srcs[0]
            elif op is Op.EXP:
                result = np.exp(srcs[0])
            elif op is Op.LOG:
                result = np.log(srcs[0])
            elif op is Op.SQRT:
                result = np.sqrt(srcs[0])
            elif op is Op.RECIP:
                result = 1 / srcs[0]
            elif op is Op.CAST:
                result = cast(srcs[0], node.dtype)
            elif op is Op.ADD:
                result = srcs[0] + srcs[1]
            elif op is Op.MUL:
                result = srcs[0] * srcs[1]
            elif op is Op.CMPLT:
                result = (srcs[0] < srcs[1]).astype(COMPUTE[node.dtype])
            elif op is Op.WHERE:
                result = np.where(srcs[0] != 0, srcs[1], srcs[2])
            elif op is Op.SUM:
                result = srcs[0].sum(axis=node.arg, keepdims=True, dtype=COMPUTE[accumulate_in(node.dtype)])
            elif op is Op.MAX:
                result = srcs[0].max(axis=node.arg, keepdims=True)
            elif op is Op.GATHER:
                result = srcs[0][srcs[1]]
            elif op is Op.SCATTER:
                result = np.zeros(node.shape, dtype=COMPUTE[node.dtype])
                if node.dtype == bfloat16:
                    scatter_rounding_each_add(result, srcs[0], srcs[1])
                else:  # float16 arithmetic already rounds every add, as limn's half array does
                    np.add.at(result, srcs[0], srcs[1])
            elif op is Op.CONTIGUOUS:
                result = np.ascontiguousarray(srcs[0])
            elif op is Op.CUSTOM:
                fn = self.custom.get(node.arg.name)
                if fn is None:
                    raise NotImplementedError(f"the numpy device has no rule for custom op {node.arg.name!r}")
                result = fn(node.arg.name, srcs, node)[node.arg.index]
            elif op is Op.ASSIGN:
                result = srcs[1]
            else:
                raise NotImplementedError(f"NumpyDevice has no rule for {op}")
            result = cast(result, node.dtype)
        assert result.shape == node.shape, f"{op.name}: interpreter produced {result.shape}, graph says {node.shape}"
        self.cache[node] = result
        return result
