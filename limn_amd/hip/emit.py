"""The HIP emitter: limn's loop-nest IR (limn_amd/codegen.py) rendered as gfx950 kernels.

One hipRTC program per plan holds every nest's kernel; `nest_runners` compiles it (cached by
source hash) and returns one launcher per nest, in order, which is the `runners()` contract of
reference `limn/jit.py:113-115`. Semantics follow the reference's compiled backends
(limn/backend_c.py:54-143, limn/cuda_emit.py:45-373, 688-733): masked reads are 0, half widths
compute in float and round to nearest even on store, a CAST to a half width rounds, MAX
propagates NaN, narrow ints wrap, reduces total at `accumulate_in` width.

How each nest maps onto the GPU (designed for wave64 CDNA4, not the reference's
one-thread-per-cell launch):

- no reduce (elementwise, CONTIGUOUS, ASSIGN, GATHER, SCATTER): a grid-stride loop over output
  cells, VEC consecutive cells of the innermost (stride-1) dim per thread so a wave's loads and
  stores cover contiguous 16-byte runs;
- a reduce is `cells x reduce-space` whatever form the IR gave it (register ACC/UPDATE or
  in-place ACCUM). GROUP threads own a cell: 1 (a thread per cell, for short reduces and for the
  ACCUM form whose kept dim is the stride-1 one, so neighbouring threads read neighbouring
  columns), 64 (a wave per cell) or 256 (a workgroup per cell, for long rows: lanes stride
  through the row with VEC-wide runs, then a fixed butterfly across the wave and a fixed fold
  across waves in LDS). Every cell's total is formed in one fixed order, so reruns give the
  same bits;
- few cells over a long reduce (the reference's split reduce, limn/cuda_emit.py:134-149):
  PARTS workgroups per cell write partials to a scratch buffer, and a second kernel folds each
  cell's partials in index order;
- a float SCATTER gives np.add.at's bits: a tiled sort of the occurrences by row, then a
  workgroup per (row, 64 columns) adds that row's values in occurrence order (`plan_scatter`);
  float16 and bfloat16 tables round their running totals to their own width after every add,
  as np.add.at into a half-width array does (the reference's GPU device declines them). An
  int32 SCATTER adds with hardware atomics, which is exact in any order. The narrow ints are
  refused, as the reference's GPU device refuses them.
"""

from __future__ import annotations

import ctypes
import math
import re
from dataclasses import dataclass, field, replace

import numpy as np

from limn_amd.hip import replay, runtime
from limn_amd.seam import DType, Index, Instr, LoopNest, Node, Op, Opcode, Valid, accumulate_in, bfloat16, float16, float32, float64, int8, int16, int32

THREADS = 256

STORE_T = {float64: "double", float32: "float", float16: "unsigned short", bfloat16: "unsigned short", int32: "int", int16: "short", int8: "signed char"}
VALUE_T = {float64: "double", float32: "float", float16: "float", bfloat16: "float", int32: "int", int16: "short", int8: "signed char"}
HALVES = (float16, bfloat16)
INTS = (int32, int16, int8)

PRELUDE = r"""
typedef long long i64;
typedef unsigned short u16;
typedef signed char i8;
// every pointer a kernel takes is the start of a device allocation (views are index arithmetic),
// so 16-byte runs along the stride-1 dim may be one vector access
#define ALIGNED __attribute__((align_value(16)))
__device__ __forceinline__ float b2f(unsigned short b) { return __uint_as_float(((unsigned)b) << 16); }
__device__ __forceinline__ unsigned short f2b(float x) { __bf16 h = (__bf16)x; return __builtin_bit_cast(unsigned short, h); }
__device__ __forceinline__ float h2f(unsigned short b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ unsigned short f2h(float x) { return __builtin_bit_cast(unsigned short, (_Float16)x); }
template <typename T> __device__ __forceinline__ T fmax_nan(T a, T b) { return (a > b || a != a) ? a : b; }
template <typename T> __device__ __forceinline__ T fadd(T a, T b) { return a + b; }
__device__ __forceinline__ int fadd(int a, int b) { return (int)((unsigned)a + (unsigned)b); }
__device__ __forceinline__ short fadd(short a, short b) { return (short)(a + b); }
__device__ __forceinline__ signed char fadd(signed char a, signed char b) { return (signed char)(a + b); }
template <typename T> __device__ __forceinline__ T wave_fold_add(T x) {
  for (int s = 32; s > 0; s >>= 1) x = fadd(x, (T)__shfl_xor(x, s));
  return x;
}
template <typename T> __device__ __forceinline__ T wave_fold_max(T x) {
  for (int s = 32; s > 0; s >>= 1) x = fmax_nan(x, (T)__shfl_xor(x, s));
  return x;
}
"""


def literal(value: float | int, dtype: DType) -> str:
    """A scalar as a literal of the dtype's compute type (a half-width literal is the float it
    rounds to)."""
    if dtype in INTS:
        v = int(value)
        bits = 8 * dtype.itemsize
        v = ((v + (1 << (bits - 1))) % (1 << bits)) - (1 << (bits - 1))
        if v == -(1 << 31):
            return "(-2147483647 - 1)"
        return f"({VALUE_T[dtype]})({v})"
    v = float(value)
    if dtype == float16:
        v = float(np.float16(v))
    elif dtype == bfloat16:
        from limn_amd.dtypes import bf16_bits, bf16_values

        v = float(bf16_values(bf16_bits(np.array([v], dtype=np.float32)))[0])
    if math.isnan(v):
        return "__builtin_nan(\"\")" if dtype == float64 else "__builtin_nanf(\"\")"
    if math.isinf(v):
        s = "-" if v < 0 else ""
        return f"({s}__builtin_inf())" if dtype == float64 else f"({s}__builtin_inff())"
    if dtype == float64:
        return repr(v)
    f = float(np.float32(v))
    if math.isinf(f):  # a finite double past float32's range
        return "(-__builtin_inff())" if f < 0 else "(__builtin_inff())"
    return repr(f) + "f"


def load_expr(dtype: DType, ref: str) -> str:
    if dtype == bfloat16:
        return f"b2f({ref})"
    if dtype == float16:
        return f"h2f({ref})"
    return ref


def store_line(ref: str, value: str, stream: bool) -> str:
    """`ref = value;`, or with `stream` the same store marked non-temporal."""
    return f"__builtin_nontemporal_store({value}, &{ref});" if stream else f"{ref} = {value};"


def store_expr(dtype: DType, value: str) -> str:
    if dtype == bfloat16:
        return f"f2b({value})"
    if dtype == float16:
        return f"f2h({value})"
    return f"({STORE_T[dtype]})({value})"


def arith(op: Op, srcs: tuple[str, ...], dtype: DType) -> str:
    """One ARITH instruction as a C expression at the value type of `dtype`. A half-width node
    (bf16, f16) is computed in float and rounded to 8 or 11 significand bits, so its EXP and RECIP
    take the hardware's approximations (v_exp_f32 on x log2 e, v_rcp_f32: within 2 ulp of float,
    far under that rounding) instead of the correctly rounded library forms, which cost ten or more
    instructions each: a composed tanh GELU over a (16384, 2048) bf16 activation is bound by them."""
    t = VALUE_T[dtype]
    wide = dtype == float64
    half = dtype in (bfloat16, float16)
    if op is Op.NEG:
        return f"({t})(-{srcs[0]})"
    if op is Op.EXP:
        return f"__expf({srcs[0]})" if half else f"{'exp' if wide else 'expf'}({srcs[0]})"
    if op is Op.LOG:
        return f"{'log' if wide else 'logf'}({srcs[0]})"
    if op is Op.SQRT:
        return f"{'sqrt' if wide else 'sqrtf'}({srcs[0]})"
    if op is Op.RECIP:
        if half:
            return f"__builtin_amdgcn_rcpf({srcs[0]})"
        return f"({'1.0' if wide else '1.0f'} / {srcs[0]})"
    if op is Op.ADD:
        return f"fadd(({t}){srcs[0]}, ({t}){srcs[1]})" if dtype in INTS else f"({srcs[0]} + {srcs[1]})"
    if op is Op.MUL:
        if dtype == int32:
            return f"(int)((unsigned){srcs[0]} * (unsigned){srcs[1]})"
        return f"({t})({srcs[0]} * {srcs[1]})"
    if op is Op.CMPLT:
        return f"({t})({srcs[0]} < {srcs[1]})"
    if op is Op.WHERE:
        return f"(({srcs[0]}) != 0 ? ({srcs[1]}) : ({srcs[2]}))"
    raise NotImplementedError(f"no HIP lowering for {op}")


@dataclass
class Buffers:
    """Element types of a nest's buffers by name (in0.., out) and whether 64-bit indexing is needed.
    `inline` maps an input's name to the producer evaluated in its place (see `inline_producers`),
    whose own inputs are the kernel's `extra` parameters, after in0.. and before out."""

    dtypes: dict[str, DType]
    wide_index: bool
    inline: dict[str, "Inlined"] = field(default_factory=dict)
    extra: list[str] = field(default_factory=list)
    # a row program's per-row values: a load of this buffer reads the named variable (the value
    # an earlier member of the program stored for this row) rounded as its store rounded it
    rowvals: dict[str, tuple[str, DType]] = field(default_factory=dict)
    # a row program's cached row: the load defining this value reads the named register instead
    cached: dict[str, str] = field(default_factory=dict)


@dataclass(frozen=True)
class Inlined:
    """A small elementwise nest evaluated where a reader loads its output: its body with every
    name prefixed, its loop variables over its output shape, and the rounding of its store."""

    space: tuple[tuple[str, int], ...]
    body: tuple[Instr, ...]
    result: str
    dtype: DType


def input_params(nest: LoopNest, bufs: Buffers) -> list[str]:
    params = [f"const {STORE_T[n.dtype]}* __restrict__ ALIGNED in{k}" for k, n in enumerate(nest.kernel.inputs)]
    return params + [f"const {STORE_T[bufs.dtypes[name]]}* __restrict__ ALIGNED {name}" for name in bufs.extra]


def render_index(index: Index, wide: bool) -> str:
    if not index.terms:
        return str(index.const)
    cast = "(i64)" if wide else ""
    parts = [f"{cast}{var}" if c == 1 else f"{cast}{var} * {c}" for var, c in index.terms]
    text = " + ".join(parts)
    if index.const:
        text += f" + {index.const}" if index.const > 0 else f" - {-index.const}"
    return text


def value_line(instr: Instr, bufs: Buffers) -> str:
    """One value-defining instruction as a declaration."""
    t = VALUE_T[instr.value_type]
    op = instr.opcode
    if op is Opcode.CONST:
        value, valid = instr.arg
        lit = literal(value, instr.value_type)
        if valid.bounds:
            return f"const {t} {instr.dest} = ({valid.render()}) ? {lit} : ({t})0;"
        return f"const {t} {instr.dest} = {lit};"
    if op is Opcode.LOAD and instr.dest in bufs.cached:
        return f"const {t} {instr.dest} = ({t}){bufs.cached[instr.dest]};"
    if op is Opcode.LOAD and instr.arg[0] in bufs.rowvals:
        var, dt = bufs.rowvals[instr.arg[0]]
        return f"const {t} {instr.dest} = ({t}){load_expr(dt, store_expr(dt, var))};"
    if op is Opcode.LOAD and instr.arg[0] in bufs.inline:
        return inline_load(instr, bufs.inline[instr.arg[0]], bufs)
    if op is Opcode.LOAD:
        buf, index, valid = instr.arg
        ref = load_expr(bufs.dtypes[buf], f"{buf}[{render_index(index, bufs.wide_index)}]")
        if valid.bounds:
            return f"const {t} {instr.dest} = ({valid.render()}) ? ({t}){ref} : ({t})0;"
        return f"const {t} {instr.dest} = ({t}){ref};"
    if op is Opcode.ARITH:
        return f"const {t} {instr.dest} = {arith(instr.arg, instr.srcs, instr.value_type)};"
    if op is Opcode.CAST:
        dt = instr.value_type
        src = instr.srcs[0]
        if dt == bfloat16:
            return f"const float {instr.dest} = b2f(f2b((float){src}));"
        if dt == float16:
            return f"const float {instr.dest} = h2f(f2h((float){src}));"
        return f"const {t} {instr.dest} = ({t})({src});"
    if op is Opcode.GATHER:
        buf, index = instr.arg
        ref = load_expr(bufs.dtypes[buf], f"{buf}[{render_index(index, True)}]")
        return f"const {t} {instr.dest} = ({t}){ref};"
    raise NotImplementedError(f"{op} does not define a value")


def inline_load(instr: Instr, src: Inlined, bufs: Buffers) -> str:
    """A load of an inlined producer's output: the producer's body evaluated at the loaded
    element (its loop variables decoded from the flat index), rounded as its store and this
    load would round it. Out of a masked load's bounds nothing is evaluated and the value is 0."""
    t = VALUE_T[instr.value_type]
    _, index, valid = instr.arg
    lines = [f"{t} {instr.dest} = ({t})0;"]
    lines.append(f"if ({valid.render()}) {{" if valid.bounds else "{")
    lines += decode(list(src.space), f"(i64)({render_index(index, True)})", "  ", True)
    lines += ["  " + value_line(i, bufs) for i in src.body]
    lines.append(f"  {instr.dest} = ({t}){load_expr(src.dtype, store_expr(src.dtype, src.result))};")
    lines.append("}")
    return "\n".join(lines)


@dataclass
class NestShape:
    """A nest read as cells x reduce-space."""

    outer: list[tuple[str, int]]
    inner: list[tuple[str, int]]
    body: list[Instr]
    write: Instr | None  # STORE/SCATTER for elementwise; the final STORE for a register reduce
    fold: Op | None  # ADD / MAX for reduces
    identity: float | int | None
    out_index: Index | None
    accum_form: bool = False
    reduce_dtype: DType | None = None
    item: str = ""


def read_nest(nest: LoopNest) -> NestShape:
    ins = list(nest.instrs)
    loops: dict[str, int] = {}
    for instr in ins:
        if instr.opcode is Opcode.LOOP:
            loops[instr.dest] = instr.arg
    if any(i.opcode is Opcode.ACCUM for i in ins):
        # STORE identity over the outer loops, then LOOP(all) ... ACCUM
        first_end = next(k for k, i in enumerate(ins) if i.opcode is Opcode.STORE)
        init = [i for i in ins[:first_end] if i.opcode is Opcode.CONST]
        identity = init[0].arg[0]
        outer_vars = [i.dest for i in ins[:first_end] if i.opcode is Opcode.LOOP]
        k = first_end
        while ins[k].opcode is not Opcode.LOOP:
            k += 1
        order_vars = []
        while ins[k].opcode is Opcode.LOOP:
            order_vars.append(ins[k].dest)
            k += 1
        accum = next(i for i in ins if i.opcode is Opcode.ACCUM)
        body = [i for i in ins[k:] if i.opcode not in (Opcode.ACCUM, Opcode.ENDLOOP, Opcode.LOOP)]
        inner = [(v, loops[v]) for v in order_vars if v not in outer_vars]
        return NestShape(
            outer=[(v, loops[v]) for v in outer_vars],
            inner=inner,
            body=body,
            write=None,
            fold=accum.arg[2],
            identity=identity,
            out_index=accum.arg[1],
            accum_form=True,
            reduce_dtype=accum.dtype,
            item=accum.srcs[0],
        )
    acc = next((i for i in ins if i.opcode is Opcode.ACC), None)
    if acc is not None:
        k_acc = ins.index(acc)
        outer_vars = [i.dest for i in ins[:k_acc] if i.opcode is Opcode.LOOP]
        update = next(i for i in ins if i.opcode is Opcode.UPDATE)
        k_upd = ins.index(update)
        inner_vars = [i.dest for i in ins[k_acc:k_upd] if i.opcode is Opcode.LOOP]
        body = [i for i in ins[k_acc:k_upd] if i.opcode not in (Opcode.LOOP, Opcode.ENDLOOP, Opcode.ACC)]
        store = next(i for i in ins[k_upd:] if i.opcode is Opcode.STORE)
        return NestShape(
            outer=[(v, loops[v]) for v in outer_vars],
            inner=[(v, loops[v]) for v in inner_vars],
            body=body,
            write=store,
            fold=update.arg,
            identity=acc.arg,
            out_index=store.arg[1],
            reduce_dtype=acc.dtype,
            item=update.srcs[0],
        )
    outer_vars = [i.dest for i in ins if i.opcode is Opcode.LOOP]
    body = [i for i in ins if i.opcode not in (Opcode.LOOP, Opcode.ENDLOOP, Opcode.STORE, Opcode.SCATTER)]
    write = next(i for i in ins if i.opcode in (Opcode.STORE, Opcode.SCATTER))
    return NestShape(outer=[(v, loops[v]) for v in outer_vars], inner=[], body=body, write=write, fold=None, identity=None, out_index=None)


def decode(vars_: list[tuple[str, int]], flat: str, indent: str, wide: bool) -> list[str]:
    """Loop variables from a flat index, the last one fastest."""
    if not vars_:
        return []
    scratch = "i64" if wide else "int"
    lines = [f"{indent}{scratch} t_ = {flat};"]
    for var, extent in reversed(vars_[1:]):
        lines.append(f"{indent}const int {var} = (int)(t_ % {extent}); t_ /= {extent};")
    lines.append(f"{indent}const int {vars_[0][0]} = (int)t_;")
    return lines


@dataclass
class Launch:
    name: str
    grid: int
    block: int
    args: str  # "io" (inputs then out), "io_scratch" (inputs then scratch), "io_scratch_out", "scratch_out"


@dataclass
class Planned:
    """What one nest became: kernels to launch in order, and the scratch bytes they share; or a
    dense contraction handed to liblimn_hip.so's MFMA kernel (`contraction`)."""

    source: str
    launches: list[Launch]
    scratch_bytes: int = 0
    notes: dict = field(default_factory=dict)
    contraction: "Contraction | None" = None


@dataclass(frozen=True)
class Contraction:
    """A SUM nest that is c[b, m, n] = sum_k a[b, m, k] * b[b, k, n] over two input buffers, with
    every stride in elements (the arguments of limn_hip_matmul)."""

    a_input: int
    b_input: int
    a_offset: int
    b_offset: int
    dtype: DType
    batch: int
    M: int
    N: int
    K: int
    a_batch: int
    a_m: int
    a_k: int
    b_batch: int
    b_k: int
    b_n: int
    c_batch: int
    c_m: int
    c_n: int


def _flat_stride(coeffs: dict[str, int], batch_vars: list[tuple[str, int]]) -> int | None:
    """One stride for the row-major flattening of the batch vars, if the operand's coefficients
    allow it (all zero is a broadcast: stride 0)."""
    if not batch_vars:
        return 0
    stride = coeffs.get(batch_vars[-1][0], 0)
    expect = stride
    for j in range(len(batch_vars) - 1, 0, -1):
        expect = expect * batch_vars[j][1]
        if coeffs.get(batch_vars[j - 1][0], 0) != expect:
            return None
    return stride


def _flat_reduce(inner: list[tuple[str, int]], ta: dict[str, int], tb: dict[str, int]) -> tuple[int, int, int] | None:
    """Several reduce vars as one k: both operands must step through them as one row-major
    index (each var's stride the next one's extent times its stride, in the same order for both),
    as a weight gradient's sum over (batch, time) does. Returns (K, k stride in a, in b)."""
    extent = dict(inner)
    if any(v not in ta or v not in tb or ta[v] <= 0 or tb[v] <= 0 for v in extent):
        return None
    order = sorted(extent, key=lambda v: -ta[v])
    for outer, nxt in zip(order, order[1:]):
        if ta[outer] != extent[nxt] * ta[nxt] or tb[outer] != extent[nxt] * tb[nxt]:
            return None
    last = order[-1]
    return math.prod(extent.values()), ta[last], tb[last]


def find_contraction(nest: LoopNest, shape: NestShape) -> Contraction | None:
    """The dense-contraction reading of a reduce nest (reference limn/cuda_emit.py:376-505
    detects the same shape, over one reduce var): a body of exactly two unmasked loads and their
    product, each load depending on every reduce var (flattened into one k, see _flat_reduce),
    the batch vars and one row var of its own."""
    if shape.fold is not Op.ADD or not shape.inner or len(shape.body) != 3:
        return None
    loads = [i for i in shape.body if i.opcode is Opcode.LOAD]
    mul = [i for i in shape.body if i.opcode is Opcode.ARITH and i.arg is Op.MUL]
    if len(loads) != 2 or len(mul) != 1 or shape.item != mul[0].dest or set(mul[0].srcs) != {loads[0].dest, loads[1].dest}:
        return None
    if any(l.arg[2].bounds for l in loads):
        return None
    dtype = loads[0].value_type
    if dtype not in (bfloat16, float16) or loads[1].value_type != dtype or shape.reduce_dtype != dtype:
        return None
    if nest.kernel.target.dtype != dtype:
        return None
    kept = sorted(shape.outer, key=lambda ve: int(ve[0][1:]))
    ta, tb = dict(loads[0].arg[1].terms), dict(loads[1].arg[1].terms)
    reduce = _flat_reduce(shape.inner, ta, tb)
    if reduce is None:
        return None
    K, red_a, red_b = reduce
    only_a = [v for v, _ in kept if v in ta and v not in tb]
    only_b = [v for v, _ in kept if v in tb and v not in ta]
    if not only_a or not only_b:
        return None
    m_var, n_var = only_a[-1], only_b[-1]  # the row dims come after any batch dims an operand broadcasts
    extent = dict(kept)
    batch_vars = [(v, e) for v, e in kept if v not in (m_var, n_var)]
    tc = dict(shape.out_index.terms)
    if tc.get(m_var, 0) == 0 or tc.get(n_var, 0) == 0 or shape.out_index.const != 0:
        return None
    a_b, b_b, c_b = (_flat_stride(t, batch_vars) for t in (ta, tb, tc))
    if a_b is None or b_b is None or c_b is None:
        return None
    batch = math.prod(e for _, e in batch_vars)
    M, N = extent[m_var], extent[n_var]
    a_in, b_in = int(loads[0].arg[0][2:]), int(loads[1].arg[0][2:])
    a_m, a_k, b_n, b_k = ta[m_var], red_a, tb[n_var], red_b
    c_m, c_n = tc[m_var], tc[n_var]
    if batch > 1 and b_b == 0 and a_b == M * a_m and c_b == M * c_m:
        M, batch, a_b, c_b = M * batch, 1, 0, 0  # a shared right operand: one taller contraction
    con = Contraction(a_in, b_in, loads[0].arg[1].const, loads[1].arg[1].const, dtype, batch, M, N, K, a_b, a_m, a_k, b_b, b_k, b_n, c_b, c_m, c_n)
    if con.a_offset % 8 or con.b_offset % 8:
        return None
    from limn_amd.dtypes import ABI_CODE

    lib = runtime.kernels()
    ok = lib.limn_hip_matmul_supported(ABI_CODE[dtype], M, N, K, a_b, a_m, a_k, b_b, b_k, b_n)
    return con if ok else None


def _vec_width(nest_shape: NestShape, bufs: Buffers, var: str, extent: int) -> int:
    """How many consecutive values of `var` one thread takes: 16 bytes of the narrowest buffer
    stepping along it, when the extent divides."""
    widths = [bufs.dtypes[b].itemsize for b in bufs.dtypes]
    v = 16 // max(1, min(widths)) if widths else 4
    v = max(1, min(v, 8))
    while v > 1 and extent % v:
        v //= 2
    return v


def signature(name: str, nest: LoopNest, out_dtype: DType, bufs: Buffers, extra: str = "") -> str:
    params = input_params(nest, bufs)
    params.append(f"{STORE_T[out_dtype]}* __restrict__ ALIGNED out")
    if extra:
        params.append(extra)
    return f'extern "C" __global__ __launch_bounds__({THREADS}) void {name}({", ".join(params)})'


def run_start(index: Index, var: str, vec: int) -> str:
    """The index of a run's first element: `var` at `var`_b * vec."""
    at0 = Index(index.const, tuple((f"({var}_b * {vec})" if v == var else v, c) for v, c in index.terms))
    return render_index(at0, True)


def run_loads(nest: LoopNest, body: list[Instr], bufs: Buffers, var: str, vec: int, indent: str) -> tuple[list[str], dict[str, list[str]]]:
    """Pointers to the first element of each VEC run of the loads that step through `var` with
    stride 1 (set before the j_ loop), and the lines that replace those loads inside it."""
    sizes = {f"in{k}": math.prod(n.shape) for k, n in enumerate(nest.kernel.inputs)}
    pre: list[str] = []
    runs: dict[str, list[str]] = {}
    for instr in body:
        if instr.opcode is not Opcode.LOAD:
            continue
        buf, index, valid = instr.arg
        if buf in bufs.inline or buf in bufs.rowvals or instr.dest in bufs.cached or any(b[0] == var for b in valid.bounds):
            continue
        if dict(index.terms).get(var) != 1 or sizes.get(buf, 0) < vec:
            continue
        d, t, dt = instr.dest, VALUE_T[instr.value_type], bufs.dtypes[buf]
        if not valid.bounds:
            pre.append(f"{indent}const {STORE_T[dt]}* {d}_p = {buf} + (i64)({run_start(index, var, vec)});")
            runs[d] = [f"const {t} {d} = ({t}){load_expr(dt, f'{d}_p[j_]')};"]
            continue
        pre.append(f"{indent}const bool {d}_ok = {valid.render()};")
        pre.append(f"{indent}const {STORE_T[dt]}* {d}_p = {buf} + ({d}_ok ? (i64)({run_start(index, var, vec)}) : (i64)0);")
        runs[d] = [f"const {t} {d}_raw = ({t}){load_expr(dt, f'{d}_p[j_]')};", f"const {t} {d} = {d}_ok ? {d}_raw : ({t})0;"]
    return pre, runs


def prefetch_row(body: list[Instr], bufs: Buffers, var: str, vec: int, tag: str,
                 indent: str) -> tuple[list[str], list[str], dict[str, str]]:
    """The plain (unmasked) loads of a nest body for one run of `vec` values of `var`, as
    registers filled ahead of the arithmetic: their declarations, the loads (in the scope where
    the loop variables are decoded and `var`_b is set) and the `Buffers.cached` entries that make
    the body read them."""
    decls: list[str] = []
    loads: list[str] = []
    cached: dict[str, str] = {}
    for instr in body:
        if instr.opcode is not Opcode.LOAD:
            continue
        buf, index, valid = instr.arg
        if buf in bufs.inline or buf in bufs.rowvals or valid.bounds:
            continue
        dt, d = bufs.dtypes[buf], instr.dest
        st, reg = STORE_T[dt], f"{tag}{instr.dest}"
        steps = dict(index.terms).get(var)
        if steps is None:
            decls.append(f"{st} {reg};")
            loads.append(f"{indent}{reg} = {buf}[{render_index(index, bufs.wide_index)}];")
            cached[d] = load_expr(dt, reg)
            continue
        decls.append(f"{st} {reg}[{vec}];")
        if steps == 1:
            loads.append(f"{indent}{{ const {st}* p_ = {buf} + (i64)({run_start(index, var, vec)});")
            loads.append(f"{indent}#pragma unroll")
            loads.append(f"{indent}  for (int j_ = 0; j_ < {vec}; j_++) {reg}[j_] = p_[j_]; }}")
        else:
            loads.append(f"{indent}#pragma unroll")
            loads.append(f"{indent}for (int j_ = 0; j_ < {vec}; j_++) {{ const int {var} = {var}_b * {vec} + j_; "
                         f"{reg}[j_] = {buf}[{render_index(index, True)}]; }}")
        cached[d] = load_expr(dt, f"{reg}[j_]")
    return decls, loads, cached


TRANSPOSE_TILE = 64  # a transposing nest's tile edge along each of its two variables
ONE_WORD = {"unsigned short": "u16", "signed char": "i8"}  # storage types as one-word names
TRANSPOSE_MIN_CELLS = 1 << 14  # the fewest output cells planned as tiles


def transposed_loads(shape: NestShape, bufs: Buffers) -> tuple[str, list[Instr]] | None:
    """The variable, and the loads, of an elementwise nest that reads across its output's rows:
    plain loads contiguous along one variable `across` other than the output's stride-1 variable,
    which they step by a stride above 1 (an optimizer reading a gradient realized transposed, a
    contiguous copy of a transposed view). Read one cell per lane along the output's rows, each
    such load touches a cache line per lane; `plan_transposed` reads them along `across`."""
    write = shape.write
    if write is None or write.opcode is not Opcode.STORE or len(shape.outer) < 2:
        return None
    inner, extent = shape.outer[-1]
    if dict(write.arg[1].terms).get(inner) != 1 or extent < 16 or math.prod(e for _, e in shape.outer) < TRANSPOSE_MIN_CELLS:
        return None
    extents = dict(shape.outer)
    across, found = None, []
    for instr in shape.body:
        if instr.opcode is not Opcode.LOAD:
            continue
        buf, index, _ = instr.arg
        if buf in bufs.inline or buf in bufs.rowvals or instr.dest in bufs.cached:
            continue
        step = dict(index.terms).get(inner)
        ones = [v for v, c in index.terms if c == 1 and v != inner and v in extents]
        if step is None or step == 1 or not ones:
            continue
        if across not in (None, ones[0]):
            return None
        across = ones[0]
        found.append(instr)
    if across is None or extents[across] < 16:
        return None
    return across, found


def plan_transposed(nest: LoopNest, shape: NestShape, bufs: Buffers, across: str, loads: list[Instr],
                    stream: bool) -> Planned:
    """An elementwise nest with loads contiguous along `across` (see transposed_loads), by tiles
    of TRANSPOSE_TILE x TRANSPOSE_TILE cells over (`across`, the output's stride-1 variable), a
    workgroup per tile, grid-strided: the lanes of a wave first read each such load along
    `across` into an LDS tile (row pitch TILE+1 elements, so the transposed reads that follow hit
    distinct banks), then compute and store a row of the output each, reading those loads from
    the tile and every other load in place. The values are the ones the plain plan computes: the
    same body, evaluated once per cell."""
    T = TRANSPOSE_TILE
    rows_per = THREADS // T
    out_dtype = nest.kernel.target.dtype
    write = shape.write
    assert write is not None
    inner, B = shape.outer[-1]
    A = dict(shape.outer)[across]
    rest = [(v, e) for v, e in shape.outer if v not in (inner, across)]
    tiles = math.prod(e for _, e in rest) * -(-A // T) * -(-B // T)
    wide = bufs.wide_index or math.prod(e for _, e in shape.outer) > (1 << 30)
    lines = [signature(nest.name, nest, out_dtype, bufs) + " {", "  const i64 bid_ = blockIdx.x, nblk_ = gridDim.x;"]
    refs = {}
    for instr in loads:
        st = ONE_WORD.get(STORE_T[bufs.dtypes[instr.arg[0]]], STORE_T[bufs.dtypes[instr.arg[0]]])
        lines.append(f"  __shared__ {st} xt_{instr.dest}[{T * (T + 1)}];")
        refs[instr.dest] = load_expr(bufs.dtypes[instr.arg[0]], f"xt_{instr.dest}[lb_ * {T + 1} + r_]")
    lines.append(f"  const int lb_ = threadIdx.x & {T - 1};")
    lines.append(f"  for (i64 tile_ = bid_; tile_ < {tiles}LL; tile_ += nblk_) {{")
    lines += decode(rest + [("ta_", -(-A // T)), ("tb_", -(-B // T))], "tile_", "    ", wide)
    lines.append("    {")
    lines.append(f"      const int {across} = ta_ * {T} + lb_;")
    lines.append("#pragma unroll 4")
    lines.append(f"      for (int r_ = threadIdx.x / {T}; r_ < {T}; r_ += {rows_per}) {{")
    lines.append(f"        const int {inner} = tb_ * {T} + r_;")
    lines.append(f"        if ({across} < {A} && {inner} < {B}) {{")
    for instr in loads:
        buf, index, valid = instr.arg
        st = STORE_T[bufs.dtypes[buf]]
        ref = f"{buf}[{render_index(index, wide)}]"
        if valid.bounds:
            ref = f"({valid.render()}) ? {ref} : ({st})0"
        lines.append(f"          xt_{instr.dest}[r_ * {T + 1} + lb_] = {ref};")
    lines += ["        }", "      }", "    }", "    __syncthreads();"]
    view = replace(bufs, cached={**bufs.cached, **refs})
    lines.append(f"    const int {inner} = tb_ * {T} + lb_;")
    lines.append("#pragma unroll 2")
    lines.append(f"    for (int r_ = threadIdx.x / {T}; r_ < {T}; r_ += {rows_per}) {{")
    lines.append(f"      const int {across} = ta_ * {T} + r_;")
    lines.append(f"      if ({across} < {A} && {inner} < {B}) {{")
    lines += ["        " + value_line(instr, view) for instr in shape.body]
    buf, index = write.arg
    lines.append(f"        {store_line(f'{buf}[{render_index(index, wide)}]', store_expr(out_dtype, write.srcs[0]), stream)}")
    lines += ["      }", "    }", "    __syncthreads();", "  }", "}"]
    grid = max(1, min(tiles, 1 << 20))
    notes: dict = {"elementwise": True, "transposed": across, "body": lines[2:-1]}
    notes["params"] = [(STORE_T[n.dtype], f"in{k}", True) for k, n in enumerate(nest.kernel.inputs)]
    notes["params"] += [(STORE_T[bufs.dtypes[name]], name, True) for name in bufs.extra]
    notes["params"].append((STORE_T[out_dtype], "out", False))
    return Planned("\n".join(lines), [Launch(nest.name, grid, THREADS, "io")], notes=notes)


def plan_elementwise(nest: LoopNest, shape: NestShape, bufs: Buffers, stream: bool = False) -> Planned:
    """One thread per run of `vec` output cells, grid-strided. With `stream`, the output goes
    out through non-temporal stores (see STREAM_BYTES). A nest that reads across its output's
    rows goes by tiles instead (see transposed_loads)."""
    across = transposed_loads(shape, bufs)
    if across is not None:
        return plan_transposed(nest, shape, bufs, across[0], across[1], stream)
    cells = math.prod(e for _, e in shape.outer)
    write = shape.write
    assert write is not None
    out_dtype = nest.kernel.target.dtype
    inner_var, inner_extent = shape.outer[-1] if shape.outer else ("", 1)
    vec = _vec_width(shape, bufs, inner_var, inner_extent) if shape.outer and write.opcode is Opcode.STORE else 1
    wide = bufs.wide_index or cells > (1 << 30)
    lines = [signature(nest.name, nest, out_dtype, bufs) + " {", "  const i64 bid_ = blockIdx.x, nblk_ = gridDim.x;"]
    groups = cells // vec
    lines.append(f"  for (i64 g = bid_ * {THREADS} + threadIdx.x; g < {groups}LL; g += nblk_ * {THREADS}) {{")
    # Loads and the store that step through the stride-1 var take a pointer to the run's first
    # element, set once per run, and index it by j_: the run is then visibly one 16-byte access
    # (computed from the full index per element, the compiler split some runs into 2-, 4- and
    # 8-byte pieces). A masked load whose mask does not involve the stride-1 var is valid for
    # the whole run or for none of it: its pointer is the buffer's start when masked (in bounds
    # for VEC elements) and the run's loads are unconditional, so they too merge into one vector
    # load instead of VEC branches around 2-byte loads.
    runs: dict[str, list[str]] = {}
    pre: list[str] = []
    store_run = None
    if shape.outer and vec > 1 and write.opcode is Opcode.STORE:
        pre, runs = run_loads(nest, shape.body, bufs, inner_var, vec, "    ")
        out_index = write.arg[1]
        if dict(out_index.terms).get(inner_var) == 1:
            pre.append(f"    {STORE_T[out_dtype]}* out_p = out + (i64)({run_start(out_index, inner_var, vec)});")
            store_run = f"      {store_line('out_p[j_]', store_expr(out_dtype, write.srcs[0]), stream)}"
    if shape.outer:
        base_vars = shape.outer[:-1] + [(inner_var + "_b", inner_extent // vec)]
        lines += decode(base_vars, "g", "    ", wide)
        lines += pre
        lines.append("#pragma unroll")
        lines.append(f"    for (int j_ = 0; j_ < {vec}; j_++) {{")
        lines.append(f"      const int {inner_var} = {inner_var}_b * {vec} + j_;")
    else:
        lines.append("    {")
    for instr in shape.body:
        if instr.dest in runs:
            lines += ["      " + ln for ln in runs[instr.dest]]
            continue
        lines.append("      " + value_line(instr, bufs))
    buf, index = write.arg
    if write.opcode is Opcode.SCATTER:
        if out_dtype not in (float32, float64, float16, bfloat16, int32):
            raise NotImplementedError(f"the hip device cannot scatter {out_dtype}; cast the table to float32 or int32")
        if out_dtype != int32:
            return plan_scatter(nest, shape, bufs)
        lines.append(f"      atomicAdd(&{buf}[{render_index(index, True)}], ({STORE_T[out_dtype]}){write.srcs[0]});")
    elif store_run is not None:
        lines.append(store_run)
    else:
        lines.append(f"      {store_line(f'{buf}[{render_index(index, wide)}]', store_expr(out_dtype, write.srcs[0]), stream)}")
    lines += ["    }", "  }", "}"]
    grid = max(1, min(-(-groups // THREADS), 1 << 20))
    notes: dict = {"elementwise": True}
    if write.opcode is Opcode.STORE:
        # the body between the block-index line and the closing brace, for merge_runs
        notes["body"] = lines[2:-1]
        notes["params"] = [(STORE_T[n.dtype], f"in{k}", True) for k, n in enumerate(nest.kernel.inputs)]
        notes["params"] += [(STORE_T[bufs.dtypes[name]], name, True) for name in bufs.extra]
        notes["params"].append((STORE_T[out_dtype], "out", False))
    return Planned("\n".join(lines), [Launch(nest.name, grid, THREADS, "io")], notes=notes)


SORT_TILE_LIMITS = ((1 << 16, 256), (1 << 20, 1024))  # occurrences -> occurrences per sorted tile
SORT_TILE_MAX = 4096
LIST_CAP = 1024  # a row's occurrences gathered in LDS per pass of the accumulating kernel


def _reads(instr: Instr) -> set[str]:
    """Every name an instruction reads: its operands, the variables of its index and of its
    bound checks."""
    names = set(instr.srcs)
    if instr.opcode in (Opcode.LOAD, Opcode.GATHER):
        names |= {v for v, _ in instr.arg[1].terms}
    if instr.opcode is Opcode.LOAD:
        names |= {b[0] for b in instr.arg[2].bounds}
    if instr.opcode is Opcode.CONST:
        names |= {b[0] for b in instr.arg[1].bounds}
    return names


def _needed(body: list[Instr], roots: set[str]) -> list[Instr]:
    """The instructions of `body` that `roots` depend on, in body order."""
    by_dest = {i.dest: i for i in body}
    need: set[str] = set()
    stack = list(roots)
    while stack:
        name = stack.pop()
        if name in need or name not in by_dest:
            continue
        need.add(name)
        stack.extend(_reads(by_dest[name]))
    return [i for i in body if i.dest in need]


def plan_scatter(nest: LoopNest, shape: NestShape, bufs: Buffers) -> Planned:
    """A float SCATTER whose totals equal np.add.at's bit for bit: every table row is the sum of
    its values in occurrence order, added one at a time onto 0 (reference limn/device.py:153-158
    is the rule; its GPU device adds with atomics in whatever order they land,
    limn/cuda_emit.py:694-703).

    The nest loops over the values, (occurrences..., column); each occurrence's row comes from
    the index instructions of the body, which read only the occurrence variables. Two kernels:

    - `<name>_sort`: a workgroup per tile of consecutive occurrences computes each one's row and
      sorts the tile in LDS by (row, occurrence), a bitonic network over unique 64-bit keys, so
      each row's occurrences in the tile come out contiguous and ascending. Rows outside the
      table (after the wrap of negatives, as numpy indexes) sort last and are never read;
    - `<name>`: a one-wave workgroup per (row, block of 64 columns) finds the row's run in 64
      tiles at a time by binary search (a lane per tile), gathers those runs into one list in
      LDS in tile order, which is occurrence order, then walks the list evaluating the value
      instructions at (occurrence, column) and adding them into one register per lane, 16
      occurrences' loads in flight at a time; the total is stored to every row, the empty
      ones as 0.

    FMA contraction is off in the accumulating kernel so a value computed by a product is
    rounded before it is added, as numpy rounds it. A float16 or bfloat16 table keeps its
    running total at its own width, rounded to nearest even after every add, which is what
    np.add.at into a half-width array does (the reference's oracle zero-fills the table at the
    node's dtype); the values themselves are the kernel's float32 results, so a scatter of
    loaded half-width values matches bit for bit and one of fused half-width arithmetic to the
    half-width tolerance."""
    out_dtype = nest.kernel.target.dtype
    table = nest.kernel.target.shape
    if len(table) != 2:
        raise NotImplementedError(f"the hip device scatters into 2-D tables, not {table}")
    rows_n, cols = table
    lead = [(f"i{d}", e) for d, e in enumerate(nest.space[:-1])]
    col_var = f"i{len(nest.space) - 1}"
    if nest.space[-1] != cols:
        raise NotImplementedError(f"scatter values {nest.space} do not end in the table's {cols} columns")
    occurrences = math.prod(e for _, e in lead)
    if occurrences >= (1 << 31):
        raise NotImplementedError(f"the hip device scatters fewer than 2^31 rows, not {occurrences}")
    write = shape.write
    index = write.arg[1]
    loop_names = {v for v, _ in shape.outer}
    row_terms = [(v, c) for v, c in index.terms if v not in loop_names]
    if len(row_terms) > 1:
        raise NotImplementedError(f"a scatter row index with several computed terms: {index}")
    row_name = row_terms[0][0] if row_terms else None
    key_body = _needed(shape.body, {row_name}) if row_name else []
    if any(col_var in _reads(i) for i in key_body):
        raise NotImplementedError("a scatter row index that depends on the column")
    value_body = _needed(shape.body, {write.srcs[0]})
    half = out_dtype in (float16, bfloat16)
    acc_t = "float" if half else STORE_T[out_dtype]
    tile = next((t for limit, t in SORT_TILE_LIMITS if occurrences <= limit), SORT_TILE_MAX)
    tiles = max(1, -(-occurrences // tile))
    block = 64  # one wave: the scan and the tile search below are lane-wide
    col_blocks = max(1, -(-cols // block))
    params = input_params(nest, bufs)

    per = tile // THREADS  # occurrences per thread, held in registers as thread * per + e
    sort = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {nest.name}_sort({", ".join(params + ["unsigned long long* __restrict__ ALIGNED runs"])}) {{']
    sort.append(f"  __shared__ unsigned long long s_[{tile}];")
    sort.append(f"  const i64 base_ = (i64)blockIdx.x * {tile};")
    sort.append("  const int th_ = threadIdx.x;")
    sort.append(f"  unsigned long long x_[{per}];")
    sort.append("#pragma unroll")
    sort.append(f"  for (int e_ = 0; e_ < {per}; e_++) {{")
    sort.append(f"    const i64 o_ = base_ + th_ * {per} + e_;")
    sort.append("    unsigned long long key_ = ~0ull;")
    sort.append(f"    if (o_ < {occurrences}LL) {{")
    sort += decode(lead, "o_", "      ", True)
    sort += ["      " + value_line(i, bufs) for i in key_body]
    sort.append(f"      long long row_ = {f'(long long){row_name}' if row_name else '0'};")
    sort.append(f"      if (row_ < 0) row_ += {rows_n}LL;")
    sort.append(f"      if (row_ < 0 || row_ >= {rows_n}LL) row_ = {rows_n}LL;")
    sort.append("      key_ = ((unsigned long long)row_ << 32) | (unsigned long long)o_;")
    sort.append("    }")
    sort.append("    x_[e_] = key_;")
    sort.append("  }")
    # bitonic network: stride j pairs element i with i ^ j; the pair runs ascending when
    # (i & k) == 0. Strides of a wave's reach or more go through LDS, shorter ones of at least
    # `per` through lane shuffles, the rest inside a thread's registers.
    sort.append(f"  for (int k_ = 2; k_ <= {tile}; k_ <<= 1) {{")
    sort.append(f"    for (int j_ = k_ >> 1; j_ >= {per}; j_ >>= 1) {{")
    sort.append(f"      if (j_ >= {64 * per}) {{")
    sort.append("#pragma unroll")
    sort.append(f"        for (int e_ = 0; e_ < {per}; e_++) s_[th_ * {per} + e_] = x_[e_];")
    sort.append("        __syncthreads();")
    sort.append("#pragma unroll")
    sort.append(f"        for (int e_ = 0; e_ < {per}; e_++) {{")
    sort.append(f"          const int i_ = th_ * {per} + e_;")
    sort.append("          const unsigned long long y_ = s_[i_ ^ j_];")
    sort.append("          const bool low_ = ((i_ & j_) == 0) == ((i_ & k_) == 0);")
    sort.append("          x_[e_] = low_ ? (x_[e_] < y_ ? x_[e_] : y_) : (x_[e_] < y_ ? y_ : x_[e_]);")
    sort.append("        }")
    sort.append("        __syncthreads();")
    sort.append("      } else {")
    sort.append("#pragma unroll")
    sort.append(f"        for (int e_ = 0; e_ < {per}; e_++) {{")
    sort.append(f"          const int i_ = th_ * {per} + e_;")
    sort.append(f"          const unsigned long long y_ = __shfl_xor(x_[e_], j_ / {per});")
    sort.append("          const bool low_ = ((i_ & j_) == 0) == ((i_ & k_) == 0);")
    sort.append("          x_[e_] = low_ ? (x_[e_] < y_ ? x_[e_] : y_) : (x_[e_] < y_ ? y_ : x_[e_]);")
    sort.append("        }")
    sort.append("      }")
    sort.append("    }")
    j = per // 2
    while j > 0:
        sort.append(f"    if ({j} < k_) {{")
        for e in range(per):
            if e & j:
                continue
            sort.append(f"      if ((x_[{e}] > x_[{e | j}]) == (((th_ * {per} + {e}) & k_) == 0)) {{ const unsigned long long y_ = x_[{e}]; x_[{e}] = x_[{e | j}]; x_[{e | j}] = y_; }}")
        sort.append("    }")
        j //= 2
    sort.append("  }")
    sort.append("#pragma unroll")
    sort.append(f"  for (int e_ = 0; e_ < {per}; e_++) runs[base_ + th_ * {per} + e_] = x_[e_];")
    sort.append("}")

    acc = [f'extern "C" __global__ __launch_bounds__({block}) void {nest.name}({", ".join(params + ["const unsigned long long* __restrict__ ALIGNED runs", f"{STORE_T[out_dtype]}* __restrict__ ALIGNED out"])}) {{']
    acc.append("#pragma clang fp contract(off)")
    acc.append("  __shared__ int lo_[64], start_[64];")
    acc.append(f"  __shared__ unsigned list_[{LIST_CAP}];")
    acc.append("  const int lane_ = threadIdx.x;")
    work = rows_n * col_blocks
    acc.append(f"  for (i64 w_ = blockIdx.x; w_ < {work}LL; w_ += gridDim.x) {{")
    acc.append(f"  const int r_ = (int)(w_ / {col_blocks});")
    acc.append(f"  const int c_ = (int)(w_ % {col_blocks}) * {block} + threadIdx.x;")
    acc.append(f"  const int {col_var} = c_ < {cols} ? c_ : {cols - 1};  // past the last column: read a valid one, store nothing")
    acc.append(f"  {acc_t} acc_ = 0;")
    acc.append(f"  for (int t0_ = 0; t0_ < {tiles}; t0_ += 64) {{")
    acc.append("    int a_ = 0, len_ = 0;")
    acc.append(f"    if (t0_ + lane_ < {tiles}) {{")
    acc.append(f"      const unsigned long long* run_ = runs + (i64)(t0_ + lane_) * {tile};")
    acc.append("      const unsigned long long first_ = (unsigned long long)r_ << 32, past_ = (unsigned long long)(r_ + 1) << 32;")
    acc.append(f"      int n_ = {tile};")
    acc.append("      while (n_ > 0) { const int h_ = n_ >> 1; if (run_[a_ + h_] < first_) { a_ += h_ + 1; n_ -= h_ + 1; } else n_ = h_; }")
    acc.append(f"      int b_ = a_; n_ = {tile} - a_;")
    acc.append("      while (n_ > 0) { const int h_ = n_ >> 1; if (run_[b_ + h_] < past_) { b_ += h_ + 1; n_ -= h_ + 1; } else n_ = h_; }")
    acc.append("      len_ = b_ - a_;")
    acc.append("    }")
    acc.append("    int incl_ = len_;  // where each tile's run starts in this row's list: a scan over the wave")
    acc.append("    for (int d_ = 1; d_ < 64; d_ <<= 1) { const int y_ = __shfl_up(incl_, d_); if (lane_ >= d_) incl_ += y_; }")
    acc.append("    const int total_ = __shfl(incl_, 63);")
    acc.append("    __syncthreads();  // the previous readers of lo_, start_ and list_ are done")
    acc.append("    lo_[lane_] = a_; start_[lane_] = incl_ - len_;")
    acc.append("    __syncthreads();")
    acc.append(f"    for (int base_ = 0; base_ < total_; base_ += {LIST_CAP}) {{")
    acc.append(f"      const int n_ = total_ - base_ < {LIST_CAP} ? total_ - base_ : {LIST_CAP};")
    acc.append("      if (base_) __syncthreads();")
    acc.append("      for (int p_ = lane_; p_ < n_; p_ += 64) {")
    acc.append("        const int q_ = base_ + p_;")
    acc.append("        int t_ = 0;  // the last tile whose run starts at or before q_")
    acc.append("        for (int s_ = 32; s_ > 0; s_ >>= 1) if (start_[t_ + s_] <= q_) t_ += s_;")
    acc.append(f"        list_[p_] = (unsigned)runs[(i64)(t0_ + t_) * {tile} + lo_[t_] + (q_ - start_[t_])];")
    acc.append("      }")
    acc.append("      __syncthreads();")
    acc.append("#pragma unroll 16")
    acc.append("      for (int j_ = 0; j_ < n_; j_++) {")
    acc.append("        const i64 o_ = (i64)list_[j_];")
    acc += decode(lead, "o_", "        ", True)
    acc += ["        " + value_line(i, bufs) for i in value_body]
    if half:  # the table's own width after every add, as np.add.at into a half array rounds
        acc.append(f"        acc_ = {load_expr(out_dtype, store_expr(out_dtype, f'acc_ + (float){write.srcs[0]}'))};")
    else:
        acc.append(f"        acc_ += ({acc_t}){write.srcs[0]};")
    acc.append("      }")
    acc.append("    }")
    acc.append("  }")
    acc.append(f"  if (c_ < {cols}) {{")
    if row_name:
        acc.append(f"    const int {row_name} = r_;")
    acc.append(f"    out[{render_index(index, True)}] = {store_expr(out_dtype, 'acc_') if half else 'acc_'};")
    acc.append("  }")
    acc.append("  }")
    acc.append("}")
    launches = [Launch(nest.name + "_sort", tiles, THREADS, "io_scratch"), Launch(nest.name, max(1, min(work, 1 << 20)), block, "io_scratch_out")]
    return Planned("\n".join(sort + acc), launches, scratch_bytes=tiles * tile * 8,
                   notes={"ordered scatter": True, "tile": tile, "tiles": tiles})


def _fold(op: Op, acc: str, x: str) -> str:
    return f"{acc} = fadd({acc}, {x});" if op is Op.ADD else f"{acc} = fmax_nan({acc}, {x});"


def stride_one_var(nest: LoopNest, shape: NestShape) -> str | None:
    """The loop variable along which the most loaded bytes are contiguous (coefficient 1)."""
    sizes = {f"in{k}": math.prod(n.shape) * n.dtype.itemsize for k, n in enumerate(nest.kernel.inputs)}
    weight: dict[str, int] = {}
    for instr in shape.body:
        if instr.opcode is Opcode.LOAD:
            buf, index, _ = instr.arg
            for var, coeff in index.terms:
                if coeff == 1:
                    weight[var] = weight.get(var, 0) + sizes.get(buf, 0)
    if not weight:
        return None
    return max(weight, key=lambda v: weight[v])


def mergeable(nest: LoopNest, bufs: Buffers, lines: list[str], notes: dict) -> dict:
    """A single-launch kernel's notes plus what merge_runs needs to place it in a merged launch:
    its body (after the block-index line, before the closing brace) and its parameters."""
    out_dtype = nest.kernel.target.dtype
    params = [(STORE_T[n.dtype], f"in{k}", True) for k, n in enumerate(nest.kernel.inputs)]
    params += [(STORE_T[bufs.dtypes[name]], name, True) for name in bufs.extra]
    params.append((STORE_T[out_dtype], "out", False))
    return {**notes, "body": lines[2:-1], "params": params}


def plan_reduce(nest: LoopNest, shape: NestShape, bufs: Buffers) -> Planned:
    cells = math.prod(e for _, e in shape.outer)
    R = math.prod(e for _, e in shape.inner)
    rdt = shape.reduce_dtype
    assert rdt is not None and shape.fold is not None
    acc_dt = accumulate_in(rdt)
    acc_t = VALUE_T[acc_dt]
    out_dtype = nest.kernel.target.dtype
    wide = bufs.wide_index or cells * R > (1 << 30)
    ident = literal(shape.identity, acc_dt)
    item = shape.item
    out_ref = f"out[{render_index(shape.out_index, wide)}]"
    fold = shape.fold
    wave_fold = "wave_fold_add" if fold is Op.ADD else "wave_fold_max"

    # how many threads own a cell: lanes go along whichever loop variable the most bytes are
    # stride-1 in. The IR's own nesting (its ACCUM form) was chosen for a CPU's inner loop and
    # can put a row index innermost merely because small per-row vectors are stride-1 along it.
    along = stride_one_var(nest, shape)
    columns = along is not None and along not in {v for v, _ in shape.inner}
    if columns:
        # cells are consecutive along the stride-1 var: decode it fastest
        shape.outer = [o for o in shape.outer if o[0] != along] + [o for o in shape.outer if o[0] == along]
    if columns and R >= 64 and cells < (1 << 18):
        return plan_columns(nest, shape, bufs, cells, R)
    if columns and cells >= 1024:
        group = 1
    elif R < 64 or (cells >= (1 << 20) and R <= 256):
        group = 1
    elif R < 4096:
        group = 64
    else:
        group = THREADS
    parts = 1
    if group == THREADS and cells < 1024 and R >= (1 << 15):
        parts = max(1, min(1024 // max(cells, 1), -(-R // (1 << 13))))

    body = ["      " + value_line(i, bufs) for i in shape.body]
    inner_var, inner_extent = shape.inner[-1]

    if group == 1:
        lines = [signature(nest.name, nest, out_dtype, bufs) + " {", "  const i64 bid_ = blockIdx.x, nblk_ = gridDim.x;"]
        lines.append(f"  for (i64 g = bid_ * {THREADS} + threadIdx.x; g < {cells}LL; g += nblk_ * {THREADS}) {{")
        lines += decode(shape.outer, "g", "    ", wide)
        lines.append(f"    {acc_t} acc = {ident};")
        for var, extent in shape.inner:
            lines.append(f"    for (int {var} = 0; {var} < {extent}; {var}++) {{")
        lines += body
        lines.append("      " + _fold(fold, "acc", f"({acc_t}){item}"))
        lines += ["    }"] * len(shape.inner)
        lines.append(f"    {out_ref} = {store_expr(out_dtype, 'acc')};")
        lines += ["  }", "}"]
        grid = max(1, min(-(-cells // THREADS), 1 << 20))
        return Planned("\n".join(lines), [Launch(nest.name, grid, THREADS, "io")], notes=mergeable(nest, bufs, lines, {"group": 1}))

    vec = _vec_width(shape, bufs, inner_var, inner_extent)
    chunks = R // vec  # vec divides the innermost extent, hence R
    per_part = -(-chunks // parts)
    base_vars = shape.inner[:-1] + [(inner_var + "_b", inner_extent // vec)]

    def strided_loop(first: str, stop: str, step: int) -> list[str]:
        out = [f"    for (i64 c_ = {first}; c_ < {stop}; c_ += {step}) {{"]
        out += decode(base_vars, "c_", "      ", True)
        out.append("#pragma unroll")
        out.append(f"      for (int j_ = 0; j_ < {vec}; j_++) {{")
        out.append(f"      const int {inner_var} = {inner_var}_b * {vec} + j_;")
        out += body
        out.append("      " + _fold(fold, "acc", f"({acc_t}){item}"))
        out += ["      }", "    }"]
        return out

    waves = THREADS // 64
    if group == 64 and chunks < 256:
        # a short row: G lanes per cell, 64 / G cells per wave, so a wave's loads cover whole
        # consecutive rows; a butterfly within each group of lanes folds the cell. Under 64
        # VEC-wide chunks G is the power of two covering them (a chunk a lane); from 64 it is a
        # quarter of that (four chunks a lane, four rows a wave for a 512-wide bf16 row: a wave a
        # row left each wave one row's loads in flight and half the rows for a second round)
        G = lane_group(chunks)
        per_wave = 64 // G
        lines = [signature(nest.name, nest, out_dtype, bufs) + " {", "  const i64 bid_ = blockIdx.x, nblk_ = gridDim.x;"]
        lines.append(f"  const int lane = threadIdx.x & 63, sub_ = lane % {G};")
        lines.append(f"  for (i64 g0 = (bid_ * {waves} + (threadIdx.x >> 6)) * {per_wave}; g0 < {cells}LL; g0 += nblk_ * {waves * per_wave}) {{")
        lines.append(f"    const i64 g = g0 + lane / {G};")
        lines.append(f"    {acc_t} acc = {ident};")
        lines.append(f"    if (g < {cells}LL) {{")
        lines += ["  " + ln for ln in decode(shape.outer, "g", "    ", wide)]
        lines += ["  " + ln for ln in strided_loop("sub_", f"{chunks}LL", G)]
        lines.append("    }")
        k = G // 2
        while k > 0:
            op = "fadd" if fold is Op.ADD else "fmax_nan"
            lines.append(f"    acc = {op}(acc, ({acc_t})__shfl_xor(acc, {k}));")
            k //= 2
        lines.append(f"    if (sub_ == 0 && g < {cells}LL) {{")
        lines += ["  " + ln for ln in decode(shape.outer, "g", "    ", wide)]
        lines.append(f"      {out_ref} = {store_expr(out_dtype, 'acc')};")
        lines += ["    }", "  }", "}"]
        grid = max(1, min(-(-cells // (waves * per_wave)), 1 << 20))
        return Planned("\n".join(lines), [Launch(nest.name, grid, THREADS, "io")], notes=mergeable(nest, bufs, lines, {"group": G, "vec": vec}))
    if group == 64:
        lines = [signature(nest.name, nest, out_dtype, bufs) + " {", "  const i64 bid_ = blockIdx.x, nblk_ = gridDim.x;"]
        lines.append("  const int lane = threadIdx.x & 63;")
        lines.append(f"  for (i64 g = bid_ * {waves} + (threadIdx.x >> 6); g < {cells}LL; g += nblk_ * {waves}) {{")
        lines += decode(shape.outer, "g", "    ", wide)
        lines.append(f"    {acc_t} acc = {ident};")
        lines += strided_loop("lane", f"{chunks}LL", 64)
        lines.append(f"    acc = {wave_fold}(acc);")
        lines.append(f"    if (lane == 0) {out_ref} = {store_expr(out_dtype, 'acc')};")
        lines += ["  }", "}"]
        grid = max(1, min(-(-cells // waves), 1 << 20))
        return Planned("\n".join(lines), [Launch(nest.name, grid, THREADS, "io")], notes=mergeable(nest, bufs, lines, {"group": 64, "vec": vec}))

    # a workgroup per (cell, part)
    def block_fold(lines: list[str]) -> None:
        lines.append(f"    acc = {wave_fold}(acc);")
        lines.append(f"    __shared__ {acc_t} lds_[{waves}];")
        lines.append("    if ((threadIdx.x & 63) == 0) lds_[threadIdx.x >> 6] = acc;")
        lines.append("    __syncthreads();")
        lines.append("    if (threadIdx.x == 0) {")
        lines.append("      acc = lds_[0];")
        for w in range(1, waves):
            lines.append("      " + _fold(fold, "acc", f"lds_[{w}]"))

    if parts == 1:
        lines = [signature(nest.name, nest, out_dtype, bufs) + " {", "  const i64 bid_ = blockIdx.x, nblk_ = gridDim.x;"]
        lines.append(f"  for (i64 g = bid_; g < {cells}LL; g += nblk_) {{")
        lines += decode(shape.outer, "g", "    ", wide)
        lines.append(f"    {acc_t} acc = {ident};")
        lines += strided_loop("threadIdx.x", f"{chunks}LL", THREADS)
        block_fold(lines)
        lines.append(f"      {out_ref} = {store_expr(out_dtype, 'acc')};")
        lines += ["    }", "    __syncthreads();", "  }", "}"]
        grid = max(1, min(cells, 1 << 20))
        return Planned("\n".join(lines), [Launch(nest.name, grid, THREADS, "io")], notes=mergeable(nest, bufs, lines, {"group": THREADS, "vec": vec}))

    # split: partials then an ordered fold per cell
    part_name = nest.name + "_part"
    params = input_params(nest, bufs)
    params.append(f"{acc_t}* __restrict__ ALIGNED scratch")
    lines = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {part_name}({", ".join(params)}) {{']
    lines.append(f"  const i64 g = blockIdx.x / {parts}, p_ = blockIdx.x % {parts};")
    lines += decode(shape.outer, "g", "  ", wide)
    lines.append(f"  {acc_t} acc = {ident};")
    lines.append(f"  const i64 stop_ = (p_ + 1) * {per_part}LL < {chunks}LL ? (p_ + 1) * {per_part}LL : {chunks}LL;")
    lines += strided_loop(f"p_ * {per_part}LL + threadIdx.x", "stop_", THREADS)
    block_fold(lines)
    lines.append("      scratch[blockIdx.x] = acc;")
    lines += ["    }", "}"]
    final, final_grid = fold_parts(nest.name, shape, acc_t, out_dtype, out_ref, wide, cells, parts, ident, "g * {parts} + p_".format(parts=parts))
    source = "\n".join(lines) + "\n" + "\n".join(final)
    launches = [
        Launch(part_name, cells * parts, THREADS, "io_scratch"),
        Launch(nest.name, final_grid, THREADS, "scratch_out"),
    ]
    return Planned(source, launches, scratch_bytes=cells * parts * acc_dt.itemsize, notes={"parts": parts, "vec": vec})


def fold_parts(name: str, shape: NestShape, acc_t: str, out_dtype: DType, out_ref: str, wide: bool, cells: int, parts: int,
               ident: str, at: str) -> tuple[list[str], int]:
    """The kernel that folds each cell's partial totals (`scratch[at]`, `at` in g and p_) and
    stores the cell. A thread per cell folds them in part order; past 16 parts a wave takes a
    cell, its lanes folding parts lane, lane + 64, ... and a fixed butterfly folding the lanes,
    so a cell's chain of dependent loads is parts / 64 long instead of parts."""
    fold = shape.fold
    lines = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {name}(const {acc_t}* __restrict__ ALIGNED scratch, {STORE_T[out_dtype]}* __restrict__ ALIGNED out) {{']
    if parts <= 16:
        lines.append(f"  for (i64 g = blockIdx.x * (i64){THREADS} + threadIdx.x; g < {cells}LL; g += (i64)gridDim.x * {THREADS}) {{")
        lines += decode(shape.outer, "g", "    ", wide)
        lines.append("    int p_ = 0;")
        lines.append(f"    {acc_t} acc = scratch[{at}];")
        lines.append(f"    for (p_ = 1; p_ < {parts}; p_++) " + _fold(fold, "acc", f"scratch[{at}]"))
        lines.append(f"    {out_ref} = {store_expr(out_dtype, 'acc')};")
        lines += ["  }", "}"]
        return lines, max(1, min(-(-cells // THREADS), 1 << 20))
    waves = THREADS // 64
    wave_fold = "wave_fold_add" if fold is Op.ADD else "wave_fold_max"
    lines.append("  const int lane = threadIdx.x & 63;")
    lines.append(f"  for (i64 g = blockIdx.x * (i64){waves} + (threadIdx.x >> 6); g < {cells}LL; g += (i64)gridDim.x * {waves}) {{")
    # each lane's parts loaded together (the last run clamped into range), then folded in order
    lines.append(f"    {acc_t} acc = {ident};")
    steps = -(-parts // 64)
    for q in range(steps):
        clamp = f"lane + {64 * q} < {parts} ? lane + {64 * q} : {parts - 1}" if 64 * (q + 1) > parts else f"lane + {64 * q}"
        lines.append(f"    {acc_t} f{q}_;")
        lines.append(f"    {{ const int p_ = {clamp}; f{q}_ = scratch[{at}]; }}")
    for q in range(steps):
        step = _fold(fold, "acc", f"f{q}_")
        lines.append(f"    if (lane + {64 * q} < {parts}) {step}" if 64 * (q + 1) > parts else f"    {step}")
    lines.append(f"    acc = {wave_fold}(acc);")
    lines.append("    if (lane == 0) {")
    lines += decode(shape.outer, "g", "      ", wide)
    lines.append(f"      {out_ref} = {store_expr(out_dtype, 'acc')};")
    lines += ["    }", "  }", "}"]
    return lines, max(1, min(-(-cells // waves), 1 << 20))


FOLD_LOADS = 64  # partials a lane of a column fold loads at once


def fold_columns(name: str, shape: NestShape, acc_t: str, out_dtype: DType, out_ref: str, wide: bool, cells: int,
                 parts: int, ident: str) -> tuple[list[str], int]:
    """The fold of a column reduce's partial totals, laid out part-major (`scratch[p_ * cells +
    g]`): a workgroup takes 64 consecutive cells, lane = cell, so each part it loads is one
    coalesced 256-byte row; wave w folds the parts w, w + 4, ... in order (up to FOLD_LOADS of
    them loaded at once: with a few hundred workgroups each wave's loads must all be in flight
    together) and wave 0 then folds the 4 waves' totals in wave order. A wave per cell, its lanes
    loading 64 parts of that cell, read one 4-byte word per 64-byte line: the GPT step's folds of
    13312 cells x 256 parts took 20 us each at 0.7 TB/s."""
    fold = shape.fold
    waves = THREADS // 64
    tiles = -(-cells // 64)
    per = -(-parts // waves)
    lines = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {name}(const {acc_t}* __restrict__ ALIGNED scratch, {STORE_T[out_dtype]}* __restrict__ ALIGNED out) {{']
    lines.append("  const int lane = threadIdx.x & 63, w_ = threadIdx.x >> 6;")
    lines.append(f"  __shared__ {acc_t} fold_[{waves}][64];")
    lines.append(f"  for (i64 t_ = blockIdx.x; t_ < {tiles}LL; t_ += gridDim.x) {{")
    lines.append("    const i64 g = t_ * 64 + lane;")
    lines.append(f"    {acc_t} acc = {ident};")
    lines.append(f"    if (g < {cells}LL) {{")
    chunk = min(per, FOLD_LOADS)
    lines.append(f"      for (int q0_ = 0; q0_ < {per}; q0_ += {chunk}) {{")
    lines.append(f"        {acc_t} f_[{chunk}];")
    lines.append("#pragma unroll")
    lines.append(f"        for (int q_ = 0; q_ < {chunk}; q_++) {{")
    lines.append(f"          const int k_ = w_ + {waves} * (q0_ + q_), p_ = k_ < {parts} ? k_ : {parts - 1};")
    lines.append(f"          f_[q_] = scratch[p_ * {cells}LL + g];")
    lines.append("        }")
    lines.append("#pragma unroll")
    lines.append(f"        for (int q_ = 0; q_ < {chunk}; q_++)")
    lines.append(f"          if (w_ + {waves} * (q0_ + q_) < {parts}) " + _fold(fold, "acc", "f_[q_]"))
    lines.append("      }")
    lines.append("    }")
    lines.append("    fold_[w_][lane] = acc;")
    lines.append("    __syncthreads();")
    lines.append(f"    if (w_ == 0 && g < {cells}LL) {{")
    lines.append("      acc = fold_[0][lane];")
    for w in range(1, waves):
        lines.append("      " + _fold(fold, "acc", f"fold_[{w}][lane]"))
    lines += decode(shape.outer, "g", "      ", wide)
    lines.append(f"      {out_ref} = {store_expr(out_dtype, 'acc')};")
    lines.append("    }")
    lines.append("    __syncthreads();")
    lines += ["  }", "}"]
    return lines, max(1, min(tiles, 1 << 20))


def lane_group(chunks: int) -> int:
    """Lanes per cell of a row reduce over `chunks` vector chunks, under 256 of them (see
    plan_reduce's short rows)."""
    G = 1
    while G < chunks:
        G *= 2
    return G if chunks < 64 else G // 4


COLUMN_TILE = 64  # cells per workgroup of a column reduce: one wave's lanes, one coalesced row piece
COLUMN_BLOCKS = 2048  # workgroups a column reduce aims for (8 per CU): tiles x row parts
COLUMN_ROWS = 16  # the fewest rows a wave of a column reduce folds
COLUMN_UNROLL = 8  # rows a wave of a column reduce loads at once


def plan_columns(nest: LoopNest, shape: NestShape, bufs: Buffers, cells: int, R: int) -> Planned:
    """A reduce whose cells run along the stride-1 var and whose reduce vars are strided (a bias
    or LayerNorm-parameter gradient: a sum over every (batch, time) row of a (.., C) tensor).
    A lane takes VEC consecutive cells (16 bytes of the narrowest input), a workgroup 64 lanes'
    worth, so each row it reads is one coalesced piece of whole-vector loads; its 4 waves take
    interleaved rows of one part of the reduce range; the parts, as many as fill the machine, are
    partial totals in scratch folded per cell in order by a second kernel (one part: written
    directly). Totals are deterministic."""
    rdt = shape.reduce_dtype
    acc_dt = accumulate_in(rdt)
    acc_t = VALUE_T[acc_dt]
    out_dtype = nest.kernel.target.dtype
    wide = bufs.wide_index or cells * R > (1 << 30)
    ident = literal(shape.identity, acc_dt)
    fold = shape.fold
    waves = THREADS // 64
    along, along_extent = shape.outer[-1]
    vec = _vec_width(shape, bufs, along, along_extent)
    per_tile = COLUMN_TILE * vec
    tiles = -(-cells // per_tile)
    # parts enough to fill the machine, each wave reading at least COLUMN_ROWS rows of its part
    parts = max(1, min(-(-COLUMN_BLOCKS // tiles), R // (COLUMN_ROWS * waves)))
    per_part = -(-R // parts)
    out_ref = f"out[{render_index(shape.out_index, wide)}]"
    base_vars = shape.outer[:-1] + [(along + "_b", along_extent // vec)]
    pre, runs = run_loads(nest, shape.body, bufs, along, vec, "        ") if vec > 1 else ([], {})
    body = []
    for instr in shape.body:
        body += ["        " + ln for ln in runs[instr.dest]] if instr.dest in runs else ["        " + value_line(instr, bufs)]
    name = nest.name if parts == 1 else nest.name + "_part"
    params = input_params(nest, bufs)
    params.append(f"{STORE_T[out_dtype]}* __restrict__ ALIGNED out" if parts == 1 else f"{acc_t}* __restrict__ ALIGNED scratch")
    lines = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {name}({", ".join(params)}) {{']
    lines.append("  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;")
    lines.append(f"  const i64 tile = blockIdx.x / {parts}, p_ = blockIdx.x % {parts};")
    lines.append(f"  const i64 gb = tile * {COLUMN_TILE} + lane;  // the lane's run of {vec} cells")
    lines.append(f"  {acc_t} acc[{vec}];")
    lines.append("#pragma unroll")
    lines.append(f"  for (int j_ = 0; j_ < {vec}; j_++) acc[j_] = {ident};")
    lines.append(f"  if (gb < {cells // vec}LL) {{")
    lines += decode(base_vars, "gb", "    ", wide)
    lines.append(f"    const i64 stop_ = (p_ + 1) * {per_part}LL < {R}LL ? (p_ + 1) * {per_part}LL : {R}LL;")
    lines.append(f"    i64 r_ = p_ * {per_part}LL + wave;")

    def row(var: str, indent: str) -> list[str]:
        """One row's loads and its fold into acc, in scope of its own."""
        out = [indent + "{"]
        out += decode(shape.inner, var, indent + "  ", True)
        out += [indent + ln[6:] for ln in pre]
        out.append("#pragma unroll")
        out.append(f"{indent}  for (int j_ = 0; j_ < {vec}; j_++) {{")
        out.append(f"{indent}    const int {along} = {along}_b * {vec} + j_;")
        out += [indent + ln[6:] for ln in body]
        out.append(f"{indent}    " + _fold(fold, "acc[j_]", f"({acc_t}){shape.item}"))
        out += [f"{indent}  }}", indent + "}"]
        return out

    # COLUMN_UNROLL of the wave's rows per step: every row's loads first, into registers, then
    # each row folded in order from them, so the rows' loads are in flight together (a row at a
    # time, a wave waits out the memory latency once per row); then the rest one at a time
    unroll = max(1, min(COLUMN_UNROLL, per_part // waves))
    if unroll > 1:
        lines.append(f"    for (; r_ + {(unroll - 1) * waves} < stop_; r_ += {unroll * waves}) {{")
        fetched = []
        for u in range(unroll):
            lines.append(f"      const i64 r{u}_ = r_ + {u * waves};")
            decls, loads, cached = prefetch_row(shape.body, bufs, along, vec, f"ra{u}_", "        ")
            lines += ["      " + d for d in decls]
            lines.append("      {")
            lines += decode(shape.inner, f"r{u}_", "        ", True)
            lines += loads
            lines.append("      }")
            fetched.append(cached)
        for u in range(unroll):
            bufs.cached = fetched[u]
            lines.append("      {")
            lines += decode(shape.inner, f"r{u}_", "        ", True)
            lines.append("#pragma unroll")
            lines.append(f"        for (int j_ = 0; j_ < {vec}; j_++) {{")
            lines.append(f"          const int {along} = {along}_b * {vec} + j_;")
            lines += ["          " + value_line(i, bufs) for i in shape.body]
            lines.append("          " + _fold(fold, "acc[j_]", f"({acc_t}){shape.item}"))
            lines += ["        }", "      }"]
        bufs.cached = {}
        lines.append("    }")
    lines.append(f"    for (; r_ < stop_; r_ += {waves}) {{")
    lines += row("r_", "      ")
    lines += ["    }", "  }"]
    # the waves' totals for each lane's cells, folded in wave order
    lines.append(f"  __shared__ {acc_t} lds_[{waves}][{64 * vec}];")
    lines.append("#pragma unroll")
    lines.append(f"  for (int j_ = 0; j_ < {vec}; j_++) lds_[wave][lane * {vec} + j_] = acc[j_];")
    lines.append("  __syncthreads();")
    lines.append(f"  if (wave == 0 && gb < {cells // vec}LL) {{")
    lines.append("#pragma unroll")
    lines.append(f"    for (int j_ = 0; j_ < {vec}; j_++) {{")
    lines.append(f"      {acc_t} t = lds_[0][lane * {vec} + j_];")
    for w in range(1, waves):
        lines.append("      " + _fold(fold, "t", f"lds_[{w}][lane * {vec} + j_]"))
    lines.append(f"      const i64 g = gb * {vec} + j_;")
    if parts == 1:
        lines += decode(shape.outer, "g", "      ", wide)
        lines.append(f"      {out_ref} = {store_expr(out_dtype, 't')};")
    else:
        lines.append(f"      scratch[p_ * {cells}LL + g] = t;  // [part][cell]: the final fold reads rows")
    lines += ["    }", "  }", "}"]
    launches = [Launch(name, tiles * parts, THREADS, "io" if parts == 1 else "io_scratch")]
    if parts == 1:
        return Planned("\n".join(lines), launches, notes={"columns": True, "parts": 1, "vec": vec})
    if parts > 16:
        final, final_grid = fold_columns(nest.name, shape, acc_t, out_dtype, out_ref, wide, cells, parts, ident)
    else:
        final, final_grid = fold_parts(nest.name, shape, acc_t, out_dtype, out_ref, wide, cells, parts, ident, f"p_ * {cells}LL + g")
    launches.append(Launch(nest.name, final_grid, THREADS, "scratch_out"))
    return Planned("\n".join(lines) + "\n" + "\n".join(final), launches, scratch_bytes=cells * parts * acc_dt.itemsize,
                   notes={"columns": True, "parts": parts, "vec": vec})


def plan_nest(nest: LoopNest, inlined: "InlineSet | None" = None, stream: bool = False) -> Planned:
    """How one nest runs. With `inlined`, loads of the outputs of the producers it names are
    evaluated in place (see inline_producers); `stream` makes an elementwise nest's stores
    non-temporal (see streamed_outputs)."""
    kernel = nest.kernel
    dtypes = {f"in{k}": n.dtype for k, n in enumerate(kernel.inputs)}
    dtypes["out"] = kernel.target.dtype
    biggest = max([math.prod(n.shape) for n in kernel.inputs] + [math.prod(kernel.target.shape)])
    bufs = Buffers(dtypes, wide_index=biggest >= (1 << 31) - 1)
    if inlined is not None:
        inlined.bind(nest, bufs)
    shape = read_nest(nest)
    if shape.fold is None:
        return plan_elementwise(nest, shape, bufs, stream)
    con = find_contraction(nest, shape)
    if con is not None:
        return Planned("", [], contraction=con, notes={"mfma": True})
    return plan_reduce(nest, shape, bufs)


def _launcher(dev, fn: int, launch: Launch, nin: int):
    api = dev.api
    nargs = nin + 1
    slots = (ctypes.c_void_p * nargs)()
    params = (ctypes.c_void_p * nargs)(*[ctypes.addressof(slots) + k * ctypes.sizeof(ctypes.c_void_p) for k in range(nargs)])
    grid, block = launch.grid, launch.block

    def run(ptrs: list[int]) -> None:
        for k, p in enumerate(ptrs):
            slots[k] = p
        runtime.check(api.hipModuleLaunchKernel(fn, grid, 1, 1, block, 1, 1, 0, None, params, None), f"launching {launch.name}")
        if dev.tape is not None:
            dev.tape.append(replay.Launch(replay.STEP_KERNEL, tuple(ptrs), function=fn, grid=grid, block=block))

    return run


def is_relu(nest: LoopNest) -> bool:
    """Whether an elementwise nest is exactly limn's relu of its one input, read at the cell it
    stores: out = where(0 < x, x, 0) (reference limn/tensor.py:365-366), nothing else."""
    body = [i for i in nest.instrs if i.opcode not in (Opcode.LOOP, Opcode.ENDLOOP)]
    if len(nest.kernel.inputs) != 1 or any(i.opcode is Opcode.ACCUM for i in body):
        return False
    loads = [i for i in body if i.opcode is Opcode.LOAD]
    stores = [i for i in body if i.opcode is Opcode.STORE]
    if len(loads) != 1 or len(stores) != 1 or loads[0].arg[0] != "in0" or loads[0].arg[2].bounds:
        return False
    x, index = loads[0].dest, stores[0].arg[1]
    if loads[0].arg[1] != index:
        return False
    zeros = {i.dest for i in body if i.opcode is Opcode.CONST and i.arg[0] == 0 and not i.arg[1].bounds}
    arith = [i for i in body if i.opcode is Opcode.ARITH]
    if len(body) != len(loads) + len(stores) + len(arith) + len(zeros) or len(arith) != 2:
        return False
    cmp, sel = arith
    return (
        cmp.arg is Op.CMPLT and cmp.srcs[0] in zeros and cmp.srcs[1] == x
        and sel.arg is Op.WHERE and sel.srcs[0] == cmp.dest and sel.srcs[1] == x and sel.srcs[2] in zeros
        and stores[0].srcs == (sel.dest,)
    )


def add_epilogue(nest: LoopNest, total: Node, N: int) -> tuple[int, int | None] | None:
    """(bias input, residual input or None) when an elementwise nest is exactly out = total + bias
    or out = res + (total + bias), at the value type of total's dtype (float for bf16 and f16, one
    rounding at the store), where total (a contraction's output, row-major, its last axis N long)
    is read at the cell the nest stores, bias along that last axis only (bias[n]), and res at the
    stored cell: what limn_hip_matmul_add computes in the contraction's store. A bias-add reader of
    a Linear layer, and one that also adds the residual stream (reference limn/nn.py:27-36 and
    limn/tensor.py:486-496 build them). Anything else, None."""
    body = [i for i in nest.instrs if i.opcode not in (Opcode.LOOP, Opcode.ENDLOOP)]
    extents = {i.dest: i.arg for i in nest.instrs if i.opcode is Opcode.LOOP}
    loads = [i for i in body if i.opcode is Opcode.LOAD]
    stores = [i for i in body if i.opcode is Opcode.STORE]
    arith = [i for i in body if i.opcode is Opcode.ARITH]
    if len(body) != len(loads) + len(stores) + len(arith) or len(stores) != 1 or len(loads) not in (2, 3):
        return None
    if len(arith) != len(loads) - 1 or any(i.arg is not Op.ADD or i.value_type != total.dtype for i in arith):
        return None
    ins = nest.kernel.inputs
    if nest.kernel.target.dtype != total.dtype or any(l.arg[2].bounds for l in loads):
        return None
    index = stores[0].arg[1]
    unit = [v for v, c in index.terms if c == 1]
    if len(unit) != 1 or extents.get(unit[0]) != N or any(c % N for v, c in index.terms if c != 1):
        return None
    n_var = unit[0]
    slot = {f"in{k}": k for k in range(len(ins))}
    role: dict[str, tuple[str, int]] = {}  # load dest -> (what it is, input index)
    for l in loads:
        k = slot.get(l.arg[0])
        if k is None or ins[k].dtype != total.dtype:
            return None
        if ins[k] is total and l.arg[1] == index:
            what = "total"
        elif l.arg[1].terms == ((n_var, 1),) and l.arg[1].const == 0:
            what = "bias"
        elif l.arg[1] == index:
            what = "res"
        else:
            return None
        role[l.dest] = (what, k)
    kinds = sorted(w for w, _ in role.values())
    if kinds not in (["bias", "total"], ["bias", "res", "total"]):
        return None
    first = arith[0]
    if sorted(role[x][0] for x in first.srcs if x in role) != ["bias", "total"] or len(set(first.srcs)) != 2:
        return None
    last = first
    if len(arith) == 2:
        second = arith[1]
        others = [x for x in second.srcs if x != first.dest]
        if len(others) != 1 or first.dest not in second.srcs or role.get(others[0], ("", 0))[0] != "res":
            return None
        last = second
    if stores[0].srcs != (last.dest,):
        return None
    bias = next(k for w, k in role.values() if w == "bias")
    res = next((k for w, k in role.values() if w == "res"), None)
    return bias, res


def batch_sum_fold(reader: LoopNest, total: Node, con: Contraction) -> Contraction | None:
    """The contraction a batched contraction and its reader make together when the reader only
    sums the contraction's output over its batch: limn's weight gradient under a batched
    activation (reference limn/tensor.py:486-496 spells a product as broadcast_to then
    reshape/expand per operand, so a weight broadcast over the batch gets one product per batch
    item, at the weight's dtype, and then a sum over the batch). Folded, the batch becomes part of
    k (both operands must step through batch and k as one row-major index) and the result goes
    straight to the reader's output, in its layout (the operands trade places when that layout has
    the contraction's rows contiguous). One difference from the two nests: the per-item products
    are not rounded to the operand dtype before the batch sum; every partial total stays in float
    until the one rounding at the store."""
    if con.batch <= 1 or con.a_batch != con.K * con.a_k or con.b_batch != con.K * con.b_k:
        return None
    shape = read_nest(reader)
    if shape.fold is not Op.ADD or not shape.inner or len(shape.body) != 1 or shape.out_index.const != 0:
        return None
    load = shape.body[0]
    if load.opcode is not Opcode.LOAD or load.dest != shape.item or load.arg[2].bounds or load.arg[1].const != 0:
        return None
    if reader.kernel.inputs[int(load.arg[0][2:])] is not total or reader.kernel.target.dtype != con.dtype:
        return None
    if shape.reduce_dtype != con.dtype or accumulate_in(con.dtype) is not float32 or con.c_m == con.c_n:
        return None
    terms, out_terms = dict(load.arg[1].terms), dict(shape.out_index.terms)
    inner = [(v, e) for v, e in shape.inner if e > 1]
    if math.prod(e for _, e in inner) != con.batch:
        return None
    order = sorted(inner, key=lambda ve: -terms.get(ve[0], 0))
    if not order or terms.get(order[-1][0], 0) != con.c_batch:
        return None
    for (outer, _), (nxt, e) in zip(order, order[1:]):
        if terms.get(outer, 0) != e * terms.get(nxt, 0):
            return None
    rows = cols = None
    for v, e in shape.outer:
        if e == 1:
            continue
        if terms.get(v) == con.c_m and e == con.M and rows is None:
            rows = out_terms.get(v, 0)
        elif terms.get(v) == con.c_n and e == con.N and cols is None:
            cols = out_terms.get(v, 0)
        else:
            return None
    if not rows or not cols:
        return None
    K = con.batch * con.K
    if cols == 1 or rows != 1:
        folded = replace(con, batch=1, K=K, a_batch=0, b_batch=0, c_batch=0, c_m=rows, c_n=cols)
    else:  # the reader's rows are the contraction's columns: c^T = b^T a^T, rows contiguous
        folded = Contraction(con.b_input, con.a_input, con.b_offset, con.a_offset, con.dtype, 1, con.N, con.M, K,
                             0, con.b_n, con.b_k, 0, con.a_k, con.a_m, 0, cols, rows)
    from limn_amd.dtypes import ABI_CODE

    lib = runtime.kernels()
    ok = lib.limn_hip_matmul_supported(ABI_CODE[folded.dtype], folded.M, folded.N, folded.K, 0, folded.a_m, folded.a_k, 0,
                                       folded.b_k, folded.b_n)
    return folded if ok else None


def epilogue_pairs(nests: list[LoopNest], plans: list[Planned], kept: set | None) -> tuple[dict[int, int], dict[int, tuple], dict[int, Contraction]]:
    """Readers to run as their contraction's epilogue: ({contraction nest: reader nest}, {reader
    nest: (bias input, residual input or None, the bias's cast nest or None)} for the readers that
    add terms, see add_epilogue and bias_cast; {reader nest: folded contraction} for the readers
    that sum a batched contraction over its batch, see batch_sum_fold; the others are relu nests).

    The reader crosses a scheduler cut (the SUM is its own kernel), so it may only move into the
    contraction's store when nothing else needs the SUM's buffer: the reader is its only reader
    among the plan's nests, and it is neither a sink nor read by a CUSTOM call (`kept`, recorded
    by the device's plan_of; None when unknown, which fuses nothing)."""
    if kept is None:
        return {}, {}, {}
    pairs: dict[int, int] = {}
    addends: dict[int, tuple] = {}
    folds: dict[int, Contraction] = {}
    for i, plan in enumerate(plans):
        con = plan.contraction
        if con is None:
            continue
        total = nests[i].kernel.target
        if total in kept:
            continue
        readers = [j for j, n in enumerate(nests) if any(src is total for src in n.kernel.inputs)]
        if len(readers) != 1 or readers[0] <= i:
            continue
        j = readers[0]
        out = nests[j].kernel.target
        if is_relu(nests[j]) and out.dtype == total.dtype and math.prod(out.shape) == math.prod(total.shape):
            pairs[i] = j
            continue
        row_major = con.c_n == 1 and con.c_m == con.N and (con.batch == 1 or con.c_batch == con.M * con.N)
        terms = add_epilogue(nests[j], total, con.N) if row_major else None
        if terms is not None and math.prod(out.shape) == math.prod(total.shape):
            pairs[i] = j
            addends[j] = (*terms, bias_cast(nests, nests[j].kernel.inputs[terms[0]], j, kept))
            continue
        folded = batch_sum_fold(nests[j], total, con)
        if folded is not None:
            pairs[i] = j
            folds[j] = folded
    return pairs, addends, folds


def bias_cast(nests: list[LoopNest], bias: Node, reader: int, kept: set) -> int | None:
    """The nest that makes an add epilogue's bias, when the epilogue can take over its work: a
    nest that only rounds a float32 vector to the bias's type (a bf16 Linear bias cast from its
    float32 parameter), read by nothing but the fused reader. limn_hip_matmul_add then reads the
    float32 vector and rounds it itself (the cast's own arithmetic), and the cast launches
    nothing; launched alone, each such cast cost a 4-5 us launch in the GPT step."""
    if bias in kept:
        return None
    makers = [p for p, n in enumerate(nests) if n.kernel.target is bias]
    if len(makers) != 1 or makers[0] >= reader:
        return None
    p = makers[0]
    if any(bias in n.kernel.inputs for k, n in enumerate(nests) if k != reader):
        return None
    nest = nests[p]
    body = [i for i in nest.instrs if i.opcode not in (Opcode.LOOP, Opcode.ENDLOOP)]
    loops = [i for i in nest.instrs if i.opcode is Opcode.LOOP]
    if len(body) != 3 or len(loops) != 1 or len(nest.kernel.inputs) != 1 or nest.kernel.inputs[0].dtype != float32:
        return None
    load, cast, store = body
    index = Index(0, ((loops[0].dest, 1),))
    if (load.opcode is not Opcode.LOAD or load.arg[0] != "in0" or load.arg[1] != index or load.arg[2].bounds
            or cast.opcode is not Opcode.CAST or cast.srcs != (load.dest,) or cast.value_type != bias.dtype
            or store.opcode is not Opcode.STORE or store.srcs != (cast.dest,) or store.arg[1] != index):
        return None
    return p


INLINE_CELLS = 1 << 16  # the largest producer evaluated in its readers instead of launched
INLINE_BODY = 24  # ... and the most instructions in its body


class InlineSet:
    """Producers evaluated inside their readers, by nest index, and the buffers each reader
    then needs: every producer it reaches (directly or through another inlined producer) hands
    its inputs over as `p<j>_in<m>` parameters."""

    def __init__(self, nests: list[LoopNest], producers: set[int]):
        self.nests = nests
        self.producers = producers
        self.by_target = {nests[j].kernel.target: j for j in producers}

    def reached(self, nest: LoopNest) -> list[int]:
        seen: set[int] = set()
        stack = [self.by_target[n] for n in nest.kernel.inputs if n in self.by_target]
        while stack:
            j = stack.pop()
            if j in seen:
                continue
            seen.add(j)
            stack += [self.by_target[n] for n in self.nests[j].kernel.inputs if n in self.by_target]
        return sorted(seen)

    def bind(self, nest: LoopNest, bufs: Buffers) -> None:
        from dataclasses import replace

        reached = self.reached(nest)
        if not reached:
            return
        names = {j: {f"in{m}": f"p{j}_in{m}" for m in range(len(self.nests[j].kernel.inputs))} for j in reached}
        for j in reached:
            for m, node in enumerate(self.nests[j].kernel.inputs):
                bufs.dtypes[names[j][f"in{m}"]] = node.dtype
                bufs.extra.append(names[j][f"in{m}"])

        def renamed(instr: Instr, prefix: str, buffers: dict[str, str]) -> Instr:
            def ix(index: Index) -> Index:
                return Index(index.const, tuple((prefix + v, c) for v, c in index.terms))

            def vd(valid: Valid) -> Valid:
                return Valid(tuple((prefix + v, lo, hi, n) for v, lo, hi, n in valid.bounds))

            arg = instr.arg
            if instr.opcode is Opcode.LOAD:
                arg = (buffers[arg[0]], ix(arg[1]), vd(arg[2]))
            elif instr.opcode is Opcode.GATHER:
                arg = (buffers[arg[0]], ix(arg[1]))
            elif instr.opcode is Opcode.CONST:
                arg = (arg[0], vd(arg[1]))
            return replace(instr, dest=prefix + instr.dest, srcs=tuple(prefix + x for x in instr.srcs), arg=arg)

        sources: dict[int, Inlined] = {}
        for j in reached:
            shape = read_nest(self.nests[j])
            prefix = f"p{j}_"
            target = self.nests[j].kernel.target
            space = tuple((prefix + f"i{d}", e) for d, e in enumerate(target.shape))
            body = tuple(renamed(i, prefix, names[j]) for i in shape.body)
            sources[j] = Inlined(space, body, prefix + shape.write.srcs[0], target.dtype)
        for k, node in enumerate(nest.kernel.inputs):
            if node in self.by_target:
                bufs.inline[f"in{k}"] = sources[self.by_target[node]]
        for j in reached:
            for m, node in enumerate(self.nests[j].kernel.inputs):
                if node in self.by_target:
                    bufs.inline[names[j][f"in{m}"]] = sources[self.by_target[node]]

    def extras(self, nest: LoopNest) -> list[tuple[int, int]]:
        """(producer, input) of each extra parameter, in order."""
        return [(j, m) for j in self.reached(nest) for m in range(len(self.nests[j].kernel.inputs))]


def _stores_its_cells(nest: LoopNest) -> bool:
    """An elementwise nest that loops over its output shape and stores each cell at its
    row-major place, so a reader's flat index decodes into its loop variables."""
    shape = read_nest(nest)
    if shape.fold is not None or shape.write is None or shape.write.opcode is not Opcode.STORE:
        return False
    target = nest.kernel.target.shape
    if tuple(nest.space) != tuple(target):
        return False
    from limn_amd.seam import contiguous_index

    return shape.write.arg[1] == contiguous_index(tuple(target), [f"i{d}" for d in range(len(target))])


def inline_producers(nests: list[LoopNest], plans: list[Planned], kept: set | None, pairs: dict[int, int]) -> set[int]:
    """Small elementwise nests to evaluate inside their readers instead of launching: the
    scheduler realizes every broadcast value (a row's max, 1/sum, a LayerNorm scale) as its own
    kernel (reference limn/schedule.py:46-141), a launch of a few microseconds for a few
    kilobytes. A producer qualifies when its output is not kept (a sink or a CUSTOM input;
    `kept` None inlines nothing), it has at most INLINE_CELLS cells and INLINE_BODY
    instructions, and every reader is an emitted nest (not a contraction, not a relu epilogue)
    that reads it by plain loads. Its inputs stay valid for the whole plan: the executor keeps
    every buffer of a transaction and commits assigns only at its end."""
    if kept is None:
        return set()
    fused = set(pairs) | set(pairs.values())
    readers: dict = {}
    for c, nest in enumerate(nests):
        for node in nest.kernel.inputs:
            readers.setdefault(node, set()).add(c)
    chosen: set[int] = set()
    for j, (nest, plan) in enumerate(zip(nests, plans)):
        target = nest.kernel.target
        if not plan.notes.get("elementwise") or j in fused or target in kept or target not in readers:
            continue
        if math.prod(target.shape) > INLINE_CELLS or len(read_nest(nest).body) > INLINE_BODY:
            continue
        if not _stores_its_cells(nest):
            continue
        ok = True
        for c in readers[target]:
            if c in fused or plans[c].contraction is not None or c <= j:
                ok = False
                break
            name = {f"in{k}" for k, n in enumerate(nests[c].kernel.inputs) if n is target}
            if any(i.opcode is Opcode.GATHER and i.arg[0] in name for i in nests[c].instrs):
                ok = False
                break
        if ok:
            chosen.add(j)
    return chosen


MERGE_GRID = 1 << 16  # the largest elementwise launch merged with its neighbours
MERGE_GROUP_GRID = 1 << 20  # the most workgroups of one merged launch
MERGE_MEMBERS = 48  # the most nests in one merged launch
MERGE_PARAMS = 400  # the most pointers one merged launch takes (3.2 KB of its 4 KB of arguments)


def merge_runs(nests: list[LoopNest], plans: list[Planned], custom_inputs: set | None, inlined: "InlineSet",
               pairs: dict[int, int], taken: set[int] = frozenset()) -> tuple[list[list[int]], list[int]]:
    """Groups of small elementwise nests that share one launch, and the nest whose runner
    launches each. Several groups are open at once, in creation order: a nest joins the first
    open group after every group holding a nest it reads (directly or through an inlined
    producer), so a group only reads groups created before it; a group launches at the latest of
    its last member and the launches of the groups it reads. A nest that is no member (it runs
    at its own place) and reads a member closes that member's group and the groups that one
    reads, which have all launched by then. No member's output is read by a CUSTOM call, which may
    sit between nests. Each member is at most MERGE_GRID workgroups, a group at most
    MERGE_MEMBERS nests, MERGE_PARAMS pointers and MERGE_GROUP_GRID workgroups. An optimizer step
    gives groups across parameters: every parameter's moments in a first few groups, every
    parameter's update from its new moments in the next few, where a run of consecutive nests
    took a launch per parameter. Column reduces (a partials kernel and a fold kernel each) form
    groups of their own kind: one launch of every member's partials, one of every fold. Nests in
    `taken` (members of row programs) never join. `custom_inputs` None merges nothing."""
    if custom_inputs is None:
        return [], []
    fused = set(pairs) | set(pairs.values())

    def reads(c: int) -> set:
        nodes = set(nests[c].kernel.inputs)
        for j in inlined.reached(nests[c]):
            nodes |= set(nests[j].kernel.inputs)
        return nodes

    groups: list[list[int]] = []
    kinds: list[str] = []  # "body" (single-launch nests) or "columns" (column reduces, two launches)
    size: list[list[int]] = []  # [workgroups, pointers] per group
    closed: list[bool] = []
    deps: list[set[int]] = []
    owner: dict = {}  # a member's output -> its group

    def close(g: int) -> None:
        stack = [g]
        while stack:
            h = stack.pop()
            if not closed[h]:
                closed[h] = True
                stack.extend(deps[h])

    for c, (nest, plan) in enumerate(zip(nests, plans)):
        if c in inlined.producers:
            continue  # launches nothing; its readers' reads() carry its inputs
        free = c not in fused and c not in taken and nest.kernel.target not in custom_inputs
        kind = None
        if free and "body" in plan.notes and len(plan.launches) == 1 and plan.launches[0].grid <= MERGE_GRID:
            kind = "body"
        elif free and plan.notes.get("columns") and len(plan.launches) == 2:
            kind = "columns"
        hit = {owner[n] for n in reads(c) if n in owner}
        if kind is None:
            for g in hit:
                close(g)
            continue
        grid, params = plan.launches[0].grid, _param_count(plan) if kind == "columns" else len(plan.notes["params"])
        lo = max(hit) + 1 if hit else 0
        target = next((g for g in range(lo, len(groups)) if not closed[g] and kinds[g] == kind
                       and len(groups[g]) < MERGE_MEMBERS and size[g][0] + grid <= MERGE_GROUP_GRID
                       and size[g][1] + params <= MERGE_PARAMS), None)
        if target is None:
            groups.append([])
            size.append([0, 0])
            closed.append(False)
            deps.append(set())
            kinds.append(kind)
            target = len(groups) - 1
        groups[target].append(c)
        size[target][0] += grid
        size[target][1] += params
        deps[target] |= hit
        owner[nest.kernel.target] = target
    launch_at: list[int] = []
    for g, members in enumerate(groups):
        launch_at.append(max([members[-1]] + [launch_at[d] for d in deps[g]]))
    # a lone member launching at its own place runs as an ordinary launch, unless other groups
    # launch from its runner
    hosts = [launch_at.count(at) for at in launch_at]
    keep = [g for g, members in enumerate(groups)
            if len(members) > 1 or launch_at[g] != members[-1] or hosts[g] > 1]
    return [groups[g] for g in keep], [launch_at[g] for g in keep]


def merged_source(name: str, nests: list[LoopNest], plans: list[Planned], run: list[int]) -> tuple[str, int]:
    """One kernel for a run of elementwise nests: each member's body in its own block range, its
    buffer names bound to its own parameters. A workgroup runs one member, so the members' LDS
    arrays (a transposing member's tiles) all start at the kernel's one `mshared_`."""
    params: list[str] = []
    segments: list[str] = []
    offset = 0
    lds = 0
    for s_, c in enumerate(run):
        plan = plans[c]
        grid = plan.launches[0].grid
        at = 0

        def shared(d) -> str:
            nonlocal at
            t, var, dims = d.group(1), d.group(2), [int(x) for x in re.findall(r"\d+", d.group(3))]
            start = -(-at // 16) * 16
            at = start + math.prod(dims) * _SIZES[t]
            return f"{t}* {var} = ({t}*)(mshared_ + {start});"

        body = [_SHARED.sub(shared, ln) for ln in plan.notes["body"]]
        lds = max(lds, at)
        binds = []
        for ctype, pname, const in plan.notes["params"]:
            q = "const " if const else ""
            params.append(f"{q}{ctype}* __restrict__ ALIGNED s{s_}_{pname}")
            binds.append(f"    {q}{ctype}* __restrict__ {pname} = ({q}{ctype}*)__builtin_assume_aligned(s{s_}_{pname}, 16);")
        cond = f"blockIdx.x < {offset + grid}"
        head = "  if" if s_ == 0 else "  } else if"
        segments.append(f"{head} ({cond}) {{" if s_ < len(run) - 1 else ("  } else {" if s_ else "  {"))
        segments += binds
        segments.append(f"    const i64 bid_ = (i64)blockIdx.x - {offset}, nblk_ = {grid};")
        segments += ["  " + ln for ln in body]
        offset += grid
    segments.append("  }")
    if lds:
        segments.insert(0, f"  __shared__ __attribute__((aligned(16))) char mshared_[{lds}];")
    source = f'extern "C" __global__ __launch_bounds__({THREADS}) void {name}({", ".join(params)}) {{\n' + "\n".join(segments) + "\n}"
    return source, offset



_KERNEL_HEAD = re.compile(r'extern "C" __global__ __launch_bounds__\(\d+\) void (\w+)\((.*?)\) \{')


_SHARED = re.compile(r"__shared__ (\w+) (\w+)((?:\[\d+\])+);")
_SIZES = {"float": 4, "double": 8, "int": 4, "i64": 8, "short": 2, "u16": 2, "i8": 1, "char": 1}


def as_device_function(source: str, grid: int) -> tuple[str, str, list[str], int]:
    """A one-kernel source as a __device__ function of the same body that takes its workgroup
    index as an argument (`mbid_`), its grid size a constant, and its LDS arrays from the caller's
    `mshared_` (a workgroup runs one such function, so the functions of a merged kernel share
    it): the function's name, its text, its parameter names in order and its LDS bytes."""
    m = _KERNEL_HEAD.search(source)
    assert m is not None, "not an emitted kernel"
    name, params = m.group(1), m.group(2)
    names = [p.split()[-1] for p in params.split(", ")]
    body = source[m.end():].replace("blockIdx.x", "mbid_").replace("gridDim.x", f"{grid}")
    at = 0

    def shared(d) -> str:
        nonlocal at
        t, var, dims = d.group(1), d.group(2), [int(x) for x in re.findall(r"\d+", d.group(3))]
        start = -(-at // 16) * 16
        at = start + math.prod(dims) * _SIZES[t]
        rest = "".join(f"[{x}]" for x in dims[1:])
        return f"{t} (*{var}){rest} = ({t} (*){rest})(mshared_ + {start});" if rest else f"{t}* {var} = ({t}*)(mshared_ + {start});"

    body = _SHARED.sub(shared, body)
    text = f"__device__ __forceinline__ void {name}_d({params}, const i64 mbid_, char* mshared_) {{" + body
    return f"{name}_d", text, names, at


def _param_count(plan: Planned) -> int:
    """The parameters of a plan's first kernel."""
    return len(_KERNEL_HEAD.search(plan.source).group(2).split(", "))


def _kernels_of(source: str) -> list[str]:
    """The kernels of a plan's source, each from its `extern "C"` to the next."""
    starts = [m.start() for m in _KERNEL_HEAD.finditer(source)]
    return [source[a:b] for a, b in zip(starts, starts[1:] + [len(source)])]


def merged_columns_source(name: str, plans: list[Planned], run: list[int]) -> tuple[str, int, int, list[int], int]:
    """Two kernels for a group of column reduces: `<name>_part` runs every member's partials
    kernel on its own range of workgroups, `<name>` every member's fold; each member's code is its
    own kernel's, as a device function given its workgroup index. The members' partials share one
    scratch buffer, at the returned byte offsets. Returns (source, partials grid, folds grid,
    offsets, scratch bytes)."""
    functions: list[str] = []
    calls = {"part": [], "fold": []}
    params = {"part": [], "fold": []}
    grids = {"part": 0, "fold": 0}
    lds = {"part": 0, "fold": 0}
    offsets, total = [], 0
    for s_, c in enumerate(run):
        plan = plans[c]
        offsets.append(total)
        total += -(-plan.scratch_bytes // 256) * 256
        part_src, fold_src = _kernels_of(plan.source)
        for kind, src, launch in (("part", part_src, plan.launches[0]), ("fold", fold_src, plan.launches[1])):
            fn, text, names, shared = as_device_function(src, launch.grid)
            lds[kind] = max(lds[kind], shared)
            functions.append(text)
            m = _KERNEL_HEAD.search(src)
            for decl, pname in zip(m.group(2).split(", "), names):
                params[kind].append(decl[: len(decl) - len(pname)] + f"s{s_}_{pname}")
            start = grids[kind]
            grids[kind] += launch.grid
            args = ", ".join(f"s{s_}_{pname}" for pname in names)
            calls[kind].append(f"  if (b_ < {grids[kind]}) {{ {fn}({args}, b_ - {start}, mshared_); return; }}")
    kernels = []
    for kind, kname in (("part", f"{name}_part"), ("fold", name)):
        kernels.append(f'extern "C" __global__ __launch_bounds__({THREADS}) void {kname}({", ".join(params[kind])}) {{\n'
                       f"  __shared__ __attribute__((aligned(16))) char mshared_[{max(lds[kind], 16)}];\n"
                       "  const i64 b_ = blockIdx.x;\n" + "\n".join(calls[kind]) + "\n}")
    return "\n".join(functions + kernels), grids["part"], grids["fold"], offsets, max(total, 256)


# ---- row programs ---------------------------------------------------------------------------
# A softmax or a LayerNorm reaches the device as a chain of nests over the same rows: row
# reductions (a max, a sum, a sum of squares) each writing one value per row, and elementwise
# nests over the rows' cells reading those values. Launched one by one, each reduction streams
# the whole input again, and each launch of a few microseconds is paid in full on short rows.
# A row program runs such a chain as one kernel: a workgroup (long rows) or a wave (rows of up to
# 64 vector chunks per lane group) takes a row and runs every member on it in plan order, each
# reduction's total kept in registers for the later members (their loads of it read the
# register, rounded as the store rounds) and stored as well. Each member's code is the code its
# own kernel would run for that row (the same strided loop, vector width and fold order), so the
# results are the same bits; the input row is re-read from the caches rather than from HBM.

@dataclass
class RowMember:
    """A nest as a member of a row program: `kind` "reduce" (one value per row, folded over the
    row's cells), "cells" (an elementwise nest over the row's cells) or "scalar" (an elementwise
    nest with one cell per row); its row loop variables, its cell variable and extent (None for
    "scalar"), and for a reduce the lanes its own kernel gives a row (THREADS or 64) and its vector
    width."""

    kind: str
    rows: tuple[int, ...]
    row_vars: list[tuple[str, int]]
    col: tuple[str, int] | None
    group: int | None
    vec: int
    shape: NestShape


def _row_strides(row_vars: list[tuple[str, int]]) -> dict[str, int]:
    strides, step = {}, 1
    for var, extent in reversed(row_vars):
        if extent > 1:
            strides[var] = step
            step *= extent
    return strides


def row_flat(index: Index, row_vars: list[tuple[str, int]], scale: int = 1) -> bool:
    """Whether `index` is the row-major position of the row (times `scale`) in `row_vars`: each
    variable of extent > 1 at its row-major stride, no constant, no other variable."""
    if index.const:
        return False
    strides = _row_strides(row_vars)
    ones = {v for v, e in row_vars if e == 1}
    seen = set()
    for var, coeff in index.terms:
        if var in strides:
            if coeff != strides[var] * scale:
                return False
            seen.add(var)
        elif var not in ones:
            return False
    return seen == set(strides)


def row_member(nest: LoopNest, plan: Planned) -> RowMember | None:
    """How a nest would run inside a row program, or None when it cannot."""
    if plan.contraction is not None or len(plan.launches) != 1 or "params" not in plan.notes:
        return None
    target = nest.kernel.target
    if target.dtype not in (float32, bfloat16, float16):
        return None
    shape = read_nest(nest)
    if shape.fold is not None:
        group = plan.notes.get("group")
        if group not in (THREADS, 64, 32, 16, 8) or plan.notes.get("columns") or len(shape.inner) != 1:
            return None
        if shape.reduce_dtype not in (float32, bfloat16, float16):
            return None
        col = shape.inner[0]
        vec = plan.notes.get("vec", 1)
        if stride_one_var(nest, shape) != col[0] or (group == 64 and col[1] // vec < 64):
            return None
        if not row_flat(shape.out_index, shape.outer):
            return None
        rows = tuple(e for _, e in shape.outer if e > 1)
        return RowMember("reduce", rows, list(shape.outer), col, group, vec, shape)
    if not plan.notes.get("elementwise") or shape.write is None or shape.write.opcode is not Opcode.STORE:
        return None
    out_index = shape.write.arg[1]
    if shape.outer and shape.outer[-1][1] > 1 and dict(out_index.terms).get(shape.outer[-1][0]) == 1:
        col = shape.outer[-1]
        rest = Index(out_index.const, tuple((v, c) for v, c in out_index.terms if v != col[0]))
        if not row_flat(rest, shape.outer[:-1], col[1]):
            return None
        rows = tuple(e for _, e in shape.outer[:-1] if e > 1)
        return RowMember("cells", rows, list(shape.outer[:-1]), col, None, 1, shape)
    if not row_flat(out_index, shape.outer):
        return None
    rows = tuple(e for _, e in shape.outer if e > 1)
    return RowMember("scalar", rows, list(shape.outer), None, None, 1, shape)


def _loads(body) -> list[Instr]:
    return [i for i in body if i.opcode in (Opcode.LOAD, Opcode.GATHER)]


def _reads_rows_only(nest: LoopNest, member: RowMember, made: set, inlined: "InlineSet") -> bool:
    """Whether every read of a value `made` earlier in the program, by the nest or by a producer
    it evaluates in place, is a plain load of this row's value."""
    producers = {inlined.nests[j].kernel.target: j for j in inlined.reached(nest)}
    # producers whose value depends on something made in the program (directly or through another)
    tainted: set = set()
    changed = True
    while changed:
        changed = False
        for target, j in producers.items():
            if target in tainted:
                continue
            if any(n in made or n in tainted for n in inlined.nests[j].kernel.inputs):
                tainted.add(target)
                changed = True
    needs = made | tainted

    def ok(body, inputs, row_vars) -> bool:
        for instr in _loads(body):
            node = inputs[int(instr.arg[0][2:])] if instr.arg[0].startswith("in") else None
            if node is None or node not in needs:
                continue
            if instr.opcode is Opcode.GATHER or instr.arg[2].bounds or not row_flat(instr.arg[1], row_vars):
                return False
        return True

    if not ok(member.shape.body, nest.kernel.inputs, member.row_vars):
        return False
    for target, j in producers.items():
        if target not in tainted:
            continue
        pn = inlined.nests[j]
        space = [(f"i{d}", e) for d, e in enumerate(pn.kernel.target.shape)]
        if not ok(read_nest(pn).body, pn.kernel.inputs, space):
            return False
    return True


def row_chains(nests: list[LoopNest], plans: list[Planned], custom_inputs: set | None, inlined: "InlineSet",
               pairs: dict[int, int]) -> list[list[int]]:
    """Runs of nests to run as row programs: consecutive in the plan (nests between members stay,
    and run before the program, unless they read a member's output, which ends the run), over
    the same rows and row length, reductions of one kind (a workgroup or a wave per row), every
    read of a member's output a plain load of the same row. A run needs a reduction and two
    members. No member's output may be a CUSTOM input; `custom_inputs` None builds none."""
    if custom_inputs is None:
        return []
    fused = set(pairs) | set(pairs.values())

    def reads(c: int) -> set:
        nodes = set(nests[c].kernel.inputs)
        for j in inlined.reached(nests[c]):
            nodes |= set(nests[j].kernel.inputs)
        return nodes

    chains: list[list[int]] = []
    run: list[int] = []
    made: set = set()
    key: dict = {}

    def close() -> None:
        kinds = [row_member(nests[c], plans[c]).kind for c in run]
        if len(run) > 1 and "reduce" in kinds:
            chains.append(list(run))
        run.clear()
        made.clear()
        key.clear()

    for c, nest in enumerate(nests):
        if c in inlined.producers:
            continue
        m = None
        if c not in fused and plans[c].launches and nest.kernel.target not in custom_inputs:
            m = row_member(nest, plans[c])
        if m is not None and run:
            fits = m.rows == key["rows"] and (m.col is None or key["cols"] in (None, m.col[1]))
            fits = fits and (m.group is None or key["group"] in (None, m.group))
            if fits and _reads_rows_only(nest, m, made, inlined) and all(
                    row_member(nests[p], plans[p]).kind != "cells" for p in run if nests[p].kernel.target in reads(c)):
                run.append(c)
                made.add(nest.kernel.target)
                key["cols"] = key["cols"] if m.col is None else m.col[1]
                key["group"] = key["group"] if m.group is None else m.group
                continue
        if run and (m is not None or reads(c) & made):
            close()
        if m is not None:
            run.append(c)
            made.add(nest.kernel.target)
            key.update(rows=m.rows, cols=None if m.col is None else m.col[1], group=m.group)
    close()
    return chains


# A row program keeps the row of each input its members read at (row, cell) in registers, up
# to this many values a thread, loaded when the row starts: the row comes from HBM once, every
# later pass over it reads the registers, and the loads of all the inputs are in flight together
# (an input first read by the last member would otherwise wait for the reductions before it).
# Re-read from memory, the passes of an 8192-float row softmax then LayerNorm (32 KB a row,
# thousands of rows in flight) missed the L2 and ran at 2.5 TB/s of algorithmic bytes; the row
# is 32 values a thread of a 256-thread workgroup.
ROW_CACHE_VALUES = 64


def _row_read(instr: Instr, inputs: list, member: RowMember, bufs: Buffers):
    """The input node that a member's LOAD reads at the member's (row, cell), unmasked - index the
    row's row-major position times the row length plus the cell - or None. Not a load of an
    inlined producer's output: that buffer is never written, the load evaluates the producer."""
    if instr.opcode is not Opcode.LOAD or not instr.arg[0].startswith("in") or member.col is None:
        return None
    if instr.arg[0] in bufs.inline:
        return None
    buf, index, valid = instr.arg
    node = inputs[int(buf[2:])]
    col_var, cols = member.col
    if valid.bounds or node.dtype not in (float32, bfloat16, float16) or dict(index.terms).get(col_var) != 1:
        return None
    rest = Index(index.const, tuple((v, c) for v, c in index.terms if v != col_var))
    return node if row_flat(rest, member.row_vars, cols) else None


def row_source(name: str, nests: list[LoopNest], plans: list[Planned], run: list[int], inlined: "InlineSet",
               streamed: set[int]) -> tuple[str, int]:
    """One kernel for a row program (see row_chains): each member's parameters bound as its own
    kernel's, its code for one row, in order, inside one loop over the rows. The inputs the members
    read along the row are loaded into registers when the row starts (ROW_CACHE_VALUES); the
    members' loops then run unrolled over the same cells in the same order, so every fold adds in
    the order of the member's own kernel."""
    members = [(c, row_member(nests[c], plans[c])) for c in run]
    group = next(m.group for _, m in members if m.kind == "reduce")
    rows = math.prod(members[0][1].rows)
    cols = next(m.col[1] for _, m in members if m.col is not None)
    threads = group  # the lanes of a row: a workgroup, a wave or a group of a wave's lanes
    tid = "threadIdx.x" if group == THREADS else "lane_" if group == 64 else "sub_"
    # each member's buffers and cells per thread step
    setup = []
    for c, m in members:
        kernel = nests[c].kernel
        dtypes = {f"in{k}": n.dtype for k, n in enumerate(kernel.inputs)}
        dtypes["out"] = kernel.target.dtype
        biggest = max([math.prod(n.shape) for n in kernel.inputs] + [math.prod(kernel.target.shape)])
        bufs = Buffers(dtypes, wide_index=biggest >= (1 << 31) - 1)
        if inlined.reached(nests[c]):
            inlined.bind(nests[c], bufs)
        vec = m.vec if m.kind == "reduce" else _vec_width(m.shape, bufs, *m.col) if m.kind == "cells" else 1
        setup.append((bufs, vec))
    # the cached rows: node -> (variable, vec, passes, member slots that read it)
    readers: dict = {}
    for s_, (c, m) in enumerate(members):
        for instr in _loads(m.shape.body):
            node = _row_read(instr, nests[c].kernel.inputs, m, setup[s_][0])
            if node is not None and s_ not in readers.setdefault(node, []):
                readers[node].append(s_)
    cache: dict = {}
    room = ROW_CACHE_VALUES
    for node, slots in readers.items():
        vec = setup[slots[0]][1]
        same = [s_ for s_ in slots if setup[s_][1] == vec]
        passes = -(-(cols // vec) // threads)
        if passes * vec > room:
            continue
        room -= passes * vec
        cache[node] = (f"rc{len(cache)}_", vec, passes, same)
    params: list[str] = []
    lines: list[str] = []
    values: dict = {}  # node -> (variable, stored dtype) of members with one value per row
    if group == THREADS:
        lines.append(f"  __shared__ float rp_fold_[{THREADS // 64}];")
        lines.append(f"  for (i64 row_ = blockIdx.x; row_ < {rows}LL; row_ += gridDim.x) {{")
        grid = max(1, min(rows, 1 << 20))
    elif group == 64:
        per = THREADS // 64
        lines.append("  const int lane_ = threadIdx.x & 63;")
        lines.append(f"  for (i64 row_ = (i64)blockIdx.x * {per} + (threadIdx.x >> 6); row_ < {rows}LL; row_ += (i64)gridDim.x * {per}) {{")
        grid = max(1, min(-(-rows // per), 1 << 20))
    else:
        # 64 / group rows a wave, one a group of lanes (the rows of a wave's groups may end
        # apart: a group's butterfly reads its own lanes only)
        per = THREADS // group
        lines.append(f"  const int lane_ = threadIdx.x & 63, sub_ = lane_ % {group};")
        lines.append(f"  for (i64 row_ = ((i64)blockIdx.x * {THREADS // 64} + (threadIdx.x >> 6)) * {64 // group} + lane_ / {group}; "
                     f"row_ < {rows}LL; row_ += (i64)gridDim.x * {per}) {{")
        grid = max(1, min(-(-rows // per), 1 << 20))
    for node, (var, vec, passes, same) in cache.items():
        first = same[0]
        k = next(k for k, n in enumerate(nests[members[first][0]].kernel.inputs) if n is node)
        st, chunks = STORE_T[node.dtype], cols // vec
        lines.append(f"    {VALUE_T[node.dtype]} {var}[{passes}][{vec}];")
        lines.append("#pragma unroll")
        lines.append(f"    for (int it_ = 0; it_ < {passes}; it_++) {{")
        lines.append(f"      const i64 c_ = {tid} + (i64)it_ * {threads};")
        if chunks % threads:
            lines.append(f"      if (c_ >= {chunks}LL) break;")
        lines.append(f"      const {st}* p_ = (const {st}*)__builtin_assume_aligned(s{first}_in{k}, 16) + row_ * {cols}LL + c_ * {vec};")
        lines.append("#pragma unroll")
        lines.append(f"      for (int j_ = 0; j_ < {vec}; j_++) {var}[it_][j_] = {load_expr(node.dtype, 'p_[j_]')};")
        lines.append("    }")

    def cell_loop(s_: int, chunks: int, indent: str) -> tuple[list[str], bool]:
        """The member's loop over its cell chunks: strided, or unrolled over the cached passes."""
        c, m = members[s_]
        bufs = setup[s_][0]
        hits = [(node, entry) for node, entry in cache.items() if s_ in entry[3]]
        if not hits:
            return [f"{indent}for (i64 c_ = {tid}; c_ < {chunks}LL; c_ += {threads}) {{"], False
        for instr in _loads(m.shape.body):
            node = _row_read(instr, nests[c].kernel.inputs, m, bufs)
            if node in cache and s_ in cache[node][3]:
                bufs.cached[instr.dest] = f"{cache[node][0]}[it_][j_]"
        passes = hits[0][1][2]
        out = ["#pragma unroll", f"{indent}for (int it_ = 0; it_ < {passes}; it_++) {{",
               f"{indent}  const i64 c_ = {tid} + (i64)it_ * {threads};"]
        if chunks % threads:
            out.append(f"{indent}  if (c_ >= {chunks}LL) break;")
        return out, True

    first_param: dict = {}  # (input node, element type) -> the first parameter that carries it
    for s_, (c, m) in enumerate(members):
        nest, plan, shape = nests[c], plans[c], m.shape
        kernel = nest.kernel
        bufs = setup[s_][0]
        names = {f"in{k}": n for k, n in enumerate(kernel.inputs)}
        for j, mm in inlined.extras(nest):
            names[f"p{j}_in{mm}"] = nests[j].kernel.inputs[mm]
        for pname, node in names.items():
            if node in values:
                bufs.rowvals[pname] = values[node]
        out_dtype = kernel.target.dtype
        wide = True
        binds = []
        for ctype, pname, const in plan.notes["params"]:
            q = "const " if const else ""
            params.append(f"{q}{ctype}* __restrict__ ALIGNED s{s_}_{pname}")
            # an input an earlier member (or name) also reads is read through that member's
            # parameter, so the compiler sees one pointer and shares the loads and the
            # arithmetic on them (a LayerNorm backward's members all scale dy by gamma)
            node = names.get(pname) if const else None
            source = first_param.setdefault((node, ctype), f"s{s_}_{pname}") if node is not None else f"s{s_}_{pname}"
            binds.append(f"      {q}{ctype}* __restrict__ {pname} = ({q}{ctype}*)__builtin_assume_aligned({source}, 16);")
        var = f"rv{s_}_"
        if m.kind != "cells":
            lines.append(f"    float {var};")
        lines.append(f"    {{  // {nest.name}")
        lines += binds
        lines += decode(m.row_vars, "row_", "      ", wide)
        if m.kind == "reduce":
            acc_dt = accumulate_in(shape.reduce_dtype)
            acc_t = VALUE_T[acc_dt]
            ident = literal(shape.identity, acc_dt)
            inner_var, inner_extent = m.col
            vec = m.vec
            chunks = inner_extent // vec
            lines.append(f"      {acc_t} acc = {ident};")
            lines += cell_loop(s_, chunks, "      ")[0]
            lines += decode([(inner_var + "_b", chunks)], "c_", "        ", True)
            lines.append("#pragma unroll")
            lines.append(f"        for (int j_ = 0; j_ < {vec}; j_++) {{")
            lines.append(f"        const int {inner_var} = {inner_var}_b * {vec} + j_;")
            lines += ["        " + value_line(i, bufs) for i in shape.body]
            lines.append("        " + _fold(shape.fold, "acc", f"({acc_t}){shape.item}"))
            lines += ["        }", "      }"]
            if group >= 64:
                lines.append(f"      acc = {'wave_fold_add' if shape.fold is Op.ADD else 'wave_fold_max'}(acc);")
            else:  # the butterfly of plan_reduce's lane groups
                k = group // 2
                while k > 0:
                    lines.append(f"      acc = {'fadd' if shape.fold is Op.ADD else 'fmax_nan'}(acc, ({acc_t})__shfl_xor(acc, {k}));")
                    k //= 2
            if group == THREADS:
                lines.append("      if ((threadIdx.x & 63) == 0) rp_fold_[threadIdx.x >> 6] = acc;")
                lines.append("      __syncthreads();")
                lines.append("      acc = rp_fold_[0];")
                for w in range(1, THREADS // 64):
                    lines.append("      " + _fold(shape.fold, "acc", f"rp_fold_[{w}]"))
                lines.append("      __syncthreads();")
            out_ref = f"out[{render_index(shape.out_index, wide)}]"
            lines.append(f"      if ({tid} == 0) {out_ref} = {store_expr(out_dtype, 'acc')};")
            lines.append(f"      {var} = (float)acc;")
            values[kernel.target] = (var, out_dtype)
        elif m.kind == "scalar":
            lines += ["      " + value_line(i, bufs) for i in shape.body]
            write = shape.write
            lines.append(f"      if ({tid} == 0) out[{render_index(write.arg[1], wide)}] = {store_expr(out_dtype, write.srcs[0])};")
            lines.append(f"      {var} = (float){write.srcs[0]};")
            values[kernel.target] = (var, out_dtype)
        else:
            col_var, extent = m.col
            vec = setup[s_][1]
            write = shape.write
            loop, _ = cell_loop(s_, extent // vec, "      ")
            pre, runs = run_loads(nest, shape.body, bufs, col_var, vec, "        ") if vec > 1 else ([], {})
            stream = c in streamed
            lines += loop
            lines.append(f"        const i64 {col_var}_b = c_;")
            lines += pre
            if vec > 1:
                lines.append(f"        {STORE_T[out_dtype]}* out_p = out + (i64)({run_start(write.arg[1], col_var, vec)});")
            lines.append("#pragma unroll")
            lines.append(f"        for (int j_ = 0; j_ < {vec}; j_++) {{")
            lines.append(f"        const int {col_var} = {col_var}_b * {vec} + j_;")
            for instr in shape.body:
                lines += ["        " + ln for ln in runs[instr.dest]] if instr.dest in runs else ["        " + value_line(instr, bufs)]
            ref = "out_p[j_]" if vec > 1 else f"out[{render_index(write.arg[1], wide)}]"
            lines.append("        " + store_line(ref, store_expr(out_dtype, write.srcs[0]), stream))
            lines += ["        }", "      }"]
        lines.append("    }")
    lines += ["  }", "}"]
    source = f'extern "C" __global__ __launch_bounds__({THREADS}) void {name}({", ".join(params)}) {{\n' + "\n".join(lines)
    return source, grid


# Outputs of at least this many bytes that nothing later in the plan reads are written with
# non-temporal stores. A plain store leaves its lines dirty in the 256 MB Infinity Cache, and
# the next kernel that streams through it pays for their write-back: in a looped row softmax
# then LayerNorm of an 8192 x 8192 float32 x (five nests) the first reduce of x ran at 4.0 TB/s
# behind the last nest's 256 MiB write and at 6.5 TB/s once that write streamed, taking the
# chain from 0.268 to 0.238 ms. Smaller outputs keep the cache: a sink that a following plan
# reads (a parameter, an activation) then comes from it.
STREAM_BYTES = 64 << 20


def streamed_outputs(nests: list[LoopNest], kept: set | None, custom_inputs: set | None) -> set[int]:
    """Elementwise nests whose output goes out non-temporally: a plan sink (`kept`, not a CUSTOM
    input) of at least STREAM_BYTES that no later nest reads. None for `kept` streams nothing."""
    if kept is None:
        return set()
    out = set()
    for k, nest in enumerate(nests):
        target = nest.kernel.target
        if target not in kept or (custom_inputs is not None and target in custom_inputs):
            continue
        if math.prod(target.shape) * target.dtype.itemsize < STREAM_BYTES:
            continue
        if any(src is target for later in nests[k + 1:] for src in later.kernel.inputs):
            continue
        out.add(k)
    return out


@dataclass
class Program:
    """A plan's nests as the device will run them (see nest_runners): each nest's Planned, the
    relu epilogues `pairs` {contraction: relu nest}, the inlined producers, the merged runs
    {last member: (members, launch)}, and the hipRTC source and kernel names of the whole plan."""

    plans: list[Planned]
    pairs: dict[int, int]
    inlined: "InlineSet"
    merged: dict[int, tuple[list[int], Launch]]
    source: str
    names: list[str]
    # the nest whose runner launches each merged run (keyed as `merged`); a run missing here
    # launches from its last member's
    launch_at: dict[int, int] = field(default_factory=dict)
    # merged column reduces (keyed as `merged`, whose launch is the partials kernel): the fold
    # launch, each member's byte offset in the shared scratch, and the scratch's size
    columns: dict[int, tuple[Launch, list[int], int]] = field(default_factory=dict)
    # the epilogue readers that add a bias (and a residual): {reader nest: (bias input, residual
    # input or None, the nest whose float32 input the epilogue rounds into the bias, or None)};
    # the other epilogues are relus
    addends: dict[int, tuple] = field(default_factory=dict)
    # the epilogue readers that sum a batched contraction over its batch: {reader nest: the
    # contraction with the batch folded into k, into the reader's output}
    folds: dict[int, "Contraction"] = field(default_factory=dict)

    def launcher_of(self, key: int) -> int:
        return self.launch_at.get(key, key)

    def launches_from(self, k: int) -> list[int]:
        """The merged runs (their keys, in launch order) that nest k's runner launches."""
        return [key for key in self.merged if self.launcher_of(key) == k]

    def role(self, k: int) -> str:
        """What nest k's runner does: 'stash' (a contraction whose relu nest launches it),
        'epilogue', 'inlined', 'deferred' (a merged run's member whose runner launches nothing),
        'merged' (it launches merged runs), 'contraction' or 'launch'."""
        if k in self.pairs:
            return "stash"
        if k in self.inlined.producers:
            return "inlined"
        if self.launches_from(k):
            return "merged"
        if any(k in run for run, _ in self.merged.values()):
            return "deferred"
        if k in set(self.pairs.values()):
            return "epilogue"
        return "contraction" if self.plans[k].contraction is not None else "launch"


def plan_program(nests: list[LoopNest], kept: set | None, custom_inputs: set | None, rows: bool = True) -> Program:
    """Plan every nest of one executor plan: contractions and their relu epilogues
    (epilogue_pairs), small broadcast producers evaluated in their readers (inline_producers),
    chains of row reductions and their readers run as one row program each (row_chains; `rows`
    False builds none), groups of small independent nests sharing a launch (merge_runs). `kept`
    is the buffers the
    plan must keep (sinks and CUSTOM inputs) and `custom_inputs` the CUSTOM inputs alone, both
    recorded by the device's plan_of; None for either turns the optimisations that need it off.
    Touches no GPU."""
    streamed = streamed_outputs(nests, kept, custom_inputs)
    plans = [plan_nest(n, stream=k in streamed) for k, n in enumerate(nests)]
    pairs, addends, folds = epilogue_pairs(nests, plans, kept)
    fused = {j: i for i, j in pairs.items()}
    for j in fused:
        plans[j] = Planned("", [], notes={"epilogue of": nests[fused[j]].name})
        if j in folds:
            plans[j].notes["batch folded into k"] = True
    absorbed = {terms[2] for terms in addends.values() if terms[2] is not None}
    inlined = InlineSet(nests, inline_producers(nests, plans, kept, pairs) | absorbed)
    for c, nest in enumerate(nests):
        if c not in inlined.producers and plans[c].launches and inlined.reached(nest):
            plans[c] = plan_nest(nest, inlined, stream=c in streamed)
    for j in inlined.producers:
        plans[j] = Planned("", [], notes={"inlined": True})
    chains = row_chains(nests, plans, custom_inputs, inlined, pairs) if rows else []
    runs, run_launch = merge_runs(nests, plans, custom_inputs, inlined, pairs, {c for chain in chains for c in chain})
    merged: dict[int, tuple[list[int], Launch]] = {}
    launch_at: dict[int, int] = {}
    merged_sources = []
    for chain in chains:
        name = f"{nests[chain[0]].name}_rows_{nests[chain[-1]].name}"
        source, grid = row_source(name, nests, plans, chain, inlined, streamed)
        merged_sources.append(source)
        merged[chain[-1]] = (chain, Launch(name, grid, THREADS, "merged"))
    runs_all = runs + chains
    columns: dict[int, tuple[Launch, list[int], int]] = {}
    for run, at in zip(runs, run_launch):
        name = f"{nests[run[0]].name}_to_{nests[run[-1]].name}"
        if plans[run[0]].notes.get("columns"):
            source, part_grid, fold_grid, offsets, scratch = merged_columns_source(name, plans, run)
            merged[run[-1]] = (run, Launch(f"{name}_part", part_grid, THREADS, "columns"))
            columns[run[-1]] = (Launch(name, fold_grid, THREADS, "columns"), offsets, scratch)
        else:
            source, grid = merged_source(name, nests, plans, run)
            merged[run[-1]] = (run, Launch(name, grid, THREADS, "merged"))
        merged_sources.append(source)
        launch_at[run[-1]] = at
    in_run = {c for run in runs_all for c in run}
    names = [launch.name for k, p in enumerate(plans) if k not in in_run for launch in p.launches]
    names += [launch.name for _, launch in merged.values()]
    names += [fold.name for fold, _, _ in columns.values()]
    kept_sources = [p.source for k, p in enumerate(plans) if k not in in_run]
    source = PRELUDE + "\n".join(kept_sources + merged_sources) if names else ""
    return Program(plans, pairs, inlined, merged, source, names, launch_at, columns, addends, folds)


def nest_runners(dev, nests: list[LoopNest]):
    """Compile every nest of a plan into one hipRTC program; one runner per nest, in order. A
    contraction whose only reader is a relu nest runs as one MFMA launch with a relu epilogue,
    from the relu nest's runner (see epilogue_pairs); small broadcast producers run inside their
    readers (inline_producers); groups of small independent elementwise nests share one launch
    from their last member's runner (merge_runs)."""
    prog = plan_program(nests, getattr(dev, "plan_kept", None), getattr(dev, "plan_custom_inputs", None),
                        getattr(dev, "row_programs", True))
    plans, pairs, inlined, merged = prog.plans, prog.pairs, prog.inlined, prog.merged
    functions = runtime.load_functions(prog.source, prog.names) if prog.names else {}
    runners = []
    operands: dict[int, list] = {}  # a fused contraction's inputs, from its call to its relu's
    producer_inputs: dict[int, list] = {}  # an inlined producer's inputs, from its call to its readers'
    deferred: dict[int, tuple] = {}  # a merged run member's (inputs, outs), from its call to the run's launch
    for k, (nest, plan) in enumerate(zip(nests, plans)):
        role = prog.role(k)
        if role == "stash":
            runners.append(_stash_runner(operands, k))
        elif role == "inlined":
            runners.append(_keep_runner(producer_inputs, k))
        elif role == "merged":
            launches = []
            for key in prog.launches_from(k):
                run, launch = merged[key]
                if key in prog.columns:
                    fold, offsets, scratch = prog.columns[key]
                    count = sum(_param_count(plans[c]) for c in run)
                    launches.append((_launcher(dev, functions[launch.name], launch, count - 1), run,
                                     (_launcher(dev, functions[fold.name], fold, 2 * len(run) - 1), offsets, scratch, [])))
                    continue
                count = sum(len(plans[c].notes["params"]) for c in run)
                launches.append((_launcher(dev, functions[launch.name], launch, count - 1), run, None))
            runners.append(_merged_runner(dev, launches, nests, inlined, producer_inputs, deferred, k))
        elif role == "deferred":
            runners.append(_defer_runner(deferred, k))
        elif role == "epilogue" and k in prog.folds:
            source = next(i for i, j in pairs.items() if j == k)
            runners.append(_fold_runner(dev, prog.folds[k], operands, source))
        elif role == "epilogue":
            source = next(i for i, j in pairs.items() if j == k)
            runners.append(_epilogue_runner(dev, plans[source].contraction, operands, source, prog.addends.get(k),
                                            producer_inputs))
        elif role == "contraction":
            runners.append(_contraction_runner(dev, plan.contraction))
        else:
            extras = inlined.extras(nest)
            nin = len(nest.kernel.inputs) + len(extras)
            launchers = []
            for launch in plan.launches:
                count = {"io": nin + 1, "io_scratch": nin + 1, "io_scratch_out": nin + 2}.get(launch.args, 2)
                launchers.append((launch.args, _launcher(dev, functions[launch.name], launch, count - 1)))
            runners.append(_make_runner(dev, launchers, plan.scratch_bytes, extras, producer_inputs))
        # the kernels this runner launches, by name (what a profile of the plan shows)
        if role == "merged":
            runners[-1].kernels = tuple(name for key in prog.launches_from(k)
                                        for name in (merged[key][1].name,) + ((prog.columns[key][0].name,) if key in prog.columns else ()))
        elif role == "launch":
            runners[-1].kernels = tuple(launch.name for launch in plan.launches)
    return runners


def _defer_runner(deferred: dict, k: int):
    """A merged run's member before its last: keep its buffers for the run's one launch."""

    def run(inputs: list, outs: list) -> None:
        deferred[k] = (inputs, outs)

    run.launches_nothing = True
    run.writes_output = True  # by the run's launch
    return run


def _merged_runner(dev, launches: list, nests: list[LoopNest], inlined: "InlineSet", producer_inputs: dict,
                   deferred: dict, k: int):
    """The runner that launches merged runs, (launch, members, columns) in order, nest k among
    their members: one launch per run over every member's buffers, in parameter order (inputs,
    an inlined producer's inputs, out). A run of column reduces (`columns` = (fold launch, scratch
    offsets, scratch bytes, held scratch)) launches its partials with each member's inputs and its
    share of the scratch, then its folds with each member's scratch share and out; the scratch
    is allocated on the first run and kept."""
    extras = {c: inlined.extras(nests[c]) for _, members, _ in launches for c in members}

    def run(inputs: list, outs: list) -> None:
        deferred[k] = (inputs, outs)
        for launch, members, columns in launches:
            ptrs: list[int] = []
            if columns is None:
                for c in members:
                    ins, outs_c = deferred.pop(c)
                    ptrs += [b.ptr for b in ins]
                    ptrs += [producer_inputs[j][m].ptr for j, m in extras[c]]
                    ptrs.append(outs_c[0].ptr)
                launch(ptrs)
                continue
            fold, offsets, scratch, held = columns
            if not held:
                held.append(dev._alloc(scratch))
            folds: list[int] = []
            for c, off in zip(members, offsets):
                ins, outs_c = deferred.pop(c)
                ptrs += [b.ptr for b in ins]
                ptrs += [producer_inputs[j][m].ptr for j, m in extras[c]]
                ptrs.append(held[0].ptr + off)
                folds += [held[0].ptr + off, outs_c[0].ptr]
            launch(ptrs)
            fold(folds)

    return run


def _keep_runner(producer_inputs: dict, k: int):
    """An inlined producer's own call: keep its inputs for its readers, launch nothing (its
    output buffer is never read)."""

    def run(inputs: list, outs: list) -> None:
        producer_inputs[k] = inputs

    run.launches_nothing = True
    return run


def _matmul_launcher(dev, con: Contraction, epilogue: int, adds: bool = False):
    """launch(inputs, out_ptr, bias_ptr, residual_ptr): the contraction through limn_hip_matmul, or
    through limn_hip_matmul_add when `adds` (the residual read at the output's strides)."""
    from limn_amd.dtypes import ABI_CODE

    lib = dev.lib
    code = ABI_CODE[con.dtype]
    size = con.dtype.itemsize
    shape = (code, con.batch, con.M, con.N, con.K, con.a_batch, con.a_m, con.a_k, con.b_batch, con.b_k, con.b_n, con.c_batch, con.c_m, con.c_n, epilogue)
    ws_bytes = int(lib.limn_hip_matmul_workspace(code, con.batch, con.M, con.N, con.K))
    held: list = []  # the split-k workspace, allocated on first use and kept with the runner

    def launch(inputs: list, out: int, bias: int | None = None, res: int | None = None, bias_code: int = code) -> None:
        if ws_bytes and not held:
            held.append(dev._alloc(ws_bytes))
        a = inputs[con.a_input].ptr + con.a_offset * size
        b = inputs[con.b_input].ptr + con.b_offset * size
        ws = held[0].ptr if held else None
        if adds:
            args = (a, b, out, *shape, bias, bias_code, 1, res, con.c_batch, con.c_m, con.c_n, ws, ws_bytes)
            runtime.check_limn(lib.limn_hip_matmul_add(*args, None))
            if dev.tape is not None:
                dev.tape.append(replay.Launch(replay.STEP_MATMUL_ADD, args))
            return
        runtime.check_limn(lib.limn_hip_matmul(a, b, out, *shape, ws, ws_bytes, None))
        if dev.tape is not None:
            dev.tape.append(replay.Launch(replay.STEP_MATMUL, (a, b, out, *shape, ws, ws_bytes)))

    return launch


def _contraction_runner(dev, con: Contraction):
    launch = _matmul_launcher(dev, con, 0)

    def run(inputs: list, outs: list) -> None:
        launch(inputs, outs[0].ptr)

    return run


def _stash_runner(operands: dict, k: int):
    """A fused contraction's own call: keep its operands for the relu nest's call, launch nothing
    (its output buffer is never read)."""

    def run(inputs: list, outs: list) -> None:
        operands[k] = inputs

    run.launches_nothing = True
    return run


def _fold_runner(dev, folded: Contraction, operands: dict, k: int):
    """The batch-sum reader's call: the batched contraction of nest k with its batch folded into
    k, stored into this nest's output (see batch_sum_fold)."""
    launch = _matmul_launcher(dev, folded, 0)

    def run(inputs: list, outs: list) -> None:
        launch(operands.pop(k), outs[0].ptr)

    run.folded = folded
    return run


def _epilogue_runner(dev, con: Contraction, operands: dict, k: int, terms: tuple | None = None,
                     producer_inputs: dict | None = None):
    """The epilogue reader's call: the contraction of nest k, stored into this nest's output with
    a relu, or (`terms` = (bias input, residual input or None, bias cast nest or None) of this
    nest) with the bias and residual added; a bias whose cast nest the epilogue took over is that
    nest's float32 input. Its layout is the contraction's: the reader reads and writes cell for
    cell."""
    if terms is None:
        launch = _matmul_launcher(dev, con, 1)

        def run(inputs: list, outs: list) -> None:
            launch(operands.pop(k), outs[0].ptr)

        return run
    launch = _matmul_launcher(dev, con, 0, adds=True)
    bias, res, cast = terms
    from limn_amd.dtypes import ABI_CODE

    bias_code = ABI_CODE[float32 if cast is not None else con.dtype]

    def run(inputs: list, outs: list) -> None:
        bias_ptr = producer_inputs[cast][0].ptr if cast is not None else inputs[bias].ptr
        launch(operands.pop(k), outs[0].ptr, bias_ptr, None if res is None else inputs[res].ptr, bias_code)

    return run


def _make_runner(dev, launchers, scratch_bytes: int, extras: list | None = None, producer_inputs: dict | None = None):
    held: list = []

    def run(inputs: list, outs: list) -> None:
        if scratch_bytes and not held:
            held.append(dev._alloc(scratch_bytes))
        ins = [b.ptr for b in inputs]
        if extras:
            ins += [producer_inputs[j][m].ptr for j, m in extras]
        for kind, launch in launchers:
            if kind == "io":
                launch(ins + [outs[0].ptr])
            elif kind == "io_scratch":
                launch(ins + [held[0].ptr])
            elif kind == "io_scratch_out":
                launch(ins + [held[0].ptr, outs[0].ptr])
            else:
                launch([held[0].ptr, outs[0].ptr])

    return run
