"""TEST INFRASTRUCTURE ONLY - the CPU baseline: limn's C backend restated over this package's IR.

Each scheduled loop nest becomes one single-threaded C function (reference
limn/backend_c.py:147-186), all of a plan's nests one shared library compiled by the host C
compiler with -O3 (and -march=native where it is accepted, reference :37-52), called through
ctypes (:239-264). It declines float16/bfloat16 like the reference (:189-208) and has no CUSTOM
kernels, so attention on it takes limn's composed path (reference limn/tensor.py:559-560).
Only tests/ and bench.py's cpu_baseline leg use this module; the hip device never imports it.

Where it departs from the reference, and why:
  - integers wrap (-fwrapv): C leaves signed overflow undefined, numpy (the oracle) wraps;
  - the innermost loop is split at mask edges (reference limn/codegen.py:404-436, `split_masked`)
    by this module's own `split_innermost`, so a padded read in that loop costs no check.
"""

from __future__ import annotations

import ctypes
import functools
import hashlib
import math
import shutil
import subprocess
import tempfile
import time
from pathlib import Path
from typing import Any, Sequence

import numpy as np

from limn_amd.seam import CompiledDevice, DType, HostDevice, Index, Instr, LoopNest, Op, Opcode, Runner, Valid, float32, float64, int8, int16, int32, loop_range

Buffer = Any

C_TYPE = {float64: "double", float32: "float", int32: "int32_t", int16: "int16_t", int8: "int8_t"}

_libraries: dict[str, ctypes.CDLL] = {}
_workdir: Path | None = None


def compiler() -> str | None:
    return shutil.which("cc") or shutil.which("gcc")


@functools.cache
def flags() -> tuple[str, ...]:
    """-O3, plus -march=native where this compiler accepts it (without it gcc targets baseline
    x86-64 and the innermost loops vectorise at SSE2 width at best), plus -fwrapv."""
    cc = compiler()
    probe = subprocess.run([cc, "-march=native", "-E", "-x", "c", "-"], input="", capture_output=True, text=True)
    return ("-O3", "-march=native", "-fwrapv") if probe.returncode == 0 else ("-O3", "-fwrapv")


def literal(value: float | int, dtype: DType) -> str:
    if dtype in (float32, float64):
        v = float(value)
        if math.isnan(v):
            return "NAN"
        if math.isinf(v):
            return "INFINITY" if v > 0 else "-INFINITY"
        return repr(v) if dtype == float64 else f"{float(np.float32(v))!r}f"
    bits = 8 * dtype.itemsize
    v = ((int(value) + (1 << (bits - 1))) % (1 << bits)) - (1 << (bits - 1))
    return "(-2147483647 - 1)" if v == -(1 << 31) else str(v)


def _math(name: str, dtype: DType) -> str:
    # float64 uses C's double functions; everything else the float ones (an int operand converts)
    return name if dtype == float64 else name + "f"


def arith(op: Op, srcs: Sequence[str], dtype: DType) -> str:
    t = C_TYPE[dtype]
    a = list(srcs)
    if op is Op.NEG:
        return f"-{a[0]}"
    if op in (Op.EXP, Op.LOG, Op.SQRT):
        return f"{_math(op.name.lower(), dtype)}({a[0]})"
    if op is Op.RECIP:
        return f"({t})1 / {a[0]}"
    if op is Op.ADD:
        return f"{a[0]} + {a[1]}"
    if op is Op.MUL:
        return f"{a[0]} * {a[1]}"
    if op is Op.CMPLT:
        return f"({t})({a[0]} < {a[1]})"
    if op is Op.WHERE:
        return f"{a[0]} != 0 ? {a[1]} : {a[2]}"
    raise NotImplementedError(f"the c device has no lowering for {op}")


def fold(op: Op, dest: str, src: str) -> str:
    """ADD, or MAX that keeps a NaN once it is in (reference limn/backend_c.py:82-91)."""
    if op is Op.ADD:
        return f"{dest} = {dest} + {src};"
    return f"{dest} = ({dest} > {src} || {dest} != {dest}) ? {dest} : {src};"


def guarded(valid: Valid, dtype: DType, expr: str) -> str:
    if not valid.bounds:
        return expr
    t = C_TYPE[dtype]
    return f"({valid.render()}) ? ({t})({expr}) : ({t})0"


# ---- mask splitting -----------------------------------------------------------------------------


def _matching_end(instrs: Sequence[Instr], start: int) -> int:
    depth = 0
    for k in range(start, len(instrs)):
        if instrs[k].opcode is Opcode.LOOP:
            depth += 1
        elif instrs[k].opcode is Opcode.ENDLOOP:
            depth -= 1
            if depth == 0:
                return k
    raise ValueError("unbalanced LOOP/ENDLOOP")


def _resolve(instr: Instr, var: str, lo: int, hi: int) -> Instr:
    """A guarded LOAD/CONST inside [lo, hi) of `var`: the checks on `var` are constant there."""
    if instr.opcode not in (Opcode.LOAD, Opcode.CONST):
        return instr
    valid: Valid = instr.arg[2] if instr.opcode is Opcode.LOAD else instr.arg[1]
    keep = []
    for bound in valid.bounds:
        bvar, blo, bhi, _ = bound
        if bvar != var:
            keep.append(bound)
        elif hi <= blo or lo >= bhi:  # wholly outside: the read is a zero
            return Instr(Opcode.CONST, instr.dest, instr.dtype, (), (0, Valid()))
        # wholly inside: the check folds away
    new_valid = Valid(tuple(keep))
    if instr.opcode is Opcode.LOAD:
        buf, index, _ = instr.arg
        return Instr(Opcode.LOAD, instr.dest, instr.dtype, instr.srcs, (buf, index, new_valid))
    value, _ = instr.arg
    return Instr(Opcode.CONST, instr.dest, instr.dtype, instr.srcs, (value, new_valid))


def split_innermost(loop: Instr, body: Sequence[Instr], end: Instr) -> list[Instr]:
    """Cut an innermost loop at every mask edge on its variable, so that in each piece every
    check on it is constant. Same iterations in the same order: bit-identical."""
    var = loop.dest
    lo, hi = loop_range(loop)
    cuts = {lo, hi}
    for instr in body:
        if instr.opcode in (Opcode.LOAD, Opcode.CONST):
            valid: Valid = instr.arg[2] if instr.opcode is Opcode.LOAD else instr.arg[1]
            for bvar, blo, bhi, _ in valid.bounds:
                if bvar == var:
                    cuts.update(c for c in (blo, bhi) if lo < c < hi)
    if len(cuts) == 2:
        return [loop, *body, end]
    points = sorted(cuts)
    out: list[Instr] = []
    for a, b in zip(points, points[1:]):
        out.append(Instr(Opcode.LOOP, var, loop.dtype, loop.srcs, (a, b)))
        out += [_resolve(instr, var, a, b) for instr in body]
        out.append(end)
    return out


def split_masked(instrs: Sequence[Instr]) -> list[Instr]:
    out: list[Instr] = []
    k = 0
    while k < len(instrs):
        instr = instrs[k]
        if instr.opcode is not Opcode.LOOP:
            out.append(instr)
            k += 1
            continue
        e = _matching_end(instrs, k)
        body = instrs[k + 1 : e]
        if any(i.opcode is Opcode.LOOP for i in body):
            out += [instr, *split_masked(body), instrs[e]]
        else:
            out += split_innermost(instr, body, instrs[e])
        k = e + 1
    return out


# ---- emission -----------------------------------------------------------------------------------


def _index(index: Index) -> str:
    return index.render()


def unsupported_dtype(nest: LoopNest) -> DType | None:
    dtypes = [node.dtype for node in nest.kernel.inputs] + [nest.kernel.target.dtype]
    dtypes += [i.dtype for i in nest.instrs if i.dtype is not None]
    return next((d for d in dtypes if d not in C_TYPE), None)


def emit_function(nest: LoopNest, split: bool = True) -> str:
    kernel = nest.kernel
    params = ", ".join([f"void* in{k}" for k in range(len(kernel.inputs))] + ["void* out"])
    lines = [f"void {nest.name}({params}) {{"]
    for k, node in enumerate(kernel.inputs):
        lines.append(f"  const {C_TYPE[node.dtype]}* _in{k} = (const {C_TYPE[node.dtype]}*)in{k};")
    # every call gets a fresh output, never an input's bytes, so it aliases nothing
    out_t = C_TYPE[kernel.target.dtype]
    lines.append(f"  {out_t}* restrict _out = ({out_t}*)out;")
    depth = 1
    for instr in split_masked(nest.instrs) if split else nest.instrs:
        pad = "  " * depth
        op = instr.opcode
        if op is Opcode.LOOP:
            lo, hi = loop_range(instr)
            lines.append(f"{pad}for (int {instr.dest} = {lo}; {instr.dest} < {hi}; {instr.dest}++) {{")
            depth += 1
        elif op is Opcode.ENDLOOP:
            depth -= 1
            lines.append("  " * depth + "}")
        elif op is Opcode.ACC:
            lines.append(f"{pad}{C_TYPE[instr.value_type]} {instr.dest} = {literal(instr.arg, instr.value_type)};")
        elif op is Opcode.CONST:
            value, valid = instr.arg
            expr = guarded(valid, instr.value_type, literal(value, instr.value_type))
            lines.append(f"{pad}const {C_TYPE[instr.value_type]} {instr.dest} = {expr};")
        elif op is Opcode.LOAD:
            buf, index, valid = instr.arg
            expr = guarded(valid, instr.value_type, f"_{buf}[{_index(index)}]")
            lines.append(f"{pad}const {C_TYPE[instr.value_type]} {instr.dest} = {expr};")
        elif op is Opcode.ARITH:
            lines.append(f"{pad}const {C_TYPE[instr.value_type]} {instr.dest} = {arith(instr.arg, instr.srcs, instr.value_type)};")
        elif op is Opcode.CAST:
            lines.append(f"{pad}const {C_TYPE[instr.value_type]} {instr.dest} = ({C_TYPE[instr.value_type]})({instr.srcs[0]});")
        elif op is Opcode.GATHER:
            buf, index = instr.arg
            lines.append(f"{pad}const {C_TYPE[instr.value_type]} {instr.dest} = _{buf}[{_index(index)}];")
        elif op is Opcode.UPDATE:
            lines.append(pad + fold(instr.arg, instr.dest, instr.srcs[0]))
        elif op is Opcode.STORE:
            buf, index = instr.arg
            lines.append(f"{pad}_{buf}[{_index(index)}] = {instr.srcs[0]};")
        elif op is Opcode.ACCUM:
            buf, index, f = instr.arg
            lines.append(pad + fold(f, f"_{buf}[{_index(index)}]", instr.srcs[0]))
        elif op is Opcode.SCATTER:
            buf, index = instr.arg
            lines.append(f"{pad}_{buf}[{_index(index)}] += {instr.srcs[0]};")
        else:
            raise NotImplementedError(f"the c device cannot emit {op}")
    lines.append("}")
    return "\n".join(lines)


def emit_c(nests: Sequence[LoopNest], split: bool = True) -> str:
    parts = ["#include <math.h>", "#include <stdint.h>", ""]
    for nest in nests:
        dtype = unsupported_dtype(nest)
        if dtype is not None:
            raise NotImplementedError(f"the c device has no {dtype}; run this graph on the numpy or hip device")
        parts += [emit_function(nest, split), ""]
    return "\n".join(parts)


def compile_c(source: str) -> ctypes.CDLL:
    global _workdir
    key = hashlib.sha256(" ".join(flags()).encode() + source.encode()).hexdigest()
    lib = _libraries.get(key)
    if lib is not None:
        return lib
    cc = compiler()
    if cc is None:
        raise RuntimeError("c device: no C compiler (cc or gcc) on PATH")
    if _workdir is None:
        _workdir = Path(tempfile.mkdtemp(prefix="limn_c_"))
    src, so = _workdir / f"{key[:16]}.c", _workdir / f"{key[:16]}.so"
    src.write_text(source)
    done = subprocess.run([cc, *flags(), "-shared", "-fPIC", "-o", str(so), str(src), "-lm"], capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"c device: compiling failed:\n{done.stderr}")
    lib = ctypes.CDLL(str(so))
    _libraries[key] = lib
    return lib


class CDevice(CompiledDevice, HostDevice):
    """Plans, caching and the assign transaction from CompiledDevice; host byte buffers; every
    nest a compiled C function run on the calling thread."""

    def __init__(self, split: bool = True) -> None:
        super().__init__()
        self.split = split
        self.seconds = 0.0  # time spent inside compiled nests (what a CPU baseline times)

    def runners(self, nests: list[LoopNest]) -> list[Runner]:
        lib = compile_c(emit_c(nests, self.split))
        out: list[Runner] = []
        for nest in nests:
            fn = getattr(lib, nest.name)
            fn.argtypes = [ctypes.c_void_p] * (len(nest.kernel.inputs) + 1)
            fn.restype = None
            out.append(lambda ins, outs, fn=fn: self._call(fn, [b.ctypes.data for b in ins] + [outs[0].ctypes.data]))
        return out

    def _call(self, fn, args: list[int]) -> None:
        t0 = time.perf_counter()
        fn(*args)
        self.seconds += time.perf_counter() - t0

    def out_alloc(self, nb: int, zero: bool) -> Buffer:
        return (np.zeros if zero else np.empty)(nb, dtype=np.uint8)

    def commit(self, target: Buffer, value: Buffer) -> None:
        target[:] = value
