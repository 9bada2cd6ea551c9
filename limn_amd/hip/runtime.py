"""ctypes bindings: the HIP runtime (libamdhip64), hipRTC (libhiprtc) and limn's kernel library.

This is the MI355X counterpart of the driver/NVRTC symbol tables of reference
`limn/backend_cuda.py:54-224`: each library is opened once, its functions get explicit
argtypes, and every status code goes through `check`, which raises
`RuntimeError("hip: <doing>: <detail>")`. Nothing here allocates device memory at import time;
`hip_unavailable()` says why the device cannot run (no library, no GPU, not gfx950) without
raising.
"""

from __future__ import annotations

import ctypes
import functools
import hashlib
from pathlib import Path

c_void_p, c_int, c_uint, c_size_t, c_char_p, c_float = (
    ctypes.c_void_p,
    ctypes.c_int,
    ctypes.c_uint,
    ctypes.c_size_t,
    ctypes.c_char_p,
    ctypes.c_float,
)
P = ctypes.POINTER
c_int64 = ctypes.c_int64

ARCH = "gfx950"
ABI_VERSION = 3  # LIMN_HIP_ABI_VERSION of include/limn_hip.h
LIBRARY = Path(__file__).resolve().parent.parent / "liblimn_hip.so"

# hipMemcpyKind
HOST_TO_DEVICE, DEVICE_TO_HOST, DEVICE_TO_DEVICE = 1, 2, 3

_HIP = {
    "hipInit": (c_int, [c_uint]),
    "hipGetDeviceCount": (c_int, [P(c_int)]),
    "hipSetDevice": (c_int, [c_int]),
    "hipGetErrorString": (c_char_p, [c_int]),
    "hipGetLastError": (c_int, []),
    "hipMalloc": (c_int, [P(c_void_p), c_size_t]),
    "hipFree": (c_int, [c_void_p]),
    "hipMemcpy": (c_int, [c_void_p, c_void_p, c_size_t, c_int]),
    "hipMemcpyAsync": (c_int, [c_void_p, c_void_p, c_size_t, c_int, c_void_p]),
    "hipMemsetAsync": (c_int, [c_void_p, c_int, c_size_t, c_void_p]),
    "hipHostMalloc": (c_int, [P(c_void_p), c_size_t, c_uint]),
    "hipHostFree": (c_int, [c_void_p]),
    "hipMemGetInfo": (c_int, [P(c_size_t), P(c_size_t)]),
    "hipDeviceSynchronize": (c_int, []),
    "hipStreamSynchronize": (c_int, [c_void_p]),
    "hipModuleLoadData": (c_int, [P(c_void_p), c_void_p]),
    "hipModuleGetFunction": (c_int, [P(c_void_p), c_void_p, c_char_p]),
    "hipModuleLaunchKernel": (
        c_int,
        [c_void_p, c_uint, c_uint, c_uint, c_uint, c_uint, c_uint, c_uint, c_void_p, P(c_void_p), P(c_void_p)],
    ),
    "hipEventCreate": (c_int, [P(c_void_p)]),
    "hipEventRecord": (c_int, [c_void_p, c_void_p]),
    "hipEventSynchronize": (c_int, [c_void_p]),
    "hipEventElapsedTime": (c_int, [P(c_float), c_void_p, c_void_p]),
    "hipEventDestroy": (c_int, [c_void_p]),
}

_RTC = {
    "hiprtcVersion": (c_int, [P(c_int), P(c_int)]),
    "hiprtcCreateProgram": (c_int, [P(c_void_p), c_char_p, c_char_p, c_int, P(c_char_p), P(c_char_p)]),
    "hiprtcCompileProgram": (c_int, [c_void_p, c_int, P(c_char_p)]),
    "hiprtcGetProgramLogSize": (c_int, [c_void_p, P(c_size_t)]),
    "hiprtcGetProgramLog": (c_int, [c_void_p, c_char_p]),
    "hiprtcGetCodeSize": (c_int, [c_void_p, P(c_size_t)]),
    "hiprtcGetCode": (c_int, [c_void_p, c_char_p]),
    "hiprtcDestroyProgram": (c_int, [P(c_void_p)]),
}

_I64 = c_int64
_LIMN = {
    "limn_hip_abi_version": (c_int, []),
    "limn_hip_last_error": (c_char_p, []),
    "limn_hip_device_info": (c_int, [c_int, c_char_p, c_int, P(c_int), P(c_int), P(c_int64)]),
    "limn_hip_sdpa_path": (c_int, [c_int, _I64, _I64]),
    "limn_hip_matmul": (c_int, [c_void_p, c_void_p, c_void_p, c_int] + [_I64] * 13 + [c_int, c_void_p, _I64, c_void_p]),
    "limn_hip_matmul_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_int] + [_I64] * 13 + [c_int, c_void_p]),
    "limn_hip_matmul_add": (c_int, [c_void_p, c_void_p, c_void_p, c_int] + [_I64] * 13
                            + [c_int, c_void_p, c_int, _I64, c_void_p, _I64, _I64, _I64, c_void_p, _I64, c_void_p]),
    "limn_hip_matmul_workspace": (_I64, [c_int, _I64, _I64, _I64, _I64]),
    "limn_hip_replay": (c_int, [c_void_p, _I64, c_void_p, _I64, c_void_p, _I64, c_void_p]),
    "limn_hip_replay_graph": (c_int, [c_void_p, _I64, c_void_p, _I64, c_void_p, _I64, c_void_p]),
    "limn_hip_replay_graph_free": (c_int, [c_void_p]),
    "limn_hip_matmul_supported": (c_int, [c_int] + [_I64] * 9),
    "limn_hip_sdpa_fwd": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, _I64, _I64, _I64, _I64, _I64, c_int,
         ctypes.c_double, c_void_p],
    ),
    "limn_hip_sdpa_bwd_q": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, _I64, _I64, _I64, _I64,
         _I64, c_int, ctypes.c_double, c_void_p],
    ),
    "limn_hip_sdpa_bwd_kv": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, _I64, _I64,
         _I64, _I64, _I64, c_int, ctypes.c_double, c_void_p],
    ),
    "limn_hip_sdpa_bwd": (
        c_int,
        [c_void_p] * 10 + [c_int, _I64, _I64, _I64, _I64, _I64, c_int, ctypes.c_double, c_int, c_void_p, _I64, c_void_p],
    ),
    "limn_hip_sdpa_bwd_workspace": (_I64, [c_int, _I64, _I64, _I64, _I64, _I64, c_int, c_int]),
}

# The C ABI's status codes (include/limn_hip.h) and the Python exception each maps to.
LIMN_OK, LIMN_EINVAL, LIMN_EUNSUPPORTED, LIMN_ERUNTIME = 0, 1, 2, 3


def _bind(lib: ctypes.CDLL, table: dict) -> ctypes.CDLL:
    for name, (restype, argtypes) in table.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = restype, argtypes
    return lib


def _open(names: list[str]) -> ctypes.CDLL | None:
    for name in names:
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    return None


@functools.cache
def hip() -> ctypes.CDLL | None:
    lib = _open(["libamdhip64.so.7", "libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"])
    return None if lib is None else _bind(lib, _HIP)


@functools.cache
def hiprtc() -> ctypes.CDLL | None:
    lib = _open(["libhiprtc.so.7", "libhiprtc.so", "/opt/rocm/lib/libhiprtc.so"])
    return None if lib is None else _bind(lib, _RTC)


@functools.cache
def kernels() -> ctypes.CDLL:
    """liblimn_hip.so, the hand-written kernels. Raises if it has not been built."""
    if not LIBRARY.exists():
        raise RuntimeError(f"{LIBRARY} is missing: build it with `python -m limn_amd.build` (hipcc, gfx950)")
    lib = _bind(ctypes.CDLL(str(LIBRARY)), _LIMN)
    if lib.limn_hip_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIBRARY} speaks ABI {lib.limn_hip_abi_version()}, this package expects {ABI_VERSION}: rebuild it")
    return lib


def check(status: int, doing: str) -> None:
    """Raise RuntimeError for a failed HIP runtime call."""
    if status == 0:
        return
    api = hip()
    detail = api.hipGetErrorString(status).decode() if api is not None else f"error {status}"
    raise RuntimeError(f"hip: {doing}: {detail}")


def check_limn(status: int) -> None:
    """Map a status from liblimn_hip.so to the exception limn raises for the same condition."""
    if status == LIMN_OK:
        return
    message = kernels().limn_hip_last_error().decode()
    if status == LIMN_EINVAL:
        raise ValueError(message)
    if status == LIMN_EUNSUPPORTED:
        raise NotImplementedError(message)
    raise RuntimeError(message)


@functools.cache
def hip_unavailable() -> str | None:
    """None when the hip device can run here, else the reason it cannot."""
    api = hip()
    if api is None:
        return "libamdhip64 not found (it ships with ROCm)"
    if hiprtc() is None:
        return "libhiprtc not found (it ships with ROCm)"
    if api.hipInit(0) != 0:
        return "hipInit failed (no usable AMD GPU driver?)"
    count = c_int()
    if api.hipGetDeviceCount(ctypes.byref(count)) != 0 or count.value == 0:
        return "no HIP device found"
    try:
        lib = kernels()
    except (OSError, RuntimeError) as err:
        return str(err)
    arch = ctypes.create_string_buffer(256)
    if lib.limn_hip_device_info(0, arch, 256, None, None, None) != 0:
        return lib.limn_hip_last_error().decode()
    name = arch.value.decode().split(":")[0]
    if name != ARCH:
        return f"device 0 is {name}; these kernels are built for {ARCH} (MI355X) only"
    return None


def has_hip() -> bool:
    return hip_unavailable() is None


# ---- hipRTC ----

_programs: dict[str, dict[str, int]] = {}
# Every floating-point operation of a generated kernel rounds on its own (no multiply-add
# contraction), as the numpy device's do: whether the compiler fuses a product into a following
# add otherwise depends on how many uses the product has, so the same nest gave different bits
# alone and inside a row program, where a value computed by several members is shared.
RTC_OPTIONS = (f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-ffp-contract=off",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")


def rtc_version() -> str:
    major, minor = c_int(), c_int()
    lib = hiprtc()
    if lib is None or lib.hiprtcVersion(ctypes.byref(major), ctypes.byref(minor)) != 0:
        return "unknown"
    return f"{major.value}.{minor.value}"


def compile_source(source: str, names: list[str]) -> bytes:
    """hipRTC-compile `source` for gfx950 and return the code object. Raises RuntimeError with
    the compiler log on failure (reference `limn/backend_cuda.py:202-209` does the same)."""
    rtc = hiprtc()
    if rtc is None:
        raise RuntimeError("hiprtc: library not found")
    prog = c_void_p()
    if rtc.hiprtcCreateProgram(ctypes.byref(prog), source.encode(), b"limn_kernels.hip", 0, None, None) != 0:
        raise RuntimeError("hiprtc: could not create a program")
    try:
        opts = (c_char_p * len(RTC_OPTIONS))(*(o.encode() for o in RTC_OPTIONS))
        if rtc.hiprtcCompileProgram(prog, len(RTC_OPTIONS), opts) != 0:
            size = c_size_t()
            rtc.hiprtcGetProgramLogSize(prog, ctypes.byref(size))
            log = ctypes.create_string_buffer(max(size.value, 1))
            rtc.hiprtcGetProgramLog(prog, log)
            raise RuntimeError(f"hiprtc failed:\n{log.value.decode(errors='replace')}")
        size = c_size_t()
        rtc.hiprtcGetCodeSize(prog, ctypes.byref(size))
        code = ctypes.create_string_buffer(size.value)
        rtc.hiprtcGetCode(prog, code)
        return code.raw
    finally:
        rtc.hiprtcDestroyProgram(ctypes.byref(prog))


def load_functions(source: str, names: list[str]) -> dict[str, int]:
    """Compile (or reuse) a program and resolve its kernels to function handles, cached by
    sha256(arch : hiprtc version : options : source) for the life of the process."""
    key = hashlib.sha256(f"{ARCH}:{rtc_version()}:{' '.join(RTC_OPTIONS)}:{source}".encode()).hexdigest()
    cached = _programs.get(key)
    if cached is not None and all(n in cached for n in names):
        return cached
    code = compile_source(source, names)
    api = hip()
    assert api is not None
    module = c_void_p()
    check(api.hipModuleLoadData(ctypes.byref(module), code), "loading a code object")
    functions: dict[str, int] = {}
    for name in names:
        fn = c_void_p()
        check(api.hipModuleGetFunction(ctypes.byref(fn), module, name.encode()), f"resolving kernel {name}")
        functions[name] = fn.value
    _programs[key] = functions
    return functions
