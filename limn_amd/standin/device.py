"""The Device protocol and the process-global device registry (reference `limn/device.py:35-60,
178-220`).

A Device owns opaque byte buffers and executes graphs against them; everything above it
(tensor, nn, optim) is device-agnostic. `set_device(name)` constructs the named device from
its factory, which checks its toolchain first and raises RuntimeError with the reason.

The registry starts empty here. Devices plug in by adding a factory under a name, as limn's own
registry takes them (`DEVICES["hip"] = factory`): `import limn_amd.hip` adds "hip", and the
tests add the numpy oracle as "numpy".
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any, Protocol

import numpy as np

from .ops import DType, Node, bfloat16, float16, float32, float64, int8, int16, int32

Buffer = Any

# Host storage per dtype. limn stores bfloat16 as ml_dtypes.bfloat16 (reference
# `limn/device.py:25-33`); without ml_dtypes a bfloat16 array is its 16-bit patterns as uint16.
NUMPY_STORAGE: dict[DType, np.dtype] = {
    float64: np.dtype(np.float64),
    float32: np.dtype(np.float32),
    float16: np.dtype(np.float16),
    bfloat16: np.dtype(np.uint16),
    int32: np.dtype(np.int32),
    int16: np.dtype(np.int16),
    int8: np.dtype(np.int8),
}


def to_numpy_storage(values: Any, dtype: DType) -> np.ndarray:
    """Host values as `dtype`'s storage, C-contiguous. bfloat16 rounds float32 to nearest even
    (the carry trick: add 0x7fff plus the kept low bit, drop 16 bits), NaN staying a quiet NaN;
    a uint16 array handed in for bfloat16 is taken as bit patterns already."""
    host = np.asarray(values)
    if dtype != bfloat16:
        return np.ascontiguousarray(host.astype(NUMPY_STORAGE[dtype]))
    if host.dtype == np.uint16:
        return np.ascontiguousarray(host)
    f = np.ascontiguousarray(host, dtype=np.float32)
    wide = f.view(np.uint32).astype(np.uint64)
    bits = ((wide + 0x7FFF + ((wide >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(f), ((wide >> 16) | 0x40).astype(np.uint16), bits)


def from_numpy_storage(raw: np.ndarray, dtype: DType, shape: tuple[int, ...]) -> np.ndarray:
    """A buffer's bytes as numbers of `dtype`; bfloat16 widens to the float32 values it holds."""
    host = np.asarray(raw).view(NUMPY_STORAGE[dtype]).reshape(shape)
    if dtype == bfloat16:
        return (host.astype(np.uint32) << 16).view(np.float32)
    return host


class Device(Protocol):
    """execute() is one transaction: every sink is computed before any ASSIGN commits."""

    def alloc(self, nbytes: int) -> Buffer: ...
    def copyin(self, buf: Buffer, array: np.ndarray) -> None: ...
    def copyout(self, buf: Buffer) -> np.ndarray: ...
    def execute(self, sinks: list[Node]) -> list[Buffer]: ...
    def has_custom(self, name: str) -> bool: ...


class HostDevice:
    """Buffers as flat host uint8 arrays."""

    def alloc(self, nbytes: int) -> Buffer:
        return np.zeros(nbytes, dtype=np.uint8)

    def copyin(self, buf: Buffer, array: np.ndarray) -> None:
        buf[:] = np.ascontiguousarray(array).view(np.uint8).reshape(-1)

    def copyout(self, buf: Buffer) -> np.ndarray:
        return buf.copy()


DEVICES: dict[str, Callable[[], Device]] = {}

active_device: Device | None = None


def active() -> Device:
    if active_device is None:
        raise RuntimeError(f"no device selected: call set_device() with one of {tuple(DEVICES)}")
    return active_device


def set_device(name: str) -> None:
    global active_device
    if name not in DEVICES:
        raise ValueError(f"unknown device {name!r}; limn has {tuple(DEVICES)}")
    active_device = DEVICES[name]()
