"""The Device protocol and the process-global device registry (reference `limn/device.py:35-60,
178-220`).

A Device owns opaque byte buffers and executes graphs against them; everything above it
(tensor, nn, optim) is device-agnostic. `set_device(name)` constructs the named device from
its factory, which checks its toolchain first and raises RuntimeError with the reason.

This package registers one device, "hip" (limn_amd/hip/device.py). limn's own numpy
interpreter is the reference every device is diffed against; here it lives with the test
oracle and is registered by the tests, not by the product.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any, Protocol

import numpy as np

from limn_amd.ops import Node

Buffer = Any


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


def _hip_device() -> Device:
    from limn_amd.hip.device import HipDevice
    from limn_amd.hip.runtime import hip_unavailable

    reason = hip_unavailable()
    if reason is not None:
        raise RuntimeError(f"the 'hip' device is unavailable: {reason}")
    return HipDevice()


DEVICES: dict[str, Callable[[], Device]] = {"hip": _hip_device}

active_device: Device | None = None


def register(name: str, factory: Callable[[], Device]) -> None:
    """Add a device factory under `name` (tests register the numpy reference this way)."""
    DEVICES[name] = factory


def active() -> Device:
    if active_device is None:
        raise RuntimeError(f"no device selected: call set_device() with one of {tuple(DEVICES)}")
    return active_device


def set_device(name: str) -> None:
    global active_device
    if name not in DEVICES:
        raise ValueError(f"unknown device {name!r}; limn has {tuple(DEVICES)}")
    active_device = DEVICES[name]()
