"""Shared test helpers.

Markers: `gpu` tests need an MI355X and the built liblimn_hip.so; they fail (not skip) when the
hip device cannot start, so a GPU run can never pass on a silent fallback. Everything else runs
on the CPU against the oracle.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from limn_amd.seam import bfloat16, float16, float32, float64, Node, Op  # noqa: E402
from limn_amd.seam import device as limn_device  # noqa: E402
from limn_amd.dtypes import STORAGE, from_storage, to_storage  # noqa: E402
from oracle.numpy_device import NumpyDevice  # noqa: E402

limn_device.DEVICES["numpy"] = NumpyDevice  # the oracle, as a selectable device for every test


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


_HIP = None


def hip_device():
    """The one HipDevice of the session; raises (never skips) when it cannot start."""
    global _HIP
    if _HIP is None:
        from limn_amd.hip.device import HipDevice
        from limn_amd.hip.runtime import hip_unavailable

        reason = hip_unavailable()
        if reason is not None:
            raise RuntimeError(f"the hip device is unavailable on this machine: {reason}")
        _HIP = HipDevice()
    return _HIP


@pytest.fixture
def hipdev():
    return hip_device()


@pytest.fixture(autouse=True)
def _restore_device():
    """Any test may switch devices; none may leak that to the next one."""
    before = limn_device.active_device
    yield
    limn_device.active_device = before


DTYPES = {"float64": float64, "float32": float32, "float16": float16, "bfloat16": bfloat16}


def upload(dev, values: np.ndarray, dtype) -> Node:
    """A BUFFER node on `dev` holding `values` rounded to `dtype`."""
    host = to_storage(values, dtype)
    buf = dev.alloc(host.nbytes)
    dev.copyin(buf, host)
    return Node(Op.BUFFER, (), dtype, tuple(values.shape), buf)


def download(dev, buf, dtype, shape) -> np.ndarray:
    """A device buffer's bytes as numbers (bfloat16 widened to float32)."""
    return from_storage(dev.copyout(buf), dtype, tuple(shape))


def storage_values(values: np.ndarray, dtype) -> np.ndarray:
    """What `values` become once stored at `dtype`, as float32/float64 numbers."""
    return from_storage(to_storage(values, dtype).view(np.uint8), dtype, values.shape).astype(
        np.float64 if dtype is float64 else np.float32
    )
