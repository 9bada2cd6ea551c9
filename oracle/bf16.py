"""bfloat16 on the host, for the oracle (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

limn stores bfloat16 through ml_dtypes (reference limn/device.py:29), whose cast rounds to
nearest even; the reference's GPU prelude does the same with the published bit method
(limn/cuda_emit.py:98-106: add 0x7fff plus the lowest kept bit, truncate; NaN stays NaN).

Pinned by tests/test_oracle.py against tests/golden/bf16_rne.npz, which torch.bfloat16 wrote
(ties both ways, subnormals, overflow to inf, NaN, signed zero).
"""

from __future__ import annotations

import numpy as np


def round_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits (uint16), round to nearest, ties to even."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    keep_lsb = (u >> np.uint64(16)) & np.uint64(1)
    out = ((u + np.uint64(0x7FFF) + keep_lsb) >> np.uint64(16)).astype(np.uint16)
    return np.where(np.isnan(f), np.uint16(0x7FC0), out).astype(np.uint16)


def widen(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bits -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def rne(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16, returned as float32."""
    return widen(round_bits(x))
