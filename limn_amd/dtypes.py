"""Host-side storage of limn dtypes as numpy arrays.

numpy has no bfloat16 (limn uses ml_dtypes for it, reference `limn/device.py:25-33`, and
ml_dtypes is not part of this stack), so a bfloat16 value lives on the host as its 16-bit
pattern in a uint16 array. `to_storage` rounds floats into a dtype's storage (round to
nearest even, NaN kept NaN); `from_storage` reads a device's bytes back as numbers, widening
bfloat16 to the float32 values it holds exactly.
"""

from __future__ import annotations

import numpy as np

from limn_amd.seam import DType, bfloat16, float16, float32, float64, int8, int16, int32

STORAGE: dict[DType, np.dtype] = {
    float64: np.dtype(np.float64),
    float32: np.dtype(np.float32),
    float16: np.dtype(np.float16),
    bfloat16: np.dtype(np.uint16),
    int32: np.dtype(np.int32),
    int16: np.dtype(np.int16),
    int8: np.dtype(np.int8),
}

# The dtype codes of include/limn_hip.h.
ABI_CODE: dict[DType, int] = {float64: 0, float32: 1, float16: 2, bfloat16: 3}


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 values -> bfloat16 bit patterns, round to nearest even; NaN -> quiet NaN."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded = np.where(nan, ((bits >> 16).astype(np.uint16) | np.uint16(0x0040)), rounded).astype(np.uint16)
    return rounded


def bf16_values(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns -> the float32 values they hold (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_storage(data, dtype: DType) -> np.ndarray:
    """Any array-like as `dtype`'s host storage (C-contiguous)."""
    array = np.asarray(data)
    if dtype == bfloat16:
        if array.dtype == np.uint16:  # already bit patterns
            return np.ascontiguousarray(array)
        return bf16_bits(array.astype(np.float32))
    return np.ascontiguousarray(array.astype(STORAGE[dtype]))


def from_storage(raw: np.ndarray, dtype: DType, shape: tuple[int, ...]) -> np.ndarray:
    """A device's flat bytes as numbers of `dtype` (bfloat16 widened to float32)."""
    arr = np.asarray(raw).view(STORAGE[dtype]).reshape(shape)
    return bf16_values(arr) if dtype == bfloat16 else arr
