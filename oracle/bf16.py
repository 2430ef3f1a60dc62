"""bf16 in numpy (test infrastructure): values are carried as float32 arrays holding bf16-exact values.

Rounding is round-to-nearest-even on the float32 bit pattern, NaN -> 0x7FC0: the rule of c10::BFloat16
(``round_to_nearest_even``), which ``Tensor.to(torch.bfloat16)`` / ``type_as`` apply.
"""

from __future__ import annotations

import numpy as np


def to_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), rounded)


def from_bits(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16 value (returned as float32)."""
    return from_bits(to_bits(x))


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` ("bf16" or "f32") and return them as float32."""
    x = np.asarray(x, dtype=np.float32)
    return round_bf16(x) if dtype == "bf16" else x
