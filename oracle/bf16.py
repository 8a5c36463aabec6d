"""Exact bf16 <-> fp32 conversions (test infrastructure).

bf16 is the upper half of an IEEE binary32; fp32 -> bf16 rounds to nearest, ties to even
(the rule the reference's bf16 test uses, tests/test_bf16_gemv.cu:8), and NaN maps to the
quiet NaN 0x7FC0. bf16 -> fp32 is exact (the reference's ix_bf16_to_f32, src/ix_compat.h:158-163).
"""
from __future__ import annotations

import numpy as np


def from_f32(x) -> np.ndarray:
    """float32 (or anything castable) -> uint16 bf16 bit patterns, round to nearest even."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(f), np.uint16(0x7FC0), r).astype(np.uint16)


def to_f32(u) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    u = np.ascontiguousarray(u, dtype=np.uint16)
    return (u.astype(np.uint32) << 16).view(np.float32)


def round_f32(x) -> np.ndarray:
    """Round float values to the nearest bf16 and return them as float32."""
    return to_f32(from_f32(x))
