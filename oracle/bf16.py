"""bf16 helpers (round-to-nearest-even), numpy.

Pinned by: exhaustive comparison against torch's CPU float32->bfloat16 cast over
all float32 bit patterns of a strided sample plus every bf16 tie case
(tests/test_oracle.py::test_bf16_round_matches_torch).
"""
from __future__ import annotations

import numpy as np


def round_bf16(x) -> np.ndarray:
    """float32 -> nearest-even bf16 value, returned as float32 (NaN stays NaN)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    r = np.where(nan, (u | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), r).astype(np.uint32)
    return r.view(np.float32)


def to_bits(x) -> np.ndarray:
    """float32 array holding bf16 values (or any float32) -> uint16 bf16 bit patterns (RNE)."""
    return (round_bf16(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def from_bits(b) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def ulp(x) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (x float), as float64.  ulp(0) is the smallest normal spacing."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def ulp_diff(a, b, floor: float = 0.0) -> np.ndarray:
    """|a - b| in units of the bf16 spacing at max(|b|, floor)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.abs(a - b) / ulp(np.maximum(np.abs(b), floor))
