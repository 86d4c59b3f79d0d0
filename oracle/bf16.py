"""bf16 helpers for the oracle (test infrastructure).

bf16 is the upper half of an IEEE binary32; rounding is to nearest, ties to
even, which is what torch's ``.bfloat16()`` (used by the reference at
src/spark_vllm_ascend/integration/weights.py:31) and the reference device
kernels' ``RoundingMode.RN`` casts do.  Pinned by known-answer tests in
tests/test_oracle_q4_0.py (ties, carries into the exponent, overflow to inf,
NaN).
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(a) -> np.ndarray:
    """float32 array -> uint16 bf16 bit patterns (RNE; NaN stays NaN)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """Round float32 values to the nearest bf16, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))
