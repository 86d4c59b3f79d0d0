"""Small decode ops for the oracle (numpy fp32; bf16 at stage outputs) --
test infrastructure.

Pins (tests/test_oracle_ops.py):
  add_rmsnorm   closed form of norm_ub, src/spark_vllm_ascend/kernels/
                linear.py:202-224; checked on constant rows (y = gamma *
                sign), scale invariance y(c*s) = y(s), and residual_out = bf16
                of the fp32 sum.
  rms_norm      the same formula per head (Qwen3-style q/k norm; no
                counterpart in the reference: pinned by the same closed forms).
  rope_cache    vLLM's get_rope construction (inv_freq = theta^(-2i/d),
                angle = pos * inv_freq, cos | sin) -- the reference consumes
                this table at src/spark_vllm_ascend/kernels/qkv.py:183-184;
                pinned by cos^2 + sin^2 = 1, row 0 = (1, 0), and the angle
                addition formula.
  apply_rope    neox rotation of src/spark_vllm_ascend/integration/rope.py:
                61-73 and kernels/qkv.py:186-187; pinned by position 0 =
                identity, pair-norm preservation, and equality with complex
                multiplication (x1 + i x2) * e^{i angle}.
  silu_mul      silu(g) * u, textbook SwiGLU (the reference model uses GELU
                instead); pinned by silu(0) = 0, silu(g) -> g for large g,
                and scipy.special.expit.
  gelu_table    the reference's 4096-entry erf-GELU table
                (src/spark_vllm_ascend/integration/model.py:13-16), here the
                correctly rounded gelu of each bf16 input (float64 erf);
                pinned by known values of gelu and against torch's
                gelu(approximate='none') table (within 1 bf16 ulp).
  gelu_mul      activate_native (src/spark_vllm_ascend/kernels/linear.py:
                540-577): table GELU of the bf16 gate times up; pinned over
                all 65536 gate bit patterns against the correctly rounded
                gelu (equal, or within 1 ulp where |g| < 2^-9 takes g / 2),
                NaN for NaN and -inf, and RNE(act * u) in float64 for u.
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16


def add_rmsnorm(x: np.ndarray, residual: np.ndarray | None, gamma: np.ndarray, eps: float):
    """x, residual, gamma: float32 values of bf16 tensors (last dim = hidden).
    Returns (y, residual_out) as float32 values of bf16."""
    s = np.asarray(x, dtype=np.float32)
    if residual is not None:
        s = (s + np.asarray(residual, dtype=np.float32)).astype(np.float32)
    hidden = s.shape[-1]
    ss = np.sum(s.astype(np.float64) ** 2, axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(np.float32(ss / hidden) + np.float32(eps))).astype(np.float32)
    y = round_bf16((s * inv).astype(np.float32) * np.asarray(gamma, dtype=np.float32))
    return y, round_bf16(s)


def rms_norm(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    y, _ = add_rmsnorm(x, None, gamma, eps)
    return y


def rope_cache(max_position: int, rot_dim: int, theta: float) -> np.ndarray:
    """cos|sin table [max_position, rot_dim] in float32 (before the bf16 cast
    the model applies)."""
    inv_freq = (1.0 / (np.float32(theta) ** (np.arange(0, rot_dim, 2, dtype=np.float32)
                                            / np.float32(rot_dim)))).astype(np.float32)
    t = np.arange(max_position, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    return np.concatenate((np.cos(freqs), np.sin(freqs)), axis=-1).astype(np.float32)


def apply_rope(x: np.ndarray, cos_sin_row: np.ndarray) -> np.ndarray:
    """neox rotation of the last dim of x with one cos|sin row; float32 in,
    bf16-rounded float32 out."""
    half = x.shape[-1] // 2
    a = np.asarray(x[..., :half], dtype=np.float32)
    b = np.asarray(x[..., half:], dtype=np.float32)
    c = np.asarray(cos_sin_row[:half], dtype=np.float32)
    s = np.asarray(cos_sin_row[half:], dtype=np.float32)
    u = (a * c - b * s).astype(np.float32)
    v = (b * c + a * s).astype(np.float32)
    return round_bf16(np.concatenate((u, v), axis=-1))


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    with np.errstate(over="ignore"):
        silu = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return round_bf16((silu * u).astype(np.float32))


GELU_LUT_ENTRIES = 4096


def gelu_f64(x: np.ndarray) -> np.ndarray:
    """gelu(x) = x (1 + erf(x / sqrt(2))) / 2 in float64."""
    from scipy.special import erf
    with np.errstate(invalid="ignore"):  # NaN inputs (signalling ones warn on the cast)
        x = np.asarray(x, dtype=np.float64)
        return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def f64_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bits rounded once to nearest even: float32 by
    round-to-odd (inexact results truncated toward zero with the last bit
    set), then RNE to bf16 -- exact, since float32 keeps more than 8 + 2
    significand bits (Boldo and Melquiond, "When double rounding is odd",
    2005)."""
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        f = v.astype(np.float32)
        u = f.view(np.uint32).copy()
        inexact = np.isfinite(v) & (f.astype(np.float64) != v)
        over = inexact & (np.abs(f.astype(np.float64)) > np.abs(v))
    u = np.where(over, u - 1, u)             # one float32 ulp toward zero
    u = np.where(inexact, u | 1, u)
    return f32_to_bf16_bits(u.astype(np.uint32).view(np.float32))


def gelu_table() -> np.ndarray:
    """bf16 bits of RNE_bf16(gelu(b)) for b = 0x3b00..0x42ff, then
    0xbb00..0xc2ff (the reference's table layout, model.py:13-16)."""
    b = np.concatenate((np.arange(0x3B00, 0x4300), np.arange(0xBB00, 0xC300))).astype(np.uint16)
    return f64_to_bf16_bits(gelu_f64(bf16_bits_to_f32(b)))


def gelu_act_bits(g_bits: np.ndarray, lut: np.ndarray) -> np.ndarray:
    """The activation of activate_native (linear.py:553-572) on bf16 gate
    bits: table lookup for 2^-9 <= |g| < 128, g / 2 below, g or -0 above,
    the NaN 0x7fff for NaN and -inf."""
    g = np.asarray(g_bits, dtype=np.uint32)
    lut = np.asarray(lut, dtype=np.uint16)
    assert lut.shape == (GELU_LUT_ENTRIES,)
    ab = g & 0x7FFF
    index = ((ab - 0x3B00) & 2047) | ((g >> 4) & 2048)     # linear.py:555-558
    out = lut[index.astype(np.int64)].astype(np.uint32)
    with np.errstate(invalid="ignore"):  # NaN lanes, replaced below
        small = f32_to_bf16_bits(np.float32(0.5) * bf16_bits_to_f32(g.astype(np.uint16)))
    out = np.where(ab < 0x3B00, small, out)                   # linear.py:562
    out = np.where(ab >= 0x4300, np.where(g < 0x8000, g, 0x8000), out)  # :561,563,566
    out = np.where((ab > 0x7F80) | (g == 0xFF80), 0x7FFF, out)           # :567-568
    return out.astype(np.uint16)


def gelu_mul(g_bits: np.ndarray, u: np.ndarray, lut: np.ndarray) -> np.ndarray:
    """bf16(act(g) * u) as float32 (linear.py:569-570); g as bf16 bits, u
    bf16-valued float32."""
    act = bf16_bits_to_f32(gelu_act_bits(g_bits, lut))
    with np.errstate(over="ignore", invalid="ignore"):  # inf and NaN gates, overflowing products
        return round_bf16((act * np.asarray(u, dtype=np.float32)).astype(np.float32))
