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
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


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
