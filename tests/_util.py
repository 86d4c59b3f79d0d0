"""Shared helpers for the tests: numpy bf16 bits <-> torch tensors."""
from __future__ import annotations

import importlib

import numpy as np

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

PKG = "spark_vllm_ascend_amd"


def pkg(mod: str):
    return importlib.import_module(f"{PKG}.{mod}")


def bf16_dev(bits: np.ndarray, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(
        torch.bfloat16).to(dev)


def bits_of(t) -> np.ndarray:
    """torch bf16 tensor -> numpy uint16 bits (host)."""
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f32_of(t) -> np.ndarray:
    return bf16_bits_to_f32(bits_of(t))


def randn_bf16(rng, shape, scale=1.0) -> np.ndarray:
    return f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))


def assert_close_rel(got, ref, rtol=1e-2, atol_frac=1e-3, what=""):
    """|got - ref| <= rtol * |ref| + atol_frac * rms(ref), elementwise."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    bound = rtol * np.abs(ref) + atol_frac * rms
    bad = np.abs(got - ref) > bound
    if bad.any():
        i = int(np.argmax(np.abs(got - ref) - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} out of tolerance; worst at {i}: "
            f"got {got.flat[i]!r} ref {ref.flat[i]!r} bound {bound.flat[i]!r}")


def bf16_ulp_diff(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two bit arrays (sign-magnitude mapped to
    a monotone integer line; +0 and -0 are 0 apart)."""
    a = np.asarray(a_bits, dtype=np.uint16).astype(np.int32)
    b = np.asarray(b_bits, dtype=np.uint16).astype(np.int32)
    ka = np.where(a & 0x8000, -(a & 0x7FFF), a)
    kb = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(ka - kb)
