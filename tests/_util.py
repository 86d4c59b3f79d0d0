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


# unit roundoff of bf16 (8 significant bits): |bf16(x) - x| <= BF16_U |x|
BF16_U = 2.0 ** -8


def assert_attention_close(got, ref, what="", rms_frac=1e-2, l2=1e-2, bf16_out=True):
    """Attention output at the 1e-2 relative bar against float64 attention:
    every element within rms_frac of the reference's RMS -- plus, for a bf16
    output, the output's own rounding (BF16_U |ref|; the reference rounds its
    output to bf16 too, and that alone reaches 1.4e-2 of the RMS at the
    largest elements) -- and the relative L2 error below l2.  Returns
    (max |err| / rms, relative L2)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2)))
    err = np.abs(got - ref)
    bound = rms_frac * rms + (BF16_U * np.abs(ref) if bf16_out else 0.0)
    bad = err > bound
    if bad.any():
        i = int(np.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} beyond {rms_frac} of the rms {rms:.4g}"
            f"{' + the bf16 rounding' if bf16_out else ''}; worst at {i}: got "
            f"{got.flat[i]!r} ref {ref.flat[i]!r} (err {err.flat[i] / rms:.4g} rms)")
    rel = float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300))
    assert rel <= l2, f"{what}: relative L2 {rel:.4g} > {l2}"
    return float(err.max() / rms), rel


def assert_partials_close(po, pl, opo, opl, what=""):
    """Split-KV partials against the oracle's restatement of the reference's
    online softmax (bf16 P): the same empty splits (lse -inf, output 0);
    every lse within 1e-4; per split, every output element within 2e-2 of
    that split's RMS and the relative L2 error below 1e-2.  (Both round P to
    bf16, at running maxima that can differ, so the element bar is twice the
    merged output's: measured up to 0.99e-2 of the RMS, L2 below 2e-3.)"""
    po, pl = np.asarray(po, np.float64), np.asarray(pl, np.float64)
    opo, opl = np.asarray(opo, np.float64), np.asarray(opl, np.float64)
    fin = np.isfinite(opl)
    np.testing.assert_array_equal(np.isfinite(pl), fin, err_msg=f"{what}: empty splits")
    if fin.any():
        lerr = float(np.max(np.abs(pl[fin] - opl[fin])))
        assert lerr < 1e-4, f"{what}: lse err {lerr:.3g}"
    assert np.all(po[~fin] == 0), f"{what}: empty split output not zero"
    for s in range(po.shape[0]):
        rows = fin[s]
        if not rows.any():
            continue
        a, b = po[s][rows], opo[s][rows]
        rms = float(np.sqrt(np.mean(b ** 2)))
        e = float(np.abs(a - b).max())
        assert e <= 2e-2 * rms, f"{what}: split {s} err {e / rms:.4g} of the rms"
        rel = float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
        assert rel <= 1e-2, f"{what}: split {s} relative L2 {rel:.4g}"


def bf16_ulp_diff(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two bit arrays (sign-magnitude mapped to
    a monotone integer line; +0 and -0 are 0 apart)."""
    a = np.asarray(a_bits, dtype=np.uint16).astype(np.int32)
    b = np.asarray(b_bits, dtype=np.uint16).astype(np.int32)
    ka = np.where(a & 0x8000, -(a & 0x7FFF), a)
    kb = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(ka - kb)


def bf16_bracket(v: np.ndarray, slack: np.ndarray):
    """The bf16 values bounding [v - slack, v + slack] from outside: (lo, hi)
    with lo <= v - slack and hi >= v + slack, each a bf16 value (float32).
    A bf16 output of an fp32-accumulated sum whose exact value is v and whose
    accumulation error is at most slack is lo, hi, or a bf16 value between."""
    v = np.asarray(v, dtype=np.float64)
    slack = np.asarray(slack, dtype=np.float64)

    def step(x, up):
        # the next bf16 value above (up) or below x, x a bf16 value (float32)
        bits = f32_to_bf16_bits(np.asarray(x, np.float32)).astype(np.int32)
        key = np.where(bits & 0x8000, -(bits & 0x7FFF), bits)  # monotone line
        key = key + (1 if up else -1)
        nb = np.where(key < 0, (-key) | 0x8000, key).astype(np.uint16)
        return bf16_bits_to_f32(nb)

    lo_t = (v - slack).astype(np.float32)
    hi_t = (v + slack).astype(np.float32)
    lo = bf16_bits_to_f32(f32_to_bf16_bits(lo_t))
    lo = np.where(lo > v - slack, step(lo, False), lo)
    hi = bf16_bits_to_f32(f32_to_bf16_bits(hi_t))
    hi = np.where(hi < v + slack, step(hi, True), hi)
    return lo.astype(np.float32), hi.astype(np.float32)


def assert_swiglu_bracketed(out_f32, g_exact, u_exact, g_slack, u_slack, silu_mul, what=""):
    """SwiGLU output of a GEMV epilogue, judged without a tolerance knob:
    the gate and up GEMV outputs are bf16 roundings of fp32 sums, so each is a
    bf16 value bracketing its exact (float64) value widened by the fp32
    accumulation bound; the output must lie within 1 bf16 ulp of
    silu_mul(g', u') over those bracketing values (silu_mul rounds to bf16)."""
    g_lo, g_hi = bf16_bracket(g_exact, g_slack)
    u_lo, u_hi = bf16_bracket(u_exact, u_slack)
    cands = np.stack([silu_mul(g, u) for g in (g_lo, g_hi) for u in (u_lo, u_hi)])
    c_bits = f32_to_bf16_bits(cands.astype(np.float32))
    o_bits = f32_to_bf16_bits(np.asarray(out_f32, np.float32))
    key = lambda b: np.where(b.astype(np.int32) & 0x8000, -(b.astype(np.int32) & 0x7FFF),
                             b.astype(np.int32))
    ok = (key(o_bits) >= key(c_bits).min(axis=0) - 1) & (key(o_bits) <= key(c_bits).max(axis=0) + 1)
    if not ok.all():
        i = int(np.argmin(ok))
        raise AssertionError(
            f"{what}: {int((~ok).sum())}/{ok.size} outside the bracket; at {i}: out "
            f"{float(np.asarray(out_f32).flat[i])!r}, candidates {cands[:, i].tolist()}, "
            f"g {float(g_exact.flat[i])!r} u {float(u_exact.flat[i])!r}")


def gemv_abs_sum(x_bits: np.ndarray, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """sum_j |x_j| |w_ij| per output row (float64): the scale of an fp32
    accumulation's rounding error for that row."""
    from oracle import q4_0 as oq
    w = np.abs(oq.dequant_f32(blocks, n, k))
    return w.astype(np.float64) @ np.abs(bf16_bits_to_f32(x_bits).astype(np.float64))


# Slack granted to an fp32-accumulated dot product, relative to its row's
# absolute sum (the per-block dot2 chains run at about 34x the magnitude of
# their result, so 2^-18 is a few hundred fp32 ulps of the result's scale).
FP32_ACC_SLACK = 2.0 ** -18


def assert_faithful_bf16(got_f32, exact, slack, what=""):
    """Every output is one of the bf16 values bracketing its exact value
    (widened by slack): the bf16 rounding of an accumulation whose error is
    below slack, at most one ulp from the exact value's own rounding."""
    lo, hi = bf16_bracket(exact, slack)
    got = np.asarray(got_f32, np.float32)
    ok = (got >= lo) & (got <= hi)
    if not ok.all():
        i = int(np.argmin(ok))
        raise AssertionError(f"{what}: {int((~ok).sum())}/{ok.size} outside the bf16 bracket; "
                             f"at {i}: got {float(got.flat[i])!r} exact "
                             f"{float(np.asarray(exact).flat[i])!r} bracket "
                             f"[{float(lo.flat[i])!r}, {float(hi.flat[i])!r}]")
