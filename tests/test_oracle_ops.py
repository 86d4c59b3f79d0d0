"""Pins for the oracle's norm, RoPE and SwiGLU restatements (CPU only)."""
import numpy as np
import pytest
from scipy.special import expit

from oracle import ops as oops
from oracle.bf16 import round_bf16


def test_rmsnorm_constant_row_gives_gamma_times_sign():
    x = np.full(2560, -3.0, np.float32)
    g = round_bf16(np.linspace(0.5, 1.5, 2560).astype(np.float32))
    y, r = oops.add_rmsnorm(x, None, g, 0.0)
    np.testing.assert_array_equal(y, round_bf16(-g))
    np.testing.assert_array_equal(r, x)


def test_rmsnorm_scale_invariance_and_residual_sum():
    rng = np.random.default_rng(0)
    s = round_bf16(rng.standard_normal(2560).astype(np.float32))
    g = round_bf16(np.ones(2560, np.float32))
    y1, _ = oops.add_rmsnorm(s, None, g, 0.0)
    y2, _ = oops.add_rmsnorm(s * 4, None, g, 0.0)  # power-of-two scale is exact
    np.testing.assert_array_equal(y1, y2)
    x = round_bf16(rng.standard_normal(2560).astype(np.float32))
    r = round_bf16(rng.standard_normal(2560).astype(np.float32))
    _, ro = oops.add_rmsnorm(x, r, g, 1e-6)
    np.testing.assert_array_equal(ro, round_bf16(x + r))
    # unit RMS after normalisation (before the bf16 rounding)
    y, _ = oops.add_rmsnorm(x, r, g, 0.0)
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 5e-3


def test_rope_table_identities():
    cs = oops.rope_cache(8192, 128, 1e6)
    c, s = cs[:, :64].astype(np.float64), cs[:, 64:].astype(np.float64)
    np.testing.assert_allclose(c * c + s * s, 1.0, atol=1e-6)
    np.testing.assert_array_equal(cs[0, :64], 1.0)
    np.testing.assert_array_equal(cs[0, 64:], 0.0)
    inv = 1e6 ** (-np.arange(0, 128, 2) / 128.0)
    np.testing.assert_allclose(cs[1, :64], np.cos(inv), atol=1e-6)
    # angle addition: row(p + q) = row(p) rotated by row(q)
    p, q = 1000, 345
    cp, sp = c[p], s[p]
    cq, sq = c[q], s[q]
    np.testing.assert_allclose(c[p + q], cp * cq - sp * sq, atol=2e-3)
    np.testing.assert_allclose(s[p + q], sp * cq + cp * sq, atol=2e-3)


def test_rope_position_zero_is_identity_and_matches_complex_multiply():
    rng = np.random.default_rng(1)
    x = round_bf16(rng.standard_normal((4, 128)).astype(np.float32))
    cs = oops.rope_cache(4096, 128, 1e6)
    np.testing.assert_array_equal(oops.apply_rope(x, cs[0]), x)
    pos = 3071
    out = oops.apply_rope(x, cs[pos])
    z = (x[:, :64].astype(np.float64) + 1j * x[:, 64:]) * (cs[pos, :64] + 1j * cs[pos, 64:])
    ref = np.concatenate((z.real, z.imag), axis=-1)
    np.testing.assert_allclose(out, ref, rtol=1e-2, atol=1e-2)
    # pair norms are preserved
    n_in = np.hypot(x[:, :64], x[:, 64:])
    n_out = np.hypot(out[:, :64], out[:, 64:])
    np.testing.assert_allclose(n_out, n_in, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("g", [0.0, -3.0, 2.5, 30.0, -30.0])
def test_silu_mul_closed_forms(g):
    u = np.float32(1.5)
    out = oops.silu_mul(np.float32([g]), np.float32([u]))[0]
    ref = g * expit(g) * u
    assert abs(out - ref) <= 1e-2 * abs(ref) + 1e-6
    if g == 0.0:
        assert out == 0.0
    if g == 30.0:
        assert out == round_bf16(np.float32([g * u]))[0]
