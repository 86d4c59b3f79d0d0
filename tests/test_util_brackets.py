"""The bracket checks the GPU parity tests use, pinned on the CPU: they accept
the bf16 rounding of an exact value and its one-ulp neighbour across the
rounding point, and reject values two ulps off and a SwiGLU that skipped a
rounding or scaled its input."""
import numpy as np
import pytest

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from oracle.ops import silu_mul

from _util import assert_faithful_bf16, assert_swiglu_bracketed, bf16_bracket


def _step(x, n):
    """x moved n bf16 ulps (x > 0)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.float32(x)) + np.uint16(n))


def test_bracket_bounds_and_width():
    rng = np.random.default_rng(0)
    v = rng.standard_normal(1000) * 10
    lo, hi = bf16_bracket(v, np.zeros_like(v))
    assert (lo <= v).all() and (hi >= v).all()
    # lo and hi are bf16 values at most one ulp apart (exact values: two)
    d = f32_to_bf16_bits(hi).astype(np.int32) - f32_to_bf16_bits(lo).astype(np.int32)
    assert set(np.abs(d).tolist()) <= {1, 2}


def test_faithful_accepts_rounding_and_neighbour_rejects_two_ulps():
    v = np.array([1.0 + 3 * 2.0 ** -10, 5.3, 1234.56])
    r = round_bf16(v.astype(np.float32))
    slack = np.zeros_like(v)
    assert_faithful_bf16(r, v, slack)
    lo, hi = bf16_bracket(v, slack)
    assert_faithful_bf16(lo, v, slack)
    assert_faithful_bf16(hi, v, slack)
    with pytest.raises(AssertionError):
        assert_faithful_bf16(_step(hi, 1), v, slack)


def test_swiglu_bracket_accepts_oracle_rejects_mistakes():
    rng = np.random.default_rng(1)
    g = rng.standard_normal(4096) * 3
    u = rng.standard_normal(4096) * 3
    slack = np.full_like(g, 1e-6)
    ok = silu_mul(round_bf16(g.astype(np.float32)), round_bf16(u.astype(np.float32)))
    assert_swiglu_bracketed(ok, g, u, slack, slack, silu_mul)
    # a gate scaled by 2% (a dropped normalisation term) fails
    bad = silu_mul(round_bf16((g * 1.02).astype(np.float32)), round_bf16(u.astype(np.float32)))
    with pytest.raises(AssertionError):
        assert_swiglu_bracketed(bad, g, u, slack, slack, silu_mul)
    # gate and up swapped fails
    with pytest.raises(AssertionError):
        assert_swiglu_bracketed(silu_mul(round_bf16(u.astype(np.float32)),
                                         round_bf16(g.astype(np.float32))),
                                g, u, slack, slack, silu_mul)
