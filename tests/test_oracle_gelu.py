"""Pins for the oracle's restatement of the reference's erf-GELU gate/up
activation (activate_native, src/spark_vllm_ascend/kernels/linear.py:540-577;
table of src/spark_vllm_ascend/integration/model.py:13-16), CPU only:
  * the float64 -> bf16 rounding is the nearest bf16 (brute force);
  * the table holds known values of gelu, and torch's gelu(approximate=
    'none') table -- the one the library's gelu_table() builds, as the
    reference does -- agrees with it within 1 ulp (x >= -3) and 2e-5 in the
    float32-cancelling tail;
  * the activation equals the correctly rounded gelu over all 65536 gate bit
    patterns (within 1 ulp where |g| < 2^-9 takes g / 2), NaN for NaN and
    -inf, g itself for g >= 128 and -0 for g <= -128;
  * the product with up is RNE(act * u) with the exact float64 product.
A planted mistake (the sign bit dropped from the index, the table halves
swapped, an off-by-one range edge) fails the whole-domain check."""
import numpy as np
import pytest

from _util import pkg
from oracle import ops as oops
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

ALL = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _nan(bits):
    return ((bits & 0x7F80) == 0x7F80) & ((bits & 0x7F) != 0)


def _ulps(a, b):
    """Distance in bf16 steps between same-signed finite bit patterns."""
    def key(x):
        x = x.astype(np.int64)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return np.abs(key(a) - key(b))


def test_f64_to_bf16_is_the_nearest_bf16():
    rng = np.random.default_rng(0)
    v = rng.standard_normal(100000) * np.exp(rng.uniform(-40, 40, 100000))
    # values exactly halfway between two bf16 neighbours go to the even one
    mid = bf16_bits_to_f32(np.uint16([0x3F80, 0x3F81])).astype(np.float64).mean()
    v = np.concatenate((v, [mid, -mid, 0.0, -0.0, 1.0]))
    b = oops.f64_to_bf16_bits(v).astype(np.int64)
    val = lambda x: bf16_bits_to_f32((x & 0xFFFF).astype(np.uint16)).astype(np.float64)
    err = lambda x: np.nan_to_num(np.abs(val(x) - v), nan=np.inf)  # NaN neighbours: never nearer
    assert (err(b) <= err(b - 1)).all() and (err(b) <= err(b + 1)).all()
    assert b[-5] == 0x3F80 and b[-4] == 0xBF80  # tie to even
    assert b[-3] == 0 and b[-2] == 0x8000 and b[-1] == 0x3F80


def test_table_known_values_and_layout():
    t = oops.gelu_table()
    assert t.shape == (4096,)
    val = lambda x: float(bf16_bits_to_f32(np.uint16([x]))[0])
    # lut[0] = gelu(2^-9), lut[(0x3f80 - 0x3b00)] = gelu(1), lut[2048 + ...] = gelu(-1)
    assert val(t[0x3F80 - 0x3B00]) == pytest.approx(0.8413447460685429, rel=4e-3)
    assert val(t[2048 + 0x3F80 - 0x3B00]) == pytest.approx(-0.15865525393145707, rel=4e-3)
    assert val(t[0x4000 - 0x3B00]) == pytest.approx(1.9544997361036416, rel=4e-3)
    assert val(t[0]) == pytest.approx(2 ** -10 * (1 + 2 ** -9 * 0.7978845608), rel=4e-3)
    assert val(t[2047]) == float(bf16_bits_to_f32(np.uint16([0x42FF]))[0])  # gelu(x) = x near 128
    assert all(val(x) <= 0 for x in t[2048:])
    assert all(val(x) > 0 for x in t[:2048])


def test_torch_table_agrees_with_the_correctly_rounded_one():
    import torch
    lib = pkg("native.torch_ops").gelu_table()
    assert lib.dtype == torch.bfloat16 and lib.shape == (4096,)
    got = lib.view(torch.int16).numpy().view(np.uint16)
    want = oops.gelu_table()
    x = bf16_bits_to_f32(np.concatenate((np.arange(0x3B00, 0x4300),
                                         np.arange(0xBB00, 0xC300))).astype(np.uint16))
    near = x >= -3.0
    assert _ulps(got[near], want[near]).max() <= 1
    assert (got[near] == want[near]).mean() > 0.99
    tail = np.abs(bf16_bits_to_f32(got[~near]).astype(np.float64) -
                  bf16_bits_to_f32(want[~near]).astype(np.float64))
    assert tail.max() < 2e-5


def _check_activation(act_bits):
    """act over ALL gate patterns against the correctly rounded gelu."""
    g = bf16_bits_to_f32(ALL)
    exact = oops.f64_to_bf16_bits(oops.gelu_f64(g))
    ab = ALL & 0x7FFF
    nan_out = _nan(ALL) | (ALL == 0xFF80)
    assert (act_bits[nan_out] == 0x7FFF).all()
    fin = ~nan_out
    small = fin & (ab < 0x3B00)
    other = fin & ~small
    np.testing.assert_array_equal(act_bits[other], exact[other])
    assert _ulps(act_bits[small], exact[small]).max() <= 1
    big = fin & (ab >= 0x4300)
    np.testing.assert_array_equal(act_bits[big], np.where(ALL[big] < 0x8000, ALL[big], 0x8000))


def test_activation_over_every_gate_bit_pattern():
    _check_activation(oops.gelu_act_bits(ALL, oops.gelu_table()))


@pytest.mark.parametrize("mistake", ["no_sign", "halves_swapped", "edge_off_by_one"])
def test_the_whole_domain_check_catches_planted_mistakes(mistake):
    lut = oops.gelu_table()
    if mistake == "no_sign":
        act = oops.gelu_act_bits(ALL & 0x7FFF, lut)  # sign bit lost before the lookup
        act = np.where(ALL & 0x8000, act | 0x8000, act)
    elif mistake == "halves_swapped":
        act = oops.gelu_act_bits(ALL, np.concatenate((lut[2048:], lut[:2048])))
    else:
        act = oops.gelu_act_bits(ALL, lut)
        act = np.where((ALL & 0x7FFF) == 0x4300, lut[0], act)  # g = 128 read from the table
    with pytest.raises(AssertionError):
        _check_activation(act)


def test_product_with_up_is_rounded_once():
    rng = np.random.default_rng(3)
    lut = oops.gelu_table()
    g = f32_to_bf16_bits((rng.standard_normal(50000) * 3).astype(np.float32))
    u = bf16_bits_to_f32(f32_to_bf16_bits((rng.standard_normal(50000) * 2).astype(np.float32)))
    got = oops.gelu_mul(g, u, lut)
    act = bf16_bits_to_f32(oops.gelu_act_bits(g, lut)).astype(np.float64)
    want = bf16_bits_to_f32(oops.f64_to_bf16_bits(act * u.astype(np.float64)))
    np.testing.assert_array_equal(got, want)
    assert (oops.gelu_mul(np.uint16([0x3F80]), np.float32([0.0]), lut) == 0).all()
