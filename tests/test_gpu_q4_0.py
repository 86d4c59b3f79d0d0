"""GPU parity of the Q4_0 kernels (dequant, GEMV, GEMV+SwiGLU) against the
oracle, through the C ABI.  Bars: dequantisation bit-exact; GEMV within 1e-2
relative of the float64 oracle (plus 1e-3 of the row RMS for cancellation),
at least 95% of outputs equal to the bf16 rounding of the fp64 result, and
every output one of the two bf16 values bracketing the exact result (an fp32
accumulation's slack added); SwiGLU within 1 bf16 ulp of silu(g) * u over
the bf16 values bracketing the exact gate and up outputs."""
import numpy as np
import pytest

from oracle import q4_0 as oq
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.ops import silu_mul as o_silu_mul

from _util import (FP32_ACC_SLACK, assert_close_rel, assert_faithful_bf16, assert_swiglu_bracketed,
                   bf16_dev, bits_of, f32_of, gemv_abs_sum, pkg, randn_bf16)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    return pkg("native.torch_ops")


def _blocks_dev(blocks, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(blocks)).to(dev)


def _kat_blocks():
    """Blocks with special scales and a nibble-order probe."""
    import numpy as np
    n, k = 8, 64
    d = np.array([[1.0, -0.0], [2.0 ** -24, 65504.0], [np.inf, -np.inf], [np.nan, 0.5],
                  [1.0, 1.0], [-2.0, 0.25], [0.0, 1e-3], [3.0, -7.5]], dtype=np.float16)
    codes = np.tile(np.arange(32, dtype=np.uint8) % 16, (n, 2, 1))
    codes[4, 0, 0] = 0xF  # byte 0 = 0x1F -> element 0 = 15 - 8, element 16 = 1 - 8
    codes[4, 0, 16] = 0x1
    return oq.pack_blocks(d, codes), n, k


@pytest.mark.parametrize("n,k", [(64, 256), (37, 96), (9728, 2560), (2560, 9728)])
def test_dequant_bit_exact(ops, dev, n, k):
    blocks = oq.make_blocks(n, k, seed=100 + n)
    out = ops.q4_0_dequant_bf16(_blocks_dev(blocks, dev), n, k)
    got = bits_of(out).reshape(n, k)
    ref = oq.c_dequant_bf16_bits(blocks, n, k)
    np.testing.assert_array_equal(got, ref)


def test_dequant_special_scales(ops, dev):
    blocks, n, k = _kat_blocks()
    got = bits_of(ops.q4_0_dequant_bf16(_blocks_dev(blocks, dev), n, k)).reshape(n, k)
    ref = oq.c_dequant_bf16_bits(blocks, n, k)
    gnan = np.isnan(bf16_bits_to_f32(got))
    rnan = np.isnan(bf16_bits_to_f32(ref))
    np.testing.assert_array_equal(gnan, rnan)
    np.testing.assert_array_equal(got[~gnan], ref[~rnan])


def _gemv_case(ops, dev, n, k, seed, x_scale=1.0):
    rng = np.random.default_rng(seed)
    blocks = oq.make_blocks(n, k, seed=seed)
    x_bits = randn_bf16(rng, k, x_scale)
    y = ops.q4_0_gemv(bf16_dev(x_bits, dev), _blocks_dev(blocks, dev), n, k)
    return f32_of(y).reshape(n), bits_of(y).reshape(n), x_bits, blocks


@pytest.mark.parametrize("n,k", [
    (64, 256), (8, 64), (37, 96), (1000, 2560), (777, 4096),
    (9728, 2560), (6144, 2560), (2560, 4096), (2560, 9728), (19456, 2560)])
def test_gemv_vs_oracle(ops, dev, n, k):
    got, got_bits, x_bits, blocks = _gemv_case(ops, dev, n, k, seed=n * 7 + k)
    ref = oq.gemv_f64(x_bits, blocks, n, k)
    assert_close_rel(got, ref, what=f"gemv {n}x{k}")
    same = np.mean(got_bits == f32_to_bf16_bits(ref.astype(np.float32)))
    assert same >= 0.95, f"only {same:.3f} of outputs equal bf16(fp64 oracle)"
    assert_faithful_bf16(got, ref, FP32_ACC_SLACK * gemv_abs_sum(x_bits, blocks, n, k),
                         what=f"gemv {n}x{k}")


def test_gemv_lm_head_shape(ops, dev):
    n, k = 151936, 2560
    got, _, x_bits, blocks = _gemv_case(ops, dev, n, k, seed=5)
    ref = oq.gemv_f64(x_bits, blocks, n, k)
    assert_close_rel(got, ref, what="head gemv")


@pytest.mark.parametrize("n,k", [(64, 256), (9728, 2560), (2560, 9728)])
def test_gemv_one_hot_selects_dequantised_column(ops, dev, n, k):
    """x = e_j makes y the bf16 of column j of the dequantised matrix exactly."""
    blocks = oq.make_blocks(n, k, seed=3)
    wref = oq.c_dequant_bf16_bits(blocks, n, k)
    wdev = _blocks_dev(blocks, dev)
    for j in [0, 1, 15, 16, 17, 31, 32, 63, k - 33, k - 1]:
        x = np.zeros(k, dtype=np.uint16)
        x[j] = 0x3F80  # 1.0
        got = bits_of(ops.q4_0_gemv(bf16_dev(x, dev), wdev, n, k)).reshape(n)
        np.testing.assert_array_equal(got, wref[:, j], err_msg=f"column {j}")


def test_gemv_matches_reference_rounding_points(ops, dev):
    """Against the reference kernel's own rounding (bf16 weights, fp32 FMA):
    the fused-dequant GEMV differs only by the weight rounding it skips."""
    n, k = 2048, 2560
    got, _, x_bits, blocks = _gemv_case(ops, dev, n, k, seed=77)
    ref_bits = oq.gemv_bf16w_bits(x_bits, blocks, n, k)
    assert_close_rel(got, bf16_bits_to_f32(ref_bits), rtol=2e-2, atol_frac=5e-3,
                     what="vs bf16-weight reference")


@pytest.mark.parametrize("x_scale", [1e-3, 10.0, 1000.0])
def test_gemv_activation_scales(ops, dev, x_scale):
    n, k = 1024, 2560
    got, _, x_bits, blocks = _gemv_case(ops, dev, n, k, seed=int(x_scale * 10) + 1, x_scale=x_scale)
    ref = oq.gemv_f64(x_bits, blocks, n, k)
    assert_close_rel(got, ref, what=f"x scale {x_scale}")


def test_gemv_output_sentinels(ops, dev):
    """Writes stay inside y: guard values around the output are untouched."""
    import torch
    n, k = 9728, 2560
    rng = np.random.default_rng(9)
    blocks = oq.make_blocks(n, k, seed=9)
    x = bf16_dev(randn_bf16(rng, k), dev)
    guard = torch.full((n + 32,), 17.0, dtype=torch.bfloat16, device=dev)
    y = guard[16:16 + n]
    ops.q4_0_gemv(x, _blocks_dev(blocks, dev), n, k, out=y)
    g = guard.float().cpu().numpy()
    assert np.all(g[:16] == 17.0) and np.all(g[16 + n:] == 17.0)


@pytest.mark.parametrize("d,k", [(32, 256), (9728, 2560), (100, 2560)])
def test_gemv_swiglu(ops, dev, d, k):
    rng = np.random.default_rng(d + k)
    blocks = oq.make_blocks(2 * d, k, seed=d)
    x_bits = randn_bf16(rng, k)
    out = ops.q4_0_gemv_swiglu(bf16_dev(x_bits, dev), _blocks_dev(blocks, dev), d, k)
    gu = oq.gemv_f64(x_bits, blocks, 2 * d, k)
    slack = FP32_ACC_SLACK * gemv_abs_sum(x_bits, blocks, 2 * d, k)
    assert_swiglu_bracketed(f32_of(out).reshape(d), gu[:d], gu[d:], slack[:d], slack[d:],
                            o_silu_mul, what=f"swiglu {d}x{k}")


def test_gemv_rejects_bad_arguments(ops, dev):
    import torch
    x = torch.zeros(256, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(64 * 8 * 18, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        ops.q4_0_gemv(x, w, 64, 255)
    with pytest.raises(ValueError):
        ops.q4_0_gemv(x.float(), w, 64, 256)
    with pytest.raises(ValueError):
        ops.q4_0_gemv(x, w[:-1], 64, 256)
