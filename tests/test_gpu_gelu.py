"""GPU parity of the reference's erf-GELU gate/up activation (activate_native,
src/spark_vllm_ascend/kernels/linear.py:540-577, over the table built at
src/spark_vllm_ascend/integration/model.py:13-16) through the C ABI:
  * smx_gelu_mul over every one of the 65536 bf16 gate bit patterns equals
    the oracle bit for bit (NaN outputs compared as NaN), and a ragged
    shape writes nothing past its output;
  * the fused epilogues -- smx_q4_0_gemv_gelu (streaming and generic
    kernels), smx_q4_0_add_rmsnorm_gemv_gelu, smx_q4_0_gemm_gelu (tile
    and word-load kernels) and smx_q4_0_gemm_packed_gelu -- equal the oracle bit for bit on one-hot
    activations, whose gate/up sums are exact (one product of at most 23
    significant bits), at magnitudes that reach the g / 2, table and
    g-or--0 regions;
  * on random activations at the 9728 x 2560 gate/up shape each output is
    exactly the oracle's activation of some gate/up pair inside the fp32
    accumulation bracket of the exact (float64) sums.
The table is the library's gelu_table() (torch's gelu, as the reference
builds it), handed to the kernels and the oracle alike."""
import numpy as np
import pytest

from oracle import ops as oops
from oracle import q4_0 as oq
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

from _util import (FP32_ACC_SLACK, bf16_bracket, bf16_dev, bits_of, gemv_abs_sum, pkg,
                   randn_bf16)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    return pkg("native.torch_ops")


@pytest.fixture(scope="module")
def lut(ops, dev):
    return ops.gelu_table(dev)


@pytest.fixture(scope="module")
def lut_bits(lut):
    return bits_of(lut)


def _w(blocks, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)).to(dev)


def _canon(bits):
    """NaN patterns -> 0x7fff (NaN payloads are not part of the contract)."""
    b = np.asarray(bits, dtype=np.uint16)
    nan = ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    return np.where(nan, np.uint16(0x7FFF), b)


def _oracle(g_bits, u_bits, lut_bits):
    return f32_to_bf16_bits(oops.gelu_mul(g_bits, bf16_bits_to_f32(u_bits), lut_bits))


def test_gelu_mul_every_gate_bit_pattern(ops, dev, lut, lut_bits):
    rows, d = 64, 1024
    rng = np.random.default_rng(1)
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(rows, d)
    u = f32_to_bf16_bits((rng.standard_normal((rows, d)) * 2).astype(np.float32))
    u[::2] = f32_to_bf16_bits(np.float32([1.0]))[0]  # half the rows: the activation itself
    gu = np.concatenate((g, u), axis=1)
    out = bits_of(ops.gelu_mul(bf16_dev(gu, dev), lut))
    want = _oracle(g, u, lut_bits)
    np.testing.assert_array_equal(_canon(out), _canon(want))


def test_gelu_mul_ragged_stays_in_bounds(ops, dev, lut, lut_bits):
    import torch
    rows, d = 3, 37
    rng = np.random.default_rng(2)
    gu = randn_bf16(rng, (rows, 2 * d), 3.0)
    buf = torch.full((rows * d + 64,), 7.0, dtype=torch.bfloat16, device=dev)
    ops.gelu_mul(bf16_dev(gu, dev), lut, out=buf[:rows * d])
    got = bits_of(buf)
    np.testing.assert_array_equal(got[:rows * d].reshape(rows, d),
                                  _oracle(gu[:, :d], gu[:, d:], lut_bits))
    assert (got[rows * d:] == f32_to_bf16_bits(np.float32([7.0]))[0]).all()


def test_gelu_table_rejects_a_wrong_size(ops, dev):
    import torch
    x = torch.zeros(1, 256, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(2 * 64 * 8 * 18, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="4096"):
        ops.q4_0_gemv_gelu(x, w, torch.zeros(4095, dtype=torch.bfloat16, device=dev), 64, 256)


# ------------------------------------------------------------ one-hot, exact
MAGNITUDES = [2.0 ** -14, 2.0 ** -6, 0.125, 1.0, 4.0, 16.0, 64.0, 256.0]


def _one_hot(k, col, value):
    x = np.zeros(k, dtype=np.uint16)
    x[col] = f32_to_bf16_bits(np.float32([value]))[0]
    return x


def _exact_gated(x_bits, blocks, d, k, lut_bits):
    """Exact sums (one nonzero product) rounded once, then the oracle."""
    gu = oq.gemv_f64(x_bits, blocks, 2 * d, k)
    gb = oops.f64_to_bf16_bits(gu[:d])
    ub = oops.f64_to_bf16_bits(gu[d:])
    return _oracle(gb, ub, lut_bits)


def _covers_regions(outs_gates):
    ab = np.concatenate(outs_gates) & 0x7FFF
    return (ab < 0x3B00).any() and ((ab >= 0x3B00) & (ab < 0x4300)).any() and (ab >= 0x4300).any()


@pytest.mark.parametrize("k", [256, 2560, 96])  # 96: the generic kernel (k % 64 != 0)
def test_gemv_gelu_one_hot_exact(ops, dev, lut, lut_bits, k):
    d = 200
    blocks = oq.make_blocks(2 * d, k, seed=k, scale=1.0)
    gates = []
    for i, a in enumerate(MAGNITUDES):
        x = _one_hot(k, (37 * i + 5) % k, a)
        out = bits_of(ops.q4_0_gemv_gelu(bf16_dev(x, dev), _w(blocks, dev), lut, d, k)).reshape(d)
        np.testing.assert_array_equal(_canon(out), _canon(_exact_gated(x, blocks, d, k, lut_bits)),
                                      err_msg=f"k={k} magnitude {a}")
        gates.append(oops.f64_to_bf16_bits(oq.gemv_f64(x, blocks, 2 * d, k)[:d]))
    assert _covers_regions(gates)


def test_add_rmsnorm_gemv_gelu_one_hot_exact(ops, dev, lut, lut_bits):
    """x one-hot, no residual, eps 0: the normalised activation is one-hot
    with value sqrt(k) * gamma_c = 16 gamma_c (k = 256), so gate and up are
    exact products; gamma_c sweeps the magnitudes."""
    import torch
    d, k = 200, 256
    blocks = oq.make_blocks(2 * d, k, seed=3, scale=1.0)
    gates = []
    for i, a in enumerate(MAGNITUDES):
        c = (53 * i + 11) % k
        x = _one_hot(k, c, -3.0 if i % 2 else 0.75)
        sign = -1.0 if i % 2 else 1.0
        gamma = f32_to_bf16_bits(np.full(k, 1.0, np.float32))
        gamma[c] = f32_to_bf16_bits(np.float32([a / 16.0]))[0]
        ro = torch.empty(1, k, dtype=torch.bfloat16, device=dev)
        out = bits_of(ops.add_rmsnorm_gemv_gelu(bf16_dev(x, dev), None, bf16_dev(gamma, dev),
                                                _w(blocks, dev), lut, d, k, 0.0,
                                                residual_out=ro)).reshape(d)
        h = _one_hot(k, c, sign * a)
        np.testing.assert_array_equal(_canon(out), _canon(_exact_gated(h, blocks, d, k, lut_bits)),
                                      err_msg=f"gamma_c {a / 16}")
        np.testing.assert_array_equal(bits_of(ro).reshape(k), x)
        gates.append(oops.f64_to_bf16_bits(oq.gemv_f64(h, blocks, 2 * d, k)[:d]))
    assert _covers_regions(gates)


@pytest.mark.parametrize("layout", ["tile", "word", "packed"])
def test_gemm_gelu_one_hot_exact(ops, dev, lut, lut_bits, layout):
    """8 rows, row r one-hot at its own column with magnitude MAGNITUDES[r]:
    the tile kernel (16-byte aligned rows), the word-load kernel (8-byte) and
    the packed-layout kernel (smx_q4_0_gemm_packed_gelu)."""
    import torch
    m, d, k = 8, 200, 512
    blocks = oq.make_blocks(2 * d, k, seed=7, scale=1.0)
    x = np.stack([_one_hot(k, (61 * r + 3) % k, a) for r, a in enumerate(MAGNITUDES)])
    buf = torch.empty(m * k + 8, dtype=torch.bfloat16, device=dev)
    off = 4 if layout == "word" else 0
    xv = buf[off:off + m * k].view(m, k)
    assert (xv.data_ptr() % 16 == 0) == (layout != "word")
    xv.copy_(bf16_dev(x, dev))
    w = _w(blocks, dev)
    if layout == "packed":
        w = ops.q4_0_repack(w, d, k, gated=True)
    out = bits_of(ops.q4_0_gemm_gelu(xv, w, lut, d, k)).reshape(m, d)
    for r in range(m):
        np.testing.assert_array_equal(_canon(out[r]),
                                      _canon(_exact_gated(x[r], blocks, d, k, lut_bits)),
                                      err_msg=f"row {r}")


# -------------------------------------------------------- random, bracketed
def _key(bits):
    b = np.asarray(bits).astype(np.int64)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def _from_key(key):
    return np.where(key < 0, (-key) | 0x8000, key).astype(np.uint16)


def assert_gelu_exact_for_some_bracketed(out_bits, g_exact, u_exact, g_slack, u_slack,
                                         lut_bits, what=""):
    """Each output must be the oracle's act(g') * u' for some bf16 g', u'
    inside the accumulation brackets of the exact gate and up sums (the
    epilogue rounds each fp32 sum to bf16 first).  A bracket wider than 8
    bf16 steps (a sum within the slack of 0, where bf16 values are dense)
    is represented by its two ends: act * u is linear in u, and gelu is
    monotone on (-0.75, inf), which such gate brackets must lie in; the
    output must then lie within 1 ulp of the range of act * u over the
    candidates.  Wide brackets must stay below 5% of the row."""
    g_lo, g_hi = (_key(f32_to_bf16_bits(v)) for v in bf16_bracket(g_exact, g_slack))
    u_lo, u_hi = (_key(f32_to_bf16_bits(v)) for v in bf16_bracket(u_exact, u_slack))
    g_wide, u_wide = (g_hi - g_lo) > 8, (u_hi - u_lo) > 8
    wide = g_wide | u_wide
    assert wide.mean() < 0.05, f"{what}: {wide.sum()} brackets wider than 8 steps"
    for end in (g_lo, g_hi):
        assert (bf16_bits_to_f32(_from_key(end[g_wide])) > -0.75).all(), what
    out = _canon(out_bits)

    def candidates(lo, hi, is_wide):
        span = int(np.where(is_wide, 1, hi - lo).max())
        return [np.where(is_wide, np.where(i == 0, lo, hi), np.minimum(lo + i, hi))
                for i in range(span + 1)]

    exact = np.zeros(out.shape, dtype=bool)
    c_min = np.full(out.shape, np.iinfo(np.int64).max)
    c_max = np.full(out.shape, np.iinfo(np.int64).min)
    for g in candidates(g_lo, g_hi, g_wide):
        for u in candidates(u_lo, u_hi, u_wide):
            o = _canon(_oracle(_from_key(g), _from_key(u), lut_bits))
            exact |= o == out
            c_min, c_max = np.minimum(c_min, _key(o)), np.maximum(c_max, _key(o))
    ok = np.where(wide, (_key(out) >= c_min - 1) & (_key(out) <= c_max + 1), exact)
    if not ok.all():
        i = int(np.argmin(ok))
        raise AssertionError(f"{what}: output {i} = {out[i]:#06x} is no bracketed act(g) * u "
                             f"(g exact {g_exact[i]}, u exact {u_exact[i]})")


def _brackets(x_bits, blocks, d, k):
    gu = oq.gemv_f64(x_bits, blocks, 2 * d, k)
    slack = FP32_ACC_SLACK * gemv_abs_sum(x_bits, blocks, 2 * d, k)
    return gu[:d], gu[d:], slack[:d], slack[d:]


@pytest.mark.parametrize("d,k", [(9728, 2560), (100, 2560), (64, 96)])
def test_gemv_gelu_random(ops, dev, lut, lut_bits, d, k):
    rng = np.random.default_rng(d + k)
    blocks = oq.make_blocks(2 * d, k, seed=d)
    x = randn_bf16(rng, k, 2.0)  # gates of a few units: mostly the table region
    out = bits_of(ops.q4_0_gemv_gelu(bf16_dev(x, dev), _w(blocks, dev), lut, d, k)).reshape(d)
    assert_gelu_exact_for_some_bracketed(out, *_brackets(x, blocks, d, k), lut_bits,
                                         what=f"gemv gelu {d}x{k}")


def test_add_rmsnorm_gemv_gelu_random(ops, dev, lut, lut_bits):
    d, k, eps = 9728, 2560, 1e-6
    rng = np.random.default_rng(5)
    blocks = oq.make_blocks(2 * d, k, seed=9)
    x = randn_bf16(rng, k)
    r = randn_bf16(rng, k, 3.0)
    g = f32_to_bf16_bits((2 + 0.2 * rng.standard_normal(k)).astype(np.float32))
    h, _ = oops.add_rmsnorm(bf16_bits_to_f32(x), bf16_bits_to_f32(r), bf16_bits_to_f32(g), eps)
    out = bits_of(ops.add_rmsnorm_gemv_gelu(bf16_dev(x, dev), bf16_dev(r, dev), bf16_dev(g, dev),
                                            _w(blocks, dev), lut, d, k, eps)).reshape(d)
    hb = f32_to_bf16_bits(h)
    assert_gelu_exact_for_some_bracketed(out, *_brackets(hb, blocks, d, k), lut_bits,
                                         what="norm gemv gelu")


def test_gemm_gelu_random(ops, dev, lut, lut_bits):
    m, d, k = 8, 9728, 2560
    rng = np.random.default_rng(6)
    blocks = oq.make_blocks(2 * d, k, seed=6)
    x = randn_bf16(rng, (m, k), 2.0)
    out = bits_of(ops.q4_0_gemm_gelu(bf16_dev(x, dev), _w(blocks, dev), lut, d, k)).reshape(m, d)
    for row in range(m):
        assert_gelu_exact_for_some_bracketed(out[row], *_brackets(x[row], blocks, d, k), lut_bits,
                                             what=f"gemm gelu row {row}")

