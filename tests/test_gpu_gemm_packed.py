"""GPU parity of the packed-layout Q4_0 GEMMs (smx_q4_0_repack and the
smx_q4_0_gemm_packed family) through the C ABI:
  * the device repack equals the oracle's packed layout byte for byte
    (plain and gated, ragged row counts);
  * each output row within 1e-2 relative of the float64 oracle GEMV of that
    activation row (the oracle reads the GGUF blocks, so this pins the layout
    end to end), for 1..16 rows and the decode shapes;
  * one-hot activations select dequantised weights bit-exactly (pins the
    lane layout of codes and scales and the MFMA operand order);
  * SwiGLU against the oracle, argmax keys against the plain packed GEMM,
    agreement with the GGUF-layout GEMM, writes in bounds, bad arguments
    refused before launch."""
import numpy as np
import pytest

from oracle import q4_0 as oq
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.ops import silu_mul as o_silu_mul

from _util import assert_close_rel, bf16_dev, bits_of, f32_of, pkg, randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    return pkg("native.torch_ops")


def _w(blocks, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)).to(dev)


def _packed(ops, blocks, n, k, dev, gated=False):
    return ops.q4_0_repack(_w(blocks, dev), n, k, gated)


@pytest.mark.parametrize("n,k,gated", [(16, 256, False), (1000, 2560, False), (37, 768, True),
                                       (9728, 2560, True), (2560, 9728, False), (5, 512, False)])
def test_repack_matches_oracle(ops, dev, n, k, gated):
    rows = 2 * n if gated else n
    blocks = oq.make_blocks(rows, k, seed=n + k + gated)
    wp = _packed(ops, blocks, n, k, dev, gated)
    assert wp.data.numel() == oq.packed_bytes(n, k, gated) == ops.q4_0_packed_bytes(n, k, gated)
    np.testing.assert_array_equal(wp.data.cpu().numpy(), oq.repack(blocks, n, k, gated))


@pytest.mark.parametrize("m", [1, 2, 5, 8, 16])
@pytest.mark.parametrize("n,k", [(64, 256), (1000, 2560), (2560, 9728), (9728, 2560), (2560, 4096)])
def test_packed_gemm_vs_oracle(ops, dev, m, n, k):
    if m in (2, 5) and n * k > 3_000_000:
        pytest.skip("covered by other row counts")
    rng = np.random.default_rng(m * 100 + n + k + 1)
    blocks = oq.make_blocks(n, k, seed=n + k + 1)
    x = randn_bf16(rng, (m, k))
    y = f32_of(ops.q4_0_gemm(bf16_dev(x, dev).view(m, k), _packed(ops, blocks, n, k, dev), n,
                             k)).reshape(m, n)
    for r in range(m):
        assert_close_rel(y[r], oq.gemv_f64(x[r], blocks, n, k), rtol=1e-2, atol_frac=5e-3,
                         what=f"row {r}")


@pytest.mark.parametrize("m", [3, 8, 9, 16])
def test_packed_gemm_one_hot_layout(ops, dev, m):
    """Row r of x one-hot at column c_r: y[r][o] = bf16(dequant(W)[o][c_r])
    exactly; the columns reach every k-group, both halves of a chunk, high
    and low nibbles and the second chunk; 40 outputs leave a partial group."""
    n, k = 40, 512
    blocks = oq.make_blocks(n, k, seed=12, scale=1.0)
    cols = np.array([0, 1, 14, 15, 16, 17, 30, 31, 100, 131, 255, 256, 300, 389, 480, 511])[:m]
    x = np.zeros((m, k), dtype=np.uint16)
    x[np.arange(m), cols] = f32_to_bf16_bits(np.float32([1.0]))[0]
    y = bits_of(ops.q4_0_gemm(bf16_dev(x, dev).view(m, k), _packed(ops, blocks, n, k, dev), n,
                              k)).reshape(m, n)
    exp = f32_to_bf16_bits(oq.dequant_f32(blocks, n, k)[:, cols].T.copy())
    np.testing.assert_array_equal(y, exp)


@pytest.mark.parametrize("m,d,k", [(8, 9728, 2560), (3, 100, 256), (16, 64, 512)])
def test_packed_gemm_swiglu(ops, dev, m, d, k):
    rng = np.random.default_rng(d + m + 1)
    blocks = oq.make_blocks(2 * d, k, seed=d + 2)
    x = randn_bf16(rng, (m, k))
    out = f32_of(ops.q4_0_gemm_swiglu(bf16_dev(x, dev).view(m, k),
                                      _packed(ops, blocks, d, k, dev, gated=True), d,
                                      k)).reshape(m, d)
    for r in range(m):
        gu = oq.gemv_f64(x[r], blocks, 2 * d, k).astype(np.float32)
        g = bf16_bits_to_f32(f32_to_bf16_bits(gu[:d]))
        u = bf16_bits_to_f32(f32_to_bf16_bits(gu[d:]))
        assert_close_rel(out[r], o_silu_mul(g, u), rtol=2e-2, atol_frac=5e-3, what=f"row {r}")


@pytest.mark.parametrize("gated", [False, True])
def test_packed_agrees_with_the_gguf_gemm(ops, dev, gated):
    """Same products, fp32 sums in another order: the bf16 outputs of the two
    layouts differ by at most one bf16 rounding step of the output, plus the
    SiLU's for the gated form."""
    m, n, k = 8, 9728, 2560
    rng = np.random.default_rng(5 + gated)
    blocks = oq.make_blocks(2 * n if gated else n, k, seed=77)
    xd = bf16_dev(randn_bf16(rng, (m, k)), dev).view(m, k)
    if gated:
        a = f32_of(ops.q4_0_gemm_swiglu(xd, _w(blocks, dev), n, k))
        b = f32_of(ops.q4_0_gemm_swiglu(xd, _packed(ops, blocks, n, k, dev, True), n, k))
    else:
        a = f32_of(ops.q4_0_gemm(xd, _w(blocks, dev), n, k))
        b = f32_of(ops.q4_0_gemm(xd, _packed(ops, blocks, n, k, dev), n, k))
    tol = 2.0 ** -7 * np.abs(a) + 1e-3 * np.abs(a).max()
    assert np.all(np.abs(a - b) <= tol), float(np.max(np.abs(a - b) - tol))
    assert np.mean(a == b) > 0.9  # most outputs round to the same bf16


@pytest.mark.parametrize("m", [1, 3, 8])
def test_packed_gemm_argmax_keys(ops, dev, m):
    """Logits equal the plain packed GEMM bit for bit; each row's largest key
    names the first index of its largest logit (rows 5 and 700 of W are equal
    and dominate: the tie goes to 5; n = 1000 leaves a partial group)."""
    import torch
    rng = np.random.default_rng(50 + m)
    n, k = 1000, 512
    blocks = oq.make_blocks(n, k, seed=22).reshape(n, -1).copy()
    top = blocks[5].reshape(-1, 18).copy()
    top[:, 0:2] = np.frombuffer(np.float16(0.5).tobytes(), dtype=np.uint8)
    top[:, 2:] = 0xFF
    blocks[5] = blocks[700] = top.reshape(-1)
    x = f32_to_bf16_bits(np.abs(bf16_bits_to_f32(randn_bf16(rng, (m, k)))))
    xd, wp = bf16_dev(x, dev).view(m, k), _packed(ops, blocks, n, k, dev)
    keys = torch.zeros((m, ops.gemm_keys_per_row(n)), dtype=torch.int64, device=dev)
    y = ops.q4_0_gemm_argmax(xd, wp, n, k, keys)
    np.testing.assert_array_equal(bits_of(y), bits_of(ops.q4_0_gemm(xd, wp, n, k)))
    kv = keys.cpu().numpy().view(np.uint64)
    yb = bits_of(y).reshape(m, n)
    for r in range(m):
        best = int(kv[r].max())
        idx = 0xFFFFFFFF - (best & 0xFFFFFFFF)
        assert idx == int(np.argmax(bf16_bits_to_f32(yb[r]))) == 5, f"row {r}"


def test_packed_gemm_output_sentinels(ops, dev):
    import torch
    m, n, k = 3, 1000, 256
    rng = np.random.default_rng(6)
    blocks = oq.make_blocks(n, k, seed=6)
    x = bf16_dev(randn_bf16(rng, (m, k)), dev).view(m, k)
    guard = torch.full((m * n + 64,), 17.0, dtype=torch.bfloat16, device=dev)
    ops.q4_0_gemm(x, _packed(ops, blocks, n, k, dev), n, k, out=guard[32:32 + m * n])
    gv = guard.float().cpu().numpy()
    assert np.all(gv[:32] == 17.0) and np.all(gv[32 + m * n:] == 17.0)
    assert np.all(np.isfinite(gv[32:32 + m * n]))


def test_packed_rejects_bad_arguments(ops, dev):
    import torch
    w = torch.zeros(64 * 10 * 18, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="256"):
        ops.q4_0_repack(w, 64, 320)
    assert ops.q4_0_packed_bytes(64, 320) == -1
    blocks = oq.make_blocks(128, 256, seed=1)
    wp = _packed(ops, blocks, 64, 256, dev, gated=True)
    x = torch.zeros((2, 256), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="gated"):
        ops.q4_0_gemm(x, wp, 64, 256)  # a gated pack in the plain GEMM
    with pytest.raises(ValueError, match="packed weights hold"):
        ops.q4_0_gemm_swiglu(x, wp, 32, 256)
    with pytest.raises(ValueError):
        ops.q4_0_gemm(torch.zeros((17, 256), dtype=torch.bfloat16, device=dev),
                      _packed(ops, blocks, 128, 256, dev), 128, 256)
    buf = torch.zeros(2 * 256 + 8, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="16-byte"):
        ops.q4_0_gemm(buf[4:4 + 512].view(2, 256), _packed(ops, blocks, 128, 256, dev), 128, 256)
    lib = pkg("native").load()
    assert lib.smx_q4_0_gemm_packed(None, x.data_ptr(), wp.data.data_ptr(), x.data_ptr(), 2, 64,
                                    320) == pkg("native").SMX_EINVAL
