"""GPU parity of the batched Q4_0 GEMM (MFMA tile kernel over the GEMV's
16-byte pair loads, up to 16 rows) through the C ABI: each output
row within 1e-2 relative of the float64 oracle GEMV of that activation row;
one-hot activations select dequantised weights bit-exactly (this pins the
MFMA operand and result layouts); SwiGLU epilogue; writes stay in bounds."""
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


@pytest.mark.parametrize("m", [1, 2, 5, 8, 16])
@pytest.mark.parametrize("n,k", [(64, 256), (1000, 2560), (2560, 9728), (9728, 2560), (2560, 4096)])
def test_gemm_vs_oracle(ops, dev, m, n, k):
    if m in (2, 5) and n * k > 3_000_000:
        pytest.skip("covered by other row counts")
    rng = np.random.default_rng(m * 100 + n + k)
    blocks = oq.make_blocks(n, k, seed=n + k)
    x = randn_bf16(rng, (m, k))
    y = f32_of(ops.q4_0_gemm(bf16_dev(x, dev), _w(blocks, dev), n, k)).reshape(m, n)
    for r in range(m):
        assert_close_rel(y[r], oq.gemv_f64(x[r], blocks, n, k), rtol=1e-2, atol_frac=5e-3,
                         what=f"row {r}")


@pytest.mark.parametrize("m", [3, 8, 16])
def test_gemm_one_hot_layout(ops, dev, m):
    """Row m of x is one-hot at column c_m: y[m][n] = bf16(dequant(W)[n][c_m])
    exactly, for up to 16 rows, 48 output rows and columns spread over both
    blocks of a pair and all nibble positions (this pins the permlane
    transpose and the MFMA operand and result layouts)."""
    n, k = 48, 256
    blocks = oq.make_blocks(n, k, seed=11, scale=1.0)
    cols = np.array([0, 1, 14, 15, 16, 17, 30, 31, 32, 33, 46, 47, 48, 63, 100, 255])[:m]
    x = np.zeros((m, k), dtype=np.uint16)
    x[np.arange(m), cols] = f32_to_bf16_bits(np.float32([1.0]))[0]
    y = bits_of(ops.q4_0_gemm(bf16_dev(x, dev), _w(blocks, dev), n, k)).reshape(m, n)
    wq = oq.dequant_f32(blocks, n, k)
    exp = f32_to_bf16_bits(wq[:, cols].T.copy())
    np.testing.assert_array_equal(y, exp)


@pytest.mark.parametrize("m", [4, 7])
@pytest.mark.parametrize("k", [64, 192, 320, 448])
def test_gemm_partial_k_tile(ops, dev, m, k):
    """A K tile holds 4 block pairs; with 1, 3, 5 or 7 pairs the last tile's
    missing pairs are clamped loads that must carry no weight.  One-hot rows
    (the first at the last column, the others spread) select dequantised
    weights exactly; random rows match the float64 oracle.  m = 4 and 7 are
    the last row counts of two activation staging widths."""
    n = 40
    blocks = oq.make_blocks(n, k, seed=k + m, scale=1.0)
    cols = (k - 1 + 37 * np.arange(m)) % k
    x = np.zeros((m, k), dtype=np.uint16)
    x[np.arange(m), cols] = f32_to_bf16_bits(np.float32([1.0]))[0]
    y = bits_of(ops.q4_0_gemm(bf16_dev(x, dev), _w(blocks, dev), n, k)).reshape(m, n)
    exp = f32_to_bf16_bits(oq.dequant_f32(blocks, n, k)[:, cols].T.copy())
    np.testing.assert_array_equal(y, exp)
    rng = np.random.default_rng(k * 10 + m)
    blocks = oq.make_blocks(200, k, seed=k + m + 1)
    xr = randn_bf16(rng, (m, k))
    yr = f32_of(ops.q4_0_gemm(bf16_dev(xr, dev), _w(blocks, dev), 200, k)).reshape(m, 200)
    for r in range(m):
        assert_close_rel(yr[r], oq.gemv_f64(xr[r], blocks, 200, k), rtol=1e-2, atol_frac=5e-3,
                         what=f"row {r}")


@pytest.mark.parametrize("m,d,k", [(8, 9728, 2560), (3, 100, 256), (16, 64, 512)])
def test_gemm_swiglu(ops, dev, m, d, k):
    rng = np.random.default_rng(d + m)
    blocks = oq.make_blocks(2 * d, k, seed=d + 1)
    x = randn_bf16(rng, (m, k))
    out = f32_of(ops.q4_0_gemm_swiglu(bf16_dev(x, dev), _w(blocks, dev), d, k)).reshape(m, d)
    for r in range(m):
        gu = oq.gemv_f64(x[r], blocks, 2 * d, k).astype(np.float32)
        g = bf16_bits_to_f32(f32_to_bf16_bits(gu[:d]))
        u = bf16_bits_to_f32(f32_to_bf16_bits(gu[d:]))
        assert_close_rel(out[r], o_silu_mul(g, u), rtol=2e-2, atol_frac=5e-3, what=f"row {r}")


@pytest.mark.parametrize("m", [2, 8])
@pytest.mark.parametrize("swiglu", [False, True])
def test_gemm_8_byte_aligned_activations(ops, dev, m, swiglu):
    """Activations that are 8- but not 16-byte aligned take the word-load
    MFMA kernel: same oracle bound as the tile kernel."""
    import torch
    n, k = 96, 512
    rng = np.random.default_rng(m + 10 * swiglu)
    blocks = oq.make_blocks(2 * n if swiglu else n, k, seed=m + 3)
    x = randn_bf16(rng, (m, k))
    buf = torch.empty(m * k + 8, dtype=torch.bfloat16, device=dev)
    xv = buf[4:4 + m * k].view(m, k)  # 8 bytes past a 16-byte aligned allocation
    assert xv.data_ptr() % 16 == 8
    xv.copy_(bf16_dev(x, dev))
    if swiglu:
        out = f32_of(ops.q4_0_gemm_swiglu(xv, _w(blocks, dev), n, k)).reshape(m, n)
    else:
        out = f32_of(ops.q4_0_gemm(xv, _w(blocks, dev), n, k)).reshape(m, n)
    for r in range(m):
        if swiglu:
            gu = oq.gemv_f64(x[r], blocks, 2 * n, k).astype(np.float32)
            ref = o_silu_mul(bf16_bits_to_f32(f32_to_bf16_bits(gu[:n])),
                             bf16_bits_to_f32(f32_to_bf16_bits(gu[n:])))
            assert_close_rel(out[r], ref, rtol=2e-2, atol_frac=5e-3, what=f"row {r}")
        else:
            assert_close_rel(out[r], oq.gemv_f64(x[r], blocks, n, k), rtol=1e-2, atol_frac=5e-3,
                             what=f"row {r}")


def test_gemm_output_sentinels(ops, dev):
    import torch
    m, n, k = 3, 1000, 256
    rng = np.random.default_rng(4)
    blocks = oq.make_blocks(n, k, seed=4)
    x = bf16_dev(randn_bf16(rng, (m, k)), dev)
    guard = torch.full((m * n + 64,), 17.0, dtype=torch.bfloat16, device=dev)
    y = guard[32:32 + m * n]
    ops.q4_0_gemm(x, _w(blocks, dev), n, k, out=y)
    gv = guard.float().cpu().numpy()
    assert np.all(gv[:32] == 17.0) and np.all(gv[32 + m * n:] == 17.0)
    assert np.all(np.isfinite(gv[32:32 + m * n]))


def test_gemm_rejects_bad_arguments(ops, dev):
    import torch
    w = torch.zeros(64 * 8 * 18, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        ops.q4_0_gemm(torch.zeros((17, 256), dtype=torch.bfloat16, device=dev), w, 64, 256)
    with pytest.raises(ValueError):
        ops.q4_0_gemm(torch.zeros((2, 256), dtype=torch.float32, device=dev), w, 64, 256)


@pytest.mark.parametrize("m", [1, 3, 8])
def test_gemm_argmax_keys(ops, dev, m):
    """The keys epilogue: logits equal the plain GEMM bit for bit, and each
    row's largest key names the first index of its largest bf16 logit; rows 5
    and 700 of W are equal and dominate, so the tie goes to 5 (n = 1000 is not
    a multiple of 16: the last group is partial)."""
    import torch
    rng = np.random.default_rng(40 + m)
    n, k = 1000, 512
    blocks = oq.make_blocks(n, k, seed=21).reshape(n, -1).copy()
    top = blocks[5].reshape(-1, 18).copy()
    top[:, 0:2] = np.frombuffer(np.float16(0.5).tobytes(), dtype=np.uint8)  # d = 0.5
    top[:, 2:] = 0xFF                                                         # every nibble 15
    blocks[5] = blocks[700] = top.reshape(-1)
    x = f32_to_bf16_bits(np.abs(bf16_bits_to_f32(randn_bf16(rng, (m, k)))))
    xd, wd = bf16_dev(x, dev).view(m, k), _w(blocks, dev)
    nk = ops.gemm_keys_per_row(n)
    assert nk == 63
    keys = torch.zeros((m, nk), dtype=torch.int64, device=dev)
    y = ops.q4_0_gemm_argmax(xd, wd, n, k, keys)
    np.testing.assert_array_equal(bits_of(y), bits_of(ops.q4_0_gemm(xd, wd, n, k)))
    kv = keys.cpu().numpy().view(np.uint64)
    yb = bits_of(y).reshape(m, n)
    for r in range(m):
        best = int(kv[r].max())
        idx = 0xFFFFFFFF - (best & 0xFFFFFFFF)
        vals = bf16_bits_to_f32(yb[r])
        assert idx == int(np.argmax(vals)) == 5, f"row {r}"
