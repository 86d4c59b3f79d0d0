"""GPU parity of the small fused ops through the C ABI.  Bars: bf16 outputs
within 1 bf16 ulp of the oracle (the kernels may contract a*b+c into one
FMA), residual sums, KV copies, gathers, argmax and the step advance exact."""
import numpy as np
import pytest

from oracle import ops as oops
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

from _util import bf16_dev, bf16_ulp_diff, bits_of, f32_of, pkg, randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    return pkg("native.torch_ops")


@pytest.mark.parametrize("rows,hidden", [(1, 2560), (3, 2560), (2, 4096), (1, 8), (1, 16384)])
@pytest.mark.parametrize("with_residual", [True, False])
def test_add_rmsnorm(ops, dev, rows, hidden, with_residual):
    rng = np.random.default_rng(rows * hidden)
    x = randn_bf16(rng, (rows, hidden))
    r = randn_bf16(rng, (rows, hidden), 3.0)
    g = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))
    y, ro = ops.add_rmsnorm(bf16_dev(x, dev), bf16_dev(r, dev) if with_residual else None,
                            bf16_dev(g, dev), 1e-6)
    ry, rro = oops.add_rmsnorm(bf16_bits_to_f32(x), bf16_bits_to_f32(r) if with_residual else None,
                               bf16_bits_to_f32(g), 1e-6)
    assert bf16_ulp_diff(bits_of(y).reshape(rows, hidden), f32_to_bf16_bits(ry)).max() <= 1
    np.testing.assert_array_equal(bits_of(ro).reshape(rows, hidden), f32_to_bf16_bits(rro))


def test_add_rmsnorm_in_place_residual(ops, dev):
    rng = np.random.default_rng(1)
    x = randn_bf16(rng, (1, 2560))
    r = randn_bf16(rng, (1, 2560))
    g = randn_bf16(rng, 2560)
    rt = bf16_dev(r, dev)
    y, ro = ops.add_rmsnorm(bf16_dev(x, dev), rt, bf16_dev(g, dev), 1e-6, residual_out=rt)
    _, rro = oops.add_rmsnorm(bf16_bits_to_f32(x), bf16_bits_to_f32(r), bf16_bits_to_f32(g), 1e-6)
    np.testing.assert_array_equal(bits_of(rt).reshape(1, 2560), f32_to_bf16_bits(rro))


def test_qknorm_rope_kv_write(ops, dev):
    import torch
    rng = np.random.default_rng(3)
    n_q, n_kv, hd, bs, nblk, T = 32, 8, 128, 128, 6, 3
    nh = n_q + 2 * n_kv
    qkv = randn_bf16(rng, (T, nh * hd))
    qg = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    kg = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    cs = f32_to_bf16_bits(oops.rope_cache(8192, hd, 1e6))
    positions = np.array([0, 4095, 7000], dtype=np.int64)
    slots = np.array([5, 130, -1], dtype=np.int64)
    kc = torch.zeros((nblk, bs, n_kv, hd), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q_out = ops.qknorm_rope_kv_write(bf16_dev(qkv, dev), bf16_dev(qg, dev), bf16_dev(kg, dev),
                                     bf16_dev(cs, dev), torch.from_numpy(positions).to(dev),
                                     torch.from_numpy(slots).to(dev), kc, vc, n_q, n_kv, 1e-6)
    qkvf = bf16_bits_to_f32(qkv).reshape(T, nh, hd)
    csf = bf16_bits_to_f32(cs)
    kcb = bits_of(kc).reshape(nblk * bs, n_kv, hd)
    vcb = bits_of(vc).reshape(nblk * bs, n_kv, hd)
    qo = bits_of(q_out).reshape(T, n_q, hd)
    for t in range(T):
        row = csf[positions[t]]
        rq = oops.apply_rope(oops.rms_norm(qkvf[t, :n_q], bf16_bits_to_f32(qg), 1e-6), row)
        assert bf16_ulp_diff(qo[t], f32_to_bf16_bits(rq)).max() <= 1
        rk = oops.apply_rope(oops.rms_norm(qkvf[t, n_q:n_q + n_kv], bf16_bits_to_f32(kg), 1e-6), row)
        if slots[t] >= 0:
            assert bf16_ulp_diff(kcb[slots[t]], f32_to_bf16_bits(rk)).max() <= 1
            np.testing.assert_array_equal(vcb[slots[t]], qkv.reshape(T, nh, hd)[t, n_q + n_kv:])
    written = set(int(s) for s in slots if s >= 0)
    for s in range(nblk * bs):
        if s not in written:
            assert not kcb[s].any() and not vcb[s].any(), f"slot {s} written"


@pytest.mark.parametrize("rows,d", [(1, 9728), (4, 100)])
def test_silu_mul(ops, dev, rows, d):
    rng = np.random.default_rng(d)
    gu = randn_bf16(rng, (rows, 2 * d), 4.0)
    out = ops.silu_mul(bf16_dev(gu, dev))
    f = bf16_bits_to_f32(gu)
    ref = oops.silu_mul(f[:, :d], f[:, d:])
    assert bf16_ulp_diff(bits_of(out).reshape(rows, d), f32_to_bf16_bits(ref)).max() <= 1


def test_embedding(ops, dev):
    import torch
    rng = np.random.default_rng(7)
    table = randn_bf16(rng, (1000, 256))
    ids = np.array([0, 999, 17, -1, 1000], dtype=np.int64)
    out = bits_of(ops.embedding(bf16_dev(table, dev), torch.from_numpy(ids).to(dev))).reshape(5, 256)
    np.testing.assert_array_equal(out[:3], table[ids[:3]])
    assert not out[3:].any()


def test_argmax(ops, dev):
    import torch
    rng = np.random.default_rng(8)
    logits = randn_bf16(rng, (3, 151936))
    logits[1, 5] = logits[1, 77] = f32_to_bf16_bits(np.float32([100.0]))[0]  # tie -> lowest index
    logits[2, 1234] = 0x7FC0  # NaN wins
    out = ops.argmax(bf16_dev(logits, dev)).cpu().numpy()
    assert out[0] == np.argmax(bf16_bits_to_f32(logits[0]))
    assert out[1] == 5
    assert out[2] == 1234


def test_argmax_ragged_vocab(ops, dev):
    """vocab 1003: row 0 is 16-byte aligned (chunks of 8 values, then a
    3-element tail), the other rows are not (element by element)."""
    rng = np.random.default_rng(9)
    v = 1003
    logits = randn_bf16(rng, (5, v))
    big = f32_to_bf16_bits(np.float32([50.0]))[0]
    logits[0, 1001] = big                     # in the tail
    logits[1, 3] = logits[1, 1002] = big      # tie across rows' elements -> lowest index
    logits[2, 999] = logits[2, 1000] = big    # tie across the chunk / tail boundary
    logits[3, 0] = 0x7FC0                     # NaN first element
    out = ops.argmax(bf16_dev(logits, dev)).cpu().numpy()
    assert out.tolist()[:4] == [1001, 3, 999, 0]
    assert out[4] == np.argmax(bf16_bits_to_f32(logits[4]))


def test_decode_advance(ops, dev):
    import torch
    table = torch.tensor([[3, 9, 4], [7, 1, 2]], dtype=torch.int32, device=dev)
    ids = torch.tensor([1, 2], dtype=torch.int64, device=dev)
    nxt = torch.tensor([42, 43], dtype=torch.int64, device=dev)
    pos = torch.tensor([127, 5], dtype=torch.int64, device=dev)
    sl = torch.tensor([128, 6], dtype=torch.int32, device=dev)
    slots = torch.zeros(2, dtype=torch.int64, device=dev)
    toks = torch.full((2, 300), -1, dtype=torch.int64, device=dev)
    ops.decode_advance(nxt, ids, pos, sl, slots, table, 128, tokens_out=toks)
    assert ids.tolist() == [42, 43]
    assert pos.tolist() == [128, 6]
    assert sl.tolist() == [129, 7]
    assert slots.tolist() == [9 * 128 + 0, 7 * 128 + 6]
    assert toks[0, 128].item() == 42 and toks[1, 6].item() == 43
    # past the end of the block table the slot becomes -1
    pos.fill_(3 * 128 - 1)
    ops.decode_advance(nxt, ids, pos, sl, slots, table, 128)
    assert slots.tolist() == [-1, -1]


def test_decode_advance_gathers_next_embedding(ops, dev):
    """With an embedding table, the advance kernel leaves the embedding row of
    each row's new id (the argmax of its keys, or the forced token), zeros
    for an id outside the vocab; the ids and positions are as without it."""
    import torch
    rng = np.random.default_rng(3)
    vocab, hidden, rows = 50, 2560, 3
    table = randn_bf16(rng, (vocab, hidden))
    tdev = bf16_dev(table, dev).view(vocab, hidden)
    keys = torch.zeros((rows, 700), dtype=torch.int64, device=dev)
    # row r's best key sits at index 500 + r with id 7 * r; ids are encoded
    # as 0xffffffff - id in the low word under a positive value key
    for r in range(rows):
        keys[r, 500 + r] = (0x9000 << 32) | (0xFFFFFFFF - 7 * r)
    nxt = torch.zeros(rows, dtype=torch.int64, device=dev)
    ids = torch.zeros(rows, dtype=torch.int64, device=dev)
    pos = torch.tensor([3, 9, 0], dtype=torch.int64, device=dev)
    sl = pos.to(torch.int32) + 1
    slots = torch.zeros(rows, dtype=torch.int64, device=dev)
    table_bt = torch.arange(rows * 4, dtype=torch.int32, device=dev).view(rows, 4)
    forced = torch.full((rows, 16), -1, dtype=torch.int64, device=dev)
    forced[1, 10] = 49          # row 1 takes a forced token
    forced[2, 1] = vocab + 5    # row 2 a forced id outside the vocab
    flen = torch.tensor([0, 11, 2], dtype=torch.int32, device=dev)
    out = torch.full((rows, hidden), 7.0, dtype=torch.bfloat16, device=dev)
    ops.decode_advance(nxt, ids, pos, sl, slots, table_bt, 128, forced_ids=forced,
                       forced_len=flen, argmax_keys=keys.view(rows, -1), embed_table=tdev,
                       embed_out=out)
    assert nxt.tolist() == [0, 7, 14]
    assert ids.tolist() == [0, 49, vocab + 5]
    assert pos.tolist() == [4, 10, 1]
    got = bits_of(out).reshape(rows, hidden)
    np.testing.assert_array_equal(got[0], table[0])
    np.testing.assert_array_equal(got[1], table[49])
    assert np.all(got[2] == 0)
