"""GPU parity of the fused decode kernels through the C ABI:

  * add+RMSNorm fused into the Q4_0 GEMV prologue (plain, SwiGLU and argmax
    epilogues): outputs within 1e-2 relative of the float64 oracle GEMV over
    the oracle's normalised activation, the new residual bit-exact;
  * the argmax epilogue + decode_advance give exactly the argmax of the
    logits the same call wrote (ties -> lowest index, across workgroups);
  * q/k RMSNorm + RoPE + KV write fused into split-KV decode: the cache
    writes equal the standalone q/k-norm kernel's, the attention output
    matches the two-launch path and the float64 oracle (every element within
    1e-2 of the output's RMS plus its bf16 rounding, relative L2 below 1e-2).
"""
import numpy as np
import pytest

from oracle import attention as oatt
from oracle import ops as oops
from oracle import q4_0 as oq
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

from _util import (FP32_ACC_SLACK, assert_attention_close, assert_close_rel, assert_swiglu_bracketed, bf16_dev,
                   bf16_ulp_diff, bits_of, f32_of, gemv_abs_sum, pkg, randn_bf16)

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    return pkg("native.torch_ops")


def _blocks_dev(blocks, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)).to(dev)


def _norm_inputs(rng, k, with_residual):
    x = randn_bf16(rng, k)
    r = randn_bf16(rng, k, 3.0) if with_residual else None
    g = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    h, res = oops.add_rmsnorm(bf16_bits_to_f32(x), bf16_bits_to_f32(r) if with_residual else None,
                              bf16_bits_to_f32(g), EPS)
    return x, r, g, h, res


@pytest.mark.parametrize("n,k", [(6144, 2560), (2560, 4096), (64, 256), (1000, 2560),
                                 (2560, 9728)])
@pytest.mark.parametrize("with_residual", [True, False])
def test_add_rmsnorm_gemv(ops, dev, n, k, with_residual):
    import torch
    rng = np.random.default_rng(n + k + with_residual)
    blocks = oq.make_blocks(n, k, seed=n ^ k)
    x, r, g, h, res = _norm_inputs(rng, k, with_residual)
    ro = torch.full((1, k), 5.0, dtype=torch.bfloat16, device=dev)
    y = ops.add_rmsnorm_gemv(bf16_dev(x, dev), bf16_dev(r, dev) if with_residual else None,
                             bf16_dev(g, dev), _blocks_dev(blocks, dev), n, k, EPS, residual_out=ro)
    ref = oq.gemv_f64(f32_to_bf16_bits(h), blocks, n, k)
    assert_close_rel(f32_of(y).reshape(n), ref, rtol=1e-2, atol_frac=5e-3, what="norm gemv")
    np.testing.assert_array_equal(bits_of(ro).reshape(k), f32_to_bf16_bits(res))
    # same result as the two-launch path (add_rmsnorm, then the GEMV)
    hy, _ = ops.add_rmsnorm(bf16_dev(x, dev).view(1, k),
                            bf16_dev(r, dev).view(1, k) if with_residual else None,
                            bf16_dev(g, dev), EPS)
    y2 = ops.q4_0_gemv(hy.view(k), _blocks_dev(blocks, dev), n, k)
    assert_close_rel(f32_of(y).reshape(n), f32_of(y2).reshape(n), rtol=1e-2, atol_frac=2e-3,
                     what="fused vs two-launch")


@pytest.mark.parametrize("d,k", [(9728, 2560), (100, 2560), (32, 256)])
def test_add_rmsnorm_gemv_swiglu(ops, dev, d, k):
    rng = np.random.default_rng(d * 7 + k)
    blocks = oq.make_blocks(2 * d, k, seed=d)
    x, r, g, h, res = _norm_inputs(rng, k, True)
    out = ops.add_rmsnorm_gemv_swiglu(bf16_dev(x, dev), bf16_dev(r, dev), bf16_dev(g, dev),
                                      _blocks_dev(blocks, dev), d, k, EPS)
    hb = f32_to_bf16_bits(h)
    gu = oq.gemv_f64(hb, blocks, 2 * d, k)
    slack = FP32_ACC_SLACK * gemv_abs_sum(hb, blocks, 2 * d, k)
    assert_swiglu_bracketed(f32_of(out).reshape(d), gu[:d], gu[d:], slack[:d], slack[d:],
                            oops.silu_mul, what=f"norm swiglu {d}x{k}")


def _argmax_via_keys(ops, dev, x, r, g, blocks, n, k):
    import torch
    nk = ops.argmax_keys_size(n, k)
    assert nk > 0
    keys = torch.empty((1, nk), dtype=torch.int64, device=dev)
    logits = ops.add_rmsnorm_gemv_argmax(bf16_dev(x, dev), bf16_dev(r, dev) if r is not None else None,
                                         bf16_dev(g, dev), _blocks_dev(blocks, dev), n, k, EPS,
                                         keys.view(-1))
    z64 = lambda: torch.zeros(1, dtype=torch.int64, device=dev)
    nxt, ids, pos, slots = z64(), z64(), z64(), z64()
    sl = torch.ones(1, dtype=torch.int32, device=dev)
    table = torch.zeros((1, 4), dtype=torch.int32, device=dev)
    ops.decode_advance(nxt, ids, pos, sl, slots, table, 128, argmax_keys=keys)
    return logits, int(ids.item()), int(nxt.item())


@pytest.mark.parametrize("n,k", [(151936, 2560), (1000, 256), (4104, 2560),
                                 (4096, 20480), (2056, 32768)])
def test_add_rmsnorm_gemv_argmax(ops, dev, n, k):
    """Head GEMV + argmax keys; K = 20480 and 32768 take 5 and 8 pair groups
    per lane (one row group per workgroup there)."""
    rng = np.random.default_rng(n)
    blocks = oq.make_blocks(n, k, seed=n)
    x, r, g, h, _ = _norm_inputs(rng, k, True)
    logits, tok, nxt = _argmax_via_keys(ops, dev, x, r, g, blocks, n, k)
    lf = f32_of(logits).reshape(n)
    ref = oq.gemv_f64(f32_to_bf16_bits(h), blocks, n, k)
    assert_close_rel(lf, ref, rtol=1e-2, atol_frac=5e-3, what="head logits")
    assert tok == nxt == int(ops.argmax(logits.view(1, n)).item()) == int(np.argmax(lf))


@pytest.mark.parametrize("first,second", [(1001, 150001), (8, 9), (151935, 151935)])
def test_argmax_ties_pick_lowest_index(ops, dev, first, second):
    """Rows `first` and `second` hold identical weights with the largest
    output: the lowest index wins, whichever workgroups own them."""
    n, k = 151936, 2560
    blocks = oq.make_blocks(n, k, seed=5).reshape(n, k // 32, 18)
    big = np.zeros((k // 32, 18), dtype=np.uint8)
    big[:, 0:2] = np.frombuffer(np.float16(0.5).tobytes(), dtype=np.uint8)
    big[:, 2:] = 0xFF  # every code 15 -> weight 7 * 0.5
    blocks[first] = big
    blocks[second] = big
    x = f32_to_bf16_bits(np.ones(k, dtype=np.float32))
    g = f32_to_bf16_bits(np.ones(k, dtype=np.float32))
    _, tok, _ = _argmax_via_keys(ops, dev, x, None, g, blocks.reshape(n, -1), n, k)
    assert tok == min(first, second)


N_Q, N_KV, HD = 32, 8, 128


def _fused_case(rng, lengths, bs, dev):
    import torch
    need = [-(-L // bs) for L in lengths]
    max_blocks = max(need) + 1
    nblk = sum(need) + 2
    perm = rng.permutation(nblk).astype(np.int32)
    table = np.zeros((len(lengths), max_blocks), dtype=np.int32)
    at = 0
    for i, nb in enumerate(need):
        table[i, :nb] = perm[at:at + nb]
        table[i, nb:] = perm[at]  # unused entries stay valid pages
        at += nb
    kc = randn_bf16(rng, (nblk, bs, N_KV, HD))
    vc = randn_bf16(rng, (nblk, bs, N_KV, HD))
    qkv = randn_bf16(rng, (len(lengths), (N_Q + 2 * N_KV) * HD), 2.0)
    qg = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32))
    kg = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32))
    cs = f32_to_bf16_bits(oops.rope_cache(8192, HD, 1e6))
    pos = np.array([L - 1 for L in lengths], dtype=np.int64)
    slots = np.array([int(table[i, p // bs]) * bs + p % bs for i, p in enumerate(pos)],
                     dtype=np.int64)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(dt).to(dev)
    return dict(qkv=bf16_dev(qkv, dev), qg=bf16_dev(qg, dev), kg=bf16_dev(kg, dev),
                cs=bf16_dev(cs, dev), pos=t(pos, torch.int64), slots=t(slots, torch.int64),
                kc=bf16_dev(kc, dev), vc=bf16_dev(vc, dev), table=t(table, torch.int32),
                sl=torch.tensor(lengths, dtype=torch.int32, device=dev),
                np=dict(qkv=qkv, qg=qg, kg=kg, cs=cs, pos=pos, slots=slots, table=table))


def _fused(ops, c, splits, kc, vc):
    import torch
    ns = c["sl"].numel()
    po = torch.empty((ns, splits, N_Q, HD), dtype=torch.float32, device=kc.device)
    pl = torch.empty((ns, splits, N_Q), dtype=torch.float32, device=kc.device)
    return ops.qknorm_rope_splitkv_decode_merged(c["qkv"], c["qg"], c["kg"], c["cs"], c["pos"],
                                                 c["slots"], kc, vc, c["table"], c["sl"], splits,
                                                 HD ** -0.5, EPS, N_Q, po, pl)


def _two_launch(ops, c, splits, kc, vc):
    import torch
    ns = c["sl"].numel()
    q = ops.qknorm_rope_kv_write(c["qkv"], c["qg"], c["kg"], c["cs"], c["pos"], c["slots"], kc, vc,
                                 N_Q, N_KV, EPS)
    po = torch.empty((ns, splits, N_Q, HD), dtype=torch.float32, device=kc.device)
    pl = torch.empty((ns, splits, N_Q), dtype=torch.float32, device=kc.device)
    return ops.splitkv_decode_merged(q.view(ns, N_Q, HD), kc, vc, c["table"], c["sl"], splits,
                                     HD ** -0.5, po, pl), q


@pytest.mark.parametrize("lengths,bs,splits", [
    ([1], 128, 1), ([300], 128, 4), ([2048], 128, 16), ([6144], 128, 32), ([6144], 128, 64),
    ([33, 129, 4096], 128, 8), ([97, 1000], 32, 4), ([6144], 128, 4), ([64, 65, 128], 64, 2)])
def test_fused_qknorm_rope_splitkv(ops, dev, lengths, bs, splits):
    rng = np.random.default_rng(sum(lengths) + splits)
    c = _fused_case(rng, lengths, bs, dev)
    kc1, vc1 = c["kc"].clone(), c["vc"].clone()
    kc2, vc2 = c["kc"].clone(), c["vc"].clone()
    out = _fused(ops, c, splits, kc1, vc1)
    out2, q = _two_launch(ops, c, splits, kc2, vc2)
    # the same cache contents (the new K/V in their slots, nothing else; the
    # two kernels may contract the RoPE products differently: 1 ulp)
    assert bf16_ulp_diff(bits_of(kc1), bits_of(kc2)).max() <= 1
    np.testing.assert_array_equal(bits_of(vc1), bits_of(vc2))
    ns = len(lengths)
    assert_close_rel(f32_of(out).reshape(ns, -1), f32_of(out2).reshape(ns, -1), rtol=1e-2,
                     atol_frac=1e-2, what="fused vs two-launch")
    # and the float64 oracle over the updated cache
    kcn = bf16_bits_to_f32(bits_of(kc1))
    vcn = bf16_bits_to_f32(bits_of(vc1))
    qf = f32_of(q).reshape(ns, N_Q, HD)
    for i, L in enumerate(lengths):
        k = oatt.gather_paged(kcn, c["np"]["table"][i], L)
        v = oatt.gather_paged(vcn, c["np"]["table"][i], L)
        ref = oatt.attention_f64(qf[i], k, v, HD ** -0.5)
        got = f32_of(out).reshape(ns, N_Q, HD)[i]
        assert_attention_close(got, ref, f"seq {i} (L={L})")


def test_fused_uses_new_kv_over_stale_slot(ops, dev):
    """The slot of the new token holds junk before the call; the result must
    use the freshly written K/V (the workgroup patches them in from LDS)."""
    rng = np.random.default_rng(42)
    lengths, bs, splits = [200, 5000], 128, 16
    c = _fused_case(rng, lengths, bs, dev)
    for s in c["np"]["slots"]:
        blk, off = divmod(int(s), bs)
        c["kc"][blk, off] = 1e4
        c["vc"][blk, off] = -1e4
    kc1, vc1 = c["kc"].clone(), c["vc"].clone()
    out = _fused(ops, c, splits, kc1, vc1)
    kc2, vc2 = c["kc"].clone(), c["vc"].clone()
    out2, _ = _two_launch(ops, c, splits, kc2, vc2)
    assert np.isfinite(f32_of(out)).all()
    assert_close_rel(f32_of(out).reshape(-1), f32_of(out2).reshape(-1), rtol=1e-2, atol_frac=1e-2,
                     what="stale slot")
    assert bf16_ulp_diff(bits_of(kc1), bits_of(kc2)).max() <= 1
    np.testing.assert_array_equal(bits_of(vc1), bits_of(vc2))


def _fused_planned(ops, c, items, splits, kc, vc):
    import torch
    ns = c["sl"].numel()
    bs = kc.shape[1]
    po = torch.full((ns, splits, N_Q, HD), float("nan"), dtype=torch.float32, device=kc.device)
    pl = torch.full((ns, splits, N_Q), float("nan"), dtype=torch.float32, device=kc.device)
    plan = ops.splitkv_plan(c["sl"], c["table"], bs, items, po, pl, positions=c["pos"],
                            slot_mapping=c["slots"])
    return ops.qknorm_rope_splitkv_decode_planned_merged(c["qkv"], c["qg"], c["kg"], c["cs"], kc, vc,
                                                         c["table"], plan, items, HD ** -0.5, EPS,
                                                         N_Q, po, pl)


@pytest.mark.parametrize("lengths,bs,items,splits", [
    ([1], 128, 8, 4), ([6144], 128, 49, 64), ([33, 129, 4096], 128, 8, 8),
    ([97, 1000, 5000, 2], 32, 24, 16), ([512, 3000, 77, 2049, 1, 700, 6000, 129], 128, 56, 16)])
def test_fused_planned(ops, dev, lengths, bs, items, splits):
    """The planned fused kernel: the same cache writes as the two-launch path
    and the float64 result over the updated cache, for ragged batches."""
    rng = np.random.default_rng(sum(lengths) + items)
    c = _fused_case(rng, lengths, bs, dev)
    kc1, vc1 = c["kc"].clone(), c["vc"].clone()
    kc2, vc2 = c["kc"].clone(), c["vc"].clone()
    out = _fused_planned(ops, c, items, splits, kc1, vc1)
    out2, q = _two_launch(ops, c, 8, kc2, vc2)
    assert bf16_ulp_diff(bits_of(kc1), bits_of(kc2)).max() <= 1
    np.testing.assert_array_equal(bits_of(vc1), bits_of(vc2))
    ns = len(lengths)
    assert_close_rel(f32_of(out).reshape(ns, -1), f32_of(out2).reshape(ns, -1), rtol=1e-2,
                     atol_frac=1e-2, what="planned fused vs two-launch")
    kcn = bf16_bits_to_f32(bits_of(kc1))
    vcn = bf16_bits_to_f32(bits_of(vc1))
    qf = f32_of(q).reshape(ns, N_Q, HD)
    for i, L in enumerate(lengths):
        k = oatt.gather_paged(kcn, c["np"]["table"][i], L)
        v = oatt.gather_paged(vcn, c["np"]["table"][i], L)
        ref = oatt.attention_f64(qf[i], k, v, HD ** -0.5)
        got = f32_of(out).reshape(ns, N_Q, HD)[i]
        assert_attention_close(got, ref, f"seq {i} (L={L})")


@pytest.mark.parametrize("given", ["none", "positions_only"])
def test_fused_planned_without_positions_poisons(ops, dev, given):
    """A plan built without positions and slots cannot drive the fused
    q/k-norm + RoPE + KV-write kernel: every sequence's output is NaN and the
    caches are left as they were (no K/V written at a made-up slot)."""
    import torch
    lengths, bs, items, splits = [300, 4096, 1], 128, 24, 8
    rng = np.random.default_rng(77)
    c = _fused_case(rng, lengths, bs, dev)
    kc, vc = c["kc"].clone(), c["vc"].clone()
    ns = len(lengths)
    po = torch.empty((ns, splits, N_Q, HD), dtype=torch.float32, device=dev)
    pl = torch.empty((ns, splits, N_Q), dtype=torch.float32, device=dev)
    kw = {} if given == "none" else {"positions": c["pos"]}
    plan = ops.splitkv_plan(c["sl"], c["table"], bs, items, po, pl, **kw)
    rec = plan.cpu().numpy().view(np.uint32)
    ref = oatt.plan_records(lengths, items, splits, c["np"]["table"], bs,
                            positions=c["np"]["pos"] if kw else None)
    np.testing.assert_array_equal(rec, ref)
    assert not (rec[:, 3] & oatt.PLAN_HAS_POSITIONS).any()
    out = ops.qknorm_rope_splitkv_decode_planned_merged(c["qkv"], c["qg"], c["kg"], c["cs"], kc,
                                                        vc, c["table"], plan, items, HD ** -0.5,
                                                        EPS, N_Q, po, pl)
    torch.cuda.synchronize()
    assert np.isnan(f32_of(out)).all()
    np.testing.assert_array_equal(bits_of(kc), bits_of(c["kc"]))
    np.testing.assert_array_equal(bits_of(vc), bits_of(c["vc"]))
