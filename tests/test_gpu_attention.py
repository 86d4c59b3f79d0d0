"""GPU parity of split-KV decode attention and the LSE merge, through the C
ABI.  Bars (tests/_util.py): the merged bf16 output against the float64
textbook attention with every element within 1e-2 of the reference's RMS
plus the output's own bf16 rounding, and relative L2 below 1e-2; per split,
lse within 1e-4 and the fp32 partial output within 2e-2 of the split's RMS
(relative L2 below 1e-2) of the oracle's restatement of the reference's
online softmax (bf16 P).  q, K, V ~ N(0,1): the output's RMS is 0.038 /
0.026 / 0.021 at contexts 2048 / 4096 / 6144."""
import numpy as np
import pytest

from oracle import attention as oatt
from oracle.bf16 import bf16_bits_to_f32

from _util import (assert_attention_close, assert_partials_close, bf16_dev, bits_of, f32_of, pkg,
                   randn_bf16)

pytestmark = pytest.mark.gpu

N_Q, N_KV, HD = 32, 8, 128


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    return pkg("native.torch_ops")


def _case(rng, lengths, bs, extra_blocks=3):
    """Random q and paged caches for several sequences with shuffled pages."""
    need = [-(-L // bs) for L in lengths]
    max_blocks = max(need) + 1
    nblk = sum(need) + extra_blocks
    perm = rng.permutation(nblk).astype(np.int32)
    table = np.full((len(lengths), max_blocks), -7, dtype=np.int32)  # junk past the end
    at = 0
    for i, nb in enumerate(need):
        table[i, :nb] = perm[at:at + nb]
        at += nb
    kc = randn_bf16(rng, (nblk, bs, N_KV, HD))
    vc = randn_bf16(rng, (nblk, bs, N_KV, HD))
    q = randn_bf16(rng, (len(lengths), N_Q, HD))
    return q, kc, vc, table


def _run(ops, dev, q, kc, vc, table, lengths, splits, scale, merged=False):
    """Separate split-KV and LSE-merge calls, or the one-call merged entry."""
    import torch
    args = (bf16_dev(q, dev), bf16_dev(kc, dev), bf16_dev(vc, dev), torch.from_numpy(table).to(dev),
            torch.tensor(lengths, dtype=torch.int32, device=dev), splits, scale)
    if merged:
        nq = q.shape[1]
        po = torch.empty((len(lengths), splits, nq, HD), dtype=torch.float32, device=dev)
        pl = torch.empty((len(lengths), splits, nq), dtype=torch.float32, device=dev)
        out = ops.splitkv_decode_merged(*args, po, pl)
    else:
        po, pl = ops.splitkv_decode(*args)
        out = ops.lse_merge(po, pl)
    return f32_of(out), po.cpu().numpy(), pl.cpu().numpy()


@pytest.mark.parametrize("merged", [False, True])
@pytest.mark.parametrize("L", [1, 2, 31, 32, 33, 127, 128, 129, 300, 2048, 4096, 6144])
@pytest.mark.parametrize("splits", [1, 4, 8, 16, 32, 64])
def test_splitkv_vs_fp64(ops, dev, L, splits, merged):
    rng = np.random.default_rng(L * 31 + splits)
    bs = 128
    q, kc, vc, table = _case(rng, [L], bs)
    scale = HD ** -0.5
    out, po, pl = _run(ops, dev, q, kc, vc, table, [L], splits, scale, merged=merged)
    qf, kf, vf = (bf16_bits_to_f32(a) for a in (q, kc, vc))
    k = oatt.gather_paged(kf, table[0], L)
    v = oatt.gather_paged(vf, table[0], L)
    ref = oatt.attention_f64(qf[0], k, v, scale)
    assert_attention_close(out.reshape(N_Q, HD), ref, f"L={L} splits={splits} merged output")
    # per-split partials against the oracle's online softmax
    bounds = oatt.split_bounds(L, splits, table.shape[1] * bs)
    opo, opl = oatt.splitkv_partials(qf[0], k, v, scale, bounds)
    assert_partials_close(po[0], pl[0], opo, opl, f"L={L} splits={splits} partials")


@pytest.mark.parametrize("bs", [32, 64, 256])
def test_block_sizes(ops, dev, bs):
    rng = np.random.default_rng(bs)
    L = 1000
    q, kc, vc, table = _case(rng, [L], bs)
    scale = HD ** -0.5
    out, _, _ = _run(ops, dev, q, kc, vc, table, [L], 8, scale)
    qf, kf, vf = (bf16_bits_to_f32(a) for a in (q, kc, vc))
    ref = oatt.attention_f64(qf[0], oatt.gather_paged(kf, table[0], L),
                             oatt.gather_paged(vf, table[0], L), scale)
    assert_attention_close(out.reshape(N_Q, HD), ref, f"block size {bs}")


@pytest.mark.parametrize("L,bs,splits", [(20000, 32, 1), (9000, 128, 1), (3000, 32, 2)])
def test_long_wave_chunks(ops, dev, L, bs, splits):
    """Waves that walk many blocks: their pages come from the entry gather
    (56 pages per wave) and, past that, from the block table (L=20000 with
    32-token pages and one split: 2500 tokens = 79 pages per wave)."""
    rng = np.random.default_rng(L + bs)
    q, kc, vc, table = _case(rng, [L], bs)
    scale = HD ** -0.5
    out, _, _ = _run(ops, dev, q, kc, vc, table, [L], splits, scale)
    qf, kf, vf = (bf16_bits_to_f32(a) for a in (q, kc, vc))
    ref = oatt.attention_f64(qf[0], oatt.gather_paged(kf, table[0], L),
                             oatt.gather_paged(vf, table[0], L), scale)
    assert_attention_close(out.reshape(N_Q, HD), ref, f"L={L} bs={bs} splits={splits}")


@pytest.mark.parametrize("merged", [False, True])
def test_ragged_batch(ops, dev, merged):
    rng = np.random.default_rng(5)
    lengths = [512, 3000, 77, 32768 // 4, 1]
    bs = 128
    q, kc, vc, table = _case(rng, lengths, bs)
    scale = HD ** -0.5
    out, _, _ = _run(ops, dev, q, kc, vc, table, lengths, 16, scale, merged=merged)
    qf, kf, vf = (bf16_bits_to_f32(a) for a in (q, kc, vc))
    out = out.reshape(len(lengths), N_Q, HD)
    for i, L in enumerate(lengths):
        ref = oatt.attention_f64(qf[i], oatt.gather_paged(kf, table[i], L),
                                 oatt.gather_paged(vf, table[i], L), scale)
        assert_attention_close(out[i], ref, f"sequence {i} (L={L})")


def test_page_permutation_invariance(ops, dev):
    """Same logical KV behind two different page orders gives the same bits."""
    import torch
    rng = np.random.default_rng(8)
    L, bs = 1500, 128
    q, kc, vc, table = _case(rng, [L], bs, extra_blocks=0)
    nb = -(-L // bs)
    perm = rng.permutation(kc.shape[0])
    inv = np.argsort(perm)
    kc2, vc2 = kc[perm], vc[perm]
    table2 = table.copy()
    table2[0, :nb] = inv[table[0, :nb]]
    a, _, _ = _run(ops, dev, q, kc, vc, table, [L], 8, HD ** -0.5)
    b, _, _ = _run(ops, dev, q, kc2, vc2, table2, [L], 8, HD ** -0.5)
    np.testing.assert_array_equal(a, b)


def test_equal_keys_give_mean_of_values(ops, dev):
    rng = np.random.default_rng(2)
    L, bs = 640, 128
    q, kc, vc, table = _case(rng, [L], bs)
    kc[:] = kc[0:1, 0:1]  # every key identical
    out, _, _ = _run(ops, dev, q, kc, vc, table, [L], 4, HD ** -0.5)
    vf = oatt.gather_paged(bf16_bits_to_f32(vc), table[0], L)
    ref = np.repeat(vf.mean(axis=0), N_Q // N_KV, axis=0)
    assert_attention_close(out.reshape(N_Q, HD), ref, "equal keys")


def test_merged_equals_two_call_path_bitwise(ops, dev):
    rng = np.random.default_rng(12)
    L = 5000
    q, kc, vc, table = _case(rng, [L], 128)
    a, _, _ = _run(ops, dev, q, kc, vc, table, [L], 32, HD ** -0.5)
    for _ in range(2):
        b, _, _ = _run(ops, dev, q, kc, vc, table, [L], 32, HD ** -0.5, merged=True)
        np.testing.assert_array_equal(a, b)


def test_bad_block_table_entry_poisons_only(ops, dev):
    """An out-of-range page id is never dereferenced; the output is NaN."""
    rng = np.random.default_rng(4)
    L, bs = 400, 128
    q, kc, vc, table = _case(rng, [L], bs)
    table[0, 1] = 1 << 20
    out, _, pl = _run(ops, dev, q, kc, vc, table, [L], 1, HD ** -0.5)
    assert np.isnan(out).all()


def test_partial_sentinels(ops, dev):
    """Kernel writes stay inside partial_o / partial_lse."""
    import torch
    rng = np.random.default_rng(6)
    L, bs, S = 700, 128, 8
    q, kc, vc, table = _case(rng, [L], bs)
    guard_o = torch.full((S * N_Q * HD + 64,), 17.0, device=dev)
    guard_l = torch.full((S * N_Q + 64,), 17.0, device=dev)
    po = guard_o[32:32 + S * N_Q * HD].view(1, S, N_Q, HD)
    pl = guard_l[32:32 + S * N_Q].view(1, S, N_Q)
    ops.splitkv_decode(bf16_dev(q, dev), bf16_dev(kc, dev), bf16_dev(vc, dev),
                       torch.from_numpy(table).to(dev),
                       torch.tensor([L], dtype=torch.int32, device=dev), S, HD ** -0.5,
                       partial_o=po, partial_lse=pl)
    go, gl = guard_o.cpu().numpy(), guard_l.cpu().numpy()
    assert np.all(go[:32] == 17) and np.all(go[-32:] == 17)
    assert np.all(gl[:32] == 17) and np.all(gl[-32:] == 17)


@pytest.mark.parametrize("merged", [False, True])
def test_zero_length_gives_zero_output(ops, dev, merged):
    """Sequences with no tokens: every split is empty and the merge has no
    weight, so the output is zero (not NaN)."""
    rng = np.random.default_rng(9)
    q, kc, vc, table = _case(rng, [1, 1], 128)
    out, _, pl = _run(ops, dev, q, kc, vc, table, [0, 0], 8, HD ** -0.5, merged=merged)
    assert np.all(out == 0)


def _planned(ops, dev, q, kc, vc, table, lengths, bs, items, splits, scale,
             positions=None, slots=None):
    """Plan + planned decode over partial buffers that start as NaN (slots
    no split writes must be cleared by the plan)."""
    import torch
    ns = len(lengths)
    po = torch.full((ns, splits, N_Q, HD), float("nan"), dtype=torch.float32, device=dev)
    pl = torch.full((ns, splits, N_Q), float("nan"), dtype=torch.float32, device=dev)
    tdev = torch.from_numpy(table).to(dev)
    t64 = lambda a: None if a is None else torch.tensor(a, dtype=torch.int64, device=dev)
    plan = ops.splitkv_plan(torch.tensor(lengths, dtype=torch.int32, device=dev), tdev, bs, items,
                            po, pl, positions=t64(positions), slot_mapping=t64(slots))
    out = ops.splitkv_decode_planned_merged(bf16_dev(q, dev), bf16_dev(kc, dev), bf16_dev(vc, dev),
                                            tdev, plan, items, scale, po, pl)
    return f32_of(out), po.cpu().numpy(), pl.cpu().numpy(), plan.cpu().numpy()


@pytest.mark.parametrize("lengths,bs,items,splits", [
    ([31075 // 8, 12494 // 8, 6639 // 8, 1, 0, 2000], 128, 24, 16),
    ([300], 32, 56, 8), ([0, 0], 128, 8, 4), ([5000, 17], 64, 3, 2),
    (list(range(0, 64 * 11, 11)), 32, 100, 8)])  # 64 sequences: every lane holds a length
def test_plan_records_match_oracle(ops, dev, lengths, bs, items, splits):
    rng = np.random.default_rng(len(lengths) * 7 + items)
    q, kc, vc, table = _case(rng, [max(L, 1) for L in lengths], bs)
    pos = [L - 1 for L in lengths]
    slots = [int(rng.integers(-1, 1 << 20)) for _ in lengths]
    _, _, _, plan = _planned(ops, dev, q, kc, vc, table, lengths, bs, items, splits,
                             HD ** -0.5, positions=pos, slots=slots)
    ref = oatt.plan_records(lengths, items, splits, table, bs, positions=pos, slots=slots)
    np.testing.assert_array_equal(plan.view(np.uint32), ref)


@pytest.mark.parametrize("lengths,bs,items,splits", [
    ([512, 3000, 77, 8192, 1, 0, 129], 128, 24, 16),
    ([512, 3000, 77, 8192, 1, 0, 129], 32, 56, 64),
    ([6144], 128, 49, 64), ([20000], 32, 1, 1), ([9000, 40], 128, 2, 2),
    ([32768, 1, 20000], 128, 88, 16), (list(range(0, 64 * 11, 11)), 32, 100, 8),
    # records (items + sequences) a multiple of 8: the records-fastest grid
    ([512, 3000, 77, 8192, 1, 0, 129], 128, 25, 16), ([32768, 1, 20000], 128, 85, 16),
    (list(range(0, 64 * 11, 11)), 32, 64, 8)])
def test_planned_vs_fp64(ops, dev, lengths, bs, items, splits):
    """Merged outputs against float64 attention, every split's partial against
    the oracle's online softmax over the plan's bounds, and the slots no
    split writes cleared to (0, -inf).  ([20000] with 32-token pages and one
    split: the waves' pages beyond the record's 55 come from the table.)
    Plans whose record count is a multiple of 8 launch records fastest (all
    kv heads of a record on one XCD), the others kv heads fastest."""
    rng = np.random.default_rng(sum(lengths) + items)
    q, kc, vc, table = _case(rng, [max(L, 1) for L in lengths], bs)
    scale = HD ** -0.5
    out, po, pl, _ = _planned(ops, dev, q, kc, vc, table, lengths, bs, items, splits, scale)
    qf, kf, vf = (bf16_bits_to_f32(a) for a in (q, kc, vc))
    out = out.reshape(len(lengths), N_Q, HD)
    _, sp = oatt.plan_splits(lengths, items, splits, table.shape[1] * bs)
    for i, L in enumerate(lengths):
        if L == 0:
            assert np.all(out[i] == 0)
        else:
            k = oatt.gather_paged(kf, table[i], L)
            v = oatt.gather_paged(vf, table[i], L)
            ref = oatt.attention_f64(qf[i], k, v, scale)
            assert_attention_close(out[i], ref, f"sequence {i} (L={L})")
            opo, opl = oatt.splitkv_partials(qf[i], k, v, scale, sp[i])
            n = len(sp[i])
            assert_partials_close(po[i, :n], pl[i, :n], opo, opl, f"sequence {i} partials")
        n = len(sp[i])
        assert np.all(po[i, n:] == 0) and np.all(pl[i, n:] == -np.inf), f"sequence {i} unused slots"


def test_planned_page_permutation_invariance(ops, dev):
    rng = np.random.default_rng(18)
    lengths, bs = [1500, 700], 128
    q, kc, vc, table = _case(rng, lengths, bs, extra_blocks=0)
    perm = rng.permutation(kc.shape[0])
    inv = np.argsort(perm)
    table2 = table.copy()
    for i, L in enumerate(lengths):
        nb = -(-L // bs)
        table2[i, :nb] = inv[table[i, :nb]]
    a = _planned(ops, dev, q, kc, vc, table, lengths, bs, 5, 8, HD ** -0.5)[0]
    b = _planned(ops, dev, q, kc[perm], vc[perm], table2, lengths, bs, 5, 8, HD ** -0.5)[0]
    np.testing.assert_array_equal(a, b)


def test_plan_rejects_bad_shapes(ops, dev):
    import torch
    SmxError = pkg("native").SmxError
    sl = torch.ones(65, dtype=torch.int32, device=dev)
    table = torch.zeros((65, 2), dtype=torch.int32, device=dev)
    po = torch.empty((65, 4, N_Q, HD), dtype=torch.float32, device=dev)
    pl = torch.empty((65, 4, N_Q), dtype=torch.float32, device=dev)
    with pytest.raises(SmxError, match="at most 64"):
        ops.splitkv_plan(sl, table, 128, 8, po, pl)


@pytest.mark.parametrize("planned", [False, True])
def test_backend_forward(dev, planned):
    """The vLLM-style backend: forward writes key/value at the slots and
    returns the merged attention, with capacity splits or with a plan built
    once for the step and shared by two layers' calls."""
    import torch
    att = pkg("integration.attention")
    rng = np.random.default_rng(21 + planned)
    lengths, bs = [700, 3000, 1], 128
    q, kc, vc, table = _case(rng, lengths, bs)
    backend = att.SplitKVDecodeBackend
    impl = backend.get_impl_cls()(N_Q, HD, HD ** -0.5, N_KV)
    kv = torch.stack([bf16_dev(kc, dev), bf16_dev(vc, dev)]).view(2, *kc.shape)
    slots = [int(table[i, (L - 1) // bs]) * bs + (L - 1) % bs for i, L in enumerate(lengths)]
    knew = randn_bf16(rng, (len(lengths), N_KV * HD))
    vnew = randn_bf16(rng, (len(lengths), N_KV * HD))
    items, splits = att.choose_plan(len(lengths), N_KV) if planned else (0, 8)
    md = att.SplitKVDecodeMetadata(
        block_tables=torch.from_numpy(table).to(dev),
        seq_lens=torch.tensor(lengths, dtype=torch.int32, device=dev),
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=dev), num_splits=splits,
        num_items=items)
    if planned:
        backend.plan(md, bs, N_Q, HD)
    outs = [impl.forward(None, bf16_dev(q, dev).view(len(lengths), -1), bf16_dev(knew, dev),
                         bf16_dev(vnew, dev), kv, md) for _ in range(2)]
    np.testing.assert_array_equal(f32_of(outs[0]), f32_of(outs[1]))
    kf = bf16_bits_to_f32(bits_of(kv[0]).reshape(kc.shape))
    vf = bf16_bits_to_f32(bits_of(kv[1]).reshape(vc.shape))
    qf = bf16_bits_to_f32(q)
    got = f32_of(outs[0]).reshape(len(lengths), N_Q, HD)
    for i, L in enumerate(lengths):
        blk, off = divmod(slots[i], bs)
        np.testing.assert_array_equal(bits_of(kv[0][blk, off]).reshape(-1), knew[i])
        ref = oatt.attention_f64(qf[i], oatt.gather_paged(kf, table[i], L),
                                 oatt.gather_paged(vf, table[i], L), HD ** -0.5)
        assert_attention_close(got[i], ref, f"sequence {i}")
