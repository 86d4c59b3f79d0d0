"""Pins for the oracle's split-KV attention (CPU only): invariants that any
correct implementation satisfies, checked against the float64 textbook
attention, which is itself checked on hand-computable cases."""
import numpy as np
import pytest

from oracle import attention as oatt
from oracle.bf16 import round_bf16


def rand_case(rng, L, n_q=8, n_kv=2, hd=128):
    q = round_bf16(rng.standard_normal((n_q, hd)).astype(np.float32))
    k = round_bf16(rng.standard_normal((L, n_kv, hd)).astype(np.float32))
    v = round_bf16(rng.standard_normal((L, n_kv, hd)).astype(np.float32))
    return q, k, v


def test_textbook_two_tokens_by_hand():
    q = np.zeros((4, 2), np.float32)
    q[:, 0] = 1.0
    k = np.array([[[0.0, 0.0]], [[np.log(3.0), 0.0]]], np.float32)  # scores 0, log 3
    v = np.array([[[1.0, 0.0]], [[0.0, 1.0]]], np.float32)
    out = oatt.attention_f64(q, k, v, 1.0)
    np.testing.assert_allclose(out[0], [0.25, 0.75], rtol=1e-7)


def test_ctx_one_gives_v0():
    rng = np.random.default_rng(0)
    q, k, v = rand_case(rng, 1)
    out = oatt.attention_f64(q, k, v, 0.1)
    np.testing.assert_allclose(out, np.repeat(v[0], 4, axis=0), rtol=1e-12)
    po, pl = oatt.splitkv_partials(q, k, v, 0.1, oatt.split_bounds(1, 4))
    np.testing.assert_allclose(round_bf16(po[0]), np.repeat(v[0], 4, axis=0), rtol=1e-2)


@pytest.mark.parametrize("L", [5, 31, 32, 33, 300, 1000])
@pytest.mark.parametrize("S", [1, 2, 3, 4, 8, 16, 32])
def test_split_count_invariance(L, S):
    rng = np.random.default_rng(L * 100 + S)
    q, k, v = rand_case(rng, L)
    ref = oatt.attention_f64(q, k, v, 128 ** -0.5)
    po, pl = oatt.splitkv_partials(q, k, v, 128 ** -0.5, oatt.split_bounds(L, S))
    out = oatt.lse_merge(po, pl)
    assert np.max(np.abs(out - ref)) < 1e-2


def test_split_bounds_cover_exactly():
    for L in (1, 31, 32, 33, 4096, 6144, 6145):
        for S in (1, 3, 4, 32, 64):
            for cap in (None, L + 100, 8192):
                b = oatt.split_bounds(L, S, cap)
                covered = [t for a, e in b for t in range(a, e)]
                assert covered == list(range(L))
                assert all(a % 32 == 0 for a, e in b if a < e)


def test_equal_keys_mean_of_values():
    rng = np.random.default_rng(2)
    q, k, v = rand_case(rng, 200)
    k[:] = k[0:1]
    ref = np.repeat(v.mean(axis=0), 4, axis=0)
    np.testing.assert_allclose(oatt.attention_f64(q, k, v, 0.2), ref, rtol=1e-6, atol=1e-6)
    po, pl = oatt.splitkv_partials(q, k, v, 0.2, oatt.split_bounds(200, 3))
    assert np.max(np.abs(oatt.lse_merge(po, pl) - ref)) < 1e-2


def test_paging_and_permutation_invariance():
    rng = np.random.default_rng(3)
    L, bs, nblk = 300, 32, 12
    kc = round_bf16(rng.standard_normal((nblk, bs, 2, 128)).astype(np.float32))
    vc = round_bf16(rng.standard_normal((nblk, bs, 2, 128)).astype(np.float32))
    q = round_bf16(rng.standard_normal((8, 128)).astype(np.float32))
    table = rng.permutation(nblk)[:10]
    a, _, _ = oatt.splitkv_decode(q, kc, vc, table, L, 4, 0.1)
    perm = rng.permutation(nblk)
    inv = np.argsort(perm)
    b, _, _ = oatt.splitkv_decode(q, kc[perm], vc[perm], inv[table], L, 4, 0.1)
    np.testing.assert_array_equal(a, b)
    # the partially filled last page: tokens >= L are ignored
    kc2 = kc.copy()
    last = table[L // bs]
    kc2[last, L % bs:] = 1e4
    c, _, _ = oatt.splitkv_decode(q, kc2, vc, table, L, 4, 0.1)
    np.testing.assert_array_equal(a, c)


def test_lse_of_single_split_is_logsumexp():
    rng = np.random.default_rng(4)
    q, k, v = rand_case(rng, 64)
    po, pl = oatt.splitkv_partials(q, k, v, 0.3, [(0, 64)])
    for h in range(8):
        s = (k[:, h // 4, :].astype(np.float64) @ q[h].astype(np.float64)) * 0.3
        lse = np.log(np.sum(np.exp(s - s.max()))) + s.max()
        assert abs(pl[0, h] - lse) < 1e-4


PLAN_CASES = [([31075, 12494, 6639, 12989, 6118, 15990, 11664, 18505], 56, 16, 32896),
              ([1], 56, 16, 128), ([0, 0, 0], 8, 4, 1024), ([512, 3000, 77, 8192, 1, 0], 24, 32, 8320),
              ([40000, 10], 8, 4, 32768), ([5, 6, 7], 1, 1, 256), ([4096] * 64, 200, 8, 4096)]


@pytest.mark.parametrize("lengths,items,splits,cap", PLAN_CASES)
def test_plan_splits_tile_and_bounds(lengths, items, splits, cap):
    chunk, sp = oatt.plan_splits(lengths, items, splits, cap)
    L = [min(max(x, 0), cap) for x in lengths]
    for l, s in zip(L, sp):
        assert [t for a, e in s for t in range(a, e)] == list(range(l))
        assert all(a % oatt.PLAN_ALIGN == 0 and e - a <= chunk for a, e in s)
        assert len(s) <= splits
    assert sum(len(s) for s in sp) <= items + len(lengths)
    # chunk is the smallest multiple of 128 meeting both bounds (brute force)
    ok = lambda c: c * items >= sum(L) and c * splits >= max(L) and c >= 1
    assert ok(chunk) and chunk % 128 == 0
    assert not any(ok(c) for c in range(128, chunk, 128))


def test_plan_records_layout():
    table = np.arange(3 * 70, dtype=np.int32).reshape(3, 70)
    rec = oatt.plan_records([300, 0, 8000], 4, 8, table, 128, positions=[299, -1, 7999],
                            slots=[5, -1, 1 << 33])
    # chunk = 128 * ceil(max(ceil(8300 / 4), ceil(8000 / 8)) / 128) = 2176
    F = oatt.PLAN_HAS_POSITIONS  # word 3 flag: positions and slots were given
    assert rec.shape == (7, oatt.PLAN_WORDS)
    assert rec[0, :5].tolist() == [0, 0, 300, F, 300]
    assert rec[0, 5:9].tolist() == [299, 0, 5, 0]
    assert rec[0, 9:12].tolist() == [0, 1, 2]
    assert rec[1, :5].tolist() == [2, 0, 2176, F, 8000]
    assert rec[1, 7:9].tolist() == [0, 2]                  # slot 2^33
    assert rec[4, :5].tolist() == [2, 6528, 8000, 3 | F, 8000]
    assert rec[4, 9] == 140 + 6528 // 128                   # page of token 6528
    assert rec[4, -1] == 140 + 69                           # clamped to the row's end
    assert rec[5, 0] == 0xFFFFFFFF and not rec[5, 1:].any()  # unused
    # without positions (or without slots) no record carries the flag
    for kw in ({}, {"positions": [299, -1, 7999]}, {"slots": [5, -1, 1 << 33]}):
        bare = oatt.plan_records([300, 0, 8000], 4, 8, table, 128, **kw)
        assert bare[0, 3] == 0 and bare[4, 3] == 3
        assert bare[0, 5:7].tolist() == ([299, 0] if "positions" in kw else [0, 0])


@pytest.mark.parametrize("lengths,items,splits", [([700, 33, 1], 6, 4), ([2000, 500], 3, 8)])
def test_planned_partials_merge_to_unsplit(lengths, items, splits):
    rng = np.random.default_rng(sum(lengths))
    _, sp = oatt.plan_splits(lengths, items, splits, 4096)
    for L, bounds in zip(lengths, sp):
        q, k, v = rand_case(rng, L)
        ref = oatt.attention_f64(q, k, v, 128 ** -0.5)
        po, pl = oatt.splitkv_partials(q, k, v, 128 ** -0.5, bounds)
        assert np.max(np.abs(oatt.lse_merge(po, pl) - ref)) < 1e-2


@pytest.mark.parametrize("L,S", [(1, 4), (33, 3), (300, 2), (1000, 8), (2500, 5)])
def test_grouped_partials_agree_with_per_head(L, S):
    """The grouped restatement (q heads of a kv head advanced together, for
    long contexts) follows the per-head recurrence: same empty splits, lse
    within a few fp32 ulps, partials within fp32 rounding of each other."""
    rng = np.random.default_rng(L + 7 * S)
    q, k, v = rand_case(rng, L)
    b = oatt.split_bounds(L, S)
    po, pl = oatt.splitkv_partials(q, k, v, 128 ** -0.5, b)
    gpo, gpl = oatt.splitkv_partials_grouped(q, k, v, 128 ** -0.5, b)
    fin = np.isfinite(pl)
    np.testing.assert_array_equal(np.isfinite(gpl), fin)
    np.testing.assert_allclose(gpl[fin], pl[fin], rtol=1e-6, atol=1e-6)
    # a bf16 rounding of p may flip when the scores differ in their last bit
    np.testing.assert_allclose(gpo, po, rtol=0, atol=4e-3 * np.abs(po).max())
    assert np.linalg.norm(gpo - po) <= 1e-3 * np.linalg.norm(po)
    assert np.all(gpo[~fin] == 0)
