"""Paged GQA decode attention for the oracle -- test infrastructure.

attention_f64     textbook softmax(q K^T * scale) V in float64 over the
                  gathered, unpaged KV.  The reference for everything else.
splitkv_partials  the reference's split-KV online softmax, AttentionStage
                  (src/spark_vllm_ascend/kernels/attention.py:59-117): per
                  tile, m' = max(m, tile max); alpha = exp(m - m'); p =
                  exp(s - m') in fp32; sum = sum * alpha + sum(p); acc = acc *
                  alpha + bf16(p) V; partial = acc / sum, lse = log(sum) + m.
splitkv_partials_grouped  the same recurrence with all heads advanced
                  together (batched products), for long-context model runs;
                  agrees with splitkv_partials to fp32 rounding.
lse_merge        merge_attention (src/spark_vllm_ascend/kernels/vector.py:
                  45-83) without the output gate: w_s = exp(lse_s - max) /
                  sum, out = bf16(sum_s w_s o_s).
plan_splits       per-sequence splits from the live lengths (the task list
                  of execute_serial, src/spark_vllm_ascend/kernels/
                  attention.py:120-128: parts = ceil(length / width)), one
                  split length for the whole batch; plan_records lays them
                  out as the device plan's records.

Pins (tests/test_oracle_attention.py): split results merged equal the
unsplit fp64 result for every split count; one split equals the unsplit
result; ctx = 1 gives v_0; equal keys give the mean of V; permuting pages
through the block table leaves the result unchanged; a partially filled last
page masks its tail.  Plans: every sequence's splits tile [0, L) exactly, no
sequence has more than num_splits splits, the batch at most num_items +
num_seqs, the split length is the smallest multiple of 128 meeting both
bounds (checked by brute force over the multiples), and the merged planned
partials equal the unsplit fp64 result.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def gather_paged(cache: np.ndarray, table: np.ndarray, length: int) -> np.ndarray:
    """cache [num_blocks, bs, n_kv, hd] -> [length, n_kv, hd] in token order."""
    bs = cache.shape[1]
    nblk = (length + bs - 1) // bs
    pages = cache[np.asarray(table[:nblk], dtype=np.int64)]
    return pages.reshape(nblk * bs, *cache.shape[2:])[:length]


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """q [n_q, hd]; k, v [L, n_kv, hd] -> out [n_q, hd] (float64)."""
    n_q = q.shape[0]
    n_kv = k.shape[1]
    g = n_q // n_kv
    out = np.empty((n_q, q.shape[1]), dtype=np.float64)
    for h in range(n_q):
        kh = k[:, h // g, :].astype(np.float64)
        vh = v[:, h // g, :].astype(np.float64)
        s = kh @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = p @ vh / p.sum()
    return out


def split_bounds(length: int, num_splits: int, capacity: int | None = None, align: int = 32):
    """Token range of each split: T = align * ceil(ceil(C / S) / align) where
    C is the block table's capacity (default: the length itself); ranges are
    clipped to the length, so splits past it are empty."""
    cap = length if capacity is None else capacity
    per = -(-cap // num_splits)
    t = -(-per // align) * align
    return [(min(length, s * t), min(length, (s + 1) * t)) for s in range(num_splits)]


def splitkv_partials(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                     bounds, tile: int = 128):
    """Per split: (partial_o [S, n_q, hd] fp32, lse [S, n_q] fp32), -inf lse
    and zero output for an empty split."""
    n_q, hd = q.shape
    n_kv = k.shape[1]
    g = n_q // n_kv
    ns = len(bounds)
    po = np.zeros((ns, n_q, hd), dtype=np.float32)
    pl = np.full((ns, n_q), -np.inf, dtype=np.float32)
    qf = q.astype(np.float32)
    for si, (a, b) in enumerate(bounds):
        if a >= b:
            continue
        for h in range(n_q):
            kh = k[a:b, h // g, :].astype(np.float32)
            vh = v[a:b, h // g, :].astype(np.float32)
            m = np.float32(-np.inf)
            ssum = np.float32(0.0)
            acc = np.zeros(hd, dtype=np.float32)
            for t0 in range(0, b - a, tile):
                s = (kh[t0:t0 + tile] @ qf[h]).astype(np.float32) * np.float32(scale)
                mn = np.float32(max(m, s.max()))
                alpha = np.float32(np.exp(m - mn)) if np.isfinite(m) else np.float32(0.0)
                p = np.exp((s - mn).astype(np.float32)).astype(np.float32)
                ssum = np.float32(ssum * alpha + p.sum(dtype=np.float32))
                acc = (acc * alpha + round_bf16(p) @ vh[t0:t0 + tile]).astype(np.float32)
                m = mn
            po[si, h] = acc / ssum
            pl[si, h] = np.float32(np.log(ssum)) + m
    return po, pl


def splitkv_partials_grouped(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                             bounds, tile: int = 128):
    """splitkv_partials with every head advanced together (per tile, one
    batched fp32 matrix product over the kv heads, each kv head's group of q
    heads as its columns) instead of one product per q head: the same
    recurrence and rounding points, for long contexts where the per-head
    loop is slow.  Products are summed in BLAS order, so results agree with
    splitkv_partials to fp32 rounding, not bit for bit
    (tests/test_oracle_attention.py checks the agreement)."""
    n_q, hd = q.shape
    n_kv = k.shape[1]
    g = n_q // n_kv
    ns = len(bounds)
    po = np.zeros((ns, n_q, hd), dtype=np.float32)
    pl = np.full((ns, n_q), -np.inf, dtype=np.float32)
    qt = q.astype(np.float32).reshape(n_kv, g, hd).transpose(0, 2, 1)  # [n_kv, hd, g]
    sc = np.float32(scale)
    for si, (a, b) in enumerate(bounds):
        if a >= b:
            continue
        kk = np.ascontiguousarray(k[a:b].astype(np.float32).transpose(1, 0, 2))  # [n_kv, t, hd]
        vv = np.ascontiguousarray(v[a:b].astype(np.float32).transpose(1, 0, 2))
        m = np.full((n_kv, g), -np.inf, dtype=np.float32)
        ssum = np.zeros((n_kv, g), dtype=np.float32)
        acc = np.zeros((n_kv, g, hd), dtype=np.float32)
        for t0 in range(0, b - a, tile):
            s = (kk[:, t0:t0 + tile] @ qt).astype(np.float32) * sc          # [n_kv, t, g]
            mn = np.maximum(m, s.max(axis=1)).astype(np.float32)
            with np.errstate(invalid="ignore"):
                alpha = np.where(np.isfinite(m), np.exp(m - mn), 0.0).astype(np.float32)
            p = np.exp((s - mn[:, None, :]).astype(np.float32)).astype(np.float32)
            ssum = (ssum * alpha + p.sum(axis=1, dtype=np.float32)).astype(np.float32)
            pv = round_bf16(p).transpose(0, 2, 1) @ vv[:, t0:t0 + tile]     # [n_kv, g, hd]
            acc = (acc * alpha[:, :, None] + pv).astype(np.float32)
            m = mn
        po[si] = (acc / ssum[:, :, None]).reshape(n_q, hd)
        pl[si] = (np.log(ssum).astype(np.float32) + m).reshape(n_q)
    return po, pl


def lse_merge(po: np.ndarray, pl: np.ndarray) -> np.ndarray:
    """(partial_o [S, n_q, hd], lse [S, n_q]) -> bf16-rounded float32 [n_q, hd]."""
    mx = pl.max(axis=0)
    z = np.where(np.isfinite(pl), np.exp((pl - mx).astype(np.float32)), 0.0).astype(np.float32)
    w = (z / z.sum(axis=0)).astype(np.float32)
    acc = np.einsum("sh,shd->hd", w, po).astype(np.float32)
    return round_bf16(acc)


def splitkv_decode(q, k_cache, v_cache, table, length, num_splits, scale, tile=128):
    """Paged convenience wrapper: gather, split (over the table's capacity),
    merge."""
    k = gather_paged(k_cache, table, length)
    v = gather_paged(v_cache, table, length)
    cap = len(table) * k_cache.shape[1]
    po, pl = splitkv_partials(q, k, v, scale, split_bounds(length, num_splits, cap), tile)
    return lse_merge(po, pl), po, pl


PLAN_WORDS = 64   # uint32 words per plan record
PLAN_PAGE0 = 9    # record words 9..63: pages from the split's first token on
PLAN_HAS_POSITIONS = 1 << 31  # word 3 flag: the record carries a position and a slot
PLAN_ALIGN = 128  # split lengths are multiples of this


def plan_splits(lengths, num_items: int, num_splits: int, capacity: int,
                align: int = PLAN_ALIGN):
    """One split length for the batch,
    chunk = align * ceil(max(ceil(T / num_items), ceil(max L / num_splits), 1) / align)
    with L = min(length, capacity) and T = sum L; sequence r gets the splits
    [j chunk, min(L_r, (j + 1) chunk)) for j < ceil(L_r / chunk).
    Returns (chunk, [[(begin, end), ...] per sequence])."""
    L = [min(max(int(x), 0), capacity) for x in lengths]
    total, lmax = sum(L), max(L)
    chunk = max(-(-total // num_items), -(-lmax // num_splits), 1)
    chunk = -(-chunk // align) * align
    return chunk, [[(j * chunk, min(l, (j + 1) * chunk)) for j in range(-(-l // chunk))]
                   for l in L]


def plan_records(lengths, num_items: int, num_splits: int, table: np.ndarray, block_size: int,
                 positions=None, slots=None) -> np.ndarray:
    """The plan's records, [num_items + num_seqs, PLAN_WORDS] uint32: per
    split (numbered sequence by sequence) the sequence, first / end token,
    split index (bit 31 set when positions and slots were both given:
    the record can drive the fused q/k-norm + RoPE + KV-write kernel),
    length, position and slot (int64 as two little-endian words; 0 and -1
    when not given) and the block-table entries from the first token's page
    on (indices clamped to the table row); past the last split, records
    with sequence -1 and zeros."""
    table = np.asarray(table)
    cap = table.shape[1] * block_size
    _, splits = plan_splits(lengths, num_items, num_splits, cap)
    nrec = num_items + len(lengths)
    rec = np.zeros((nrec, PLAN_WORDS), dtype=np.uint32)
    rec[:, 0] = 0xFFFFFFFF
    b = 0
    for r, sp in enumerate(splits):
        L = min(max(int(lengths[r]), 0), cap)
        p = int(positions[r]) if positions is not None else 0
        s = int(slots[r]) if slots is not None else -1
        for j, (tb, te) in enumerate(sp):
            flag = PLAN_HAS_POSITIONS if positions is not None and slots is not None else 0
            head = [r, tb, te, j | flag, L, p & 0xFFFFFFFF, (p >> 32) & 0xFFFFFFFF,
                    s & 0xFFFFFFFF, (s >> 32) & 0xFFFFFFFF]
            rec[b, :PLAN_PAGE0] = head
            idx = np.minimum(tb // block_size + np.arange(PLAN_WORDS - PLAN_PAGE0),
                             table.shape[1] - 1)
            rec[b, PLAN_PAGE0:] = table[r, idx].astype(np.int64) & 0xFFFFFFFF
            b += 1
    assert b <= nrec
    return rec
