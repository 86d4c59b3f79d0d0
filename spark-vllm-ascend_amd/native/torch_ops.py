"""Torch-tensor wrappers over the C ABI (the role of the reference's
TORCH_LIBRARY wrapper, src/spark_vllm_ascend/native/head/extension.cpp:6-14).

Each wrapper checks device, dtype, contiguity and element counts before the
call (raising ValueError, as TORCH_CHECK raises c10::Error), passes raw data
pointers plus the current HIP stream of the tensor's device, and returns the
output tensor.  Outputs can be passed in (``out=``) so that a captured graph
reuses fixed buffers; otherwise they are freshly allocated, as the
reference's custom ops do (src/spark_vllm_ascend/integration/head.py:8-9).
"""
from __future__ import annotations

import torch

from . import call

BF16 = torch.bfloat16


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _check(t: torch.Tensor, name: str, dtype: torch.dtype, numel: int | None = None,
           device: torch.device | None = None) -> None:
    _need(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _need(t.is_cuda, f"{name} must be on a GPU device")
    _need(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _need(t.is_contiguous(), f"{name} must be contiguous")
    if numel is not None:
        _need(t.numel() == numel, f"{name} must have {numel} elements, got {t.numel()}")
    if device is not None:
        _need(t.device == device, f"{name} must be on {device}, got {t.device}")


def q4_0_row_bytes(k: int) -> int:
    """Bytes of one Q4_0 row of k weights (k/32 blocks of 18 bytes)."""
    return k // 32 * 18


def q4_0_dequant_bf16(w: torch.Tensor, n: int, k: int, out: torch.Tensor | None = None) -> torch.Tensor:
    _need(k % 32 == 0 and k > 0 and n > 0, "need n > 0 and k a positive multiple of 32")
    _check(w, "w", torch.uint8, n * q4_0_row_bytes(k))
    if out is None:
        out = torch.empty((n, k), dtype=BF16, device=w.device)
    _check(out, "out", BF16, n * k, w.device)
    call("smx_q4_0_dequant_bf16", _stream(w), w.data_ptr(), out.data_ptr(), n, k)
    return out


def q4_0_gemv(x: torch.Tensor, w: torch.Tensor, n: int, k: int,
              out: torch.Tensor | None = None) -> torch.Tensor:
    _need(k % 32 == 0 and k > 0 and n > 0, "need n > 0 and k a positive multiple of 32")
    _check(x, "x", BF16, k)
    _check(w, "w", torch.uint8, n * q4_0_row_bytes(k), x.device)
    if out is None:
        out = torch.empty((1, n), dtype=BF16, device=x.device)
    _check(out, "out", BF16, n, x.device)
    call("smx_q4_0_gemv", _stream(x), x.data_ptr(), w.data_ptr(), out.data_ptr(), n, k)
    return out


GELU_LUT_ENTRIES = 4096


def gelu_table(device: torch.device | str = "cpu") -> torch.Tensor:
    """The reference's erf-GELU activation table (src/spark_vllm_ascend/
    integration/model.py:13-16): gelu(approximate='none') of the bf16 bit
    patterns 0x3b00..0x42ff, then of 0xbb00..0xc2ff, as 4096 bf16 values.
    Evaluated by torch on the CPU (the reference evaluates it on its device),
    then copied to `device`."""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(BF16)
    full = torch.nn.functional.gelu(bits, approximate="none")
    return torch.cat((full[0x3B00:0x4300], full[0xBB00:0xC300])).contiguous().to(device)


def _lut_checked(lut: torch.Tensor, device: torch.device) -> int:
    _check(lut, "lut", BF16, GELU_LUT_ENTRIES, device)
    return lut.data_ptr()


def _gemv_gated(x, w, d, k, out, lut):
    _need(k % 32 == 0 and k > 0 and d > 0, "need d > 0 and k a positive multiple of 32")
    _check(x, "x", BF16, k)
    _check(w, "w", torch.uint8, 2 * d * q4_0_row_bytes(k), x.device)
    if out is None:
        out = torch.empty((1, d), dtype=BF16, device=x.device)
    _check(out, "out", BF16, d, x.device)
    if lut is None:
        call("smx_q4_0_gemv_swiglu", _stream(x), x.data_ptr(), w.data_ptr(), out.data_ptr(), d, k)
    else:
        call("smx_q4_0_gemv_gelu", _stream(x), x.data_ptr(), w.data_ptr(),
             _lut_checked(lut, x.device), out.data_ptr(), d, k)
    return out


def q4_0_gemv_swiglu(x: torch.Tensor, w: torch.Tensor, d: int, k: int,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    return _gemv_gated(x, w, d, k, out, None)


def q4_0_gemv_gelu(x: torch.Tensor, w: torch.Tensor, lut: torch.Tensor, d: int, k: int,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """out [1, d] = act(x W_gate^T) * (x W_up^T), act the table GELU
    (gelu_table)."""
    return _gemv_gated(x, w, d, k, out, lut)


def splitkv_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   block_table: torch.Tensor, seq_lens: torch.Tensor, num_splits: int,
                   scale: float, partial_o: torch.Tensor | None = None,
                   partial_lse: torch.Tensor | None = None):
    """Split-KV partials.  q [S, n_q, 128]; caches [blocks, bs, n_kv, 128]."""
    _need(q.dim() == 3 and k_cache.dim() == 4, "q must be [seqs, n_q, hd], caches 4-D")
    num_seqs, n_q, hd = q.shape
    num_blocks, bs, n_kv, hd2 = k_cache.shape
    _need(hd == hd2, "head_dim mismatch between q and the cache")
    _need(tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ")
    _check(q, "q", BF16)
    _check(k_cache, "k_cache", BF16, device=q.device)
    _check(v_cache, "v_cache", BF16, device=q.device)
    _check(block_table, "block_table", torch.int32, device=q.device)
    _need(block_table.dim() == 2 and block_table.shape[0] == num_seqs, "block_table must be [seqs, max_blocks]")
    _check(seq_lens, "seq_lens", torch.int32, num_seqs, q.device)
    if partial_o is None:
        partial_o = torch.empty((num_seqs, num_splits, n_q, hd), dtype=torch.float32, device=q.device)
    if partial_lse is None:
        partial_lse = torch.empty((num_seqs, num_splits, n_q), dtype=torch.float32, device=q.device)
    _check(partial_o, "partial_o", torch.float32, num_seqs * num_splits * n_q * hd, q.device)
    _check(partial_lse, "partial_lse", torch.float32, num_seqs * num_splits * n_q, q.device)
    call("smx_splitkv_decode", _stream(q), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
         block_table.data_ptr(), seq_lens.data_ptr(), partial_o.data_ptr(), partial_lse.data_ptr(),
         num_seqs, num_splits, block_table.shape[1], num_blocks, bs, n_q, n_kv, hd, float(scale))
    return partial_o, partial_lse


def splitkv_decode_merged(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                          block_table: torch.Tensor, seq_lens: torch.Tensor, num_splits: int,
                          scale: float, partial_o: torch.Tensor, partial_lse: torch.Tensor,
                          out: torch.Tensor | None = None) -> torch.Tensor:
    """Split-KV decode then the LSE merge, enqueued by one call; partial_o /
    partial_lse are the workspace between the two kernels."""
    _need(q.dim() == 3 and k_cache.dim() == 4, "q must be [seqs, n_q, hd], caches 4-D")
    num_seqs, n_q, hd = q.shape
    num_blocks, bs, n_kv, hd2 = k_cache.shape
    _need(hd == hd2, "head_dim mismatch between q and the cache")
    _need(tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ")
    _check(q, "q", BF16)
    _check(k_cache, "k_cache", BF16, device=q.device)
    _check(v_cache, "v_cache", BF16, device=q.device)
    _check(block_table, "block_table", torch.int32, device=q.device)
    _need(block_table.dim() == 2 and block_table.shape[0] == num_seqs, "block_table must be [seqs, max_blocks]")
    _check(seq_lens, "seq_lens", torch.int32, num_seqs, q.device)
    _check(partial_o, "partial_o", torch.float32, num_seqs * num_splits * n_q * hd, q.device)
    _check(partial_lse, "partial_lse", torch.float32, num_seqs * num_splits * n_q, q.device)
    if out is None:
        out = torch.empty((num_seqs, n_q, hd), dtype=BF16, device=q.device)
    _check(out, "out", BF16, num_seqs * n_q * hd, q.device)
    call("smx_splitkv_decode_merged", _stream(q), q.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(), partial_o.data_ptr(),
         partial_lse.data_ptr(), out.data_ptr(), num_seqs, num_splits,
         block_table.shape[1], num_blocks, bs, n_q, n_kv, hd, float(scale))
    return out


def lse_merge(partial_o: torch.Tensor, partial_lse: torch.Tensor,
              out: torch.Tensor | None = None) -> torch.Tensor:
    _need(partial_o.dim() == 4, "partial_o must be [seqs, splits, n_q, hd]")
    num_seqs, num_splits, n_q, hd = partial_o.shape
    _check(partial_o, "partial_o", torch.float32)
    _check(partial_lse, "partial_lse", torch.float32, num_seqs * num_splits * n_q, partial_o.device)
    if out is None:
        out = torch.empty((num_seqs, n_q, hd), dtype=BF16, device=partial_o.device)
    _check(out, "out", BF16, num_seqs * n_q * hd, partial_o.device)
    call("smx_lse_merge", _stream(partial_o), partial_o.data_ptr(), partial_lse.data_ptr(),
         out.data_ptr(), num_seqs, num_splits, n_q, hd)
    return out


PLAN_WORDS = 64  # uint32 words per split-plan record (SMX_SPLITKV_PLAN_WORDS)


def splitkv_plan(seq_lens: torch.Tensor, block_table: torch.Tensor, block_size: int,
                 num_items: int, partial_o: torch.Tensor, partial_lse: torch.Tensor,
                 positions: torch.Tensor | None = None, slot_mapping: torch.Tensor | None = None,
                 plan: torch.Tensor | None = None) -> torch.Tensor:
    """Per-sequence split plan from the live lengths (device-side; one call
    per decode step serves every layer).  partial_o [seqs, num_splits, n_q,
    hd] / partial_lse fix num_splits and must be the buffers the planned
    attention calls use: slots no split writes are cleared here.  Returns
    the plan, int32 [num_items + seqs, PLAN_WORDS] (uint32 words)."""
    num_seqs = seq_lens.numel()
    _need(partial_o.dim() == 4 and partial_o.shape[0] == num_seqs,
          "partial_o must be [seqs, splits, n_q, hd]")
    _, num_splits, n_q, hd = partial_o.shape
    _check(seq_lens, "seq_lens", torch.int32, num_seqs)
    _check(block_table, "block_table", torch.int32, device=seq_lens.device)
    _need(block_table.dim() == 2 and block_table.shape[0] == num_seqs, "block_table must be [seqs, max_blocks]")
    _check(partial_o, "partial_o", torch.float32, device=seq_lens.device)
    _check(partial_lse, "partial_lse", torch.float32, num_seqs * num_splits * n_q, seq_lens.device)
    for t, name in ((positions, "positions"), (slot_mapping, "slot_mapping")):
        if t is not None:
            _check(t, name, torch.int64, num_seqs, seq_lens.device)
    nrec = num_items + num_seqs
    if plan is None:
        plan = torch.empty((nrec, PLAN_WORDS), dtype=torch.int32, device=seq_lens.device)
    _check(plan, "plan", torch.int32, nrec * PLAN_WORDS, seq_lens.device)
    call("smx_splitkv_plan", _stream(seq_lens), seq_lens.data_ptr(), _ptr(positions),
         _ptr(slot_mapping), block_table.data_ptr(), plan.data_ptr(), partial_o.data_ptr(),
         partial_lse.data_ptr(), num_seqs, num_items, num_splits, block_table.shape[1],
         block_size, n_q, hd)
    return plan


def splitkv_decode_planned_merged(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                  block_table: torch.Tensor, plan: torch.Tensor, num_items: int,
                                  scale: float, partial_o: torch.Tensor, partial_lse: torch.Tensor,
                                  out: torch.Tensor | None = None) -> torch.Tensor:
    """splitkv_decode_merged over the splits of a plan (splitkv_plan with the
    same block table, num_items and partial buffers)."""
    _need(q.dim() == 3 and k_cache.dim() == 4, "q must be [seqs, n_q, hd], caches 4-D")
    num_seqs, n_q, hd = q.shape
    num_blocks, bs, n_kv, hd2 = k_cache.shape
    _need(hd == hd2, "head_dim mismatch between q and the cache")
    _need(tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ")
    _check(q, "q", BF16)
    _check(k_cache, "k_cache", BF16, device=q.device)
    _check(v_cache, "v_cache", BF16, device=q.device)
    _check(block_table, "block_table", torch.int32, device=q.device)
    _need(block_table.dim() == 2 and block_table.shape[0] == num_seqs, "block_table must be [seqs, max_blocks]")
    _check(plan, "plan", torch.int32, (num_items + num_seqs) * PLAN_WORDS, q.device)
    _need(partial_o.dim() == 4 and partial_o.shape[0] == num_seqs, "partial_o must be [seqs, splits, n_q, hd]")
    num_splits = partial_o.shape[1]
    _check(partial_o, "partial_o", torch.float32, num_seqs * num_splits * n_q * hd, q.device)
    _check(partial_lse, "partial_lse", torch.float32, num_seqs * num_splits * n_q, q.device)
    if out is None:
        out = torch.empty((num_seqs, n_q, hd), dtype=BF16, device=q.device)
    _check(out, "out", BF16, num_seqs * n_q * hd, q.device)
    call("smx_splitkv_decode_planned_merged", _stream(q), q.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), block_table.data_ptr(), plan.data_ptr(), partial_o.data_ptr(),
         partial_lse.data_ptr(), out.data_ptr(), num_seqs, num_items, num_splits,
         block_table.shape[1], num_blocks, bs, n_q, n_kv, hd, float(scale))
    return out


def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor | None, gamma: torch.Tensor, eps: float,
                out: torch.Tensor | None = None, residual_out: torch.Tensor | None = None):
    """Returns (y, residual_out).  With residual=None: y = RMSNorm(x), residual_out = x."""
    _need(x.dim() >= 1, "x must have a hidden dimension")
    hidden = x.shape[-1]
    rows = x.numel() // hidden
    _check(x, "x", BF16)
    _check(gamma, "gamma", BF16, hidden, x.device)
    if residual is not None:
        _check(residual, "residual", BF16, x.numel(), x.device)
    if out is None:
        out = torch.empty_like(x)
    _check(out, "out", BF16, x.numel(), x.device)
    if residual is not None and residual_out is None:
        residual_out = torch.empty_like(x)
    if residual_out is not None:
        _check(residual_out, "residual_out", BF16, x.numel(), x.device)
    call("smx_add_rmsnorm", _stream(x), x.data_ptr(),
         residual.data_ptr() if residual is not None else None, gamma.data_ptr(), out.data_ptr(),
         residual_out.data_ptr() if residual_out is not None else None, rows, hidden, float(eps))
    return out, (residual_out if residual is not None else x)


def qknorm_rope_kv_write(qkv: torch.Tensor, q_gamma: torch.Tensor, k_gamma: torch.Tensor,
                         cos_sin: torch.Tensor, positions: torch.Tensor, slot_mapping: torch.Tensor,
                         k_cache: torch.Tensor, v_cache: torch.Tensor, n_q: int, n_kv: int,
                         eps: float, q_out: torch.Tensor | None = None) -> torch.Tensor:
    num_blocks, bs, n_kv2, hd = k_cache.shape
    _need(n_kv2 == n_kv, "cache kv-head count mismatch")
    num_tokens = positions.numel()
    _check(qkv, "qkv", BF16, num_tokens * (n_q + 2 * n_kv) * hd)
    _check(q_gamma, "q_gamma", BF16, hd, qkv.device)
    _check(k_gamma, "k_gamma", BF16, hd, qkv.device)
    _check(cos_sin, "cos_sin", BF16, device=qkv.device)
    _need(cos_sin.dim() == 2 and cos_sin.shape[1] == hd, "cos_sin must be [max_position, head_dim]")
    _check(positions, "positions", torch.int64, num_tokens, qkv.device)
    _check(slot_mapping, "slot_mapping", torch.int64, num_tokens, qkv.device)
    _check(k_cache, "k_cache", BF16, device=qkv.device)
    _check(v_cache, "v_cache", BF16, device=qkv.device)
    _need(tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ")
    if q_out is None:
        q_out = torch.empty((num_tokens, n_q, hd), dtype=BF16, device=qkv.device)
    _check(q_out, "q_out", BF16, num_tokens * n_q * hd, qkv.device)
    call("smx_qknorm_rope_kv_write", _stream(qkv), qkv.data_ptr(), q_gamma.data_ptr(),
         k_gamma.data_ptr(), cos_sin.data_ptr(), positions.data_ptr(), slot_mapping.data_ptr(),
         q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), num_tokens, n_q, n_kv, hd,
         num_blocks, bs, cos_sin.shape[0], float(eps))
    return q_out


def _gated_mul(gate_up, out, lut):
    _check(gate_up, "gate_up", BF16)
    d2 = gate_up.shape[-1]
    _need(d2 % 2 == 0, "last dimension must be even")
    rows = gate_up.numel() // d2
    if out is None:
        out = torch.empty((*gate_up.shape[:-1], d2 // 2), dtype=BF16, device=gate_up.device)
    _check(out, "out", BF16, rows * d2 // 2, gate_up.device)
    if lut is None:
        call("smx_silu_mul", _stream(gate_up), gate_up.data_ptr(), out.data_ptr(), rows, d2 // 2)
    else:
        call("smx_gelu_mul", _stream(gate_up), gate_up.data_ptr(),
             _lut_checked(lut, gate_up.device), out.data_ptr(), rows, d2 // 2)
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    return _gated_mul(gate_up, out, None)


def gelu_mul(gate_up: torch.Tensor, lut: torch.Tensor,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """The table GELU (gelu_table) of a [..., 2d] gate|up tensor times up."""
    return _gated_mul(gate_up, out, lut)


def embedding(table: torch.Tensor, ids: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    _check(table, "table", BF16)
    _need(table.dim() == 2, "table must be [vocab, hidden]")
    _check(ids, "ids", torch.int64, device=table.device)
    vocab, hidden = table.shape
    if out is None:
        out = torch.empty((ids.numel(), hidden), dtype=BF16, device=table.device)
    _check(out, "out", BF16, ids.numel() * hidden, table.device)
    call("smx_embedding", _stream(table), table.data_ptr(), ids.data_ptr(), out.data_ptr(),
         ids.numel(), vocab, hidden)
    return out


def argmax(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    _check(logits, "logits", BF16)
    vocab = logits.shape[-1]
    rows = logits.numel() // vocab
    if out is None:
        out = torch.empty((rows,), dtype=torch.int64, device=logits.device)
    _check(out, "out", torch.int64, rows, logits.device)
    call("smx_argmax_bf16", _stream(logits), logits.data_ptr(), rows, vocab, out.data_ptr())
    return out


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """key, value: [num_tokens, n_kv, head_dim]; caches [blocks, bs, n_kv, head_dim]."""
    num_blocks, bs, n_kv, hd = k_cache.shape
    num_tokens = slot_mapping.numel()
    _check(key, "key", BF16, num_tokens * n_kv * hd)
    _check(value, "value", BF16, num_tokens * n_kv * hd, key.device)
    _check(k_cache, "k_cache", BF16, device=key.device)
    _check(v_cache, "v_cache", BF16, device=key.device)
    _need(tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ")
    _check(slot_mapping, "slot_mapping", torch.int64, num_tokens, key.device)
    call("smx_reshape_and_cache", _stream(key), key.data_ptr(), value.data_ptr(),
         k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(), num_tokens, n_kv, hd,
         num_blocks, bs)


def decode_advance(next_ids: torch.Tensor, ids: torch.Tensor, positions: torch.Tensor,
                   seq_lens: torch.Tensor, slot_mapping: torch.Tensor, block_table: torch.Tensor,
                   block_size: int, tokens_out: torch.Tensor | None = None,
                   forced_ids: torch.Tensor | None = None,
                   forced_len: torch.Tensor | None = None,
                   argmax_keys: torch.Tensor | None = None,
                   embed_table: torch.Tensor | None = None,
                   embed_out: torch.Tensor | None = None) -> None:
    """forced_ids [rows, max_len] int64 with forced_len [rows] int32 on the
    device; tokens_out [rows, max_len] int64 (same max_len); argmax_keys
    [rows, num_keys] int64 from add_rmsnorm_gemv_argmax (next_ids is then
    written with the argmax); embed_table [vocab, hidden] bf16 with embed_out
    [rows, hidden]: the embedding rows of the new ids for the next step."""
    rows = ids.numel()
    _check(next_ids, "next_ids", torch.int64, rows)
    _check(ids, "ids", torch.int64, rows, next_ids.device)
    _check(positions, "positions", torch.int64, rows, next_ids.device)
    _check(seq_lens, "seq_lens", torch.int32, rows, next_ids.device)
    _check(slot_mapping, "slot_mapping", torch.int64, rows, next_ids.device)
    _check(block_table, "block_table", torch.int32, device=next_ids.device)
    _need(block_table.dim() == 2 and block_table.shape[0] == rows, "block_table must be [rows, max_blocks]")
    _need((forced_ids is None) == (forced_len is None), "forced_ids and forced_len go together")
    max_len = 0
    for name, t in (("tokens_out", tokens_out), ("forced_ids", forced_ids)):
        if t is not None:
            _check(t, name, torch.int64, device=next_ids.device)
            _need(t.dim() == 2 and t.shape[0] == rows, f"{name} must be [rows, max_len]")
            _need(max_len in (0, t.shape[1]), "tokens_out and forced_ids need the same max_len")
            max_len = t.shape[1]
    if forced_len is not None:
        _check(forced_len, "forced_len", torch.int32, rows, next_ids.device)
    num_keys = 0
    if argmax_keys is not None:
        _check(argmax_keys, "argmax_keys", torch.int64, device=next_ids.device)
        _need(argmax_keys.dim() == 2 and argmax_keys.shape[0] == rows, "argmax_keys must be [rows, n]")
        num_keys = argmax_keys.shape[1]
    _need((embed_table is None) == (embed_out is None), "embed_table and embed_out go together")
    vocab = hidden = 0
    if embed_table is not None:
        _check(embed_table, "embed_table", BF16, device=next_ids.device)
        _need(embed_table.dim() == 2, "embed_table must be [vocab, hidden]")
        vocab, hidden = embed_table.shape
        _check(embed_out, "embed_out", BF16, rows * hidden, next_ids.device)
    call("smx_decode_advance", _stream(ids), next_ids.data_ptr(),
         argmax_keys.data_ptr() if argmax_keys is not None else None, num_keys,
         forced_ids.data_ptr() if forced_ids is not None else None,
         forced_len.data_ptr() if forced_len is not None else None, ids.data_ptr(),
         positions.data_ptr(), seq_lens.data_ptr(), slot_mapping.data_ptr(), block_table.data_ptr(),
         tokens_out.data_ptr() if tokens_out is not None else None, rows, block_table.shape[1],
         block_size, max_len, _ptr(embed_table), _ptr(embed_out), vocab, hidden)


def _norm_gemv_checks(x, residual, gamma, residual_out, k):
    _check(x, "x", BF16, k)
    _check(gamma, "gamma", BF16, k, x.device)
    if residual is not None:
        _check(residual, "residual", BF16, k, x.device)
    if residual_out is not None:
        _check(residual_out, "residual_out", BF16, k, x.device)
        _need(residual_out.data_ptr() not in (x.data_ptr(),
                                               residual.data_ptr() if residual is not None else -1),
              "residual_out must not alias x or residual")


def _ptr(t):
    return t.data_ptr() if t is not None else None


def add_rmsnorm_gemv(x: torch.Tensor, residual: torch.Tensor | None, gamma: torch.Tensor,
                     w: torch.Tensor, n: int, k: int, eps: float,
                     residual_out: torch.Tensor | None = None,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """y = W . (RMSNorm(x + residual) * gamma); residual_out = bf16(x + residual)."""
    _norm_gemv_checks(x, residual, gamma, residual_out, k)
    _check(w, "w", torch.uint8, n * q4_0_row_bytes(k), x.device)
    if out is None:
        out = torch.empty((1, n), dtype=BF16, device=x.device)
    _check(out, "out", BF16, n, x.device)
    call("smx_q4_0_add_rmsnorm_gemv", _stream(x), x.data_ptr(), _ptr(residual), gamma.data_ptr(),
         _ptr(residual_out), w.data_ptr(), out.data_ptr(), n, k, float(eps))
    return out


def add_rmsnorm_gemv_swiglu(x: torch.Tensor, residual: torch.Tensor | None, gamma: torch.Tensor,
                            w: torch.Tensor, d: int, k: int, eps: float,
                            residual_out: torch.Tensor | None = None,
                            out: torch.Tensor | None = None,
                            lut: torch.Tensor | None = None) -> torch.Tensor:
    """add+RMSNorm, gate/up GEMV and SwiGLU -- or, given the GELU table
    (gelu_table) as lut, the reference's table GELU in place of SiLU."""
    _norm_gemv_checks(x, residual, gamma, residual_out, k)
    _check(w, "w", torch.uint8, 2 * d * q4_0_row_bytes(k), x.device)
    if out is None:
        out = torch.empty((1, d), dtype=BF16, device=x.device)
    _check(out, "out", BF16, d, x.device)
    if lut is None:
        call("smx_q4_0_add_rmsnorm_gemv_swiglu", _stream(x), x.data_ptr(), _ptr(residual),
             gamma.data_ptr(), _ptr(residual_out), w.data_ptr(), out.data_ptr(), d, k, float(eps))
    else:
        call("smx_q4_0_add_rmsnorm_gemv_gelu", _stream(x), x.data_ptr(), _ptr(residual),
             gamma.data_ptr(), _ptr(residual_out), w.data_ptr(), _lut_checked(lut, x.device),
             out.data_ptr(), d, k, float(eps))
    return out


def add_rmsnorm_gemv_gelu(x: torch.Tensor, residual: torch.Tensor | None, gamma: torch.Tensor,
                          w: torch.Tensor, lut: torch.Tensor, d: int, k: int, eps: float,
                          residual_out: torch.Tensor | None = None,
                          out: torch.Tensor | None = None) -> torch.Tensor:
    """NativeUp.execute as one launch: add+RMSNorm, gate/up GEMV, table GELU."""
    return add_rmsnorm_gemv_swiglu(x, residual, gamma, w, d, k, eps, residual_out, out, lut)


def argmax_keys_size(n: int, k: int) -> int:
    from . import load
    return int(load().smx_q4_0_argmax_keys_size(n, k))


def add_rmsnorm_gemv_argmax(x: torch.Tensor, residual: torch.Tensor | None, gamma: torch.Tensor,
                            w: torch.Tensor, n: int, k: int, eps: float, keys: torch.Tensor,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """Logits = W . RMSNorm(x + residual) * gamma, plus per-workgroup argmax
    keys [argmax_keys_size(n, k)] int64 for decode_advance."""
    _norm_gemv_checks(x, residual, gamma, None, k)
    _check(w, "w", torch.uint8, n * q4_0_row_bytes(k), x.device)
    _check(keys, "keys", torch.int64, device=x.device)
    if out is None:
        out = torch.empty((1, n), dtype=BF16, device=x.device)
    _check(out, "out", BF16, n, x.device)
    call("smx_q4_0_add_rmsnorm_gemv_argmax", _stream(x), x.data_ptr(), _ptr(residual),
         gamma.data_ptr(), w.data_ptr(), out.data_ptr(), keys.data_ptr(), keys.numel(), n, k,
         float(eps))
    return out


def qknorm_rope_splitkv_decode_merged(qkv: torch.Tensor, q_gamma: torch.Tensor,
                                      k_gamma: torch.Tensor, cos_sin: torch.Tensor,
                                      positions: torch.Tensor, slot_mapping: torch.Tensor,
                                      k_cache: torch.Tensor, v_cache: torch.Tensor,
                                      block_table: torch.Tensor, seq_lens: torch.Tensor,
                                      num_splits: int, scale: float, eps: float, n_q: int,
                                      partial_o: torch.Tensor, partial_lse: torch.Tensor,
                                      out: torch.Tensor | None = None) -> torch.Tensor:
    """q/k RMSNorm + RoPE + KV write + split-KV decode + merge for one decode
    token per sequence (qkv: raw QKV projection [num_seqs, (n_q+2n_kv)*hd])."""
    num_blocks, bs, n_kv, hd = k_cache.shape
    num_seqs = seq_lens.numel()
    _check(qkv, "qkv", BF16, num_seqs * (n_q + 2 * n_kv) * hd)
    _check(q_gamma, "q_gamma", BF16, hd, qkv.device)
    _check(k_gamma, "k_gamma", BF16, hd, qkv.device)
    _check(cos_sin, "cos_sin", BF16, device=qkv.device)
    _need(cos_sin.dim() == 2 and cos_sin.shape[1] == hd, "cos_sin must be [max_position, head_dim]")
    _check(positions, "positions", torch.int64, num_seqs, qkv.device)
    _check(slot_mapping, "slot_mapping", torch.int64, num_seqs, qkv.device)
    _check(k_cache, "k_cache", BF16, device=qkv.device)
    _check(v_cache, "v_cache", BF16, device=qkv.device)
    _need(tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ")
    _check(block_table, "block_table", torch.int32, device=qkv.device)
    _need(block_table.dim() == 2 and block_table.shape[0] == num_seqs, "block_table must be [seqs, max_blocks]")
    _check(seq_lens, "seq_lens", torch.int32, num_seqs, qkv.device)
    _check(partial_o, "partial_o", torch.float32, num_seqs * num_splits * n_q * hd, qkv.device)
    _check(partial_lse, "partial_lse", torch.float32, num_seqs * num_splits * n_q, qkv.device)
    if out is None:
        out = torch.empty((num_seqs, n_q, hd), dtype=BF16, device=qkv.device)
    _check(out, "out", BF16, num_seqs * n_q * hd, qkv.device)
    call("smx_qknorm_rope_splitkv_decode_merged", _stream(qkv), qkv.data_ptr(), q_gamma.data_ptr(),
         k_gamma.data_ptr(), cos_sin.data_ptr(), positions.data_ptr(), slot_mapping.data_ptr(),
         k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(),
         partial_o.data_ptr(), partial_lse.data_ptr(), out.data_ptr(), num_seqs, num_splits,
         block_table.shape[1], num_blocks, bs, n_q, n_kv, hd, cos_sin.shape[0], float(eps),
         float(scale))
    return out


def qknorm_rope_splitkv_decode_planned_merged(qkv: torch.Tensor, q_gamma: torch.Tensor,
                                              k_gamma: torch.Tensor, cos_sin: torch.Tensor,
                                              k_cache: torch.Tensor, v_cache: torch.Tensor,
                                              block_table: torch.Tensor, plan: torch.Tensor,
                                              num_items: int, scale: float, eps: float, n_q: int,
                                              partial_o: torch.Tensor, partial_lse: torch.Tensor,
                                              out: torch.Tensor | None = None) -> torch.Tensor:
    """qknorm_rope_splitkv_decode_merged over the splits of a plan; the
    positions and slots come from the plan (splitkv_plan given them)."""
    num_blocks, bs, n_kv, hd = k_cache.shape
    num_seqs = block_table.shape[0]
    _check(qkv, "qkv", BF16, num_seqs * (n_q + 2 * n_kv) * hd)
    _check(q_gamma, "q_gamma", BF16, hd, qkv.device)
    _check(k_gamma, "k_gamma", BF16, hd, qkv.device)
    _check(cos_sin, "cos_sin", BF16, device=qkv.device)
    _need(cos_sin.dim() == 2 and cos_sin.shape[1] == hd, "cos_sin must be [max_position, head_dim]")
    _check(k_cache, "k_cache", BF16, device=qkv.device)
    _check(v_cache, "v_cache", BF16, device=qkv.device)
    _need(tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ")
    _check(block_table, "block_table", torch.int32, device=qkv.device)
    _need(block_table.dim() == 2, "block_table must be [seqs, max_blocks]")
    _check(plan, "plan", torch.int32, (num_items + num_seqs) * PLAN_WORDS, qkv.device)
    _need(partial_o.dim() == 4 and partial_o.shape[0] == num_seqs, "partial_o must be [seqs, splits, n_q, hd]")
    num_splits = partial_o.shape[1]
    _check(partial_o, "partial_o", torch.float32, num_seqs * num_splits * n_q * hd, qkv.device)
    _check(partial_lse, "partial_lse", torch.float32, num_seqs * num_splits * n_q, qkv.device)
    if out is None:
        out = torch.empty((num_seqs, n_q, hd), dtype=BF16, device=qkv.device)
    _check(out, "out", BF16, num_seqs * n_q * hd, qkv.device)
    call("smx_qknorm_rope_splitkv_decode_planned_merged", _stream(qkv), qkv.data_ptr(),
         q_gamma.data_ptr(), k_gamma.data_ptr(), cos_sin.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), block_table.data_ptr(), plan.data_ptr(), partial_o.data_ptr(),
         partial_lse.data_ptr(), out.data_ptr(), num_seqs, num_items, num_splits,
         block_table.shape[1], num_blocks, bs, n_q, n_kv, hd, cos_sin.shape[0], float(eps),
         float(scale))
    return out


def compute_slot_mapping(query_start_loc: torch.Tensor, positions: torch.Tensor,
                         block_table: torch.Tensor, block_size: int, max_tokens: int | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """int64 slots [max_tokens] of a ragged batch (-1 for padding and for
    positions past the block table)."""
    num_reqs = query_start_loc.numel() - 1
    _need(num_reqs >= 1, "query_start_loc needs num_reqs + 1 entries")
    _check(query_start_loc, "query_start_loc", torch.int32)
    _need(positions.dtype == torch.int64 and positions.device == query_start_loc.device
          and positions.is_contiguous(), "positions must be contiguous int64 on the same device")
    _check(block_table, "block_table", torch.int32, device=query_start_loc.device)
    _need(block_table.dim() == 2 and block_table.shape[0] >= num_reqs, "block_table must be [reqs, max_blocks]")
    num_tokens = positions.numel()
    max_tokens = num_tokens if max_tokens is None else max_tokens
    if out is None:
        out = torch.empty(max(max_tokens, 1), dtype=torch.int64, device=positions.device)
    _check(out, "out", torch.int64, device=positions.device)
    _need(out.numel() >= max_tokens, "out must hold max_tokens entries")
    pos_ptr = positions.data_ptr() if num_tokens else out.data_ptr()  # never read when empty
    call("smx_compute_slot_mapping", _stream(out), query_start_loc.data_ptr(), num_reqs,
         pos_ptr, block_table.data_ptr(), out.data_ptr(), num_tokens,
         max(max_tokens, 1), block_table.shape[1], block_size)
    return out


class PackedQ4_0:
    """A Q4_0 matrix in the packed layout of the MFMA GEMMs (smx_q4_0_repack):
    ``data`` uint8 [packed_bytes], the [n, k] matrix it holds (gated: the
    [2n, k] gate|up matrix, n = d).  q4_0_gemm, q4_0_gemm_swiglu and
    q4_0_gemm_argmax take one in place of the GGUF tensor."""

    __slots__ = ("data", "n", "k", "gated")

    def __init__(self, data: torch.Tensor, n: int, k: int, gated: bool):
        self.data, self.n, self.k, self.gated = data, int(n), int(k), bool(gated)


def q4_0_packed_bytes(n: int, k: int, gated: bool = False) -> int:
    """Bytes of the packed form of an [n, k] Q4_0 matrix (gated: [2n, k]);
    -1 when unsupported (k not a positive multiple of 256)."""
    from . import load
    return int(load().smx_q4_0_packed_bytes(n, k, 1 if gated else 0))


def q4_0_repack(w: torch.Tensor, n: int, k: int, gated: bool = False,
                out: torch.Tensor | None = None) -> PackedQ4_0:
    """Repack GGUF Q4_0 weights (n rows; gated: the 2n gate|up rows) into the
    packed layout; lossless (the same codes and fp16 scales, moved)."""
    nbytes = q4_0_packed_bytes(n, k, gated)
    _need(nbytes > 0, "the packed layout needs k a positive multiple of 256")
    _check(w, "w", torch.uint8, (2 * n if gated else n) * q4_0_row_bytes(k))
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    _check(out, "out", torch.uint8, nbytes, w.device)
    _need(out.data_ptr() % 16 == 0, "out must be 16-byte aligned")
    call("smx_q4_0_repack", _stream(w), w.data_ptr(), out.data_ptr(), n, k, 1 if gated else 0)
    return PackedQ4_0(out, n, k, gated)


def _gemm_x(x: torch.Tensor, k: int, align: int) -> None:
    _need(x.dim() == 2 and x.shape[1] == k and 1 <= x.shape[0] <= 16, "x must be [m <= 16, k]")
    _check(x, "x", BF16)
    _need(x.data_ptr() % align == 0, f"x must be {align}-byte aligned")


def _packed_checked(w: PackedQ4_0, n: int, k: int, gated: bool, device) -> int:
    _need(w.n == n and w.k == k and w.gated == gated,
          f"packed weights hold [{w.n}, {w.k}] (gated={w.gated}), the call wants [{n}, {k}] "
          f"(gated={gated})")
    _check(w.data, "w.data", torch.uint8, q4_0_packed_bytes(n, k, gated), device)
    return w.data.data_ptr()


def q4_0_gemm(x: torch.Tensor, w: torch.Tensor | PackedQ4_0, n: int, k: int,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """y [m, n] = x [m, k] . W^T for m <= 16 rows (MFMA kernel); W GGUF Q4_0
    or packed (q4_0_repack)."""
    packed = isinstance(w, PackedQ4_0)
    _gemm_x(x, k, 16 if packed else 8)
    if out is None:
        out = torch.empty((x.shape[0], n), dtype=BF16, device=x.device)
    _check(out, "out", BF16, x.shape[0] * n, x.device)
    if packed:
        call("smx_q4_0_gemm_packed", _stream(x), x.data_ptr(),
             _packed_checked(w, n, k, False, x.device), out.data_ptr(), x.shape[0], n, k)
    else:
        _check(w, "w", torch.uint8, n * q4_0_row_bytes(k), x.device)
        call("smx_q4_0_gemm", _stream(x), x.data_ptr(), w.data_ptr(), out.data_ptr(),
             x.shape[0], n, k)
    return out


def q4_0_gemm_swiglu(x: torch.Tensor, w: torch.Tensor | PackedQ4_0, d: int, k: int,
                     out: torch.Tensor | None = None,
                     lut: torch.Tensor | None = None) -> torch.Tensor:
    """out [m, d] = silu(x W_gate^T) * (x W_up^T), W = [gate; up] [2d, k] (GGUF
    Q4_0, or packed gated by q4_0_repack); given the GELU table (gelu_table)
    as lut, the table GELU in place of SiLU."""
    packed = isinstance(w, PackedQ4_0)
    _gemm_x(x, k, 16 if packed else 8)
    if out is None:
        out = torch.empty((x.shape[0], d), dtype=BF16, device=x.device)
    _check(out, "out", BF16, x.shape[0] * d, x.device)
    if packed:
        wp = _packed_checked(w, d, k, True, x.device)
        if lut is None:
            call("smx_q4_0_gemm_packed_swiglu", _stream(x), x.data_ptr(), wp, out.data_ptr(),
                 x.shape[0], d, k)
        else:
            call("smx_q4_0_gemm_packed_gelu", _stream(x), x.data_ptr(), wp,
                 _lut_checked(lut, x.device), out.data_ptr(), x.shape[0], d, k)
        return out
    _check(w, "w", torch.uint8, 2 * d * q4_0_row_bytes(k), x.device)
    if lut is None:
        call("smx_q4_0_gemm_swiglu", _stream(x), x.data_ptr(), w.data_ptr(), out.data_ptr(),
             x.shape[0], d, k)
    else:
        call("smx_q4_0_gemm_gelu", _stream(x), x.data_ptr(), w.data_ptr(),
             _lut_checked(lut, x.device), out.data_ptr(), x.shape[0], d, k)
    return out


def q4_0_gemm_gelu(x: torch.Tensor, w: torch.Tensor | PackedQ4_0, lut: torch.Tensor, d: int, k: int,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    return q4_0_gemm_swiglu(x, w, d, k, out, lut)


def gemm_keys_per_row(n: int) -> int:
    """Greedy-argmax keys q4_0_gemm_argmax writes per row (one per 16 outputs)."""
    from . import load
    return int(load().smx_q4_0_gemm_keys_per_row(n))


def q4_0_gemm_argmax(x: torch.Tensor, w: torch.Tensor | PackedQ4_0, n: int, k: int,
                     keys: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = x W^T (m <= 16 rows; W GGUF Q4_0 or packed) plus keys [m, ceil(n / 16)]
    int64 (uint64 bits), the greedy-argmax keys decode_advance(argmax_keys=keys)
    reduces."""
    _gemm_x(x, k, 16)
    m = x.shape[0]
    _check(keys, "keys", torch.int64, m * gemm_keys_per_row(n), x.device)
    if out is None:
        out = torch.empty((m, n), dtype=BF16, device=x.device)
    _check(out, "out", BF16, m * n, x.device)
    if isinstance(w, PackedQ4_0):
        call("smx_q4_0_gemm_packed_argmax", _stream(x), x.data_ptr(),
             _packed_checked(w, n, k, False, x.device), out.data_ptr(), keys.data_ptr(), m, n, k)
    else:
        _check(w, "w", torch.uint8, n * q4_0_row_bytes(k), x.device)
        call("smx_q4_0_gemm_argmax", _stream(x), x.data_ptr(), w.data_ptr(), out.data_ptr(),
             keys.data_ptr(), m, n, k)
    return out
