"""Split-KV decode attention backend over a paged bf16 KV cache.

The reference does not register a backend of its own: its decode layer pulls
``(metadata, impl, kv_cache)`` from vLLM-Ascend through
``get_attention_context(layer_name)`` and reads ``metadata.block_tables``,
``metadata.slot_mapping`` and ``kv_cache[0] / kv_cache[1]`` viewed as
[num_blocks, 128, kv_heads, head_dim] (src/spark_vllm_ascend/integration/
model.py:46-68,118-139).  Here that surface is an explicit backend with
vLLM's AttentionBackend / AttentionImpl method names:

  SplitKVDecodeBackend.get_kv_cache_shape(num_blocks, block_size,
      num_kv_heads, head_size) -> (2, num_blocks, block_size, kv, head)
  SplitKVDecodeImpl.forward(layer, query, key, value, kv_cache,
      attn_metadata, output=None)
      writes key/value at slot_mapping, runs split-KV decode and the LSE
      merge (HIP kernels), returns [num_tokens, n_q * head_dim] bf16.
  SplitKVDecodeBackend.plan(attn_metadata, block_size, num_heads, head_size)
      once per step for a batch: cuts the live tokens into per-sequence
      splits of one length (a device kernel), which every layer's forward
      then uses (the reference's device-side task list, parts = ceil(length
      / width): src/spark_vllm_ascend/kernels/attention.py:120-128).

Metadata lives in device tensors (block tables, sequence lengths, slots) so
a captured graph can replay with new values; only ``num_splits`` (and a
plan's ``num_items``) is fixed at capture time.  The split partials are a
workspace shared by every layer (layers run one after another on a stream):
a plan clears the slots its splits do not write, once for all layers.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ..native import torch_ops


@dataclass
class SplitKVDecodeMetadata:
    block_tables: torch.Tensor    # int32 [num_seqs, max_blocks]
    seq_lens: torch.Tensor        # int32 [num_seqs]
    slot_mapping: torch.Tensor    # int64 [num_tokens], -1 = skip
    num_splits: int
    max_seq_len: int = 0          # host hint used only to choose num_splits
    num_items: int = 0            # a plan's split budget (SplitKVDecodeBackend.plan)
    plan: torch.Tensor | None = None  # int32 [num_items + num_seqs, 64] plan records
    plan_positions: torch.Tensor | None = None  # the positions the plan's records carry


def choose_num_splits(capacity: int, tokens_per_split: int = 128, num_seqs: int = 1) -> int:
    """Split count for a block table addressing `capacity` tokens.  Splits
    are cut from the capacity (not the current length), so one captured graph
    serves every step.  Measured on MI355X:
      * one sequence: 128 tokens per split (four waves of one 32-token block
        each, two workgroups per CU) is best at 2k..6k (49 splits at a
        6272-token capacity; 32 or 33 splits of 224 / 192 tokens put one
        8-wave workgroup on a CU, and past 256 workgroups the rest run in a
        second round);
      * several sequences: about 25 long splits whatever the capacity (8
        sequences at 512..32768 tokens, 32896-token capacity: 25 splits of
        1344 tokens 5.47 ms per step, 17 / 33 splits 5.52 / 5.56 ms, 257
        splits of 128 tokens 6.14 ms): the KV stream is large, so fewer
        workgroups, partials and merge inputs win.  A per-sequence split
        plan (choose_plan, SplitKVDecodeBackend.plan) does better still."""
    n = int(max(1, -(-capacity // tokens_per_split)))
    return min(n, 25) if num_seqs > 1 else n


def choose_plan(num_seqs: int, n_kv: int = 8) -> tuple[int, int]:
    """(num_items, num_splits) of a per-sequence split plan: an item budget
    of (num_items + num_seqs) * n_kv ~= 768 workgroups and at most 16 splits
    per sequence.  With long sequences the 16-split cap sets the split length
    (the 8-sequence bench at contexts 512..32768: 2048-token splits, 61
    items).  Measured there: 16 splits 5.06 ms against 5.14 with 32 (the
    merge reads num_seqs * num_splits partial slots, the unused ones
    cleared), 5.01 with 12 and 4.94 with 24 (2-wave workgroups); 56 / 120 /
    184 items at 32 splits 5.13-5.19 ms; capacity splits 5.34 ms."""
    return max(1, 768 // n_kv - num_seqs), 16


_WORKSPACES: dict = {}


def split_partials(num_seqs: int, num_splits: int, num_heads: int, head_size: int, device):
    """Split partials, allocated once per shape and shared by every layer
    (the reference likewise allocates its workspaces once per compile key,
    src/spark_vllm_ascend/integration/model.py:128-131)."""
    key = (num_seqs, num_splits, num_heads, head_size, torch.device(device))
    if key not in _WORKSPACES:
        _WORKSPACES[key] = (
            torch.empty((num_seqs, num_splits, num_heads, head_size), dtype=torch.float32,
                        device=device),
            torch.empty((num_seqs, num_splits, num_heads), dtype=torch.float32, device=device))
    return _WORKSPACES[key]


class SplitKVDecodeImpl:
    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 **unused):
        if head_size != 128:
            raise ValueError("split-KV decode supports head_size 128")
        if num_heads != 4 * num_kv_heads:
            raise ValueError("split-KV decode supports GQA 4:1")
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads

    def forward(self, layer, query: torch.Tensor, key: torch.Tensor | None,
                value: torch.Tensor | None, kv_cache: torch.Tensor,
                attn_metadata: SplitKVDecodeMetadata, output: torch.Tensor | None = None):
        """query [num_seqs, n_q*hd] (one decode token per sequence)."""
        k_cache, v_cache = kv_cache[0], kv_cache[1]
        num_seqs = attn_metadata.seq_lens.numel()
        if key is not None and value is not None:
            torch_ops.reshape_and_cache(key.reshape(-1, self.num_kv_heads, self.head_size),
                                        value.reshape(-1, self.num_kv_heads, self.head_size),
                                        k_cache, v_cache, attn_metadata.slot_mapping)
        q = query.reshape(num_seqs, self.num_heads, self.head_size)
        po, pl = split_partials(num_seqs, attn_metadata.num_splits, self.num_heads,
                                self.head_size, query.device)
        out = output.view(num_seqs, self.num_heads, self.head_size) if output is not None else None
        if attn_metadata.plan is not None:
            out = torch_ops.splitkv_decode_planned_merged(
                q, k_cache, v_cache, attn_metadata.block_tables, attn_metadata.plan,
                attn_metadata.num_items, self.scale, po, pl, out=out)
        else:
            out = torch_ops.splitkv_decode_merged(q, k_cache, v_cache, attn_metadata.block_tables,
                                                  attn_metadata.seq_lens,
                                                  attn_metadata.num_splits, self.scale, po, pl,
                                                  out=out)
        return out.view(num_seqs, self.num_heads * self.head_size)


class SplitKVDecodeBackend:
    @staticmethod
    def get_name() -> str:
        return "SMX_SPLITKV_DECODE"

    @staticmethod
    def get_impl_cls():
        return SplitKVDecodeImpl

    @staticmethod
    def get_metadata_cls():
        return SplitKVDecodeMetadata

    @staticmethod
    def plan(attn_metadata: SplitKVDecodeMetadata, block_size: int, num_heads: int,
             head_size: int, positions: torch.Tensor | None = None) -> SplitKVDecodeMetadata:
        """Per-sequence split plan for this step's metadata (num_items > 0,
        at most 64 sequences), enqueued on the current stream; every layer's
        forward with this metadata then runs over the plan's splits.  With
        `positions` (int64, one per sequence) the records also carry each
        sequence's position and KV slot (metadata.slot_mapping), which the
        fused q/k-norm + RoPE + KV-write attention needs; a plan built
        without them makes that kernel return NaN."""
        if attn_metadata.num_items <= 0:
            raise ValueError("set num_items (choose_plan) before planning")
        num_seqs = attn_metadata.seq_lens.numel()
        po, pl = split_partials(num_seqs, attn_metadata.num_splits, num_heads, head_size,
                            attn_metadata.seq_lens.device)
        attn_metadata.plan = torch_ops.splitkv_plan(
            attn_metadata.seq_lens, attn_metadata.block_tables, block_size,
            attn_metadata.num_items, po, pl, positions=positions,
            slot_mapping=attn_metadata.slot_mapping if positions is not None else None,
            plan=attn_metadata.plan)
        attn_metadata.plan_positions = positions
        return attn_metadata

    @staticmethod
    def get_supported_head_sizes() -> list[int]:
        return [128]

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                           head_size: int) -> tuple[int, ...]:
        if block_size < 32 or block_size & (block_size - 1):
            raise ValueError("block_size must be a power of two >= 32")
        return (2, num_blocks, block_size, num_kv_heads, head_size)
