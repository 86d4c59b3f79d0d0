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

Metadata lives in device tensors (block tables, sequence lengths, slots) so
a captured graph can replay with new values; only ``num_splits`` is fixed at
capture time.
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
        workgroups, partials and merge inputs win."""
    n = int(max(1, -(-capacity // tokens_per_split)))
    return min(n, 25) if num_seqs > 1 else n


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
        self._workspaces = {}

    def _workspace(self, num_seqs: int, num_splits: int, device):
        """Split partials, allocated once per shape (the reference likewise
        allocates its workspaces once per compile key,
        src/spark_vllm_ascend/integration/model.py:128-131)."""
        key = (num_seqs, num_splits, device)
        if key not in self._workspaces:
            self._workspaces[key] = (
                torch.empty((num_seqs, num_splits, self.num_heads, self.head_size),
                            dtype=torch.float32, device=device),
                torch.empty((num_seqs, num_splits, self.num_heads), dtype=torch.float32,
                            device=device))
        return self._workspaces[key]

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
        po, pl = self._workspace(num_seqs, attn_metadata.num_splits, query.device)
        out = output.view(num_seqs, self.num_heads, self.head_size) if output is not None else None
        out = torch_ops.splitkv_decode_merged(q, k_cache, v_cache, attn_metadata.block_tables,
                                              attn_metadata.seq_lens, attn_metadata.num_splits,
                                              self.scale, po, pl, out=out)
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
    def get_supported_head_sizes() -> list[int]:
        return [128]

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                           head_size: int) -> tuple[int, ...]:
        if block_size < 32 or block_size & (block_size - 1):
            raise ValueError("block_size must be a power of two >= 32")
        return (2, num_blocks, block_size, num_kv_heads, head_size)
