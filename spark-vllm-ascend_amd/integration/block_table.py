"""Paged KV block allocation and per-sequence block tables for decode.

The reference runs one request and takes vLLM's block tables as given
(``metadata.block_tables``, src/spark_vllm_ascend/integration/model.py:64),
computing slots with its Triton slot-mapping kernel
(src/spark_vllm_ascend/integration/slot_mapping.py:8-55).  For
multi-sequence decode this module keeps the host side of that: a free list of
physical pages, each sequence's pages in order, and the device block table
``[max_seqs, max_blocks]`` int32 the attention kernel reads (unused entries
are -1).  Slots for a step come from ``torch_ops.compute_slot_mapping``.
"""
from __future__ import annotations

from collections import deque

import torch


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int, max_seqs: int, max_blocks_per_seq: int,
                 device):
        if num_blocks < 1 or block_size < 1 or max_seqs < 1 or max_blocks_per_seq < 1:
            raise ValueError("sizes must be >= 1")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.max_seqs = max_seqs
        self.max_blocks = max_blocks_per_seq
        self.device = torch.device(device)
        self._free = deque(range(num_blocks))
        self._pages: dict[int, list[int]] = {}
        self._len: dict[int, int] = {}
        self._row: dict[int, int] = {}
        self._free_rows = deque(range(max_seqs))
        self.table_host = torch.full((max_seqs, max_blocks_per_seq), -1, dtype=torch.int32)
        self.block_table = self.table_host.to(self.device)

    # ------------------------------------------------------------ queries
    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    def pages(self, seq_id: int) -> list[int]:
        return list(self._pages[seq_id])

    def length(self, seq_id: int) -> int:
        return self._len[seq_id]

    def row(self, seq_id: int) -> int:
        return self._row[seq_id]

    def slot(self, seq_id: int, pos: int) -> int:
        """Physical slot of position `pos` of a sequence (host arithmetic)."""
        return self._pages[seq_id][pos // self.block_size] * self.block_size + pos % self.block_size

    # ------------------------------------------------------------ updates
    def _grow(self, seq_id: int, new_len: int) -> None:
        need = -(-new_len // self.block_size)
        pages = self._pages[seq_id]
        if need > self.max_blocks:
            raise ValueError(f"sequence {seq_id} would need {need} blocks > {self.max_blocks}")
        if need - len(pages) > len(self._free):
            raise MemoryError("out of KV cache blocks")
        r = self._row[seq_id]
        while len(pages) < need:
            p = self._free.popleft()
            self.table_host[r, len(pages)] = p
            pages.append(p)
        self._len[seq_id] = new_len

    def add_sequence(self, seq_id: int, length: int) -> None:
        if seq_id in self._pages:
            raise ValueError(f"sequence {seq_id} exists")
        if not self._free_rows:
            raise MemoryError("no free block-table row")
        self._pages[seq_id] = []
        self._row[seq_id] = self._free_rows.popleft()
        try:
            self._grow(seq_id, length)
        except Exception:
            self.free(seq_id)
            raise

    def append_tokens(self, seq_id: int, n: int = 1) -> None:
        self._grow(seq_id, self._len[seq_id] + n)

    def free(self, seq_id: int) -> None:
        r = self._row.pop(seq_id)
        self._free.extend(self._pages.pop(seq_id))
        self._len.pop(seq_id, None)
        self.table_host[r] = -1
        self._free_rows.append(r)

    def sync(self) -> torch.Tensor:
        """Copy the host block table to the device tensor (same address)."""
        self.block_table.copy_(self.table_host, non_blocking=False)
        return self.block_table

    def decode_batch(self, seq_ids: list[int]) -> dict:
        """Device metadata of one decode step where each sequence feeds its
        newest token (position length - 1): rows of the block table in batch
        order, positions, seq_lens, query_start_loc."""
        rows = torch.tensor([self._row[s] for s in seq_ids], dtype=torch.int64)
        pos = torch.tensor([self._len[s] - 1 for s in seq_ids], dtype=torch.int64)
        dev = self.device
        return dict(block_table=self.table_host[rows].contiguous().to(dev),
                    positions=pos.to(dev),
                    seq_lens=(pos + 1).to(torch.int32).to(dev),
                    query_start_loc=torch.arange(len(seq_ids) + 1, dtype=torch.int32).to(dev))
