"""Tied LM head as a Q4_0 GEMV, plus greedy sampling on the device.

Mirrors Q6HeadMethod (src/spark_vllm_ascend/integration/head.py:12-16,31):
the head layer keeps its tied bf16 embedding weight, gains a packed
quantized buffer, and its ``quant_method`` is swapped for a method whose
``apply`` serves batch-1 bf16 input with the native kernel and defers to a
plain bf16 matmul otherwise.  The quantized head here is Q4_0
[vocab, hidden] (the reference model's head is Q6_K), and the tied
embedding is bf16(dequantized head), the tying the reference prepares at
src/tools/deployment/prepare_head.py:27.
"""
from __future__ import annotations

import torch

from ..native import torch_ops
from .weights import dequantize_bf16, row_bytes


class Q4_0HeadMethod:
    def apply(self, layer: torch.nn.Module, x: torch.Tensor,
              bias: torch.Tensor | None = None) -> torch.Tensor:
        vocab, hidden = layer.weight.shape
        if x.shape == (1, hidden) and x.dtype == torch.bfloat16 and bias is None:
            return torch_ops.q4_0_gemv(x.contiguous(), layer.q4_0_head, vocab, hidden)
        out = torch.nn.functional.linear(x, layer.weight)
        return out if bias is None else out + bias


class TiedQ4_0Head(torch.nn.Module):
    """Embedding/LM-head pair sharing one Q4_0 tensor."""

    def __init__(self, q4_0_blocks: torch.Tensor, vocab: int, hidden: int):
        super().__init__()
        if tuple(q4_0_blocks.shape) != (vocab, row_bytes(hidden)):
            raise ValueError("head blocks must be uint8 [vocab, hidden/32*18]")
        self.register_buffer("q4_0_head", q4_0_blocks.contiguous())
        self.weight = torch.nn.Parameter(dequantize_bf16(self.q4_0_head, vocab, hidden),
                                         requires_grad=False)
        self.quant_method = Q4_0HeadMethod()

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        return self.quant_method.apply(self, x)

    def embed(self, ids: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        return torch_ops.embedding(self.weight, ids, out=out)


def greedy_sample(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """argmax over the vocabulary (temperature 0), lowest index on ties."""
    return torch_ops.argmax(logits, out=out)
