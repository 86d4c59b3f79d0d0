"""Graph-safe torch custom ops over the HIP kernels.

The reference wraps its device calls as ``torch.library.custom_op(...,
mutates_args=())`` with a ``register_fake`` that returns ``empty_like``
shapes, and allocates every output freshly per call, so torch.compile and
graph capture can trace through them (src/spark_vllm_ascend/integration/
model.py:37-44,46-82; integration/head.py:6-11).  The same contract here,
under the namespace ``smx``:

  smx::q4_0_gemv(x, w, n, k) -> y                      bf16 [1, n]
  smx::q4_0_gemv_swiglu(x, w, d, k) -> y               bf16 [1, d]
  smx::q4_0_gemv_gelu(x, w, lut, d, k) -> y            bf16 [1, d] (the
      reference model's table GELU; lut = torch_ops.gelu_table(device))
  smx::add_rmsnorm(x, residual, gamma, eps) -> (y, residual_out)
  smx::splitkv_decode_attention(q, k_cache, v_cache, block_table, seq_lens,
                                num_splits, scale) -> out   bf16 [seqs, n_q, hd]
  smx::argmax(logits) -> ids                           int64 [rows]
  smx::layer_run(x, residual, positions, layer_name) -> (y, residual_out)
      one decoder layer's decode step over the layers layer_run.install()
      registered (src/spark_vllm_ascend/integration/model.py:46-82)

register() defines them once per process; calling it again is a no-op.
"""
from __future__ import annotations

import torch

from ..native import torch_ops

_NS = "smx"
_done = False


def register() -> None:
    global _done
    if _done:
        return

    @torch.library.custom_op(f"{_NS}::q4_0_gemv", mutates_args=())
    def q4_0_gemv(x: torch.Tensor, w: torch.Tensor, n: int, k: int) -> torch.Tensor:
        return torch_ops.q4_0_gemv(x.contiguous(), w, n, k)

    @q4_0_gemv.register_fake
    def _(x, w, n, k):
        return x.new_empty((1, n))

    @torch.library.custom_op(f"{_NS}::q4_0_gemv_swiglu", mutates_args=())
    def q4_0_gemv_swiglu(x: torch.Tensor, w: torch.Tensor, d: int, k: int) -> torch.Tensor:
        return torch_ops.q4_0_gemv_swiglu(x.contiguous(), w, d, k)

    @q4_0_gemv_swiglu.register_fake
    def _(x, w, d, k):
        return x.new_empty((1, d))

    @torch.library.custom_op(f"{_NS}::q4_0_gemv_gelu", mutates_args=())
    def q4_0_gemv_gelu(x: torch.Tensor, w: torch.Tensor, lut: torch.Tensor, d: int,
                       k: int) -> torch.Tensor:
        return torch_ops.q4_0_gemv_gelu(x.contiguous(), w, lut, d, k)

    @q4_0_gemv_gelu.register_fake
    def _(x, w, lut, d, k):
        return x.new_empty((1, d))

    @torch.library.custom_op(f"{_NS}::add_rmsnorm", mutates_args=())
    def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, gamma: torch.Tensor,
                    eps: float) -> tuple[torch.Tensor, torch.Tensor]:
        y, r = torch_ops.add_rmsnorm(x.contiguous(), residual.contiguous(), gamma, eps)
        return y, r

    @add_rmsnorm.register_fake
    def _(x, residual, gamma, eps):
        return torch.empty_like(x), torch.empty_like(x)

    @torch.library.custom_op(f"{_NS}::splitkv_decode_attention", mutates_args=())
    def splitkv_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                 block_table: torch.Tensor, seq_lens: torch.Tensor,
                                 num_splits: int, scale: float) -> torch.Tensor:
        po, pl = torch_ops.splitkv_decode(q.contiguous(), k_cache, v_cache, block_table, seq_lens,
                                          num_splits, scale)
        return torch_ops.lse_merge(po, pl)

    @splitkv_decode_attention.register_fake
    def _(q, k_cache, v_cache, block_table, seq_lens, num_splits, scale):
        return torch.empty_like(q)

    @torch.library.custom_op(f"{_NS}::argmax", mutates_args=())
    def argmax(logits: torch.Tensor) -> torch.Tensor:
        return torch_ops.argmax(logits.contiguous())

    @argmax.register_fake
    def _(logits):
        rows = logits.numel() // logits.shape[-1]
        return logits.new_empty((rows,), dtype=torch.int64)

    @torch.library.custom_op(f"{_NS}::layer_run", mutates_args=())
    def layer_run(x: torch.Tensor, residual: torch.Tensor, positions: torch.Tensor,
                  layer_name: str) -> tuple[torch.Tensor, torch.Tensor]:
        from . import layer_run as lr
        return lr.layer_run(x, residual, positions, layer_name)

    @layer_run.register_fake
    def _(x, residual, positions, layer_name):
        return torch.empty_like(x), torch.empty_like(residual)

    _done = True
