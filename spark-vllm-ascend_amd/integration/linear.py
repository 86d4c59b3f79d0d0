"""Q4_0 linear quant method: the plugin's operator surface for the GEMVs.

The reference swaps a layer's ``quant_method`` for a class whose
``apply(layer, x, bias=None)`` serves the fast path for batch-1 bf16 input
and defers to the stock method otherwise (Q6HeadMethod,
src/spark_vllm_ascend/integration/head.py:12-16,31).  This module offers the
same hook for Q4_0 linears on vLLM's LinearMethodBase contract:

  create_weights(layer, input_size_per_partition, output_partition_sizes,
                 input_size, output_size, params_dtype, **extra)
      registers ``layer.qweight``: uint8 [sum(output_partition_sizes),
      input_size_per_partition/32*18], GGUF Q4_0 blocks as stored in the file.
  process_weights_after_loading(layer)
      validates the loaded blocks; the GEMVs stream GGUF blocks directly, so
      no repack happens here unless the config asks for the batched GEMM's
      packed layout (Q4_0Config(pack_for_batch=True): pack(layer) below).
  pack(layer, gated=False)
      on request, for batched decode: adds ``layer.q4_0_packed``, the packed
      layout of the MFMA GEMM (torch_ops.q4_0_repack; gated for a merged
      gate|up layer's SwiGLU GEMM), as the reference repacks its weights for
      its own kernel (src/spark_vllm_ascend/integration/weights.py:42-54).
      The GGUF blocks stay: the one-row GEMV reads them.
  apply(layer, x, bias=None) -> [..., N] bf16
      one HIP launch: the Q4_0 GEMV for one activation row, the MFMA Q4_0
      GEMM for 2..16 rows (K % 64 == 0; over the packed weights when pack()
      made them); more rows (prefill) go through the
      bf16 weights the reference's stock path uses (dequantised on the
      device, then a library GEMM), as Q6HeadMethod defers to the stock
      method outside its one-row case.  Bias added after.

vLLM is not installed in this image; when it is, the class derives from its
LinearMethodBase so vLLM's loaders accept it unchanged.
"""
from __future__ import annotations

import torch

from ..native import torch_ops
from .weights import row_bytes

try:  # pragma: no cover - vLLM is absent here
    from vllm.model_executor.layers.linear import LinearMethodBase as _Base
except Exception:  # noqa: BLE001
    class _Base:  # minimal stand-in with vLLM's method names
        def create_weights(self, layer, *args, **kwargs):
            raise NotImplementedError

        def apply(self, layer, x, bias=None):
            raise NotImplementedError

        def process_weights_after_loading(self, layer):
            return None


#: activation rows one MFMA Q4_0 GEMM launch serves (the kernel's m limit)
GEMM_MAX_ROWS = 16


class Q4_0Config:
    """Quantization config naming the method, as vLLM's QuantizationConfig.
    pack_for_batch=True makes every linear also hold the packed layout of
    the batched GEMM (built in process_weights_after_loading): faster
    2..16-row decode for twice the weight memory."""

    def __init__(self, pack_for_batch: bool = False):
        self.pack_for_batch = bool(pack_for_batch)

    @classmethod
    def get_name(cls) -> str:
        return "q4_0"

    @classmethod
    def get_supported_act_dtypes(cls):
        return [torch.bfloat16]

    def get_quant_method(self, layer, prefix: str = ""):
        return Q4_0LinearMethod(pack_for_batch=self.pack_for_batch)


class Q4_0LinearMethod(_Base):
    """Q4_0 weights, bf16 activations, fp32 accumulation, bf16 output."""

    def __init__(self, pack_for_batch: bool = False):
        self.pack_for_batch = bool(pack_for_batch)

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: list[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs) -> None:
        k = int(input_size_per_partition)
        n = int(sum(output_partition_sizes))
        if params_dtype not in (torch.bfloat16,):
            raise ValueError(f"Q4_0 linears take bf16 activations, got {params_dtype}")
        device = extra_weight_attrs.pop("device", None)
        qweight = torch.nn.Parameter(
            torch.empty((n, row_bytes(k)), dtype=torch.uint8, device=device), requires_grad=False)
        layer.register_parameter("qweight", qweight)
        layer.q4_0_n = n
        layer.q4_0_k = k
        layer.output_partition_sizes = list(output_partition_sizes)
        for key, val in extra_weight_attrs.items():
            setattr(qweight, key, val)

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        w = layer.qweight
        if w.dtype != torch.uint8 or tuple(w.shape) != (layer.q4_0_n, row_bytes(layer.q4_0_k)):
            raise ValueError(f"qweight must be uint8 {(layer.q4_0_n, row_bytes(layer.q4_0_k))}, "
                             f"got {w.dtype} {tuple(w.shape)}")
        if not w.is_contiguous():
            layer.qweight = torch.nn.Parameter(w.contiguous(), requires_grad=False)
        if self.pack_for_batch:
            self.pack(layer)

    def pack(self, layer: torch.nn.Module, gated: bool = False) -> bool:
        """Build ``layer.q4_0_packed`` for the batched GEMM (K % 256 == 0;
        gated: a merged [gate, up] layer of equal halves).  Returns whether
        the layer has one afterwards."""
        n, k = layer.q4_0_n, layer.q4_0_k
        if k % 256 != 0:
            return False
        if gated:
            sizes = layer.output_partition_sizes
            if len(sizes) != 2 or sizes[0] != sizes[1]:
                raise ValueError("a gated pack needs a merged [gate, up] layer of equal halves")
            n = sizes[0]
        layer.q4_0_packed = torch_ops.q4_0_repack(layer.qweight.reshape(-1), n, k, gated)
        return True

    def apply(self, layer: torch.nn.Module, x: torch.Tensor,
              bias: torch.Tensor | None = None) -> torch.Tensor:
        n, k = layer.q4_0_n, layer.q4_0_k
        if x.shape[-1] != k:
            raise ValueError(f"expected last dim {k}, got {x.shape[-1]}")
        if x.dtype != torch.bfloat16:
            raise ValueError(f"expected bf16 activations, got {x.dtype}")
        rows = x.reshape(-1, k).contiguous()
        m = rows.shape[0]
        w = layer.qweight.reshape(-1)
        if m == 0:
            out = torch.empty((0, n), dtype=torch.bfloat16, device=x.device)
        elif m == 1:
            out = torch_ops.q4_0_gemv(rows, w, n, k)
        elif m <= GEMM_MAX_ROWS and k % 64 == 0:
            if rows.data_ptr() % 16:
                rows = rows.clone()  # the tile kernel stages 16-byte activation chunks
            out = torch_ops.q4_0_gemm(rows, gemm_weight(layer), n, k)
        elif m <= GEMM_MAX_ROWS:
            # K % 64 != 0: the GEMV (any K % 32 == 0), one launch per row
            out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
            for i in range(m):
                torch_ops.q4_0_gemv(rows[i], w, n, k, out=out[i])
        else:
            w_bf16 = torch_ops.q4_0_dequant_bf16(w, n, k)
            out = torch.nn.functional.linear(rows, w_bf16.view(n, k))
        out = out.reshape(*x.shape[:-1], n)
        if bias is not None:
            out = out + bias
        return out

    def apply_swiglu(self, layer: torch.nn.Module, x: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
        """Merged gate|up layer (two equal partitions): silu(gate) * up fused
        into the GEMV epilogue, for one activation row."""
        sizes = layer.output_partition_sizes
        if len(sizes) != 2 or sizes[0] != sizes[1]:
            raise ValueError("apply_swiglu needs a merged [gate, up] layer of equal halves")
        return torch_ops.q4_0_gemv_swiglu(x.reshape(-1), layer.qweight.reshape(-1), sizes[0],
                                          layer.q4_0_k, out=out)


def gemm_weight(layer: torch.nn.Module, gated: bool = False):
    """The weights a batched GEMM of the layer reads: its packed form when
    pack() made one of that kind, else the GGUF blocks."""
    p = getattr(layer, "q4_0_packed", None)
    if p is not None and p.gated == gated:
        return p
    return layer.qweight.reshape(-1)


class Q4_0Linear(torch.nn.Module):
    """A bare linear layer driven by Q4_0LinearMethod (used by the decode
    model and tests in place of vLLM's parallel linear classes)."""

    def __init__(self, input_size: int, output_partition_sizes: list[int], device=None):
        super().__init__()
        self.quant_method = Q4_0LinearMethod()
        self.quant_method.create_weights(self, input_size, output_partition_sizes, input_size,
                                         sum(output_partition_sizes), torch.bfloat16,
                                         device=device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.quant_method.apply(self, x)
