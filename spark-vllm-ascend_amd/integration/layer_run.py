"""The reference's per-layer decode seam: ``layer_run(x, residual,
positions, layer_name) -> (y, residual)``.

The reference replaces each decoder layer's decode step with one custom op
(``spark_v43::layer_run``, src/spark_vllm_ascend/integration/model.py:46-82,
``register_fake`` returning ``empty_like`` pairs), registered per layer by
``install(model)`` under the attention layer's name together with the norm
that follows the layer (the next layer's input norm, the model's final norm
after the last layer: :84-95), and called by the model loop after the first
input norm (src/spark_vllm_ascend/plugin/spark2_5.py:369-376):

  x           bf16 [T, hidden]  the layer input, already normalised by the
                                layer's input norm
  residual    bf16 [T, hidden]  the residual stream entering the layer
  positions   int64 [T]         the token positions
  layer_name  the key install() registered the layer under
  returns     (y, residual_out): residual_out = bf16(mlp_out + h) where h is
              the residual after the attention add, and y = the next norm of
              (mlp_out, h) -- the next layer's normalised input, or the final
              norm's output after the last layer.

Outputs are freshly allocated per call; the intermediate buffers are
allocated once per shape and shared by every layer, as the reference
allocates its workspaces once per compile key (:128-131).

The attention metadata comes from the layer's attention context, as the
reference's ``get_attention_context(layer_name)`` (:49): the caller
publishes the step's metadata with set_attention_metadata() (vLLM publishes
its forward context the same way) and the KV cache is the one registered
with the layer.

Kernel sequence (HIP launches):
  T == 1: QKV GEMV -> q/k RMSNorm + RoPE + KV write fused into split-KV
          attention, LSE merge -> o_proj GEMV -> add + RMSNorm(post norm)
          fused into the gate|up GEMV with SwiGLU -> down GEMV -> add +
          RMSNorm(next norm): 7 launches.
  2 <= T <= 16 (one decode token per sequence, over the per-sequence split
          plan SplitKVDecodeBackend.plan built for this step, with the
          positions and slots; the GEMMs read a layer's packed weights when
          its linears were packed, Q4_0LinearMethod.pack): QKV GEMM -> fused planned split-KV + merge
          -> o_proj GEMM -> add + RMSNorm -> gate|up GEMM with SwiGLU -> down
          GEMM -> add + RMSNorm(next norm).
Other calls -- no published metadata, more than 16 rows, or rows that are
not one decode token per sequence (prefill) -- go to the stock layer, as the
reference's op runs vLLM's attention, post-attention norm, MLP and next norm
for ``x.shape[0] != 1`` or missing metadata (:50-61): install() takes the
stock layer as a callable ``stock_layer(index, x, residual, positions) ->
(y, residual_out)`` with the same contract as layer_run.  Without one, such
calls raise.  With several sequences the positions and KV slots come from
the step's plan (SplitKVDecodeBackend.plan), so layer_run checks that
``positions`` is what the plan was built with.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

from ..native import torch_ops
from .attention import SplitKVDecodeMetadata, split_partials
from .linear import gemm_weight

_layers: dict = {}
_metadata: SplitKVDecodeMetadata | None = None
_workspaces: dict = {}


@dataclass
class _Entry:
    layer: object          # model.DecoderLayer
    next_norm: torch.Tensor
    cfg: object            # model.DecoderConfig
    cos_sin: torch.Tensor
    scale: float
    index: int
    act_lut: torch.Tensor | None  # the GELU table of a GELU model (None: SwiGLU)
    stock: Callable | None  # stock_layer(index, x, residual, positions) for other calls


def install(model, stock_layer: Callable | None = None) -> list[str]:
    """Register every layer of a DecodeModel under its attention layer name
    with the norm that follows it, and the stock layer that serves the calls
    the decode kernels do not (prefill); returns the names in layer order."""
    names = []
    n = len(model.layers)
    for i, L in enumerate(model.layers):
        nxt = model.layers[i + 1].input_norm if i + 1 < n else model.final_norm
        _layers[L.name] = _Entry(L, nxt, model.cfg, model.cos_sin, model.scale, i,
                                 getattr(model, "act_lut", None), stock_layer)
        names.append(L.name)
    return names


def uninstall() -> None:
    """Forget every installed layer and the published metadata."""
    global _metadata
    _layers.clear()
    _workspaces.clear()
    _metadata = None


def set_attention_metadata(metadata: SplitKVDecodeMetadata | None) -> None:
    """Publish this step's attention metadata (block tables, sequence
    lengths, slots, split count; a plan for several sequences)."""
    global _metadata
    _metadata = metadata


def get_attention_context(layer_name: str):
    """(metadata, kv_cache) of an installed layer: the published metadata
    and the layer's [2, num_blocks, block_size, n_kv, head_dim] cache."""
    if layer_name not in _layers:
        raise KeyError(f"layer {layer_name!r} is not installed")
    return _metadata, _layers[layer_name].layer.kv_cache


def _workspace(cfg, rows: int, num_splits: int, device) -> dict:
    key = (rows, num_splits, cfg.hidden, cfg.qkv_rows, cfg.intermediate, cfg.n_q,
           torch.device(device))
    ws = _workspaces.get(key)
    if ws is None:
        bf = dict(dtype=torch.bfloat16, device=device)
        c = cfg
        ws = {"qkv": torch.empty((rows, c.qkv_rows), **bf),
              "attn": torch.empty((rows, c.n_q, c.head_dim), **bf),
              "o": torch.empty((rows, c.hidden), **bf),
              "h2": torch.empty((rows, c.hidden), **bf),
              "res_a": torch.empty((rows, c.hidden), **bf),
              "act": torch.empty((rows, c.intermediate), **bf),
              "d": torch.empty((rows, c.hidden), **bf)}
        # the split partials are the attention backend's own buffers: a
        # step's plan (SplitKVDecodeBackend.plan) clears the slots its splits
        # leave unwritten in exactly these
        ws["po"], ws["pl"] = split_partials(rows, num_splits, c.n_q, c.head_dim, device)
        _workspaces[key] = ws
    return ws


def _check_plan_positions(md: SplitKVDecodeMetadata, positions: torch.Tensor) -> None:
    """Several sequences take their RoPE positions and KV slots from the
    plan's records, not from `positions`: the two must agree.  The same
    tensor (what a step passes) passes at once; another tensor is compared
    by value, which needs a synchronisation, so it is refused under graph
    capture."""
    pp = md.plan_positions
    if md.plan is None or pp is None:
        raise ValueError("several sequences need this step's split plan built with their "
                         "positions (SplitKVDecodeBackend.plan(..., positions=...))")
    if (pp.data_ptr() == positions.data_ptr() and pp.numel() == positions.numel()
            and pp.dtype == positions.dtype):
        return
    if torch.cuda.is_current_stream_capturing():
        raise ValueError("positions is not the tensor the plan was built with (values cannot "
                         "be compared during graph capture)")
    if not torch.equal(pp.to(positions.device).view(-1), positions.view(-1)):
        raise ValueError("positions differ from those the step's plan was built with")


def layer_run(x: torch.Tensor, residual: torch.Tensor, positions: torch.Tensor,
              layer_name: str) -> tuple[torch.Tensor, torch.Tensor]:
    """One decoder layer's decode step; see the module docstring."""
    if layer_name not in _layers:
        raise KeyError(f"layer {layer_name!r} is not installed")
    e = _layers[layer_name]
    md = _metadata
    T = x.shape[0] if x.dim() == 2 else -1
    decode = md is not None and 1 <= T <= 16 and md.seq_lens.numel() == T
    if not decode:
        if e.stock is not None:  # prefill and unpublished metadata: the stock layer
            return e.stock(e.index, x, residual, positions)
        if md is None:
            raise RuntimeError("no attention metadata published: call set_attention_metadata() "
                               "for this step (or install a stock layer)")
    c, L = e.cfg, e.layer
    if x.dim() != 2 or x.shape[1] != c.hidden or x.dtype != torch.bfloat16:
        raise ValueError(f"x must be bf16 [T, {c.hidden}], got {x.dtype} {tuple(x.shape)}")
    if tuple(residual.shape) != tuple(x.shape) or residual.dtype != torch.bfloat16:
        raise ValueError("residual must be bf16 of x's shape")
    if positions.numel() != T or positions.dtype != torch.int64:
        raise ValueError("positions must be int64 [T]")
    if md.seq_lens.numel() != T:
        raise ValueError(f"the metadata describes {md.seq_lens.numel()} sequences, x has {T} "
                         "rows (one decode token per sequence); install a stock layer for "
                         "prefill")
    if not 1 <= T <= 16:
        raise ValueError("decode layer_run serves 1..16 sequences; install a stock layer for "
                         "prefill")
    if T > 1:
        _check_plan_positions(md, positions)
    x = x.contiguous()
    residual = residual.contiguous()
    ws = _workspace(c, T, md.num_splits, x.device)
    kc, vc = L.kv_cache[0], L.kv_cache[1]
    ops = torch_ops
    y = torch.empty_like(x)
    r_out = torch.empty_like(residual)
    if T == 1:
        ops.q4_0_gemv(x, L.qkv.qweight, c.qkv_rows, c.hidden, out=ws["qkv"])
        ops.qknorm_rope_splitkv_decode_merged(
            ws["qkv"], L.q_norm, L.k_norm, e.cos_sin, positions, md.slot_mapping, kc, vc,
            md.block_tables, md.seq_lens, md.num_splits, e.scale, c.eps, c.n_q, ws["po"],
            ws["pl"], out=ws["attn"])
        ops.q4_0_gemv(ws["attn"], L.o_proj.qweight, c.hidden, c.n_q * c.head_dim, out=ws["o"])
        ops.add_rmsnorm_gemv_swiglu(ws["o"], residual, L.post_norm, L.gate_up.qweight,
                                    c.intermediate, c.hidden, c.eps, residual_out=ws["res_a"],
                                    out=ws["act"], lut=e.act_lut)
        ops.q4_0_gemv(ws["act"], L.down.qweight, c.hidden, c.intermediate, out=ws["d"])
    else:
        if md.num_items <= 0:
            raise ValueError("several sequences need this step's split plan "
                             "(SplitKVDecodeBackend.plan with positions and slots)")
        ops.q4_0_gemm(x, gemm_weight(L.qkv), c.qkv_rows, c.hidden, out=ws["qkv"])
        ops.qknorm_rope_splitkv_decode_planned_merged(
            ws["qkv"], L.q_norm, L.k_norm, e.cos_sin, kc, vc, md.block_tables, md.plan,
            md.num_items, e.scale, c.eps, c.n_q, ws["po"], ws["pl"], out=ws["attn"])
        ops.q4_0_gemm(ws["attn"].view(T, -1), gemm_weight(L.o_proj), c.hidden,
                      c.n_q * c.head_dim, out=ws["o"])
        ops.add_rmsnorm(ws["o"], residual, L.post_norm, c.eps, out=ws["h2"],
                        residual_out=ws["res_a"])
        ops.q4_0_gemm_swiglu(ws["h2"], gemm_weight(L.gate_up, gated=True), c.intermediate,
                             c.hidden, out=ws["act"], lut=e.act_lut)
        ops.q4_0_gemm(ws["act"], gemm_weight(L.down), c.hidden, c.intermediate, out=ws["d"])
    ops.add_rmsnorm(ws["d"], ws["res_a"], e.next_norm, c.eps, out=y, residual_out=r_out)
    return y, r_out
