"""One decoder layer and an N-layer greedy decode for the oracle -- test
infrastructure.

Wiring follows the reference's decode layer (src/spark_vllm_ascend/kernels/
layer.py:48-103, the phases QKV -> RoPE/KV write -> attention -> merge ->
o_proj -> add+RMSNorm -> gate/up + activation -> down -> add + next norm) and
the decoder residual wiring of src/spark_vllm_ascend/plugin/spark2_5.py:
287-297,369-376 (the first input norm outside the loop, each layer's output
normalised by the next layer's input norm, the final norm after the last
layer).  Shapes and ops are those of the 4B Q4_0 decoder (per-head q/k
RMSNorm, neox RoPE over the full head, SwiGLU -- or the reference model's
table GELU, cfg activation "gelu"); rounding to bf16 happens at
every stage output, as in the reference's stage outputs.  GEMVs are float64
over exactly dequantised weights (q4_0.gemv_f64).

Pins: the layer is a composition of functions pinned in the other oracle
modules; tests/test_oracle_model.py additionally checks that a layer with
zero weights passes the residual through, and that the model is invariant
to the split count.  Greedy decode compares tokens teacher-forced and
classifies a disagreement as a near-tie when the float64 top-2 margin is
below 2e-2 of the top logit (two logits each within the 1e-2 GEMV tolerance
cannot swap order above that margin).
"""
from __future__ import annotations

import numpy as np

from . import attention as oatt
from . import ops as oops
from . import q4_0 as oq
from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16

NEAR_TIE_REL = 2e-2


def _gemv(x_f32: np.ndarray, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """bf16 output of the Q4_0 GEMV (float64 accumulation)."""
    return round_bf16(oq.gemv_f64(f32_to_bf16_bits(x_f32), blocks, n, k).astype(np.float32))


class OracleDecoder:
    """cfg: dict with hidden, n_layers, n_q, n_kv, head_dim, intermediate,
    vocab, eps; optional activation ("swiglu" or "gelu") and gelu_lut.  weights: dict of numpy arrays --
      layers.{i}.qkv / o_proj / gate_up / down : uint8 Q4_0 blocks
      layers.{i}.norm0..3 : float32 values of bf16 (input, post, q, k norms)
      final_norm : float32 values of bf16; head : uint8 Q4_0 blocks
    cos_sin: float32 values of the bf16 rotary table [max_position, head_dim].
    """

    def __init__(self, cfg: dict, weights: dict, cos_sin: np.ndarray, num_splits: int = 1,
                 capacity: int | None = None, grouped_attention: bool = False):
        self.c = cfg
        self.w = weights
        self.cos_sin = cos_sin
        self.num_splits = num_splits
        self.capacity = capacity  # KV capacity the splits are cut from (None: the length)
        # long contexts: the grouped split-KV restatement (q heads of a kv
        # head together; agrees with the per-head one to fp32 rounding)
        self._partials = (oatt.splitkv_partials_grouped if grouped_attention
                          else oatt.splitkv_partials)
        # activation "gelu": the bf16 table of the reference model's GELU
        # (cfg "gelu_lut", bits; default the correctly rounded table)
        self.gelu_lut = cfg.get("gelu_lut")
        if cfg.get("activation") == "gelu" and self.gelu_lut is None:
            self.gelu_lut = oops.gelu_table()
        c = cfg
        # the tied embedding: bf16 of the dequantised head (the C restatement,
        # which tests/test_oracle_q4_0.py checks bit for bit against numpy's)
        self.embed = bf16_bits_to_f32(oq.c_dequant_bf16_bits(weights["head"], c["vocab"],
                                                             c["hidden"]))
        self.reset()

    def reset(self):
        c = self.c
        self.k = [np.zeros((0, c["n_kv"], c["head_dim"]), np.float32) for _ in range(c["n_layers"])]
        self.v = [np.zeros((0, c["n_kv"], c["head_dim"]), np.float32) for _ in range(c["n_layers"])]

    def _append_kv(self, i: int, k: np.ndarray, v: np.ndarray) -> None:
        """self.k[i] / self.v[i] grow by one token.  They are views of
        backing arrays with spare rows, so a step copies one token, not the
        whole cache (a caller may also assign self.k[i] an array of its own:
        it is moved into a new backing array on the next append)."""
        if not hasattr(self, "_kv_back"):
            self._kv_back = {}
        n = self.k[i].shape[0]
        back = self._kv_back.get(i)
        if (back is None or self.k[i].base is not back[0] or self.v[i].base is not back[1]
                or back[0].shape[0] <= n):
            cap = max(2 * n, n + 256)
            kb = np.empty((cap,) + self.k[i].shape[1:], np.float32)
            vb = np.empty((cap,) + self.v[i].shape[1:], np.float32)
            kb[:n] = self.k[i]
            vb[:n] = self.v[i]
            back = self._kv_back[i] = (kb, vb)
        back[0][n] = k
        back[1][n] = v
        self.k[i] = back[0][:n + 1]
        self.v[i] = back[1][:n + 1]

    def layer(self, i: int, h: np.ndarray, res: np.ndarray, pos: int):
        c, w = self.c, self.w
        nq, nkv, hd, H, I = c["n_q"], c["n_kv"], c["head_dim"], c["hidden"], c["intermediate"]
        eps = c["eps"]
        qkv = _gemv(h, w[f"layers.{i}.qkv"], (nq + 2 * nkv) * hd, H)
        q = qkv[:nq * hd].reshape(nq, hd)
        k = qkv[nq * hd:(nq + nkv) * hd].reshape(nkv, hd)
        v = qkv[(nq + nkv) * hd:].reshape(nkv, hd)
        row = self.cos_sin[pos]
        qr = oops.apply_rope(oops.rms_norm(q, w[f"layers.{i}.norm2"], eps), row)
        kr = oops.apply_rope(oops.rms_norm(k, w[f"layers.{i}.norm3"], eps), row)
        self._append_kv(i, kr, v)
        L = pos + 1
        po, pl = self._partials(qr, self.k[i][:L], self.v[i][:L], hd ** -0.5,
                                oatt.split_bounds(L, self.num_splits, self.capacity))
        attn = oatt.lse_merge(po, pl).reshape(nq * hd)
        o = _gemv(attn, w[f"layers.{i}.o_proj"], H, nq * hd)
        h2, res = oops.add_rmsnorm(o, res, w[f"layers.{i}.norm1"], eps)
        gu = _gemv(h2, w[f"layers.{i}.gate_up"], 2 * I, H)
        if c.get("activation", "swiglu") == "gelu":  # the reference model's table GELU
            act = oops.gelu_mul(f32_to_bf16_bits(gu[:I]), gu[I:], self.gelu_lut)
        else:
            act = oops.silu_mul(gu[:I], gu[I:])
        d = _gemv(act, w[f"layers.{i}.down"], H, I)
        nxt = w[f"layers.{i + 1}.norm0"] if i + 1 < c["n_layers"] else w["final_norm"]
        return oops.add_rmsnorm(d, res, nxt, eps)

    def step(self, token: int, pos: int) -> np.ndarray:
        """Feed `token` at `pos`; returns float64 logits."""
        c, w = self.c, self.w
        x = self.embed[token]
        h, res = oops.add_rmsnorm(x, None, w["layers.0.norm0"], c["eps"])
        res = x
        for i in range(c["n_layers"]):
            h, res = self.layer(i, h, res, pos)
        self.last_hidden = h
        return oq.gemv_f64(f32_to_bf16_bits(h), w["head"], c["vocab"], c["hidden"])


def top2_margin(logits64: np.ndarray) -> tuple[int, float]:
    """(argmax, (top1 - top2) / |top1|) of float64 logits."""
    order = np.argsort(-logits64, kind="stable")
    t1, t2 = logits64[order[0]], logits64[order[1]]
    return int(order[0]), float((t1 - t2) / max(abs(t1), 1e-30))


def bf16_argmax(logits64: np.ndarray) -> int:
    """argmax of the bf16-rounded logits, lowest index on ties."""
    return int(np.argmax(round_bf16(logits64.astype(np.float32))))
