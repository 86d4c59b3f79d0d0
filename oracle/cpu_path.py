"""The reference's PyTorch CPU path for one decode step -- the CPU baseline
(test infrastructure; bench.py's cpu_baseline leg times it).

The reference deploys Q4_0 weights by dequantising them with gguf and
casting to bf16 (src/spark_vllm_ascend/integration/weights.py:28-32,
src/tools/deployment/prepare_model.py:62-64) and runs vLLM's stock modules
on them (``F.linear`` for every projection); its own CPU threads are pinned
with OMP_NUM_THREADS=4 (src/tools/deployment/run_user.sh:35).  This class
restates that path on torch CPU at the 4B decoder's shapes: bf16 weights,
F.linear, fp32 softmax attention over a contiguous bf16 KV cache, RMSNorm
and RoPE in fp32 with bf16 stage outputs, greedy argmax.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def _rms(x: torch.Tensor, gamma: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * inv * gamma.float()).to(torch.bfloat16)


def _rope(x: torch.Tensor, cs: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    a, b = x[..., :half].float(), x[..., half:].float()
    c, s = cs[:half].float(), cs[half:].float()
    return torch.cat((a * c - b * s, b * c + a * s), dim=-1).to(torch.bfloat16)


class CpuDecoder:
    """weights: per layer dict(qkv, o_proj, gate_up, down: bf16 [out, in];
    input_norm, post_norm, q_norm, k_norm: bf16), plus final_norm and the
    tied bf16 head/embedding [vocab, hidden]."""

    def __init__(self, cfg, layers: list[dict], final_norm: torch.Tensor, head: torch.Tensor,
                 cos_sin: torch.Tensor, max_len: int):
        self.c = cfg
        self.layers = layers
        self.final_norm = final_norm
        self.head = head
        self.cos_sin = cos_sin
        kv_shape = (max_len, cfg.n_kv, cfg.head_dim)
        self.k = [torch.zeros(kv_shape, dtype=torch.bfloat16) for _ in layers]
        self.v = [torch.zeros(kv_shape, dtype=torch.bfloat16) for _ in layers]

    def fill_cache(self, length: int, seed: int = 0) -> None:
        g = torch.Generator().manual_seed(seed)
        for k, v in zip(self.k, self.v):
            k[:length] = torch.randn(k[:length].shape, generator=g).to(torch.bfloat16)
            v[:length] = torch.randn(v[:length].shape, generator=g).to(torch.bfloat16)

    @torch.inference_mode()
    def step(self, token: int, pos: int) -> int:
        c = self.c
        nq, nkv, hd = c.n_q, c.n_kv, c.head_dim
        x = self.head[token].view(1, -1)
        res = x.float()
        h = _rms(x, self.layers[0]["input_norm"], c.eps)
        cs = self.cos_sin[pos]
        for i, L in enumerate(self.layers):
            qkv = F.linear(h, L["qkv"])
            q = _rope(_rms(qkv[:, :nq * hd].view(nq, hd), L["q_norm"], c.eps), cs)
            k = _rope(_rms(qkv[:, nq * hd:(nq + nkv) * hd].view(nkv, hd), L["k_norm"], c.eps), cs)
            v = qkv[:, (nq + nkv) * hd:].view(nkv, hd)
            self.k[i][pos] = k
            self.v[i][pos] = v
            kk = self.k[i][:pos + 1].float().repeat_interleave(nq // nkv, dim=1)  # [L, nq, hd]
            vv = self.v[i][:pos + 1].float().repeat_interleave(nq // nkv, dim=1)
            s = torch.einsum("hd,lhd->hl", q.float(), kk) / math.sqrt(hd)
            attn = torch.einsum("hl,lhd->hd", torch.softmax(s, dim=-1), vv).to(torch.bfloat16)
            o = F.linear(attn.view(1, -1), L["o_proj"])
            res = res + o.float()
            h2 = _rms(res, L["post_norm"], c.eps)
            res = res.to(torch.bfloat16).float()
            gu = F.linear(h2, L["gate_up"])
            g, u = gu[:, :c.intermediate].float(), gu[:, c.intermediate:].float()
            act = (F.silu(g) * u).to(torch.bfloat16)
            d = F.linear(act, L["down"])
            res = res + d.float()
            nxt = self.layers[i + 1]["input_norm"] if i + 1 < len(self.layers) else self.final_norm
            h = _rms(res, nxt, c.eps)
            res = res.to(torch.bfloat16).float()
        logits = F.linear(h, self.head)
        return int(torch.argmax(logits.float()))
