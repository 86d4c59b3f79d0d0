"""Pins for the oracle decoder (CPU only): its greedy tokens against the
independently written torch CPU path (the reference's bf16 F.linear path),
a zero-weight layer passing the residual through, and split-count
invariance of the logits."""
from types import SimpleNamespace

import numpy as np
import torch

from oracle import model as omodel
from oracle import ops as oops
from oracle import q4_0 as oq
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from oracle.cpu_path import CpuDecoder

CFG = dict(hidden=256, n_layers=2, n_q=8, n_kv=2, head_dim=128, intermediate=512, vocab=1000,
           eps=1e-6)


def make_weights(seed=0, zero=False):
    c = CFG
    rng = np.random.default_rng(seed)
    w = {}
    shapes = {"qkv": ((c["n_q"] + 2 * c["n_kv"]) * c["head_dim"], c["hidden"]),
              "o_proj": (c["hidden"], c["n_q"] * c["head_dim"]),
              "gate_up": (2 * c["intermediate"], c["hidden"]),
              "down": (c["hidden"], c["intermediate"])}
    for i in range(c["n_layers"]):
        for j, (name, (n, k)) in enumerate(shapes.items()):
            b = oq.make_blocks(n, k, seed=seed * 100 + i * 10 + j)
            if zero:
                b = b.reshape(n, k // 32, 18).copy()
                b[:, :, :2] = 0
                b = b.reshape(n, -1)
            w[f"layers.{i}.{name}"] = b
        for j, n in enumerate((c["hidden"], c["hidden"], c["head_dim"], c["head_dim"])):
            w[f"layers.{i}.norm{j}"] = round_bf16((1 + 0.1 * rng.standard_normal(n)).astype(np.float32))
    w["final_norm"] = round_bf16((1 + 0.1 * rng.standard_normal(c["hidden"])).astype(np.float32))
    w["head"] = oq.make_blocks(c["vocab"], c["hidden"], seed=seed * 100 + 99)
    return w


def cos_sin(max_pos=64):
    return round_bf16(oops.rope_cache(max_pos, 128, 1e6))


def as_bf16(a):
    return torch.from_numpy(f32_to_bf16_bits(np.asarray(a, np.float32)).view(np.int16)).view(torch.bfloat16)


def cpu_decoder(w, max_len=64):
    c = CFG
    deq = lambda b, n, k: torch.from_numpy(oq.dequant_bf16_bits(b, n, k).view(np.int16)).view(torch.bfloat16)
    layers = []
    for i in range(c["n_layers"]):
        layers.append({
            "qkv": deq(w[f"layers.{i}.qkv"], (c["n_q"] + 2 * c["n_kv"]) * 128, c["hidden"]),
            "o_proj": deq(w[f"layers.{i}.o_proj"], c["hidden"], c["n_q"] * 128),
            "gate_up": deq(w[f"layers.{i}.gate_up"], 2 * c["intermediate"], c["hidden"]),
            "down": deq(w[f"layers.{i}.down"], c["hidden"], c["intermediate"]),
            "input_norm": as_bf16(w[f"layers.{i}.norm0"]), "post_norm": as_bf16(w[f"layers.{i}.norm1"]),
            "q_norm": as_bf16(w[f"layers.{i}.norm2"]), "k_norm": as_bf16(w[f"layers.{i}.norm3"])})
    head = deq(w["head"], c["vocab"], c["hidden"])
    cfg = SimpleNamespace(**c)
    return CpuDecoder(cfg, layers, as_bf16(w["final_norm"]), head, as_bf16(cos_sin(max_len)), max_len)


def test_oracle_decoder_agrees_with_torch_cpu_path():
    w = make_weights(seed=1)
    orc = omodel.OracleDecoder(CFG, w, cos_sin(), num_splits=2)
    cpu = cpu_decoder(w)
    rng = np.random.default_rng(5)
    seq = rng.integers(0, CFG["vocab"], 24)
    disagree = 0
    for pos, tok in enumerate(seq):
        lo = orc.step(int(tok), pos)
        tc = cpu.step(int(tok), pos)
        to = omodel.bf16_argmax(lo)
        if tc != to:
            _, margin = omodel.top2_margin(lo)
            assert margin < omodel.NEAR_TIE_REL, f"pos {pos}: {tc} vs {to}, margin {margin}"
            disagree += 1
    assert disagree <= 3


def test_zero_weight_layer_passes_residual_through():
    w = make_weights(seed=2, zero=True)
    orc = omodel.OracleDecoder(CFG, w, cos_sin(), num_splits=1)
    rng = np.random.default_rng(0)
    h = round_bf16(rng.standard_normal(CFG["hidden"]).astype(np.float32))
    res = round_bf16(rng.standard_normal(CFG["hidden"]).astype(np.float32))
    y, r = orc.layer(0, h, res, 0)
    np.testing.assert_array_equal(r, res)
    ref, _ = oops.add_rmsnorm(res, None, w["layers.1.norm0"], CFG["eps"])
    np.testing.assert_array_equal(y, ref)


def test_logits_invariant_to_split_count():
    w = make_weights(seed=3)
    a = omodel.OracleDecoder(CFG, w, cos_sin(), num_splits=1)
    b = omodel.OracleDecoder(CFG, w, cos_sin(), num_splits=4)
    for pos, tok in enumerate([5, 17, 900, 3, 3, 41, 7, 8, 100, 2]):
        la, lb = a.step(tok, pos), b.step(tok, pos)
        assert np.max(np.abs(la - lb)) <= 2e-2 * np.max(np.abs(la))
