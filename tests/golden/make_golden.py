"""Writes the golden fixtures of this directory from the oracle (run from the
repository root: ``python tests/golden/make_golden.py``).

The reference ships no golden vectors for Q4_0 decode, the Q4_0 GEMV,
split-KV attention, RMSNorm, RoPE or SwiGLU, so these fixtures are produced
by the oracle, whose functions are pinned independently by closed forms and
invariants (tests/test_oracle_*.py).  Each file holds inputs and expected
outputs only (numpy .npz, no pickles):

  q4_0_kat.npz        GGUF Q4_0 known-answer blocks (unit scale, nibble order,
                      -0, fp16 subnormal, 65504, +-inf, NaN scales) with their
                      exact fp32 values and bf16 bits.
  gemv_64x256.npz     Q4_0 GEMV N=64, K=256: blocks, x, float64 y and bf16 y.
  attention_ctx300.npz  split-KV decode at context 300 (a partial last page),
                      1 kv head / 4 q heads, block size 32, shuffled block
                      table: float64 textbook output, the split partials and
                      merged bf16 output for 2 and 3 splits.
  model_tiny.npz      a 2-layer decoder (hidden 128, 4 q / 1 kv heads of 128,
                      SwiGLU 128, vocab 256, block size 32): all weights, the
                      rotary table, 8 teacher-forced tokens, float64 logits
                      and greedy tokens of every step.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle import attention as oatt  # noqa: E402
from oracle import model as omodel  # noqa: E402
from oracle import ops as oops  # noqa: E402
from oracle import q4_0 as oq  # noqa: E402
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits  # noqa: E402

TINY = dict(hidden=128, n_layers=2, n_q=4, n_kv=1, head_dim=128, intermediate=128, vocab=256,
            eps=1e-6, block_size=32, max_len=64, theta=1e6)


def kat_blocks() -> np.ndarray:
    codes = (np.arange(32) % 16).astype(np.uint8)
    rows = []
    for d in (1.0, -0.0, 2.0 ** -24, 65504.0, np.inf, -np.inf, np.nan, 0.5):
        rows.append(oq.pack_blocks(np.array([[d]], dtype=np.float16), codes.reshape(1, 1, 32)))
    nib = np.zeros((1, 18), dtype=np.uint8)  # byte 0 = 0x1F: element 0 -> 7, element 16 -> -7
    nib[0, 0:2] = np.array([1.0], dtype="<f2").view(np.uint8)
    nib[0, 2] = 0x1F
    nib[0, 3:] = 0x88
    rows.append(nib)
    return np.concatenate(rows, axis=0)


def make_kat(out: Path) -> None:
    blocks = kat_blocks()
    n = blocks.shape[0]
    with np.errstate(invalid="ignore"):  # inf * (8 - 8) is NaN by definition
        f32 = oq.dequant_f32(blocks, n, 32)
        bf16 = oq.dequant_bf16_bits(blocks, n, 32)
    np.savez(out / "q4_0_kat.npz", blocks=blocks, f32_bits=f32.view(np.uint32), bf16_bits=bf16)


def make_gemv(out: Path) -> None:
    n, k = 64, 256
    blocks = oq.make_blocks(n, k, seed=64)
    x = f32_to_bf16_bits(np.random.default_rng(256).standard_normal(k).astype(np.float32))
    y64 = oq.gemv_f64(x, blocks, n, k)
    np.savez(out / "gemv_64x256.npz", blocks=blocks, x_bits=x, y_f64=y64,
             y_bf16_bits=f32_to_bf16_bits(y64.astype(np.float32)), n=n, k=k)


def make_attention(out: Path) -> None:
    rng = np.random.default_rng(300)
    L, bs, n_q, n_kv, hd = 300, 32, 4, 1, 128
    need = -(-L // bs)
    nblk = need + 2
    table = rng.permutation(nblk).astype(np.int32)[:need + 1]  # one spare entry past the end
    kc = f32_to_bf16_bits(rng.standard_normal((nblk, bs, n_kv, hd)).astype(np.float32))
    vc = f32_to_bf16_bits(rng.standard_normal((nblk, bs, n_kv, hd)).astype(np.float32))
    q = f32_to_bf16_bits(rng.standard_normal((n_q, hd)).astype(np.float32))
    scale = hd ** -0.5
    kf, vf, qf = bf16_bits_to_f32(kc), bf16_bits_to_f32(vc), bf16_bits_to_f32(q)
    ref = oatt.attention_f64(qf, oatt.gather_paged(kf, table, L), oatt.gather_paged(vf, table, L),
                             scale)
    res = dict(q_bits=q, k_bits=kc, v_bits=vc, table=table, length=L, scale=scale, out_f64=ref)
    for s in (2, 3):
        o, po, pl = oatt.splitkv_decode(qf, kf, vf, table, L, s, scale)
        res[f"out{s}_bf16_bits"] = f32_to_bf16_bits(o)
        res[f"partial_o{s}"] = po
        res[f"partial_lse{s}"] = pl
    np.savez(out / "attention_ctx300.npz", **res)


def tiny_weights(rng) -> dict:
    c = TINY
    hd, H, I = c["head_dim"], c["hidden"], c["intermediate"]
    w = {}
    for i in range(c["n_layers"]):
        s = 1000 + 10 * i
        w[f"layers.{i}.qkv"] = oq.make_blocks((c["n_q"] + 2 * c["n_kv"]) * hd, H, seed=s)
        w[f"layers.{i}.o_proj"] = oq.make_blocks(H, c["n_q"] * hd, seed=s + 1)
        w[f"layers.{i}.gate_up"] = oq.make_blocks(2 * I, H, seed=s + 2)
        w[f"layers.{i}.down"] = oq.make_blocks(H, I, seed=s + 3)
        for j, n in enumerate((H, H, hd, hd)):
            w[f"layers.{i}.norm{j}"] = f32_to_bf16_bits(
                (1 + 0.1 * rng.standard_normal(n)).astype(np.float32))
    w["final_norm"] = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    w["head"] = oq.make_blocks(c["vocab"], H, seed=999, scale=0.05)
    return w


def make_model(out: Path) -> None:
    c = TINY
    rng = np.random.default_rng(2)
    w = tiny_weights(rng)
    cs = f32_to_bf16_bits(oops.rope_cache(c["max_len"], c["head_dim"], c["theta"]))
    wf = {k: (bf16_bits_to_f32(v) if v.dtype == np.uint16 else v) for k, v in w.items()}
    cfg = {k: c[k] for k in ("hidden", "n_layers", "n_q", "n_kv", "head_dim", "intermediate",
                             "vocab", "eps")}
    cap = -(-c["max_len"] // c["block_size"]) * c["block_size"]
    dec = omodel.OracleDecoder(cfg, wf, bf16_bits_to_f32(cs), num_splits=2, capacity=cap)
    tokens = rng.integers(0, c["vocab"], 8).astype(np.int64)
    logits, greedy, margin = [], [], []
    for pos, tok in enumerate(tokens):
        lg = dec.step(int(tok), pos)
        logits.append(lg)
        greedy.append(omodel.bf16_argmax(lg))
        margin.append(omodel.top2_margin(lg)[1])
    np.savez(out / "model_tiny.npz", **{f"w.{k}": v for k, v in w.items()}, cos_sin_bits=cs,
             tokens=tokens, logits_f64=np.array(logits), greedy=np.array(greedy, dtype=np.int64),
             margin=np.array(margin), num_splits=2,
             **{f"cfg.{k}": v for k, v in c.items()})


def main() -> None:
    make_kat(HERE)
    make_gemv(HERE)
    make_attention(HERE)
    make_model(HERE)
    for p in sorted(HERE.glob("*.npz")):
        print(f"{p.name}: {p.stat().st_size} bytes")


if __name__ == "__main__":
    main()
