"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the oracle).

CPU: the oracle still reproduces every fixture, and the fixtures agree with
textbook forms computed here independently (a float64 matmul over the
dequantised weights, the float64 softmax attention).
GPU: the HIP path on the fixture inputs against the fixture outputs --
dequant bit-exact, the GEMV within 1e-2 relative, attention partials within
1e-4 (lse) / 2e-2 of each split's RMS, the merged output within 1e-2 of its
RMS plus its bf16 rounding, the tiny decoder's logits within 2e-2 with
greedy tokens equal except at near-ties.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import model as omodel
from oracle import q4_0 as oq
from oracle.bf16 import bf16_bits_to_f32

from _util import (assert_attention_close, assert_close_rel, assert_partials_close, bf16_dev,
                   f32_of, pkg)

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


# ----------------------------------------------------------------- CPU side
def test_kat_fixture_matches_oracle():
    g = load("q4_0_kat.npz")
    b = g["blocks"]
    n = b.shape[0]
    with np.errstate(invalid="ignore"):
        np.testing.assert_array_equal(oq.dequant_f32(b, n, 32).view(np.uint32), g["f32_bits"])
        np.testing.assert_array_equal(oq.c_dequant_f32(b, n, 32).view(np.uint32), g["f32_bits"])
        np.testing.assert_array_equal(oq.dequant_bf16_bits(b, n, 32), g["bf16_bits"])
    f = g["f32_bits"].view(np.float32)
    np.testing.assert_array_equal(f[0], (np.arange(32) % 16 - 8).astype(np.float32))
    assert np.all(np.isnan(f[4][np.arange(32) % 16 == 8]))  # inf * 0
    assert f[8][0] == 7 and f[8][16] == -7  # byte 0x1F


def test_gemv_fixture_matches_textbook():
    g = load("gemv_64x256.npz")
    n, k = int(g["n"]), int(g["k"])
    np.testing.assert_array_equal(oq.gemv_f64(g["x_bits"], g["blocks"], n, k), g["y_f64"])
    w = oq.dequant_f32(g["blocks"], n, k).astype(np.float64)
    np.testing.assert_allclose(w @ bf16_bits_to_f32(g["x_bits"]).astype(np.float64), g["y_f64"],
                               rtol=1e-12, atol=1e-12)


def test_attention_fixture_matches_textbook():
    g = load("attention_ctx300.npz")
    kf, vf, qf = (bf16_bits_to_f32(g[x]) for x in ("k_bits", "v_bits", "q_bits"))
    L = int(g["length"])
    ref = oatt.attention_f64(qf, oatt.gather_paged(kf, g["table"], L),
                             oatt.gather_paged(vf, g["table"], L), float(g["scale"]))
    np.testing.assert_allclose(ref, g["out_f64"], rtol=0, atol=1e-12)
    for s in (2, 3):
        o, po, pl = oatt.splitkv_decode(qf, kf, vf, g["table"], L, s, float(g["scale"]))
        np.testing.assert_array_equal(po, g[f"partial_o{s}"])
        np.testing.assert_array_equal(pl, g[f"partial_lse{s}"])
        assert np.abs(bf16_bits_to_f32(g[f"out{s}_bf16_bits"]) - g["out_f64"]).max() < 1e-2


def _tiny(g):
    c = {k[4:]: g[k] for k in g if k.startswith("cfg.")}
    w = {k[2:]: g[k] for k in g if k.startswith("w.")}
    return c, w


def test_model_fixture_matches_oracle():
    g = load("model_tiny.npz")
    c, w = _tiny(g)
    wf = {k: (bf16_bits_to_f32(v) if v.dtype == np.uint16 else v) for k, v in w.items()}
    cfg = {k: int(c[k]) for k in ("hidden", "n_layers", "n_q", "n_kv", "head_dim",
                                  "intermediate", "vocab")}
    cfg["eps"] = float(c["eps"])
    cap = -(-int(c["max_len"]) // int(c["block_size"])) * int(c["block_size"])
    dec = omodel.OracleDecoder(cfg, wf, bf16_bits_to_f32(g["cos_sin_bits"]),
                               num_splits=int(g["num_splits"]), capacity=cap)
    for pos, tok in enumerate(g["tokens"]):
        lg = dec.step(int(tok), pos)
        np.testing.assert_allclose(lg, g["logits_f64"][pos], rtol=1e-9, atol=1e-9)
        assert omodel.bf16_argmax(lg) == g["greedy"][pos]


# ----------------------------------------------------------------- GPU side
@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _u8(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.gpu
def test_gpu_dequant_kat(dev):
    ops = pkg("native.torch_ops")
    g = load("q4_0_kat.npz")
    n = g["blocks"].shape[0]
    out = ops.q4_0_dequant_bf16(_u8(g["blocks"], dev), n, 32)
    import torch
    got = out.view(torch.int16).cpu().numpy().view(np.uint16).reshape(n, 32)
    np.testing.assert_array_equal(got, g["bf16_bits"])


@pytest.mark.gpu
def test_gpu_gemv_fixture(dev):
    ops = pkg("native.torch_ops")
    g = load("gemv_64x256.npz")
    n, k = int(g["n"]), int(g["k"])
    y = ops.q4_0_gemv(bf16_dev(g["x_bits"], dev), _u8(g["blocks"], dev), n, k)
    assert_close_rel(f32_of(y).reshape(n), g["y_f64"], rtol=1e-2, atol_frac=5e-3, what="gemv")


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [2, 3])
def test_gpu_attention_fixture(dev, splits):
    import torch
    ops = pkg("native.torch_ops")
    g = load("attention_ctx300.npz")
    L = int(g["length"])
    q = bf16_dev(g["q_bits"], dev).view(1, 4, 128)
    table = torch.from_numpy(g["table"]).view(1, -1).to(dev)
    sl = torch.tensor([L], dtype=torch.int32, device=dev)
    po, pl = ops.splitkv_decode(q, bf16_dev(g["k_bits"], dev), bf16_dev(g["v_bits"], dev), table,
                                sl, splits, float(g["scale"]))
    out = ops.lse_merge(po, pl)
    pl_ref = g[f"partial_lse{splits}"]
    assert_partials_close(po.cpu().numpy().reshape(g[f"partial_o{splits}"].shape),
                          pl.cpu().numpy().reshape(pl_ref.shape), g[f"partial_o{splits}"], pl_ref,
                          f"{splits} splits")
    assert_attention_close(f32_of(out).reshape(4, 128), g["out_f64"], "merged output")


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [True, False])
def test_gpu_tiny_model_fixture(dev, fused):
    import torch
    m = pkg("integration.model")
    g = load("model_tiny.npz")
    c, w = _tiny(g)
    weights = {k: (bf16_dev(v, dev) if v.dtype == np.uint16 else _u8(v, dev)) for k, v in w.items()}
    cfg = m.DecoderConfig(hidden=int(c["hidden"]), n_layers=int(c["n_layers"]), n_q=int(c["n_q"]),
                          n_kv=int(c["n_kv"]), head_dim=int(c["head_dim"]),
                          intermediate=int(c["intermediate"]), vocab=int(c["vocab"]),
                          eps=float(c["eps"]), rope_theta=float(c["theta"]),
                          block_size=int(c["block_size"]))
    model = m.DecodeModel(cfg, dev, max_len=int(c["max_len"]), num_splits=int(g["num_splits"]),
                          weights=weights, fused=fused)
    model.reset(torch.from_numpy(g["tokens"]))
    for pos in range(len(g["tokens"])):
        model.step()
        torch.cuda.synchronize()
        ref = g["logits_f64"][pos]
        assert_close_rel(f32_of(model.logits).reshape(-1), ref, rtol=2e-2, atol_frac=2e-2,
                         what=f"logits at {pos}")
        tok = int(model.state.next_ids.item())
        if tok != g["greedy"][pos]:
            assert g["margin"][pos] < omodel.NEAR_TIE_REL, f"step {pos}: {tok} vs {g['greedy'][pos]}"
