"""GGUF reader/writer and the decoder tensor mapping.

The reader is pinned against a file assembled byte by byte here from the
GGUF v3 layout (independently of write_gguf): header, typed metadata
(scalar, string, array), tensor infos, alignment padding, tensor data.
gguf-py (the reference's reader, gguf==0.19.0) is not installed, so
equality with it is not checked: parity with it is unpinned beyond the file
format itself."""
import struct

import numpy as np
import pytest

from oracle import q4_0 as oq

from _util import pkg


def gf():
    return pkg("integration.gguf_file")


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def handmade(tmp_path, alignment=32):
    """One F32 [2, 3] tensor and one Q4_0 [2, 64] tensor, by hand."""
    f32 = np.arange(6, dtype="<f4").reshape(2, 3)
    q4 = oq.make_blocks(2, 64, seed=1)
    md = [(_s("general.architecture"), 8, _s("qwen3")),
          (_s("qwen3.block_count"), 4, struct.pack("<I", 7)),
          (_s("some.floats"), 9, struct.pack("<IQ", 6, 2) + struct.pack("<2f", 1.5, -2.0))]
    if alignment != 32:
        md.append((_s("general.alignment"), 4, struct.pack("<I", alignment)))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, len(md))
    for k, t, v in md:
        head += k + struct.pack("<I", t) + v
    head += _s("a.f32") + struct.pack("<I", 2) + struct.pack("<QQ", 3, 2) + struct.pack("<IQ", 0, 0)
    off2 = -(-f32.nbytes // alignment) * alignment
    head += _s("b.q4") + struct.pack("<I", 2) + struct.pack("<QQ", 64, 2) + struct.pack("<IQ", 2, off2)
    data_start = -(-len(head) // alignment) * alignment
    blob = head + b"\0" * (data_start - len(head)) + f32.tobytes()
    blob += b"\0" * (data_start + off2 - len(blob)) + q4.tobytes()
    p = tmp_path / "hand.gguf"
    p.write_bytes(blob)
    return p, f32, q4


@pytest.mark.parametrize("alignment", [32, 64])
def test_reader_on_handmade_file(tmp_path, alignment):
    p, f32, q4 = handmade(tmp_path, alignment)
    g = gf().GGUFFile(p)
    assert g.version == 3 and g.alignment == alignment
    assert g.metadata["general.architecture"] == "qwen3"
    assert g.metadata["qwen3.block_count"] == 7
    np.testing.assert_array_equal(g.metadata["some.floats"], np.float32([1.5, -2.0]))
    a = g.tensor("a.f32")
    assert a.shape == (2, 3) and a.dims == (3, 2)
    np.testing.assert_array_equal(a.float32(), f32)
    b = g.tensor("b.q4")
    assert b.shape == (2, 64)
    np.testing.assert_array_equal(b.q4_0_blocks(), q4)
    assert g.data_offset % alignment == 0


def test_writer_round_trip(tmp_path):
    m = gf()
    q = oq.make_blocks(8, 256, seed=3)
    h = np.random.default_rng(0).standard_normal(256).astype("<f2")
    tensors = [("w.q4", m.GGML_Q4_0, (8, 256), q), ("n.f16", m.GGML_F16, (256,), h.view(np.uint8)),
               ("e.f32", m.GGML_F32, (3,), np.float32([1, 2, 3]).view(np.uint8))]
    md = {"general.architecture": "qwen3", "x.u": 5, "x.f": 0.25, "x.s": "hi", "x.b": True,
          "x.arr": np.int32([1, -2, 3]), "x.strs": ["a", "bc"]}
    p = tmp_path / "rt.gguf"
    m.write_gguf(p, md, tensors, alignment=64)
    g = m.GGUFFile(p)
    assert g.alignment == 64
    for k, v in md.items():
        got = g.metadata[k]
        if isinstance(v, np.ndarray):
            np.testing.assert_array_equal(got, v)
        elif isinstance(v, float):
            assert got == pytest.approx(v)
        else:
            assert got == v
    np.testing.assert_array_equal(g.tensor("w.q4").q4_0_blocks(), q)
    np.testing.assert_array_equal(g.tensor("n.f16").float32(), h.astype(np.float32))
    np.testing.assert_array_equal(g.tensor("e.f32").float32(), [1, 2, 3])
    assert [t.name for t in g.tensors] == ["w.q4", "n.f16", "e.f32"]
    assert all(t.offset % 64 == 0 for t in g.tensors)


def test_reader_rejects_bad_files(tmp_path):
    m = gf()
    p, _, _ = handmade(tmp_path)
    blob = p.read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + blob[4:])
    with pytest.raises(ValueError, match="not a GGUF"):
        m.GGUFFile(bad)
    bad.write_bytes(blob[:-10])
    with pytest.raises(ValueError):
        m.GGUFFile(bad)
    bad.write_bytes(blob[:40])
    with pytest.raises(ValueError, match="truncated"):
        m.GGUFFile(bad)
    with pytest.raises(ValueError, match="not Q4_0"):
        m.GGUFFile(p).tensor("a.f32").q4_0_blocks()


def tiny_qwen3_file(tmp_path, layers=2, hidden=128, n_q=4, n_kv=1, hd=128, inter=128, vocab=256):
    m = gf()
    rng = np.random.default_rng(9)
    md = {"general.architecture": "qwen3", "qwen3.embedding_length": hidden,
          "qwen3.block_count": layers, "qwen3.attention.head_count": n_q,
          "qwen3.attention.head_count_kv": n_kv, "qwen3.attention.key_length": hd,
          "qwen3.feed_forward_length": inter, "qwen3.attention.layer_norm_rms_epsilon": 1e-6,
          "qwen3.rope.freq_base": 1e6}
    ts = []
    seed = 100

    def q4(name, n, k):
        nonlocal seed
        seed += 1
        ts.append((name, m.GGML_Q4_0, (n, k), oq.make_blocks(n, k, seed=seed)))

    def nrm(name, n):
        ts.append((name, m.GGML_F32, (n,),
                   (1 + 0.1 * rng.standard_normal(n)).astype("<f4").view(np.uint8)))
    q4("token_embd.weight", vocab, hidden)
    for i in range(layers):
        b = f"blk.{i}."
        q4(b + "attn_q.weight", n_q * hd, hidden)
        q4(b + "attn_k.weight", n_kv * hd, hidden)
        q4(b + "attn_v.weight", n_kv * hd, hidden)
        q4(b + "attn_output.weight", hidden, n_q * hd)
        q4(b + "ffn_gate.weight", inter, hidden)
        q4(b + "ffn_up.weight", inter, hidden)
        q4(b + "ffn_down.weight", hidden, inter)
        for n, sz in (("attn_norm", hidden), ("ffn_norm", hidden), ("attn_q_norm", hd),
                      ("attn_k_norm", hd)):
            nrm(b + n + ".weight", sz)
    nrm("output_norm.weight", hidden)
    p = tmp_path / "tiny.gguf"
    m.write_gguf(p, md, ts)
    return p, dict((t[0], t[3]) for t in ts)


def test_decoder_mapping(tmp_path):
    m = gf()
    p, raw = tiny_qwen3_file(tmp_path)
    g = m.GGUFFile(p)
    cfg = m.decoder_config(g)
    assert cfg == dict(hidden=128, n_layers=2, n_q=4, n_kv=1, head_dim=128, intermediate=128,
                       vocab=256, eps=pytest.approx(1e-6), rope_theta=1e6)
    w = m.decoder_weights(g, 2)
    np.testing.assert_array_equal(
        w["layers.1.qkv"], np.concatenate([raw[f"blk.1.attn_{x}.weight"] for x in "qkv"]))
    np.testing.assert_array_equal(
        w["layers.0.gate_up"], np.concatenate([raw["blk.0.ffn_gate.weight"], raw["blk.0.ffn_up.weight"]]))
    np.testing.assert_array_equal(w["head"], raw["token_embd.weight"])  # tied
    np.testing.assert_array_equal(w["layers.0.norm2"], raw["blk.0.attn_q_norm.weight"].view("<f4"))


@pytest.mark.gpu
@pytest.mark.parametrize("activation", ["swiglu", "gelu"])
def test_model_from_gguf_against_oracle(tmp_path, activation):
    """A decoder loaded from a GGUF file, teacher-forced against the oracle
    decoder built from the same file's tensors -- with SwiGLU, and with the
    reference model's table GELU named at load time."""
    import torch
    from oracle import model as omodel
    from oracle.bf16 import round_bf16
    from _util import assert_close_rel, f32_of
    p, _ = tiny_qwen3_file(tmp_path)
    mm = pkg("integration.model")
    dev = torch.device("cuda:0")
    model = mm.DecodeModel.from_gguf(p, dev, max_len=64, num_splits=2, block_size=32,
                                     activation=activation)
    assert model.cfg.activation == activation and (model.act_lut is not None) == (
        activation == "gelu")
    g = gf().GGUFFile(p)
    cfg = gf().decoder_config(g)
    w = {k: (round_bf16(v) if v.dtype == np.float32 else v)
         for k, v in gf().decoder_weights(g, cfg["n_layers"]).items()}
    ocfg = {k: cfg[k] for k in ("hidden", "n_layers", "n_q", "n_kv", "head_dim", "intermediate",
                                "vocab", "eps")}
    ocfg["activation"] = activation
    if activation == "gelu":
        from _util import bits_of
        ocfg["gelu_lut"] = bits_of(model.act_lut)
    cap = model.state.block_table.shape[1] * 32
    oracle = omodel.OracleDecoder(ocfg, w, f32_of(model.cos_sin), num_splits=2, capacity=cap)
    seq = np.array([3, 17, 200, 5, 77, 128, 9, 250])
    model.reset(torch.from_numpy(seq))
    for pos, tok in enumerate(seq):
        model.step()
        torch.cuda.synchronize()
        ol = oracle.step(int(tok), pos)
        assert_close_rel(f32_of(model.logits).reshape(-1), ol, rtol=2e-2, atol_frac=2e-2,
                         what=f"logits at {pos}")


@pytest.mark.gpu
def test_batched_model_from_gguf_against_oracle(tmp_path):
    """The same file decoding two sequences per step (MFMA GEMMs; the 512-k
    o_proj over the packed layout, the 128-k linears and head over GGUF
    blocks), each row teacher-forced against its own oracle decoder."""
    import torch
    from oracle import model as omodel
    from oracle.bf16 import round_bf16
    from _util import assert_close_rel, f32_of
    p, _ = tiny_qwen3_file(tmp_path)
    mm = pkg("integration.model")
    dev = torch.device("cuda:0")
    model = mm.DecodeModel.from_gguf(p, dev, max_len=64, block_size=32, batch=2)
    L0 = model.layers[0]
    assert L0.o_proj.q4_0_packed is not None and not hasattr(L0.qkv, "q4_0_packed")
    g = gf().GGUFFile(p)
    cfg = gf().decoder_config(g)
    w = {k: (round_bf16(v) if v.dtype == np.float32 else v)
         for k, v in gf().decoder_weights(g, cfg["n_layers"]).items()}
    ocfg = {k: cfg[k] for k in ("hidden", "n_layers", "n_q", "n_kv", "head_dim", "intermediate",
                                "vocab", "eps")}
    cap = model.state.block_table.shape[1] * 32
    oracles = [omodel.OracleDecoder(ocfg, w, f32_of(model.cos_sin), num_splits=2, capacity=cap)
               for _ in range(2)]
    seqs = np.array([[3, 17, 200, 5, 77, 128, 9, 250], [41, 0, 255, 90, 12, 33, 7, 64]])
    model.reset([torch.from_numpy(s) for s in seqs])
    for pos in range(seqs.shape[1]):
        model.step()
        torch.cuda.synchronize()
        gl = f32_of(model.logits).reshape(2, -1)
        for r in range(2):
            ol = oracles[r].step(int(seqs[r, pos]), pos)
            assert_close_rel(gl[r], ol, rtol=2e-2, atol_frac=2e-2, what=f"row {r} at {pos}")


def test_from_gguf_rejects_an_unknown_activation(tmp_path):
    mm = pkg("integration.model")
    with pytest.raises(ValueError, match="activation"):
        mm.DecodeModel.from_gguf(tmp_path / "unused.gguf", "cpu", activation="relu")
