"""GPU tests of the plugin boundary around the kernels:

  * Q4_0LinearMethod.apply serves one activation row with one GEMV launch,
    2..16 rows with one MFMA GEMM launch, other row counts as the reference's
    stock path would (bf16 weights, dequantised on the device); every row
    matches the float64 oracle GEMV;
  * torch.ops.smx.layer_run -- the reference's per-layer decode seam,
    layer_run(x, residual, positions, layer_name) -> (y, residual) -- chained
    over a model's layers: one sequence, teacher-forced, against the decode
    model's own step (logits within bf16 tolerance, greedy tokens equal
    except near-ties) and the float64 oracle; several sequences, bit for bit
    against the decode model's batched step (the same kernels in the same
    order); the chain captured once in a CUDA graph and replayed at every
    position, bit for bit against the eager chain; a full-size layer at
    context 4096 against the oracle layer.
"""
import numpy as np
import pytest

from oracle import model as omodel
from oracle import ops as oops
from oracle import q4_0 as oq
from oracle.bf16 import bf16_bits_to_f32

from _util import assert_close_rel, bf16_dev, bits_of, f32_of, pkg, randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _count_calls(monkeypatch):
    """Record every C-ABI function the torch wrappers call."""
    ops = pkg("native.torch_ops")
    seen = []
    real = ops.call

    def counting(name, *args):
        seen.append(name)
        return real(name, *args)
    monkeypatch.setattr(ops, "call", counting)
    return seen


@pytest.mark.parametrize("m,n,k,launches", [
    (1, 6144, 2560, ["smx_q4_0_gemv"]),
    (2, 6144, 2560, ["smx_q4_0_gemm"]),
    (8, 6144, 2560, ["smx_q4_0_gemm"]),
    (16, 2560, 4096, ["smx_q4_0_gemm"]),
    (3, 512, 2592, ["smx_q4_0_gemv"] * 3),        # K % 64 != 0: the GEMV per row
    (40, 1024, 2560, ["smx_q4_0_dequant_bf16"]),  # prefill-sized: bf16 weights + library GEMM
])
def test_apply_dispatch(dev, monkeypatch, m, n, k, launches):
    import torch
    lin_mod = pkg("integration.linear")
    layer = lin_mod.Q4_0Linear(k, [n], device=dev)
    blocks = oq.make_blocks(n, k, seed=m * 31 + n)
    layer.qweight.data.copy_(torch.from_numpy(blocks))
    layer.quant_method.process_weights_after_loading(layer)
    rng = np.random.default_rng(m + k)
    x_bits = randn_bf16(rng, (m, k))
    x = bf16_dev(x_bits, dev)
    seen = _count_calls(monkeypatch)
    y = layer(x)
    torch.cuda.synchronize()
    assert seen == launches
    assert tuple(y.shape) == (m, n) and y.dtype == torch.bfloat16
    got = f32_of(y).reshape(m, n)
    if launches == ["smx_q4_0_dequant_bf16"]:
        # the stock path's operands: the bf16-rounded weights (RNE of d*q,
        # src/spark_vllm_ascend/integration/weights.py:28-32), float64 product
        w = bf16_bits_to_f32(oq.dequant_bf16_bits(blocks, n, k)).astype(np.float64)
        refs = bf16_bits_to_f32(x_bits).astype(np.float64) @ w.T
    else:
        refs = [oq.gemv_f64(x_bits[r], blocks, n, k) for r in range(m)]
    for r in range(m):
        assert_close_rel(got[r], refs[r], rtol=1e-2, atol_frac=5e-3, what=f"row {r}")
    # a leading batch shape is kept, and bias is added after the product
    bias = torch.randn(n, device=dev).to(torch.bfloat16)
    y3 = layer.quant_method.apply(layer, x.view(1, m, k), bias=bias)
    assert tuple(y3.shape) == (1, m, n)
    torch.testing.assert_close(y3.view(m, n), y + bias, rtol=0, atol=0)


@pytest.mark.parametrize("m,n,k,launches", [
    (1, 6144, 2560, ["smx_q4_0_gemv"]),
    (8, 6144, 2560, ["smx_q4_0_gemm_packed"]),
    (16, 2560, 4096, ["smx_q4_0_gemm_packed"]),
    (3, 512, 2592, ["smx_q4_0_gemv"] * 3),        # K % 256 != 0: not packed
    (4, 512, 320, ["smx_q4_0_gemm"]),             # K % 64 == 0 but not packed: GGUF GEMM
])
def test_apply_dispatch_with_packed_weights(dev, monkeypatch, m, n, k, launches):
    """Q4_0Config(pack_for_batch=True): process_weights_after_loading adds the
    packed layout where K % 256 == 0, and apply() runs the packed GEMM for
    2..16 rows, the GEMV for one, against the same float64 oracle."""
    import torch
    lin_mod = pkg("integration.linear")
    layer = lin_mod.Q4_0Linear(k, [n], device=dev)
    layer.quant_method = lin_mod.Q4_0Config(pack_for_batch=True).get_quant_method(layer)
    blocks = oq.make_blocks(n, k, seed=m * 37 + n)
    layer.qweight.data.copy_(torch.from_numpy(blocks))
    layer.quant_method.process_weights_after_loading(layer)
    assert hasattr(layer, "q4_0_packed") == (k % 256 == 0)
    rng = np.random.default_rng(m + k + 1)
    x_bits = randn_bf16(rng, (m, k))
    seen = _count_calls(monkeypatch)
    y = layer(bf16_dev(x_bits, dev))
    torch.cuda.synchronize()
    assert seen == launches
    got = f32_of(y).reshape(m, n)
    for r in range(m):
        assert_close_rel(got[r], oq.gemv_f64(x_bits[r], blocks, n, k), rtol=1e-2,
                         atol_frac=5e-3, what=f"row {r}")


def _tiny_cfg():
    m = pkg("integration.model")
    return m.DecoderConfig(hidden=256, n_layers=2, n_q=8, n_kv=2, head_dim=128,
                           intermediate=512, vocab=1000, block_size=32)


def _metadata(model, positions, num_items=0, plan=False):
    """The step's attention metadata for the sequences of `model` at
    `positions` (one decode token each)."""
    import torch
    att = pkg("integration.attention")
    st, bs = model.state, model.cfg.block_size
    pos = torch.as_tensor(positions, dtype=torch.int64, device=model.device)
    rows = torch.arange(pos.numel(), device=model.device)
    slots = st.block_table[rows, pos // bs].to(torch.int64) * bs + pos % bs
    md = att.SplitKVDecodeMetadata(block_tables=st.block_table,
                                   seq_lens=(pos + 1).to(torch.int32), slot_mapping=slots,
                                   num_splits=model.num_splits, num_items=num_items)
    if plan:
        c = model.cfg
        att.SplitKVDecodeBackend.plan(md, bs, c.n_q, c.head_dim, positions=pos)
    return md, pos


def _chain(model, ids, positions, md):
    """The reference's model loop over torch.ops.smx.layer_run: the first
    input norm outside, then one layer_run per layer; returns the final
    norm's output and the logits of the Q4_0 head."""
    import torch
    ops = pkg("native.torch_ops")
    lr = pkg("integration.layer_run")
    c = model.cfg
    lr.set_attention_metadata(md)
    e = model.head.embed(torch.as_tensor(ids, dtype=torch.int64, device=model.device))
    y, r = ops.add_rmsnorm(e, None, model.layers[0].input_norm, c.eps)
    for L in model.layers:
        y, r = torch.ops.smx.layer_run(y, r, positions, L.name)
    if y.shape[0] == 1:
        logits = ops.q4_0_gemv(y, model.head.q4_0_head, c.vocab, c.hidden)
    else:
        logits = ops.q4_0_gemm(y, model.head.q4_0_head, c.vocab, c.hidden)
    return y, logits


@pytest.mark.parametrize("activation", ["swiglu", "gelu"])
def test_layer_run_one_sequence_matches_step_and_oracle(dev, activation):
    """layer_run (the reference's seam) against the decode step and the
    oracle, with SwiGLU and with the reference model's table GELU."""
    import torch
    m = pkg("integration.model")
    pkg("integration.custom_ops").register()
    lr = pkg("integration.layer_run")
    from test_gpu_model import oracle_from
    cfg = _tiny_cfg()
    cfg.activation = activation
    a = m.DecodeModel(cfg, dev, seed=21, max_len=64, num_splits=2)
    b = m.DecodeModel(cfg, dev, seed=21, max_len=64, num_splits=2)
    oracle = oracle_from(b, num_splits=2)
    lr.uninstall()
    names = lr.install(b)
    assert names == [L.name for L in b.layers]
    seq = np.random.default_rng(21).integers(0, 1000, 24)
    a.reset(torch.from_numpy(seq))
    ties = 0
    try:
        for pos, tok in enumerate(seq):
            a.step()
            md, p = _metadata(b, [pos])
            _, logits = _chain(b, [int(tok)], p, md)
            torch.cuda.synchronize()
            gl = f32_of(logits).reshape(-1)
            al = f32_of(a.logits).reshape(-1)
            ol = oracle.step(int(tok), pos)
            assert_close_rel(gl, al, rtol=2e-2, atol_frac=2e-2, what=f"vs step at {pos}")
            assert_close_rel(gl, ol, rtol=2e-2, atol_frac=2e-2, what=f"vs oracle at {pos}")
            if int(np.argmax(gl)) != omodel.bf16_argmax(ol):
                assert omodel.top2_margin(ol)[1] < omodel.NEAR_TIE_REL
                ties += 1
        # both wrote the same K/V (the fused kernel's writes are exact copies
        # of the same arithmetic on the same inputs up to the first layer's
        # norm rounding): compare the caches within bf16 tolerance
        for La, Lb in zip(a.layers, b.layers):
            assert_close_rel(f32_of(Lb.kv_cache[:, :, :]).reshape(-1),
                             f32_of(La.kv_cache[:, :, :]).reshape(-1), rtol=2e-2, atol_frac=2e-2,
                             what="kv cache")
    finally:
        lr.uninstall()
    assert ties <= 3


@pytest.mark.parametrize("activation", ["swiglu", "gelu"])
def test_layer_run_batched_bitwise_against_batched_step(dev, activation):
    """Three sequences: layer_run over the plan computes exactly what the
    decode model's batched step computes (same kernels, same order), so the
    final normalised hidden state is equal bit for bit at every step (with
    either activation)."""
    import torch
    m = pkg("integration.model")
    pkg("integration.custom_ops").register()
    lr = pkg("integration.layer_run")
    B, T = 3, 10
    cfg = _tiny_cfg()
    cfg.activation = activation
    a = m.DecodeModel(cfg, dev, seed=23, max_len=64, num_splits=3, batch=B)
    b = m.DecodeModel(cfg, dev, seed=23, max_len=64, num_splits=3, batch=B)
    lr.uninstall()
    lr.install(b)
    seqs = np.random.default_rng(23).integers(0, 1000, (B, T))
    a.reset([torch.from_numpy(s) for s in seqs])
    try:
        for pos in range(T):
            a.step()
            md, p = _metadata(b, [pos] * B, num_items=b.num_items, plan=True)
            y, logits = _chain(b, seqs[:, pos].tolist(), p, md)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits_of(y), bits_of(a.h), err_msg=f"step {pos}")
            assert_close_rel(f32_of(logits).reshape(-1), f32_of(a.logits).reshape(-1),
                             rtol=1e-2, atol_frac=1e-2, what=f"logits at {pos}")
        for La, Lb in zip(a.layers, b.layers):
            np.testing.assert_array_equal(bits_of(Lb.kv_cache), bits_of(La.kv_cache))
    finally:
        lr.uninstall()


def test_layer_run_chain_replays_in_a_graph(dev):
    """The seam is graph-safe, as the reference's op is: the model loop over
    torch.ops.smx.layer_run captured once in a CUDA graph, replayed at every
    position with the step's positions / lengths / slots updated in place
    (and the captured chain reading the new embedding row), equals the eager
    chain bit for bit -- normalised output, logits and the KV cache."""
    import torch
    m = pkg("integration.model")
    pkg("integration.custom_ops").register()
    ops = pkg("native.torch_ops")
    lr = pkg("integration.layer_run")
    T = 12
    seq = np.random.default_rng(29).integers(0, 1000, T).tolist()

    # eager reference: model e, every position
    e = m.DecodeModel(_tiny_cfg(), dev, seed=29, max_len=64, num_splits=2)
    lr.uninstall()
    lr.install(e)
    want_y, want_logits = [], []
    try:
        for pos, tok in enumerate(seq):
            md, p = _metadata(e, [pos])
            y, logits = _chain(e, [tok], p, md)
            want_y.append(bits_of(y))
            want_logits.append(bits_of(logits))
        want_kv = [bits_of(L.kv_cache) for L in e.layers]
    finally:
        lr.uninstall()
    del e

    # the same chain captured once over static inputs: model g
    g = m.DecodeModel(_tiny_cfg(), dev, seed=29, max_len=64, num_splits=2)
    c, bs = g.cfg, g.cfg.block_size
    lr.install(g)
    try:
        md, pos_t = _metadata(g, [0])
        emb = torch.empty((1, c.hidden), dtype=torch.bfloat16, device=dev)
        lr.set_attention_metadata(md)

        def chain():
            y, r = ops.add_rmsnorm(emb, None, g.layers[0].input_norm, c.eps)
            for L in g.layers:
                y, r = torch.ops.smx.layer_run(y, r, pos_t, L.name)
            return y, ops.q4_0_gemv(y, g.head.q4_0_head, c.vocab, c.hidden)

        def set_step(pos, tok):
            emb.copy_(g.head.embed(torch.tensor([tok], dtype=torch.int64, device=dev)))
            pos_t.fill_(pos)
            md.seq_lens.fill_(pos + 1)
            md.slot_mapping.fill_(int(g.state.block_table[0, pos // bs]) * bs + pos % bs)

        # warm-up outside the graph writes position 0 once; the replays
        # below rewrite it with the same values
        set_step(0, seq[0])
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            chain()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y_s, logits_s = chain()
        for pos, tok in enumerate(seq):
            set_step(pos, tok)
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits_of(y_s), want_y[pos], err_msg=f"y at {pos}")
            np.testing.assert_array_equal(bits_of(logits_s), want_logits[pos],
                                          err_msg=f"logits at {pos}")
        for L, kv in zip(g.layers, want_kv):
            np.testing.assert_array_equal(bits_of(L.kv_cache), kv)
    finally:
        lr.uninstall()


def test_layer_run_full_size_layer_at_4096(dev):
    """One full-size layer (hidden 2560, 32q/8kv, SwiGLU 9728) through
    layer_run at position 4095 over a seeded cache, against the oracle layer
    at the 1e-2 bar (elementwise 1e-2 relative + 1e-2 of the rms, relative L2
    below 1e-2)."""
    import torch
    m = pkg("integration.model")
    pkg("integration.custom_ops").register()
    lr = pkg("integration.layer_run")
    from test_gpu_model import fill_kv, oracle_from
    cfg = m.DecoderConfig(n_layers=1, vocab=512)
    L = 4096
    model = m.DecodeModel(cfg, dev, seed=9, max_len=L + 128, num_splits=16)
    oracle = oracle_from(model, num_splits=16)
    pos = L - 1
    fill_kv(model, oracle, pos, 9)
    lr.uninstall()
    lr.install(model)
    try:
        md, p = _metadata(model, [pos])
        lr.set_attention_metadata(md)
        x = (3 * torch.randn((1, cfg.hidden), generator=torch.Generator().manual_seed(9))).to(
            torch.bfloat16)
        ops = pkg("native.torch_ops")
        h, res = ops.add_rmsnorm(x.to(dev), None, model.layers[0].input_norm, cfg.eps)
        y, r = torch.ops.smx.layer_run(h, res, p, model.layers[0].name)
        torch.cuda.synchronize()
    finally:
        lr.uninstall()
    xf = x.float().numpy()[0]
    h0, _ = oops.add_rmsnorm(xf, None, f32_of(model.layers[0].input_norm), cfg.eps)
    y_ref, res_ref = oracle.layer(0, h0, xf, pos)
    for what, got, ref in (("residual", f32_of(r).reshape(-1), res_ref),
                           ("layer out", f32_of(y).reshape(-1), y_ref)):
        assert_close_rel(got, ref, rtol=1e-2, atol_frac=1e-2, what=what)
        rel_l2 = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel_l2 < 1e-2, f"{what}: relative L2 {rel_l2:.3g}"


def test_layer_run_rejects_what_it_cannot_serve(dev):
    import torch
    m = pkg("integration.model")
    lr = pkg("integration.layer_run")
    model = m.DecodeModel(_tiny_cfg(), dev, seed=1, max_len=64, num_splits=2)
    lr.uninstall()
    lr.install(model)
    try:
        name = model.layers[0].name
        x = torch.zeros((1, 256), dtype=torch.bfloat16, device=dev)
        p = torch.zeros(1, dtype=torch.int64, device=dev)
        with pytest.raises(RuntimeError, match="metadata"):
            lr.layer_run(x, x, p, name)
        md, p = _metadata(model, [0])
        lr.set_attention_metadata(md)
        with pytest.raises(KeyError):
            lr.layer_run(x, x, p, "no.such.layer")
        with pytest.raises(ValueError, match="rows"):
            lr.layer_run(torch.zeros((2, 256), dtype=torch.bfloat16, device=dev),
                         torch.zeros((2, 256), dtype=torch.bfloat16, device=dev),
                         torch.zeros(2, dtype=torch.int64, device=dev), name)
    finally:
        lr.uninstall()


def test_layer_run_defers_to_the_stock_layer(dev):
    """As the reference's op runs the stock layer for x.shape[0] != 1 or
    missing metadata (src/spark_vllm_ascend/integration/model.py:50-61), the
    seam hands prefill-shaped calls and calls without published metadata to
    the installed stock layer, with its arguments unchanged; decode calls
    never reach it."""
    import torch
    m = pkg("integration.model")
    lr = pkg("integration.layer_run")
    model = m.DecodeModel(_tiny_cfg(), dev, seed=1, max_len=64, num_splits=2)
    calls = []

    def stock(index, x, residual, positions):
        calls.append((index, tuple(x.shape), positions.tolist()))
        return x + 1, residual

    lr.uninstall()
    names = lr.install(model, stock_layer=stock)
    try:
        h = torch.zeros((1, 256), dtype=torch.bfloat16, device=dev)
        p = torch.zeros(1, dtype=torch.int64, device=dev)
        y, r = lr.layer_run(h, h, p, names[1])  # no metadata published
        assert calls == [(1, (1, 256), [0])] and float(y.float().min()) == 1.0
        md, p1 = _metadata(model, [4])
        lr.set_attention_metadata(md)
        x20 = torch.zeros((20, 256), dtype=torch.bfloat16, device=dev)
        p20 = torch.arange(20, device=dev)
        lr.layer_run(x20, x20, p20, names[0])  # more rows than the decode kernels serve
        x3 = torch.zeros((3, 256), dtype=torch.bfloat16, device=dev)
        lr.layer_run(x3, x3, p20[:3], names[0])  # three tokens of one sequence: prefill
        assert [c[:2] for c in calls[1:]] == [(0, (20, 256)), (0, (3, 256))]
        lr.layer_run(torch.randn((1, 256), device=dev).to(torch.bfloat16), h, p1, names[0])
        torch.cuda.synchronize()
        assert len(calls) == 3  # the decode token ran the HIP kernels
    finally:
        lr.uninstall()


def test_layer_run_checks_positions_against_the_plan(dev):
    """Several sequences take positions and slots from the step's plan:
    layer_run accepts the plan's own positions tensor or an equal one, and
    refuses positions that differ from the plan's."""
    import torch
    m = pkg("integration.model")
    lr = pkg("integration.layer_run")
    B = 3
    model = m.DecodeModel(_tiny_cfg(), dev, seed=2, max_len=64, num_splits=3, batch=B)
    lr.uninstall()
    names = lr.install(model)
    try:
        md, pos = _metadata(model, [5, 9, 2], num_items=model.num_items, plan=True)
        lr.set_attention_metadata(md)
        x = torch.randn((B, 256), device=dev).to(torch.bfloat16)
        y1, _ = lr.layer_run(x, x, pos, names[0])
        y2, _ = lr.layer_run(x, x, pos.clone(), names[0])
        torch.cuda.synchronize()
        assert y1.shape == y2.shape == (B, 256)
        with pytest.raises(ValueError, match="differ"):
            lr.layer_run(x, x, pos + 1, names[0])
        md_np, _ = _metadata(model, [5, 9, 2], num_items=model.num_items, plan=False)
        lr.set_attention_metadata(md_np)
        with pytest.raises(ValueError, match="plan"):
            lr.layer_run(x, x, pos, names[0])
    finally:
        lr.uninstall()
