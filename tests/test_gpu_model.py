"""GPU parity of the whole decode step against the oracle decoder.

  * a 2-layer model (hidden 256): logits within 2e-2 of the float64 oracle
    at every teacher-forced step, greedy tokens equal except near-ties --
    with SwiGLU, and with the reference model's table GELU;
  * graph replay equals eager execution bit for bit;
  * one full-size layer (hidden 2560, 32q/8kv, intermediate 9728) at context
    4096 against the oracle layer, within 1e-2;
  * the 36-layer 4B-shape model: greedy tokens teacher-forced against the
    oracle, disagreements only at near-ties (float64 top-2 margin below 2e-2
    of the top logit), from an empty cache and at contexts 2048-2051 and
    4093-4096 over a seeded cache, and on the step runner in the decode
    benchmark's configuration (6272-token block table, 49 splits) at its
    last positions 6138-6143 and over a 64-token greedy run across a page
    boundary;
  * eight 4B sequences at seeded contexts in 512..32768 decoded together
    (the ragged batch) give each row what the sequence gets decoded alone.
"""
import numpy as np
import pytest

from oracle import attention as oatt
from oracle import model as omodel
from oracle import ops as oops
from oracle.bf16 import bf16_bits_to_f32

from _util import assert_close_rel, bits_of, f32_of, pkg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _m():
    return pkg("integration.model")


def tiny_cfg(n_layers=2):
    return _m().DecoderConfig(hidden=256, n_layers=n_layers, n_q=8, n_kv=2, head_dim=128,
                              intermediate=512, vocab=1000, block_size=32)


def oracle_from(model, num_splits, grouped=False):
    c = model.cfg
    w = {}
    for i, L in enumerate(model.layers):
        w[f"layers.{i}.qkv"] = L.qkv.qweight.cpu().numpy()
        w[f"layers.{i}.o_proj"] = L.o_proj.qweight.cpu().numpy()
        w[f"layers.{i}.gate_up"] = L.gate_up.qweight.cpu().numpy()
        w[f"layers.{i}.down"] = L.down.qweight.cpu().numpy()
        for j, t in enumerate((L.input_norm, L.post_norm, L.q_norm, L.k_norm)):
            w[f"layers.{i}.norm{j}"] = f32_of(t)
    w["final_norm"] = f32_of(model.final_norm)
    w["head"] = model.head.q4_0_head.cpu().numpy()
    cfg = dict(hidden=c.hidden, n_layers=c.n_layers, n_q=c.n_q, n_kv=c.n_kv, head_dim=c.head_dim,
               intermediate=c.intermediate, vocab=c.vocab, eps=c.eps, activation=c.activation,
               gelu_lut=None if model.act_lut is None else bits_of(model.act_lut))
    cap = model.state.block_table.shape[1] * c.block_size
    return omodel.OracleDecoder(cfg, w, f32_of(model.cos_sin), num_splits=num_splits, capacity=cap,
                                grouped_attention=grouped)


def teacher_forced(model, oracle, seq):
    """Run both on `seq`; returns per-step (gpu argmax, oracle logits64,
    gpu logits)."""
    import torch
    model.reset(torch.tensor(seq))
    out = []
    for pos, tok in enumerate(seq):
        model.step()
        torch.cuda.synchronize()
        gl = f32_of(model.logits).reshape(-1)
        gid = int(model.state.next_ids.item())
        ol = oracle.step(int(tok), pos)
        out.append((gid, ol, gl))
    return out


def check_greedy(records, what):
    ties = 0
    for pos, (gid, ol, gl) in enumerate(records):
        assert_close_rel(gl, ol, rtol=2e-2, atol_frac=2e-2, what=f"{what} logits at {pos}")
        oid = omodel.bf16_argmax(ol)
        if gid != oid:
            top, margin = omodel.top2_margin(ol)
            assert margin < omodel.NEAR_TIE_REL, (
                f"{what}: step {pos} token {gid} != oracle {oid} with margin {margin:.3g}")
            ties += 1
    return ties


@pytest.mark.parametrize("fused", [True, False])
def test_tiny_model_teacher_forced(dev, fused):
    m = _m()
    model = m.DecodeModel(tiny_cfg(), dev, seed=3, max_len=64, num_splits=2, fused=fused)
    oracle = oracle_from(model, num_splits=2)
    rng = np.random.default_rng(0)
    seq = rng.integers(0, model.cfg.vocab, 40)
    recs = teacher_forced(model, oracle, seq)
    ties = check_greedy(recs, "tiny")
    assert ties <= 4


@pytest.mark.parametrize("fused", [True, False])
def test_tiny_model_gelu_teacher_forced(dev, fused):
    """The reference model's activation (table erf-GELU) in the whole step:
    same bar as the SwiGLU model; the oracle reads the model's table."""
    m = _m()
    cfg = tiny_cfg()
    cfg.activation = "gelu"
    model = m.DecodeModel(cfg, dev, seed=4, max_len=64, num_splits=2, fused=fused)
    oracle = oracle_from(model, num_splits=2)
    seq = np.random.default_rng(2).integers(0, model.cfg.vocab, 40)
    ties = check_greedy(teacher_forced(model, oracle, seq), f"tiny gelu fused={fused}")
    assert ties <= 4


def test_graph_replay_matches_eager(dev):
    import torch
    m = _m()
    prompt = torch.tensor(np.random.default_rng(1).integers(0, 1000, 7))
    a = m.DecodeModel(tiny_cfg(), dev, seed=5, max_len=64, num_splits=2)
    eager = a.generate(prompt, 30).cpu().numpy()
    eager_logits = bits_of(a.logits)
    a.capture()
    graph = a.generate(prompt, 30).cpu().numpy()
    np.testing.assert_array_equal(eager, graph)
    np.testing.assert_array_equal(eager_logits, bits_of(a.logits))
    # replays after unrelated eager work still agree
    torch.randn(1000, device=dev).sum().item()
    again = a.generate(prompt, 30).cpu().numpy()
    np.testing.assert_array_equal(eager, again)
    assert np.all(eager[:7] == prompt.numpy())


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("seed", [7, 8])
def test_full_size_layer_at_4096(dev, fused, seed):
    """One full-size layer (hidden 2560, 32q/8kv, SwiGLU 9728) at position
    4095 over a seeded cache, against the oracle layer, at the 1e-2 bar:
    elementwise within 1e-2 relative plus 1e-2 of the output rms, and within
    1e-2 in relative L2.  Measured on MI355X (seeds 7-9, both paths): relative
    L2 3.2-3.7e-3, the largest error 1.4-2.2e-2 of the rms -- bf16 outputs of
    two implementations whose GEMVs accumulate in different orders differ by
    one ulp at about half the elements of each stage (0.39% of an element),
    and a residual element near zero carries the absolute part."""
    import torch
    m = _m()
    cfg = m.DecoderConfig(n_layers=1, vocab=512)
    L = 4096
    model = m.DecodeModel(cfg, dev, seed=seed, max_len=L + 128, num_splits=16, fused=fused)
    oracle = oracle_from(model, num_splits=16)
    pos = L - 1
    fill_kv(model, oracle, pos, seed)  # positions < pos
    table = model.state.block_table[0].cpu().numpy()
    st = model.state
    st.positions.fill_(pos)
    st.seq_lens.fill_(pos + 1)
    st.slot_mapping.fill_(int(table[pos // cfg.block_size]) * cfg.block_size + pos % cfg.block_size)
    x = (3 * torch.randn((1, cfg.hidden), generator=torch.Generator().manual_seed(seed))).to(
        torch.bfloat16)  # layer 0 input: the embedding
    model.x.copy_(x.to(dev))
    model.layer_run(0)
    # the next consumer (here the head) adds and normalises (down, residual)
    y_dev, r_dev = pkg("native.torch_ops").add_rmsnorm(model.d, model.res_b, model.final_norm,
                                                       cfg.eps)
    torch.cuda.synchronize()
    xf = x.float().numpy()[0]
    h0, _ = oops.add_rmsnorm(xf, None, f32_of(model.layers[0].input_norm), cfg.eps)
    y, res = oracle.layer(0, h0, xf, pos)
    for what, got, ref in (("residual", f32_of(r_dev).reshape(-1), res),
                           ("layer out", f32_of(y_dev).reshape(-1), y)):
        assert_close_rel(got, ref, rtol=1e-2, atol_frac=1e-2, what=what)
        rel_l2 = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel_l2 < 1e-2, f"{what}: relative L2 {rel_l2:.3g}"


@pytest.mark.parametrize("num_splits", [2, 3])
def test_fused_and_unfused_steps_agree(dev, num_splits):
    """The fused kernel sequence and the one-op-per-launch sequence give the
    same greedy tokens and logits within bf16 noise."""
    m = _m()
    prompt_np = np.random.default_rng(4).integers(0, 1000, 9)
    import torch
    prompt = torch.tensor(prompt_np)
    runs = []
    for fused in (True, False):
        model = m.DecodeModel(tiny_cfg(), dev, seed=6, max_len=64, num_splits=num_splits,
                              fused=fused)
        toks = model.generate(prompt, 25).cpu().numpy()
        runs.append((toks, f32_of(model.logits).reshape(-1)))
    np.testing.assert_array_equal(runs[0][0], runs[1][0])
    assert_close_rel(runs[0][1], runs[1][1], rtol=2e-2, atol_frac=2e-2, what="final logits")


def test_4b_model_greedy_tokens(dev):
    m = _m()
    model = m.DecodeModel(m.DecoderConfig(), dev, seed=1, max_len=64, num_splits=4)
    oracle = oracle_from(model, num_splits=4)
    rng = np.random.default_rng(11)
    seq = rng.integers(0, model.cfg.vocab, 6)
    recs = teacher_forced(model, oracle, seq)
    check_greedy(recs, "4B")


def fill_kv(model, oracle, length: int, seed: int) -> None:
    """Seeded N(0,1) bf16 K and V for positions < length in every layer,
    written through the model's block table (row 0) and given to the oracle
    as its cache."""
    import torch
    c = model.cfg
    bs = c.block_size
    pages = model.state.block_table[0, :(length + bs - 1) // bs].long()
    g = torch.Generator(device=model.device).manual_seed(seed)
    for i, L in enumerate(model.layers):
        kv = torch.randn((2, pages.numel() * bs, c.n_kv, c.head_dim), generator=g,
                         device=model.device).to(torch.bfloat16)
        kv[:, length:] = 0
        L.kv_cache[:, pages] = kv.view(2, pages.numel(), bs, c.n_kv, c.head_dim)
        host = kv[:, :length].float().cpu().numpy()
        oracle.k[i] = host[0]
        oracle.v[i] = host[1]


@pytest.mark.parametrize("start", [2048, 4093])
def test_4b_model_teacher_forced_at_long_context(dev, start):
    """The 36-layer 4B model at the contexts a decode benchmark times (the
    2048-token prompt's KV in the cache, then four teacher-forced tokens, and
    again near 4096): every step's logits against the float64 oracle decoder
    holding the same cache, greedy tokens equal except at near-ties.  The
    block table's capacity is 6144 tokens (48 splits of 128), as in the
    benchmark."""
    import torch
    m = _m()
    model = m.DecodeModel(m.DecoderConfig(), dev, seed=2, max_len=6144)
    oracle = oracle_from(model, num_splits=model.num_splits)
    fill_kv(model, oracle, start, seed=start)
    T = 4
    seq = np.random.default_rng(start).integers(0, model.cfg.vocab, T)
    st = model.state
    model.set_context([start], ids=[int(seq[0])])
    st.forced[0, start + 1:start + T] = torch.from_numpy(seq[1:]).to(dev)
    st.forced_len.fill_(start + T)
    model.capture()
    model.set_context([start], ids=[int(seq[0])])
    st.forced_len.fill_(start + T)
    recs = []
    for j in range(T):
        model.step()
        torch.cuda.synchronize()
        gl = f32_of(model.logits).reshape(-1)
        gid = int(st.next_ids.item())
        recs.append((gid, oracle.step(int(seq[j]), start + j), gl))
        print(f"4B ctx {start + j}: step checked", flush=True)
    # the tokens fed are the forced ones, by position
    np.testing.assert_array_equal(st.tokens[0, start + 1:start + T].cpu().numpy(), seq[1:])
    check_greedy(recs, f"4B at {start}")


@pytest.mark.parametrize("batch,activation", [(3, "swiglu"), (8, "swiglu"), (12, "swiglu"),
                                              (8, "gelu")])
def test_batched_decode_against_per_sequence_oracle(dev, batch, activation):
    """batch sequences decoded together (MFMA GEMM path: activations staged
    per wave up to 8 rows, read from global memory above), teacher-forced
    with different token streams: every row's logits match that sequence's
    own oracle decoder at every step (SwiGLU, and the reference model's
    table GELU in the GEMM epilogue)."""
    import torch
    m = _m()
    cfg = tiny_cfg()
    cfg.activation = activation
    model = m.DecodeModel(cfg, dev, seed=8, max_len=64, num_splits=3, batch=batch)
    oracles = [oracle_from(model, num_splits=3) for _ in range(batch)]
    rng = np.random.default_rng(batch)
    T = 12
    seqs = rng.integers(0, model.cfg.vocab, (batch, T))
    model.reset([torch.from_numpy(s) for s in seqs])
    ties = 0
    for pos in range(T):
        model.step()
        torch.cuda.synchronize()
        gl = f32_of(model.logits).reshape(batch, -1)
        gid = model.state.next_ids.cpu().numpy()
        for r in range(batch):
            ol = oracles[r].step(int(seqs[r, pos]), pos)
            assert_close_rel(gl[r], ol, rtol=2e-2, atol_frac=2e-2, what=f"row {r} step {pos}")
            if gid[r] != omodel.bf16_argmax(ol):
                assert omodel.top2_margin(ol)[1] < omodel.NEAR_TIE_REL
                ties += 1
    # each mismatch above is a near-tie of the fp64 logits; a few per hundred
    # comparisons are expected from the random tiny model's flat logits
    assert ties <= max(3, batch * T // 25)


@pytest.mark.parametrize("activation", ["swiglu", "gelu"])
def test_batched_packed_and_gguf_layouts_agree(dev, activation):
    """A batched model packs every layer linear (gate|up gated) and the head
    and runs the packed-layout GEMMs; packed=False runs the GGUF-layout GEMMs
    over the same weights.  The logits of the two agree at every
    teacher-forced step to within the bf16 rounding of differently ordered
    fp32 sums, and the greedy tokens match except at near-ties."""
    import torch
    m = _m()
    cfg = tiny_cfg()
    cfg.activation = activation
    B, T = 5, 10
    a = m.DecodeModel(cfg, dev, seed=9, max_len=64, num_splits=3, batch=B)
    b = m.DecodeModel(cfg, dev, seed=9, max_len=64, num_splits=3, batch=B, packed=False)
    for L in a.layers:
        for lin in (L.qkv, L.o_proj, L.down):
            assert not lin.q4_0_packed.gated
        assert L.gate_up.q4_0_packed.gated
    assert a.head_packed is not None and b.head_packed is None
    assert not hasattr(b.layers[0].qkv, "q4_0_packed")
    seqs = np.random.default_rng(9).integers(0, cfg.vocab, (B, T))
    prompts = [torch.from_numpy(s) for s in seqs]
    a.reset(prompts)
    b.reset(prompts)
    diff = 0
    for pos in range(T):
        a.step()
        b.step()
        torch.cuda.synchronize()
        la, lb = f32_of(a.logits).reshape(B, -1), f32_of(b.logits).reshape(B, -1)
        for r in range(B):
            assert_close_rel(la[r], lb[r], rtol=2e-2, atol_frac=2e-2, what=f"row {r} step {pos}")
        ia, ib = a.state.next_ids.cpu().numpy(), b.state.next_ids.cpu().numpy()
        for r in np.nonzero(ia != ib)[0]:
            assert omodel.top2_margin(lb[r].astype(np.float64))[1] < omodel.NEAR_TIE_REL
            diff += 1
    assert diff <= 2


def test_batched_graph_replay_and_ragged_prompts(dev):
    """Prompts of different lengths in one batch; graph replay equals eager;
    each row's prompt is fed before its own generated tokens."""
    import torch
    m = _m()
    prompts = [torch.tensor([5, 6, 7]), torch.tensor([9]), torch.tensor([1, 2, 3, 4, 5, 6])]
    a = m.DecodeModel(tiny_cfg(), dev, seed=9, max_len=64, num_splits=2, batch=3)
    eager = a.generate(prompts, 10).cpu().numpy()
    a.capture()
    graph = a.generate(prompts, 10).cpu().numpy()
    np.testing.assert_array_equal(eager, graph)
    for r, p in enumerate(prompts):
        np.testing.assert_array_equal(eager[r, :p.numel()], p.numpy())
    assert (eager[:, :16] >= 0).all() and (eager[:, :16] < 1000).all()


def test_batched_plan_splits_change_under_graph_replay(dev):
    """Through the captured graph, each step's plan re-cuts the splits from
    the grown lengths: with 8 plan items a sequence has 1 split up to 128
    tokens, then 2, then 3 (three sequences, 280 steps).  Every row's logits
    match its own oracle decoder (checked every 7th step and at the end)."""
    import torch
    m = _m()
    batch, T = 3, 280
    model = m.DecodeModel(tiny_cfg(), dev, seed=11, max_len=320, batch=batch, plan_items=8,
                          num_splits=4)
    oracles = [oracle_from(model, num_splits=3) for _ in range(batch)]
    rng = np.random.default_rng(11)
    seqs = rng.integers(0, model.cfg.vocab, (batch, T))
    model.capture()
    model.reset([torch.from_numpy(s) for s in seqs])
    splits_seen = set()
    for pos in range(T):
        model.step()
        ols = [oracles[r].step(int(seqs[r, pos]), pos) for r in range(batch)]
        if pos % 7 == 6 or pos == T - 1:
            torch.cuda.synchronize()
            gl = f32_of(model.logits).reshape(batch, -1)
            for r in range(batch):
                assert_close_rel(gl[r], ols[r], rtol=2e-2, atol_frac=2e-2, what=f"row {r} step {pos}")
        cap = model.state.block_table.shape[1] * model.cfg.block_size
        _, sp = oatt.plan_splits([pos + 1] * batch, 8, 4, cap)
        splits_seen.add(len(sp[0]))
    assert {1, 2, 3} <= splits_seen


def test_4b_batched_matches_single_sequence(dev):
    """At the full 4B size, 8 sequences teacher-forced together (m = 8 GEMMs,
    split plan: 3 splits of 128 tokens each by the end) give each row the
    logits the same sequence gets decoded alone (GEMVs, capacity splits),
    within 2e-2 of the logits' scale, and the same greedy token unless the
    top two are a near-tie.  Same seed, so the same weights."""
    import torch
    m = _m()
    B, T = 8, 260
    seqs = np.random.default_rng(17).integers(0, m.DecoderConfig().vocab, (B, T))
    batch = m.DecodeModel(m.DecoderConfig(), dev, seed=3, max_len=300, batch=B)
    batch.reset([torch.from_numpy(s) for s in seqs])
    for _ in range(T):
        batch.step()
    torch.cuda.synchronize()
    bl = f32_of(batch.logits).reshape(B, -1)
    del batch
    torch.cuda.empty_cache()
    single = m.DecodeModel(m.DecoderConfig(), dev, seed=3, max_len=300)
    for r in range(B):
        single.reset(torch.from_numpy(seqs[r]))
        for _ in range(T):
            single.step()
        torch.cuda.synchronize()
        sl = f32_of(single.logits).reshape(-1)
        assert_close_rel(bl[r], sl, rtol=2e-2, atol_frac=2e-2, what=f"row {r}")
        if int(np.argmax(bl[r])) != int(np.argmax(sl)):
            top = np.sort(sl)[-2:]
            assert top[1] - top[0] < 2e-2 * abs(top[1]), f"row {r}: greedy tokens differ"


def _runner_records(model, oracle, start, seq, forced):
    """Steps of `model` on its recorded step runner from position `start`
    (token seq[0] fed first), each run and read back alone; with forced,
    seq[1:] are fed next, else the model's own greedy tokens.  Each step's
    fed token also goes to the oracle.  Returns check_greedy records."""
    import torch
    st = model.state
    T = len(seq)
    model.set_context([start], ids=[int(seq[0])])
    if forced:
        st.forced[0, start + 1:start + T] = torch.from_numpy(np.asarray(seq[1:])).to(model.device)
        st.forced_len.fill_(start + T)
    recs = []
    for j in range(T):
        model.run_steps(1, "acquire")
        gl = f32_of(model.logits).reshape(-1)
        gid = int(st.next_ids.item())
        # set_context feeds seq[0] as the id itself; each later token was
        # written at its position by the previous step's advance kernel
        fed = int(seq[0]) if j == 0 else int(st.tokens[0, start + j].item())
        assert fed == (int(seq[j]) if forced or j == 0 else recs[-1][0])
        recs.append((gid, oracle.step(fed, start + j), gl))
        print(f"4B runner ctx {start + j}: step checked", flush=True)
    return recs


def test_4b_model_at_the_protocol_end_on_the_runner(dev):
    """The decode benchmark's configuration -- a 6272-token block table (49
    pages), 49 splits of 128, the step runner with acquire-only fences --
    at the last positions its protocol decodes (6138-6143), teacher-forced
    over a seeded cache: every step's logits against the float64 oracle,
    greedy tokens equal except at near-ties."""
    m = _m()
    model = m.DecodeModel(m.DecoderConfig(), dev, seed=4, max_len=6272)
    assert model.num_splits == 49
    oracle = oracle_from(model, num_splits=model.num_splits, grouped=True)
    start, T = 6138, 6
    fill_kv(model, oracle, start, seed=start)
    seq = np.random.default_rng(start).integers(0, model.cfg.vocab, T)
    model.record_runner()
    try:
        recs = _runner_records(model, oracle, start, seq, forced=True)
    finally:
        model.runner.close()
    check_greedy(recs, f"4B runner at {start}")


def test_4b_greedy_run_across_a_page_boundary_on_the_runner(dev):
    """64 greedy steps on the step runner (the benchmark's configuration)
    from position 4064 over a seeded cache, crossing the page boundary at
    4096: the oracle is fed the model's own tokens, and every step's token
    equals the oracle's greedy choice except at near-ties, with the logits
    within the bar throughout (as the reference checks its whole 4096-token
    run for identical tokens, src/tools/deployment/verify_results.py:31,49)."""
    m = _m()
    model = m.DecodeModel(m.DecoderConfig(), dev, seed=6, max_len=6272)
    oracle = oracle_from(model, num_splits=model.num_splits, grouped=True)
    start, T = 4064, 64
    fill_kv(model, oracle, start, seed=start)
    seq = [int(np.random.default_rng(start).integers(0, model.cfg.vocab))] + [0] * (T - 1)
    model.record_runner()
    try:
        recs = _runner_records(model, oracle, start, seq, forced=False)
    finally:
        model.runner.close()
    ties = check_greedy(recs, f"4B greedy run from {start}")
    assert ties <= 2
    pages = {(start + j) // model.cfg.block_size for j in range(T)}
    assert len(pages) == 2


def test_4b_batched_at_ragged_long_contexts_matches_single_sequence(dev):
    """Eight 4B sequences at seeded contexts drawn from 512..32768 (the
    ragged-batch workload) over a seeded cache, decoded together for 4
    teacher-forced steps on the step runner (m = 8 GEMMs, per-sequence split
    plan): each row's logits at every step match that sequence decoded alone
    from the same cache contents (GEMVs, capacity splits), within 2e-2 of
    the logits' scale, with the same greedy token unless the top two are a
    near-tie.  Same seed, so the same weights."""
    import torch
    m = _m()
    B, T = 8, 4
    rng = np.random.default_rng(33)
    ctx = rng.integers(512, 32768 - T, B)
    seqs = rng.integers(0, m.DecoderConfig().vocab, (B, T))
    max_len = int(ctx.max()) + T + 1
    batch = m.DecodeModel(m.DecoderConfig(), dev, seed=7, max_len=max_len, batch=B)
    batch.fill_kv(int(ctx.sum()))
    st = batch.state
    batch.record_runner()
    blogits = []
    try:
        batch.set_context(ctx.tolist(), ids=seqs[:, 0].tolist())
        for r in range(B):
            st.forced[r, ctx[r] + 1:ctx[r] + T] = torch.from_numpy(seqs[r, 1:]).to(dev)
        st.forced_len.copy_(torch.from_numpy(ctx + T).to(torch.int32))
        for _ in range(T):
            batch.run_steps(1, "acquire")
            blogits.append(f32_of(batch.logits).reshape(B, -1))
    finally:
        batch.runner.close()
    print(f"batched 8 x 4 steps at contexts {ctx.tolist()} done", flush=True)
    single = m.DecodeModel(m.DecoderConfig(), dev, seed=7, max_len=max_len)
    sst = single.state
    bs = single.cfg.block_size
    nb = -(-max_len // bs)
    for r in range(B):
        src = st.block_table[r, :nb].long()
        dst = sst.block_table[0, :nb].long()
        for Lb, Ls in zip(batch.layers, single.layers):
            Ls.kv_cache[:, dst] = Lb.kv_cache[:, src]
        # the batched steps wrote positions ctx..ctx+T-1; the single decode
        # writes the same values there (compared below through the logits)
        single.set_context([int(ctx[r])], ids=[int(seqs[r, 0])])
        sst.forced[0, ctx[r] + 1:ctx[r] + T] = torch.from_numpy(seqs[r, 1:]).to(dev)
        sst.forced_len.fill_(int(ctx[r]) + T)
        for j in range(T):
            single.step()
            sl = f32_of(single.logits).reshape(-1)
            assert_close_rel(blogits[j][r], sl, rtol=2e-2, atol_frac=2e-2,
                             what=f"row {r} (ctx {ctx[r]}) step {j}")
            if int(np.argmax(blogits[j][r])) != int(np.argmax(sl)):
                top = np.sort(sl)[-2:]
                assert top[1] - top[0] < 2e-2 * abs(top[1]), f"row {r} step {j}: tokens differ"
        print(f"row {r} (ctx {ctx[r]}): 4 steps checked", flush=True)
