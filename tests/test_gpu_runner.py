"""GPU tests of the step runner (native/runner.py, smx_runner_* in
include/smx.h): one decode step recorded once and replayed as AQL dispatch
packets must give eager execution's results bit for bit -- tokens, logits,
decode state and every KV cache slot -- for the fused and unfused
one-sequence steps and the batched step, over many steps per replay call and
over several calls, with SwiGLU and with the table-GELU activation, and the
36-layer 4B-shape model at contexts near 4000 (one sequence and eight);
recording launches nothing; a recording that allocates device memory,
launches anything outside the library or raises is refused.  (Eager execution is the reference: a
graph replays it bit for bit too, but capture() runs a warm-up step that
writes one KV slot outside the sequences' block tables.)"""
import numpy as np
import pytest

from _util import bits_of, pkg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _m():
    return pkg("integration.model")


def tiny_cfg(activation="swiglu"):
    return _m().DecoderConfig(hidden=256, n_layers=2, n_q=8, n_kv=2, head_dim=128,
                              intermediate=512, vocab=1000, block_size=32, activation=activation)


def _state_bits(model):
    st = model.state
    out = {"tokens": st.tokens.cpu().numpy(), "positions": st.positions.cpu().numpy(),
           "seq_lens": st.seq_lens.cpu().numpy(), "slots": st.slot_mapping.cpu().numpy(),
           "logits": bits_of(model.logits), "x": bits_of(model.x)}
    for i, L in enumerate(model.layers):
        out[f"k{i}"] = bits_of(L.kv_cache[0])
        out[f"v{i}"] = bits_of(L.kv_cache[1])
    return out


def _assert_same(a, b, what):
    assert a.keys() == b.keys()
    for k in a:
        np.testing.assert_array_equal(a[k], b[k], err_msg=f"{what}: {k}")


def _eager_vs_runner(dev, fences, *, fused=True, batch=1, steps=30, chunks=(30,), seed=5,
                     activation="swiglu"):
    import torch
    m = _m()
    kw = dict(seed=seed, max_len=64, num_splits=2, fused=fused)
    if batch > 1:
        kw.update(batch=batch)
    e = m.DecodeModel(tiny_cfg(activation), dev, **kw)
    r = m.DecodeModel(tiny_cfg(activation), dev, **kw)
    rng = np.random.default_rng(seed)
    prompts = [torch.tensor(rng.integers(0, 1000, 3 + i)) for i in range(batch)]
    prompt = prompts[0] if batch == 1 else prompts
    e.reset(prompt)
    for _ in range(steps):
        e.step()
    torch.cuda.synchronize()
    want = _state_bits(e)
    r.reset(prompt)
    n = r.record_runner().num_packets
    assert n > 0
    assert sum(chunks) == steps
    for c in chunks:
        r.run_steps(c, fences)
    _assert_same(want, _state_bits(r), f"{fences} fences, fused={fused}, batch={batch}")
    r.runner.close()
    return n


FENCES = ["agent", "acquire"]


@pytest.mark.parametrize("fences", FENCES)
@pytest.mark.parametrize("fused", [True, False])
def test_runner_replays_the_step(dev, fused, fences):
    n = _eager_vs_runner(dev, fences, fused=fused)
    # fused: per layer QKV, attention, merge, o_proj, gate/up, down; head + advance
    if fused:
        assert n == 2 * 6 + 2


@pytest.mark.parametrize("fences", FENCES)
def test_runner_batched_step(dev, fences):
    _eager_vs_runner(dev, fences, batch=3, chunks=(1, 12, 17))


@pytest.mark.parametrize("fused,batch", [(True, 1), (False, 1), (False, 3)])
def test_runner_replays_the_gelu_model(dev, fused, batch):
    """The reference model's table-GELU activation (the table pointer is a
    recorded kernel argument) in the fused, unfused and batched steps."""
    _eager_vs_runner(dev, "acquire", fused=fused, batch=batch, chunks=(10, 20), seed=8,
                     activation="gelu")


@pytest.mark.parametrize("fences", FENCES)
def test_runner_steps_per_call_do_not_matter(dev, fences):
    _eager_vs_runner(dev, fences, chunks=(1, 1, 5, 23), seed=6)


def test_recording_launches_nothing(dev):
    import torch
    m = _m()
    model = m.DecodeModel(tiny_cfg(), dev, seed=4, max_len=64, num_splits=2)
    model.reset(torch.tensor([5, 6, 7]))
    torch.cuda.synchronize()
    before = _state_bits(model)
    model.record_runner()
    torch.cuda.synchronize()
    _assert_same(before, _state_bits(model), "after recording")
    model.runner.close()


def test_recording_refuses_allocations_and_errors(dev):
    import torch
    native = pkg("native")
    ops = pkg("native.torch_ops")
    StepRunner = pkg("native.runner").StepRunner
    x = torch.randn(1, 256, device=dev).to(torch.bfloat16)
    w = torch.zeros(64, 8 * 18, dtype=torch.uint8, device=dev)
    with StepRunner() as runner:
        # an output allocated inside the recording would dangle after it
        with pytest.raises(RuntimeError, match="allocated"):
            runner.record(lambda: ops.q4_0_gemv(x, w, 64, 256))
        with pytest.raises(RuntimeError, match="nothing recorded"):
            runner.replay(1)
        # a failing library call stops the recording and propagates
        with pytest.raises(native.SmxError, match="multiple of 32"):
            runner.record(lambda: native.call("smx_q4_0_gemv", None, 16, 16, 16, 64, 100))
        y = torch.empty(1, 64, dtype=torch.bfloat16, device=dev)
        # a launch outside the library (here torch's fill_ into a preallocated
        # buffer) would run once and vanish from every replay: refused, and
        # it did not run while recording either
        y.fill_(2.0)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="outside this library"):
            runner.record(lambda: (ops.q4_0_gemv(x, w, 64, 256, out=y), y.fill_(5.0)))
        torch.cuda.synchronize()
        assert float(y.float().min()) == 2.0 and float(y.float().max()) == 2.0
        with pytest.raises(RuntimeError, match="nothing recorded"):
            runner.replay(1)
        assert runner.record(lambda: ops.q4_0_gemv(x, w, 64, 256, out=y)) == 1
        y.fill_(1.0)
        runner.run(3)
        assert float(y.float().abs().max()) == 0.0  # zero weights: y = 0
        runner.wait(1.0)  # idle: returns at once


# models whose buffers a broken runner's already-written packets may still read: kept alive
# for the rest of the process
_KEEP = []


def test_a_replay_that_cannot_drain_breaks_the_runner(dev):
    """Forced from the host: with a zero drain timeout, a replay of far more packets than the
    runner's queue holds (16384) gives up at the first full queue while the GPU works through
    the packets already written (they all run to the end: the model's block table covers
    every position they reach).  The runner then refuses replay, wait, elapsed and a new
    recording with the reason, and closing it leaves it allocated instead of waiting on a
    completion signal that the unwritten last packet would have sent."""
    import time
    import torch
    SmxError = pkg("native").SmxError
    m = _m()
    model = m.DecodeModel(tiny_cfg(), dev, seed=4, max_len=4096, num_splits=2)
    model.reset(torch.tensor([5, 6, 7]))
    runner = model.record_runner()
    _KEEP.append((model, runner))
    runner.set_drain_timeout(0.0)
    reps = 3000  # 3000 steps x 14 packets; positions stay below max_len even if all ran
    assert runner.num_packets * reps > 2 * 16384
    with pytest.raises(SmxError, match="did not drain"):
        runner.replay(reps, "acquire")
    for fn in (lambda: runner.wait(1.0), runner.elapsed, lambda: runner.replay(1, "acquire")):
        with pytest.raises(SmxError, match="broken"):
            fn()
    with pytest.raises(SmxError, match="broken"):
        runner.record(model.enqueue_step)
    time.sleep(0.5)  # the written packets finish meanwhile (tiny kernels, a few ms)
    runner.close()   # left allocated, with a message; returns at once
    with pytest.raises(pkg("native").SmxError):
        pkg("native").call("smx_runner_set_drain_timeout", None, 1.0)


def test_runner_elapsed_is_gpu_time_of_the_last_replay(dev):
    import time
    import torch
    m = _m()
    model = m.DecodeModel(tiny_cfg(), dev, seed=4, max_len=64, num_splits=2)
    model.reset(torch.tensor([5, 6, 7]))
    runner = model.record_runner()
    with pytest.raises(pkg("native").SmxError, match="nothing replayed"):
        runner.elapsed()
    for steps in (1, 40):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        runner.replay(steps, "acquire", sync=False)
        runner.wait(30.0)
        wall = time.perf_counter() - t0
        gpu = runner.elapsed()
        assert 0.0 < gpu <= wall
    runner.close()


@pytest.mark.parametrize("batch", [1, 8])
def test_runner_4b_model_matches_eager(dev, batch):
    """The 36-layer 4B-shape model at real kernel shapes (49 capacity splits
    for one sequence; the per-sequence plan, MFMA GEMMs and the batched head
    for 8): 6 steps from contexts near 4000 through the runner (either fence
    mode) equal 6 eager steps bit for bit -- tokens, logits, decode state
    and the K/V slots the steps wrote."""
    import torch
    m = _m()
    model = m.DecodeModel(m.DecoderConfig(), dev, seed=2, max_len=6272, batch=batch)
    model.fill_kv(21)
    ctx = [4000 + 97 * r for r in range(batch)]
    ids = [1 + 13 * r for r in range(batch)]
    steps = 6

    def run(step_fn):
        model.set_context(ctx, ids=ids)
        step_fn()
        torch.cuda.synchronize()
        st = model.state
        bs = model.cfg.block_size
        slots = [int(st.block_table[r, p // bs]) * bs + p % bs
                 for r in range(batch) for p in range(ctx[r], ctx[r] + steps)]
        idx = torch.tensor(slots, device=dev)
        kv = [bits_of(L.kv_cache.flatten(1, 2)[:, idx]) for L in model.layers]
        return {"tokens": st.tokens.cpu().numpy(), "positions": st.positions.cpu().numpy(),
                "slots": st.slot_mapping.cpu().numpy(), "logits": bits_of(model.logits),
                "x": bits_of(model.x), **{f"kv{i}": a for i, a in enumerate(kv)}}

    want = run(lambda: [model.step() for _ in range(steps)])
    model.record_runner()
    for fences in FENCES:
        got = run(lambda: model.run_steps(steps, fences))
        _assert_same(want, got, f"4B model, batch {batch}, {fences} fences")
    model.runner.close()


def test_recording_is_per_thread(dev):
    """While one thread records, a library call on another thread launches
    as usual (the recording runner is the calling thread's).  The other
    thread launches on a stream of its own and does not synchronise the
    device meanwhile: HIP refuses a device-wide synchronisation while the
    recording's capture runs."""
    import threading
    import torch
    native = pkg("native")
    ops = pkg("native.torch_ops")
    StepRunner = pkg("native.runner").StepRunner
    x = torch.randn(1, 256, device=dev).to(torch.bfloat16)
    w = torch.zeros(64, 8 * 18, dtype=torch.uint8, device=dev)
    y_rec = torch.full((1, 64), 1.0, dtype=torch.bfloat16, device=dev)
    y_other = torch.full((1, 64), 1.0, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    inside, done = threading.Event(), threading.Event()
    other_stream = torch.cuda.Stream(device=dev)

    def other():
        inside.wait(30)
        with torch.cuda.stream(other_stream):
            ops.q4_0_gemv(x, w, 64, 256, out=y_other)  # launched now, on this thread's stream
        done.set()

    t = threading.Thread(target=other)
    t.start()
    with StepRunner() as runner:
        def fn():
            ops.q4_0_gemv(x, w, 64, 256, out=y_rec)
            inside.set()
            assert done.wait(30)
        assert runner.record(fn) == 1
        t.join(30)
        torch.cuda.synchronize()
        assert float(y_other.float().abs().max()) == 0.0  # the other thread's GEMV ran
        assert float(y_rec.float().min()) == 1.0  # the recorded one did not
        runner.run(1)
        assert float(y_rec.float().abs().max()) == 0.0
    assert native.load() is not None


def test_generate_on_the_runner(dev):
    """generate() through the runner (one replay for prompt + new tokens)
    returns the graph's tokens, for one sequence and for three ragged ones."""
    import torch
    m = _m()
    rng = np.random.default_rng(17)
    for batch in (1, 3):
        kw = dict(seed=9, max_len=64, num_splits=2) if batch == 1 else \
            dict(seed=9, max_len=64, batch=batch)
        g = m.DecodeModel(tiny_cfg(), dev, **kw)
        r = m.DecodeModel(tiny_cfg(), dev, **kw)
        prompts = [torch.tensor(rng.integers(0, 1000, 4 + 2 * i)) for i in range(batch)]
        prompt = prompts[0] if batch == 1 else prompts
        g.capture()
        want = g.generate(prompt, 20).cpu().numpy()
        r.record_runner()
        got = r.generate(prompt, 20, fences="acquire").cpu().numpy()
        r.runner.close()
        np.testing.assert_array_equal(want, got, err_msg=f"batch {batch}")
