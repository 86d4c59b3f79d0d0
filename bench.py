"""Benchmark: batch-1 greedy decode TPOT of the 4B Q4_0 decoder on one MI355X.

Workload (the configuration the headline metric is quoted on): 36-layer
decoder, hidden 2560, 32 q / 8 kv heads of 128, SwiGLU 9728, tied vocab
151936 with a Q4_0 head, random-init weights, BF16 paged KV (block 128) over a
block table of 49 pages (6272 tokens: the 2048 + 4096 tokens of the protocol,
whatever --steps is, so the kernels' split count does not follow the run's
length).  TPOT is the reference's: time per generated token after the first
((t_last - t_first) / 4095, src/tools/benchmark/benchmark.py:123).
  --steps 4095 (the default): the protocol itself -- a 2048-token random
      prompt fed through the decode step, the first generated token untimed,
      the next 4095 timed.
  --steps K < 4095: K timed tokens spread over the protocol's contexts --
      up to 4 segments starting at contexts from 2049 to 6144 - K/4, each
      after --warmup untimed tokens, over a KV cache pre-filled with seeded
      random bf16 -- so a short run reports the protocol's mean context, not
      its first tokens.
The median over --runs independent runs is reported.  The steps run on the
library's step runner (the recorded step replayed as AQL packets on its own
HSA queue, agent-scope acquire and no release between kernels); the same
steps then run once through the captured graph (graph_ms_per_step, with a
token comparison).  Both executors are timed the same way: host wall-clock
from a synchronised device to the last step's completion (the replay and
its wait, or the graph replays and a device synchronise).  The runner's
packet-processor timestamps of the same replays (first kernel's start to
last kernel's end, no host dispatch or wake-up) are reported beside them
(runner_gpu_ms_per_step).  Without a runner (no HSA queue) the graph is
timed alone.

Also reported, on the same box in the same run:
  roofline      the Q4_0 GEMV [9728 x 2560] (the dominant kernel class:
                2.26 of the 2.87 GB a token streams) timed with HIP events
                over a captured graph of launches that rotate through 24
                weight sets (336 MB, larger than the 256 MB Infinity Cache);
                achieved = 14,032,896 algorithmic bytes / mean launch time;
                ceiling = a streaming-read kernel over the same weight sets;
                sustained = the same kernel at the head's 151936 x 2560 shape
                (218.8 MB per launch), where the launch floor is amortised;
  attention     split-KV decode + LSE merge at contexts 2048 / 4096 / 6144
                over rotating KV sets (> 256 MB), for each split count, with
                the streaming-read ceiling of the same bytes;
  step          bytes a decode step streams vs the HBM-bound step time;
  batch_decode  8 sequences at seeded ragged contexts in one step;
  cpu_baseline  the reference's PyTorch CPU path (bf16 weights, F.linear) on
                this host's cores: decode steps on all cores and on 4 threads
                (the reference's OMP_NUM_THREADS=4), the single GEMV
                (F.linear and the fp32-accumulating restatement), and split-free
                fp32 attention at 6144.
One JSON line is printed.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
# the benchmark measures the library as built, before any validation record
os.environ.setdefault("SMX_ALLOW_UNVALIDATED", "1")

HBM_PEAK_GBS = 8000.0
GEMV_N, GEMV_K = 9728, 2560
GEMV_W_BYTES = GEMV_N * GEMV_K // 32 * 18                # 14,008,320
GEMV_BYTES = GEMV_W_BYTES + GEMV_K * 2 + GEMV_N * 2      # 14,032,896
ATTN_CTXS = (2048, 4096, 6144)
ATTN_SPLITS = (4, 8, 16, 32, 48, 64)
ROTATE_BYTES = 300 << 20    # rotating sets exceed the 256 MB Infinity Cache
PROMPT, GENERATED = 2048, 4096
CAPACITY = 6272             # 49 pages of 128: the protocol's 6144 tokens + the last token id


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_graph(fn, launches_per_call: int, reps: int, warm: int = 2):
    """Capture fn() (which enqueues `launches_per_call` launches) in a graph,
    replay it, and return the mean time per launch in microseconds."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (reps * launches_per_call)


def read_ceiling(bufs, nbytes: int, reps: int):
    """Streaming-read ceiling of `nbytes` per launch over the rotating buffers
    `bufs` (16-byte aligned device tensors of at least nbytes): the fastest
    loads-per-lane setting of the read probe, timed like the kernels."""
    import torch
    from spark_vllm_ascend_amd.native import probe
    best = None
    for loads in (2, 4, 8, 16):
        sink = torch.empty(probe.read_probe_sink_size(nbytes, loads), dtype=torch.int32,
                           device=bufs[0].device)

        def fn():
            for b in bufs:
                probe.read_probe(b, nbytes, sink, loads)
        us = time_graph(fn, len(bufs), reps)
        if best is None or us < best[0]:
            best = (us, loads)
    us, loads = best
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"bytes": nbytes, "us": round(us, 3), "gbs": round(gbs, 1),
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "loads_per_lane": loads}


def gemv_roofline(dev, reps: int):
    import torch
    from spark_vllm_ascend_amd.integration.weights import synthetic_q4_0
    from spark_vllm_ascend_amd.native import torch_ops as ops
    sets = 24
    ws = [synthetic_q4_0(GEMV_N, GEMV_K, 500 + i, dev) for i in range(sets)]
    x = torch.randn(GEMV_K, device=dev).to(torch.bfloat16)
    y = torch.empty((1, GEMV_N), dtype=torch.bfloat16, device=dev)

    def fn():
        for w in ws:
            ops.q4_0_gemv(x, w, GEMV_N, GEMV_K, out=y)
    us = time_graph(fn, sets, reps)
    gbs = GEMV_BYTES / (us * 1e-6) / 1e9
    ceil = read_ceiling([w.view(-1) for w in ws], GEMV_W_BYTES, reps)
    del ws
    # The same kernel where the per-launch floor is amortised: the 151936x2560
    # head shape (218.8 MB per launch), two rotating sets (beyond the 256 MB
    # Infinity Cache), timed the same way.
    hn = 151936
    hw = [synthetic_q4_0(hn, GEMV_K, 900 + i, dev) for i in range(2)]
    hy = torch.empty((1, hn), dtype=torch.bfloat16, device=dev)

    def head_fn():
        for w in hw:
            ops.q4_0_gemv(x, w, hn, GEMV_K, out=hy)
    h_us = time_graph(head_fn, len(hw), max(2, reps // 4))
    h_bytes = hn * GEMV_K // 32 * 18 + GEMV_K * 2 + hn * 2
    del hw, hy
    torch.cuda.empty_cache()
    sustained = {"kernel": "q4_0_gemv_kernel, Q4_0 GEMV 151936x2560 (the head's shape)",
                 "bytes_per_launch": h_bytes, "us_per_launch": round(h_us, 3),
                 "gbs": round(h_bytes / (h_us * 1e-6) / 1e9, 1),
                 "frac_of_peak": round(h_bytes / (h_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
            "ceiling_gbs": ceil["gbs"], "frac_of_ceiling": round(gbs / ceil["gbs"], 4),
            "ceiling": ceil, "sustained": sustained,
            "kernel": "q4_0_gemv_kernel (Q4_0 GEMV 9728x2560, x bf16, y bf16)",
            "bytes_per_launch": GEMV_BYTES, "us_per_launch": round(us, 3),
            "timing": "HIP events over a captured graph of 24 launches on rotating weight sets "
                      "(336 MB), mean per launch including dispatch gaps; ceiling: the "
                      "streaming-read probe over the same 24 weight buffers; sustained: the "
                      "same kernel at the head's 218.8 MB shape over 2 rotating sets"}


def attention_roofline(dev, reps: int, ctxs=ATTN_CTXS, splits_list=ATTN_SPLITS):
    import torch
    from spark_vllm_ascend_amd.native import torch_ops as ops
    n_q, n_kv, hd, bs = 32, 8, 128, 128
    out = {}
    for ctx in ctxs:
        nblk = ctx // bs
        kv_bytes = 2 * ctx * n_kv * hd * 2
        sets = max(2, -(-ROTATE_BYTES // kv_bytes))
        g = torch.Generator(device=dev).manual_seed(7)
        planes = []  # K and V of one set in one allocation (the ceiling reads both at once)
        for _ in range(sets):
            kv = torch.empty((2, nblk, bs, n_kv, hd), dtype=torch.bfloat16, device=dev)
            kv.normal_(generator=g)
            planes.append(kv)
        caches = [(kv[0], kv[1]) for kv in planes]
        table = torch.randperm(nblk, generator=torch.Generator().manual_seed(3)).to(torch.int32)
        table = table.view(1, -1).to(dev)
        q = torch.randn((1, n_q, hd), device=dev).to(torch.bfloat16)
        seq_lens = torch.tensor([ctx], dtype=torch.int32, device=dev)
        o = torch.empty((1, n_q, hd), dtype=torch.bfloat16, device=dev)
        algo = kv_bytes + 2 * n_q * hd * 2  # K+V + q + out
        res = {}
        for S in splits_list:
            po = torch.empty((1, S, n_q, hd), dtype=torch.float32, device=dev)
            pl = torch.empty((1, S, n_q), dtype=torch.float32, device=dev)

            def fn():
                for kc, vc in caches:
                    ops.splitkv_decode_merged(q, kc, vc, table, seq_lens, S, hd ** -0.5, po, pl,
                                              out=o)
            us = time_graph(fn, sets, reps)
            gbs = algo / (us * 1e-6) / 1e9
            res[S] = {"us": round(us, 3), "achieved_gbs": round(gbs, 1),
                      "frac": round(gbs / HBM_PEAK_GBS, 4)}
        best = min(res, key=lambda s: res[s]["us"])
        # the read ceiling over the same bytes: each set's K and V read in one launch
        ceil = read_ceiling([kv.view(-1) for kv in planes], kv_bytes, reps)
        out[ctx] = {"bytes_per_call": algo, "sets": sets, "best_splits": best, **res[best],
                    "ceiling_gbs": ceil["gbs"], "ceiling_us": ceil["us"],
                    "frac_of_ceiling": round(algo / (res[best]["us"] * 1e-6) / 1e9 / ceil["gbs"], 4),
                    "sweep": res}
        del caches, planes
        torch.cuda.empty_cache()
    return {"by_ctx": out, "ctx": 6144, **{k: out[6144][k] for k in
                                           ("bytes_per_call", "best_splits", "us",
                                            "achieved_gbs", "frac", "ceiling_gbs")},
            "timing": "split-KV kernel + LSE merge kernel per call, HIP events over a graph of "
                      "calls on rotating KV sets (> 300 MB per context); ceiling: the "
                      "streaming-read probe over the same K and V planes"}


COPY_BYTES = 64 << 20


def counter_workload(dev, steps: int = 2):
    """Eager launches for a hardware-counter run (rocprofv3 --pmc), each part
    at the configuration it is reported for:
      * a plain device copy of COPY_BYTES, five times (the calibration
        kernel: it reads and writes exactly COPY_BYTES);
      * the 9728x2560 GEMV over 24 weight sets, twice, then the
        streaming-read probe over the same sets (the roofline kernel);
      * split-KV decode + LSE merge at context 6144 with the decode step's
        49 capacity splits (a 49-page block table), over 12 KV sets;
      * `steps` decode steps of the 36-layer 4B model at the benchmark's
        configuration (49-page block table, 49 splits, seeded KV cache,
        context 4096): every kernel of the step, 36 times per step;
      * `steps` steps of the 8-sequence batch at seeded contexts in
        512..32768 (MFMA GEMMs at m = 8, per-sequence split plan).
    rocprofv3 reads counters per dispatch with cold caches, so no part
    rotates buffers for cache reasons; the parts are told apart by kernel
    name and grid size."""
    import torch
    from spark_vllm_ascend_amd.integration.model import DecodeModel, DecoderConfig
    from spark_vllm_ascend_amd.integration.weights import synthetic_q4_0
    from spark_vllm_ascend_amd.native import probe
    from spark_vllm_ascend_amd.native import torch_ops as ops
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    ws = [synthetic_q4_0(GEMV_N, GEMV_K, 500 + i, dev) for i in range(24)]
    x = torch.randn(GEMV_K, device=dev).to(torch.bfloat16)
    y = torch.empty((1, GEMV_N), dtype=torch.bfloat16, device=dev)
    for _ in range(2):
        for w in ws:
            ops.q4_0_gemv(x, w, GEMV_N, GEMV_K, out=y)
    torch.cuda.synchronize()
    sink = torch.empty(probe.read_probe_sink_size(GEMV_W_BYTES, 8), dtype=torch.int32, device=dev)
    for w in ws:
        probe.read_probe(w.view(-1), GEMV_W_BYTES, sink, 8)
    torch.cuda.synchronize()
    del ws
    n_q, n_kv, hd, bs = 32, 8, 128, 128
    nblk = CAPACITY // bs  # 49 pages: the step's table and split count
    S = nblk
    caches = [(torch.randn((nblk, bs, n_kv, hd), device=dev).to(torch.bfloat16),
               torch.randn((nblk, bs, n_kv, hd), device=dev).to(torch.bfloat16))
              for _ in range(12)]
    table = torch.randperm(nblk, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    table = table.view(1, -1).to(dev)
    q = torch.randn((1, n_q, hd), device=dev).to(torch.bfloat16)
    seq_lens = torch.tensor([6144], dtype=torch.int32, device=dev)
    po = torch.empty((1, S, n_q, hd), dtype=torch.float32, device=dev)
    pl = torch.empty((1, S, n_q), dtype=torch.float32, device=dev)
    for kc, vc in caches:
        ops.splitkv_decode_merged(q, kc, vc, table, seq_lens, S, hd ** -0.5, po, pl)
    torch.cuda.synchronize()
    del caches
    # the decode step at the benchmark's configuration
    model = DecodeModel(DecoderConfig(), dev, seed=0, max_len=CAPACITY)
    model.fill_kv(1234)
    model.set_context([4095], ids=[1])
    for _ in range(steps):
        model.step()
    torch.cuda.synchronize()
    step_splits = model.num_splits
    del model
    torch.cuda.empty_cache()
    # the 8-sequence batch
    ctx = torch.randint(512, 32768, (8,), generator=torch.Generator().manual_seed(5))
    bm = DecodeModel(DecoderConfig(), dev, seed=5, max_len=int(ctx.max()) + steps + 2, batch=8)
    bm.fill_kv(5)
    bm.set_context(ctx.tolist())
    for _ in range(steps):
        bm.step()
    torch.cuda.synchronize()
    plan = (bm.num_items, bm.num_splits)
    del bm
    torch.cuda.empty_cache()
    return {"copy_bytes": COPY_BYTES, "gemv_bytes": GEMV_BYTES, "gemv_launches": 48,
            "read_probe_launches": 24, "attn_launches": 12, "attn_splits": S,
            "step": {"context": 4096, "steps": steps, "num_splits": step_splits},
            "batch": {"contexts": ctx.tolist(), "steps": steps, "plan": plan}}


def build_model(dev, max_len: int, num_splits: int | None, seed: int = 0):
    from spark_vllm_ascend_amd.integration.model import DecodeModel, DecoderConfig
    return DecodeModel(DecoderConfig(), dev, seed=seed, max_len=max_len, num_splits=num_splits)


#: fences between two kernels of a step-runner replay: agent-scope acquire,
#: no release (every kernel writes what a later one reads with agent-scope
#: stores, so no boundary needs an L2 write-back)
RUNNER_FENCES = "acquire"


def record_runner(model):
    """Record the model's decode step into a step runner; returns (executor,
    reason): ("runner", None), or ("graph", why) when no runner could be made
    (for instance no HSA queue), in which case the captured graph is timed."""
    try:
        model.record_runner()
        return "runner", None
    except Exception as exc:  # the graph executor still measures the same kernels
        return "graph", f"{type(exc).__name__}: {exc}"


EXECUTORS = {"runner": "step runner: AQL packets on the library's own HSA queue, agent-scope "
                       "acquire and no release between kernels",
             "graph": "HIP graph replay (agent-scope acquire and release between kernels)"}


def _untimed_steps(model, n: int, executor: str = "graph") -> None:
    if n <= 0:
        return
    if executor == "runner":
        model.run_steps(n, RUNNER_FENCES)
    else:
        for _ in range(n):
            model.step()


#: GPU-side seconds of the runner's timed replays (packet-processor
#: timestamps, first kernel's start to last kernel's end), summed by
#: _timed_steps beside the wall-clock figure both executors are timed by
RUNNER_GPU_S = []


def _timed_steps(model, n: int, executor: str = "graph") -> float:
    """Seconds for n decode steps, timed the same way for both executors:
    host wall-clock from a synchronised device to the completion of the
    n-th step (n graph replays then a device synchronise, or one step-runner
    replay of n steps then its wait).  For the runner, the GPU's own
    timestamps of the same replay go to RUNNER_GPU_S."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if executor == "runner":
        model.runner.replay(n, RUNNER_FENCES, sync=False)  # the device is synchronised
        model.runner.wait(120.0)
        dt = time.perf_counter() - t0
        RUNNER_GPU_S.append(model.runner.elapsed())
        return dt
    for _ in range(n):
        model.step()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def run_protocol(model, prompt, warmup: int, steps: int, executor: str = "graph"):
    """Feed the prompt, run `warmup` generated steps untimed, time `steps`;
    returns (seconds per step, tokens, positions timed)."""
    model.reset(prompt)
    _untimed_steps(model, prompt.numel() - 1 + warmup, executor)
    p0 = prompt.numel() - 1 + warmup
    dt = _timed_steps(model, steps, executor)
    total = prompt.numel() + warmup + steps
    return dt / steps, model.state.tokens[0, :total].clone().cpu(), list(range(p0, p0 + steps))


def spread_segments(steps: int, lo: int = PROMPT, hi: int = PROMPT + GENERATED - 2):
    """Up to 4 segments of timed positions covering [lo, hi] evenly: (first
    position, length) pairs whose lengths sum to `steps`."""
    n = min(4, steps)
    lens = [steps // n + (1 if i < steps % n else 0) for i in range(n)]
    if n == 1:
        return [(lo + (hi - lo - lens[0] + 1) // 2, lens[0])]
    span = hi - lo - lens[-1] + 1
    return [(lo + round(i * span / (n - 1)), lens[i]) for i in range(n)]


def run_spread(model, warmup: int, segments, executor: str = "graph"):
    """Time each segment's positions after `warmup` untimed steps before it,
    on the model's pre-filled KV cache; returns (seconds per step, tokens
    generated in the timed steps, positions timed)."""
    total_t, toks, positions = 0.0, [], []
    for p0, n in segments:
        model.set_context([p0 - warmup], ids=[1])
        _untimed_steps(model, warmup, executor)
        total_t += _timed_steps(model, n, executor)
        toks.append(model.state.tokens[0, p0 + 1:p0 + n + 1].clone().cpu())
        positions += list(range(p0, p0 + n))
    import torch
    return total_t / len(positions), torch.cat(toks), positions


def batch_breakdown(model, ctx, reps: int = 10):
    """Unprofiled per-class times of the batched step, as step_breakdown does
    for one sequence: each kernel class of a layer in a captured graph of its
    36 launches (each layer's own weights and KV cache), per-launch means
    including the gap to the next launch; the head (final add+RMSNorm + head
    GEMM with argmax keys) and the advance kernel by difference against the
    36 gate/up launches.  Resets the contexts first, and leaves the model's
    state advanced."""
    from spark_vllm_ascend_amd.native import torch_ops as ops
    from spark_vllm_ascend_amd.integration.linear import gemm_weight as gw
    m, c, st, L = model, model.cfg, model.state, model.layers
    n, B = len(L), model.batch
    head_w = m.head_packed if m.head_packed is not None else m.head.q4_0_head
    m.set_context(list(ctx))
    ops.splitkv_plan(st.seq_lens, st.block_table, c.block_size, m.num_items, m.partial_o,
                     m.partial_lse, positions=st.positions, slot_mapping=st.slot_mapping,
                     plan=m.plan)
    kernels = {
        "norm_in": ("residual add + input RMSNorm, B rows", 1, lambda i: ops.add_rmsnorm(
            m.d, m.res_b, L[i].input_norm, c.eps, out=m.h, residual_out=m.res_a)),
        "qkv": ("QKV GEMM 6144x2560 (packed weights), m = B", 1, lambda i: ops.q4_0_gemm(
            m.h, gw(L[i].qkv), c.qkv_rows, c.hidden, out=m.qkv_out)),
        "attention": ("q/k norm + RoPE + KV write + split-KV over the plan, then the LSE merge "
                      "(two launches)", 2, lambda i: ops.qknorm_rope_splitkv_decode_planned_merged(
            m.qkv_out, L[i].q_norm, L[i].k_norm, m.cos_sin, L[i].kv_cache[0], L[i].kv_cache[1],
            st.block_table, m.plan, m.num_items, m.scale, c.eps, c.n_q, m.partial_o,
            m.partial_lse, out=m.attn)),
        "o_proj": ("o_proj GEMM 2560x4096 (packed weights), m = B", 1, lambda i: ops.q4_0_gemm(
            m.attn.view(B, -1), gw(L[i].o_proj), c.hidden, c.n_q * c.head_dim, out=m.o)),
        "norm_post": ("residual add + post-attention RMSNorm, B rows", 1, lambda i: ops.add_rmsnorm(
            m.o, m.res_a, L[i].post_norm, c.eps, out=m.h2, residual_out=m.res_b)),
        "gate_up": ("gate/up GEMM 19456x2560 + SwiGLU (packed weights), m = B", 1, lambda i: ops.q4_0_gemm_swiglu(
            m.h2, gw(L[i].gate_up, gated=True), c.intermediate, c.hidden, out=m.act)),
        "down": ("down GEMM 2560x9728 (packed weights), m = B", 1, lambda i: ops.q4_0_gemm(
            m.act, gw(L[i].down), c.hidden, c.intermediate, out=m.d)),
    }
    rb = lambda rows, k: rows * k // 32 * 18
    weight_bytes = {"qkv": rb(c.qkv_rows, c.hidden), "o_proj": rb(c.hidden, c.n_q * c.head_dim),
                    "gate_up": rb(2 * c.intermediate, c.hidden),
                    "down": rb(c.hidden, c.intermediate)}
    out = {}
    for key, (what, launches, f) in kernels.items():
        us = time_graph(lambda: [f(i) for i in range(n)], n * launches, reps) * launches
        out[key] = {"what": what, "us_per_layer": round(us, 3)}
        if key in weight_bytes:  # the GEMMs: Q4_0 weight bytes streamed per microsecond
            out[key]["weight_gbs"] = round(weight_bytes[key] / us / 1e3, 1)
    gu = kernels["gate_up"][2]

    def head():
        ops.add_rmsnorm(m.d, m.res_b, m.final_norm, c.eps, out=m.h)
        ops.q4_0_gemm_argmax(m.h, head_w, c.vocab, c.hidden, m.argmax_keys, out=m.logits)

    def advance():
        ops.decode_advance(st.next_ids, st.ids, st.positions, st.seq_lens, st.slot_mapping,
                           st.block_table, c.block_size, tokens_out=st.tokens,
                           forced_ids=st.forced, forced_len=st.forced_len,
                           argmax_keys=m.argmax_keys, embed_table=m.head.weight, embed_out=m.x)
    base = time_graph(lambda: [gu(i) for i in range(n)], n, reps) * n
    with_head = time_graph(lambda: ([gu(i) for i in range(n)], head()), n + 2, reps) * (n + 2)
    out["head"] = {"what": "final add+RMSNorm + Q4_0 head GEMM 151936x2560 (packed weights) + argmax keys",
                   "us_per_step": round(with_head - base, 3)}
    m.set_context(list(ctx))
    with_adv = time_graph(lambda: ([gu(i) for i in range(n)], advance()), n + 1, reps) * (n + 1)
    out["advance"] = {"what": "argmax reduction, step advance, next embedding rows",
                      "us_per_step": round(with_adv - base, 3)}
    per_layer = sum(v["us_per_layer"] for v in out.values() if "us_per_layer" in v)
    total = n * per_layer + out["head"]["us_per_step"] + out["advance"]["us_per_step"]
    return {"kernels": out, "us_per_layer": round(per_layer, 3),
            "per_step_sum_ms": round(total / 1e3, 4),
            "timing": "HIP events over captured graphs of each kernel class's 36 launches, "
                      "per-launch mean including the gap to the next launch; the head and the "
                      "advance kernel by difference; one plan launch per step not included"}


def batch_decode(dev, steps: int = 64, warmup: int = 4, batch: int = 8, seed: int = 5,
                 breakdown: bool = True, executor: str = "runner"):
    """Config-5 style throughput: `batch` sequences at seeded ragged contexts
    ~U[512, 32768] decoded together through the captured step graph (MFMA
    GEMM path, split-KV over per-sequence block tables), over a KV cache
    filled with seeded random bf16; with `breakdown`, the unprofiled
    per-class times of that step (batch_breakdown).  executor "graph"
    times the captured graph only (no step runner is recorded)."""
    import torch
    from spark_vllm_ascend_amd.integration.model import DecodeModel, DecoderConfig
    ctx = torch.randint(512, 32768, (batch,), generator=torch.Generator().manual_seed(seed))
    max_len = int(ctx.max()) + warmup + steps + 2
    model = DecodeModel(DecoderConfig(), dev, seed=seed, max_len=max_len, batch=batch)
    model.fill_kv(seed)
    model.set_context(ctx.tolist())
    model.capture()
    runner_error = None
    if executor == "runner":
        executor, runner_error = record_runner(model)
    model.set_context(ctx.tolist())
    _untimed_steps(model, warmup, executor)
    dt = _timed_steps(model, steps, executor) / steps
    toks = model.state.tokens.clone().cpu()
    graph_dt = same = None
    if executor == "runner":  # the same steps through the graph, for comparison
        model.set_context(ctx.tolist())
        _untimed_steps(model, warmup, "graph")
        graph_dt = _timed_steps(model, steps, "graph") / steps
        same = bool(torch.equal(toks, model.state.tokens.cpu()))
        model.runner.close()
    c = model.cfg
    rb = lambda n, k: n * k // 32 * 18
    weights = c.n_layers * (rb(c.qkv_rows, c.hidden) + rb(c.hidden, c.n_q * c.head_dim)
                            + rb(2 * c.intermediate, c.hidden) + rb(c.hidden, c.intermediate)) \
        + rb(c.vocab, c.hidden)
    mid = ctx.to(torch.float64) + warmup + steps / 2
    kv = int((mid * 2 * c.n_kv * c.head_dim * 2 * c.n_layers).sum())
    model_items, model_splits = model.num_items, model.num_splits
    bd = batch_breakdown(model, ctx.tolist()) if breakdown else None
    del model
    torch.cuda.empty_cache()
    extra = {"step_breakdown": bd} if bd else {}
    if graph_dt is not None:
        extra.update(graph_ms_per_step=round(graph_dt * 1e3, 4),
                     tokens_equal_graph_vs_runner=same)
    if runner_error:
        extra["runner_error"] = runner_error
    return {**extra, "batch": batch, "contexts": ctx.tolist(), "steps": steps,
            "executor": EXECUTORS[executor],
            "ms_per_step": round(dt * 1e3, 4),
            "tok_s": round(batch / dt, 2),
            # every sequence advances one token per step: its TPOT is the step time
            "tpot_ms_per_sequence": [round(dt * 1e3, 4)] * batch,
            "plan": {"num_items": model_items, "num_splits": model_splits},
            "bytes_per_step": weights + kv,
            "achieved_gbs": round((weights + kv) / dt / 1e9, 1),
            "note": "8 sequences, contexts ~U[512, 32768] (seeded), KV cache filled with seeded "
                    "random bf16, greedy; split-KV over a per-sequence split plan"}


def step_breakdown(model, ctx: int, reps: int = 10):
    """Unprofiled per-kernel times of one decode step at context ctx: each
    kernel class of a layer timed alone in a captured graph of its 36
    launches (one per layer, so every launch streams that layer's own
    weights and KV cache, beyond the 256 MB Infinity Cache), the head as the
    difference between a graph of the 36 gate/up launches with and without
    it.  Per-launch times include the gap to the next launch, as in the
    step, so their per-step sum can be set against the measured TPOT
    (rocprofv3's kernel trace inflates every dispatch)."""
    import torch
    from spark_vllm_ascend_amd.native import torch_ops as ops
    c, st, L = model.cfg, model.state, model.layers
    n = len(L)
    model.set_context([ctx - 1], ids=[1])
    keys = model.argmax_keys.view(-1)
    kernels = {
        "qkv": ("add+RMSNorm + QKV GEMV 6144x2560", lambda i: ops.add_rmsnorm_gemv(
            model.d, model.res_b, L[i].input_norm, L[i].qkv.qweight, c.qkv_rows, c.hidden, c.eps,
            residual_out=model.res_a, out=model.qkv_out)),
        "attention": ("q/k norm + RoPE + KV write + split-KV decode, then the LSE merge "
                      "(two launches)", lambda i: ops.qknorm_rope_splitkv_decode_merged(
            model.qkv_out, L[i].q_norm, L[i].k_norm, model.cos_sin, st.positions, st.slot_mapping,
            L[i].kv_cache[0], L[i].kv_cache[1], st.block_table, st.seq_lens, model.num_splits,
            model.scale, c.eps, c.n_q, model.partial_o, model.partial_lse, out=model.attn)),
        "o_proj": ("o_proj GEMV 2560x4096", lambda i: ops.q4_0_gemv(
            model.attn, L[i].o_proj.qweight, c.hidden, c.n_q * c.head_dim, out=model.o)),
        "gate_up": ("add+RMSNorm + gate/up GEMV 19456x2560 + SwiGLU", lambda i: ops.add_rmsnorm_gemv_swiglu(
            model.o, model.res_a, L[i].post_norm, L[i].gate_up.qweight, c.intermediate, c.hidden,
            c.eps, residual_out=model.res_b, out=model.act)),
        "down": ("down GEMV 2560x9728", lambda i: ops.q4_0_gemv(
            model.act, L[i].down.qweight, c.hidden, c.intermediate, out=model.d)),
    }
    out = {}
    for key, (what, f) in kernels.items():
        us = time_graph(lambda: [f(i) for i in range(n)], n, reps)
        out[key] = {"what": what, "us_per_layer": round(us, 3)}
    gu = kernels["gate_up"][1]

    def head():
        ops.add_rmsnorm_gemv_argmax(model.d, model.res_b, model.final_norm, model.head.q4_0_head,
                                    c.vocab, c.hidden, c.eps, keys, out=model.logits)

    def advance():
        ops.decode_advance(st.next_ids, st.ids, st.positions, st.seq_lens, st.slot_mapping,
                           st.block_table, c.block_size, tokens_out=st.tokens,
                           forced_ids=st.forced, forced_len=st.forced_len,
                           argmax_keys=model.argmax_keys, embed_table=model.head.weight,
                           embed_out=model.x)
    base = time_graph(lambda: [gu(i) for i in range(n)], n, reps) * n
    with_head = time_graph(lambda: ([gu(i) for i in range(n)], head()), n + 1, reps) * (n + 1)
    out["head"] = {"what": "final add+RMSNorm + Q4_0 head GEMV 151936x2560 + argmax keys",
                   "us_per_step": round(with_head - base, 3)}
    with_adv = time_graph(lambda: ([gu(i) for i in range(n)], advance()), n + 1, reps) * (n + 1)
    out["advance"] = {"what": "argmax reduction, step advance, next embedding row",
                      "us_per_step": round(with_adv - base, 3)}
    per_layer = sum(v["us_per_layer"] for v in out.values() if "us_per_layer" in v)
    total = n * per_layer + out["head"]["us_per_step"] + out["advance"]["us_per_step"]
    model.set_context([ctx - 1], ids=[1])
    return {"context": ctx, "kernels": out, "us_per_layer": round(per_layer, 3),
            "per_step_sum_ms": round(total / 1e3, 4),
            "timing": "HIP events over captured graphs of each kernel class's 36 launches (each "
                      "layer's own weights / KV cache), per-launch mean including the gap to "
                      "the next launch; the head and the advance kernel by difference"}


def step_bytes(cfg, ctx: int) -> int:
    c = cfg
    rb = lambda n, k: n * k // 32 * 18
    layer = (rb(c.qkv_rows, c.hidden) + rb(c.hidden, c.n_q * c.head_dim)
             + rb(2 * c.intermediate, c.hidden) + rb(c.hidden, c.intermediate))
    kv = 2 * ctx * c.n_kv * c.head_dim * 2
    norms = (2 * c.hidden + 2 * c.head_dim) * 2
    return c.n_layers * (layer + kv + norms) + rb(c.vocab, c.hidden) + c.hidden * 2 * 2


def _median_time(fn, reps: int, warm: int = 3) -> float:
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(model, ctx: int, reps: int, budget_s: float):
    """The reference's CPU path on this host: bf16 weights (RNE(d*q), the
    bytes the reference deploys) + F.linear, timed per decode step on all
    cores and on 4 threads; plus the single-GEMV and attention legs."""
    import numpy as np
    import torch
    from oracle.cpu_path import CpuDecoder
    from oracle import q4_0 as oq
    from spark_vllm_ascend_amd.integration.weights import dequantize_bf16, synthetic_q4_0
    cores = len(os.sched_getaffinity(0))
    c = model.cfg
    layers = []
    for L in model.layers:
        layers.append({
            "qkv": dequantize_bf16(L.qkv.qweight, c.qkv_rows, c.hidden).cpu(),
            "o_proj": dequantize_bf16(L.o_proj.qweight, c.hidden, c.n_q * c.head_dim).cpu(),
            "gate_up": dequantize_bf16(L.gate_up.qweight, 2 * c.intermediate, c.hidden).cpu(),
            "down": dequantize_bf16(L.down.qweight, c.hidden, c.intermediate).cpu(),
            "input_norm": L.input_norm.cpu(), "post_norm": L.post_norm.cpu(),
            "q_norm": L.q_norm.cpu(), "k_norm": L.k_norm.cpu()})
    dec = CpuDecoder(c, layers, model.final_norm.cpu(), model.head.weight.cpu(),
                     model.cos_sin.cpu(), ctx + 2 * reps + 8)
    dec.fill_cache(ctx)

    def steps_at(threads: int):
        torch.set_num_threads(threads)
        dec.step(1, ctx)  # warm-up (first touch, thread pool)
        times, tok, t_start = [], 1, time.perf_counter()
        for i in range(reps):
            t0 = time.perf_counter()
            tok = dec.step(tok, ctx + 1 + i)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - t_start > budget_s and len(times) >= 5:
                break
        return statistics.median(times), len(times)

    med_all, n_all = steps_at(cores)
    log(f"  decode step, {cores} threads: {med_all * 1e3:.1f} ms (median of {n_all})")
    med_4, n_4 = steps_at(4)
    log(f"  decode step, 4 threads: {med_4 * 1e3:.1f} ms (median of {n_4})")

    # config 1: the single GEMV on pre-dequantised bf16 weights (F.linear),
    # and the fp32/fp64-accumulating restatement the oracle uses
    blocks = synthetic_q4_0(GEMV_N, GEMV_K, 500, model.device)
    w_bf16 = dequantize_bf16(blocks, GEMV_N, GEMV_K).cpu()
    x = torch.randn((1, GEMV_K)).to(torch.bfloat16)
    legs = {}
    for threads in (cores, 4):
        torch.set_num_threads(threads)
        t = _median_time(lambda: torch.nn.functional.linear(x, w_bf16), max(reps, 20))
        legs[f"gemv_9728x2560_f_linear_bf16_{threads}t"] = {
            "us": round(t * 1e6, 1), "gbs_of_q4_0_bytes": round(GEMV_BYTES / t / 1e9, 2)}
    blocks_np = blocks.cpu().numpy()
    x_bits = x.view(torch.int16).numpy().view(np.uint16).reshape(-1)
    t = _median_time(lambda: oq.gemv_f64(x_bits, blocks_np, GEMV_N, GEMV_K), max(reps, 20), 1)
    legs["gemv_9728x2560_oracle_c_f64"] = {"us": round(t * 1e6, 1),
                                           "gbs_of_q4_0_bytes": round(GEMV_BYTES / t / 1e9, 2)}
    # config 2: fp32 attention at 6144 over a gathered cache (one q head per kv
    # head group, softmax(q K^T s) V)
    n_q, n_kv, hd, L = 32, 8, 128, 6144
    q = torch.randn((n_q, hd))
    kk = torch.randn((L, n_kv, hd)).to(torch.bfloat16)
    vv = torch.randn((L, n_kv, hd)).to(torch.bfloat16)

    def attn():
        k = kk.float().repeat_interleave(n_q // n_kv, dim=1)
        v = vv.float().repeat_interleave(n_q // n_kv, dim=1)
        s = torch.bmm(q.unsqueeze(1), k.permute(1, 2, 0).contiguous()).squeeze(1) * hd ** -0.5
        return torch.bmm(torch.softmax(s, -1).unsqueeze(1), v.permute(1, 0, 2).contiguous())
    for threads in (cores, 4):
        torch.set_num_threads(threads)
        t = _median_time(attn, max(reps, 20))
        legs[f"attention_ctx6144_fp32_{threads}t"] = {"us": round(t * 1e6, 1)}
    torch.set_num_threads(cores)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(1.0 / med_all, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "ms_per_token": round(med_all * 1e3, 2), "cpu": cpu_model,
            "threads_4": {"value": round(1.0 / med_4, 3), "ms_per_token": round(med_4 * 1e3, 2),
                          "steps": n_4},
            "legs": legs,
            "sample": f"median of {n_all} decode steps of the 36-layer model at context "
                      f"{ctx + 1}.. (KV cache pre-filled with seeded random bf16), torch "
                      f"{torch.__version__} CPU, bf16 F.linear, {cores} threads; the same on 4 "
                      f"threads ({n_4} steps); legs: the 9728x2560 GEMV and fp32 attention at "
                      f"6144, median of >= 20"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=GENERATED - 1)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--runs", type=int, default=3)
    ap.add_argument("--prompt-len", type=int, default=PROMPT)
    ap.add_argument("--num-splits", type=int, default=0, help="0 = backend default")
    ap.add_argument("--phase", choices=["all", "roofline", "decode", "counters", "batch", "cpu"],
                    default="all",
                    help="counters: eager launches for a rocprofv3 --pmc run, no timing")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-breakdown", action="store_true",
                    help="no per-kernel step breakdown (e.g. under a profiler)")
    ap.add_argument("--cpu-budget", type=float, default=25.0,
                    help="seconds per decode-step leg of the CPU baseline")
    ap.add_argument("--executor", choices=["runner", "graph"], default="runner",
                    help="batch phase: time the step runner (and the graph beside it), or the "
                         "captured graph alone (rocprofv3's kernel trace does not run the "
                         "runner's replays of the 8-sequence step)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode path has no multi-GPU launch (it would "
              "shard the GEMVs by output rows and the attention by kv heads)",
              file=sys.stderr)
        return 2

    import torch
    import __graft_entry__
    __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    result = {}

    if args.phase == "counters":
        print(json.dumps(counter_workload(dev)))
        return 0
    if args.phase == "batch":
        print(json.dumps(batch_decode(dev, breakdown=not args.skip_breakdown,
                                      executor=args.executor)))
        return 0

    if args.phase in ("all", "roofline"):
        log("GEMV roofline (9728x2560, 24 rotating weight sets)")
        result["roofline"] = gemv_roofline(dev, reps=20)
        r = result["roofline"]
        log(f"  {r['us_per_launch']} us/launch, {r['achieved']} GB/s; read ceiling "
            f"{r['ceiling']['us']} us ({r['ceiling_gbs']} GB/s)")
        log("attention roofline (ctx 2048 / 4096 / 6144, rotating KV sets)")
        result["attention"] = attention_roofline(dev, reps=20)
        for ctx, a in result["attention"]["by_ctx"].items():
            log(f"  ctx {ctx}: best splits {a['best_splits']}: {a['us']} us "
                f"({a['achieved_gbs']} GB/s, ceiling {a['ceiling_gbs']} GB/s)")
        pmc = ROOT / "profiles" / "q4_0_gemv_9728x2560_traffic.json"
        if pmc.exists():
            result["roofline"]["traffic"] = json.loads(pmc.read_text()).get("traffic_bytes")
        torch.cuda.empty_cache()
        if args.phase == "roofline":
            print(json.dumps(result))
            return 0

    protocol = args.steps >= GENERATED - 1 and args.prompt_len == PROMPT
    max_len = max(CAPACITY, args.prompt_len + args.warmup + args.steps + 1)
    log(f"building the 4B model (block table {-(-max_len // 128)} pages)")
    model = build_model(dev, max_len, args.num_splits or None)
    model.capture()
    executor, runner_error = record_runner(model)
    log(f"executor: {EXECUTORS[executor]}" + (f" ({runner_error})" if runner_error else ""))
    c = model.cfg
    if protocol:
        prompt = torch.randint(0, c.vocab, (args.prompt_len,),
                               generator=torch.Generator().manual_seed(1234))
        how = (f"prompt {args.prompt_len} random ids through the decode graph, TPOT over the "
               f"{args.steps} tokens after {args.warmup} warmup")
    else:
        model.fill_kv(1234)
        segments = spread_segments(args.steps)
        how = (f"TPOT over {args.steps} tokens in {len(segments)} segments at positions "
               f"{', '.join(f'{p}..{p + n - 1}' for p, n in segments)} (each after "
               f"{args.warmup} untimed tokens) over a seeded random KV cache, spread over the "
               f"protocol's {PROMPT + 1}..{PROMPT + GENERATED} contexts")
    def one_run(ex):
        if protocol:
            return run_protocol(model, prompt, args.warmup, args.steps, ex)
        return run_spread(model, args.warmup, segments, ex)

    tpots, token_runs, gpu_runs = [], [], []
    for r in range(args.runs):
        RUNNER_GPU_S.clear()
        tpot, toks, positions = one_run(executor)
        if RUNNER_GPU_S:
            gpu_runs.append(sum(RUNNER_GPU_S) / len(positions))
        tpots.append(tpot)
        token_runs.append(toks)
        log(f"run {r}: TPOT {tpot * 1e3:.4f} ms ({1 / tpot:.1f} tok/s)")
    tpot = statistics.median(tpots)
    deterministic = all(torch.equal(token_runs[0], t) for t in token_runs[1:])
    graph_cmp = {}
    if gpu_runs:  # the GPU's own clock over the same replays (no host dispatch or wake-up)
        graph_cmp["runner_gpu_ms_per_step"] = round(statistics.median(gpu_runs) * 1e3, 4)
    if executor == "runner":  # the same steps once through the captured graph
        g_tpot, g_toks, _ = one_run("graph")
        graph_cmp.update({"graph_ms_per_step": round(g_tpot * 1e3, 4),
                          "tokens_equal_graph_vs_runner": bool(torch.equal(g_toks,
                                                                           token_runs[0]))})
        log(f"graph: TPOT {g_tpot * 1e3:.4f} ms")
        model.runner.close()
    gen = token_runs[0][args.prompt_len:] if protocol else token_runs[0]
    valid = bool(((gen >= 0) & (gen < c.vocab)).all())
    mean_bytes = statistics.fmean(step_bytes(c, p + 1) for p in positions)
    bound_ms = mean_bytes / (HBM_PEAK_GBS * 1e9) * 1e3
    out = {
        "metric": "batch-1 decode TPOT ms/token (tok/s) 4B Q4_0; GEMV+attn HBM GB/s vs peak",
        "value": round(1.0 / tpot, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(tpot * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, seeded random prompt ids / KV contents)",
        "config": {"workload": "4B Q4_0 decoder: 36 layers, hidden 2560, 32q/8kv x 128, SwiGLU "
                               "9728, vocab 151936 Q4_0 head, BF16 paged KV block 128, block "
                               f"table {model.state.block_table.shape[1]} pages; greedy decode, "
                               f"{how}; median of {args.runs} runs",
                   "global_batch": 1, "seq_len": max(positions) + 1,
                   "contexts": [min(positions) + 1, max(positions) + 1],
                   "mean_context": round(statistics.fmean(positions) + 1, 1),
                   "parallelism": "single GPU", "num_splits": model.num_splits},
        "executor": EXECUTORS[executor],
        **graph_cmp,
        **({"runner_error": runner_error} if runner_error else {}),
        "tpot_ms_runs": [round(t * 1e3, 4) for t in tpots],
        "tokens_deterministic_across_runs": deterministic,
        "tokens_in_vocab": valid,
        "step": {"mean_bytes_per_token": int(mean_bytes), "hbm_bound_ms": round(bound_ms, 4),
                 "frac_of_bound": round(bound_ms / (tpot * 1e3), 4),
                 "achieved_gbs": round(mean_bytes / tpot / 1e9, 1)},
        "reference_published": {"tpot_ms": 2.909848, "tok_s": 343.661,
                                "note": "Spark-X2.6-4B Q4_0 on Ascend 950 (a different model "
                                        "shape), README.en.md:87; not this exact workload"},
    }
    out.update(result)
    if not args.skip_breakdown:
        log("step breakdown (each kernel class alone, at the timed steps' mean context)")
        out["step_breakdown"] = step_breakdown(model, int(round(statistics.fmean(positions))) + 1)
        sb = out["step_breakdown"]
        # the breakdown replays graphs: set it against the graph executor's step
        sb["measured_ms"] = graph_cmp.get("graph_ms_per_step", round(tpot * 1e3, 4))
        log(f"  per layer {sb['us_per_layer']} us; per step {sb['per_step_sum_ms']} ms "
            f"(graph step measured {sb['measured_ms']} ms)")
    if args.phase == "all":
        log("batched decode (8 ragged sequences)")
        out["batch_decode"] = batch_decode(dev, breakdown=not args.skip_breakdown)
        log(f"  {out['batch_decode']['tok_s']} tok/s aggregate")
    if not args.skip_cpu and args.phase in ("all", "cpu", "decode"):
        log("CPU baseline")
        out["cpu_baseline"] = cpu_baseline(model, ctx=PROMPT + GENERATED // 2, reps=21,
                                           budget_s=args.cpu_budget)
        log(f"  {out['cpu_baseline']['ms_per_token']} ms/token on "
            f"{out['cpu_baseline']['cores']} cores")
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
