"""Benchmark: batch-1 greedy decode TPOT of the 4B Q4_0 decoder on one MI355X.

Workload (the configuration the headline metric is quoted on): 36-layer
decoder, hidden 2560, 32 q / 8 kv heads of 128, SwiGLU 9728, tied vocab
151936 with a Q4_0 head, random-init weights, BF16 paged KV (block 128).
A 2048-token random prompt is fed through the decode graph, the first
generated token is the untimed warmup, and K further greedy tokens are timed:
TPOT = time / K, as the reference defines it over SSE events
((t_last - t_first) / 4095, src/tools/benchmark/benchmark.py:123).  The
median over --runs independent runs is reported.

Also reported, on the same box in the same run:
  roofline      the Q4_0 GEMV [9728 x 2560] (the dominant kernel class:
                2.26 of the 2.87 GB a token streams) timed with HIP events
                over a captured graph of launches that rotate through 24
                weight sets (336 MB, larger than the 256 MB Infinity Cache);
                achieved = 14,032,896 algorithmic bytes / mean launch time;
  attention     split-KV decode + LSE merge at context 6144 (25.2 MB of KV)
                over 12 rotating KV sets, for each split count;
  step          bytes a decode step streams vs the HBM-bound step time;
  cpu_baseline  the reference's PyTorch CPU path (bf16 weights, F.linear)
                on this host's cores, on a bounded sample of decode steps.
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

HBM_PEAK_GBS = 8000.0
GEMV_N, GEMV_K = 9728, 2560
GEMV_BYTES = GEMV_N * GEMV_K // 32 * 18 + GEMV_K * 2 + GEMV_N * 2  # 14,032,896
ATTN_CTX = 6144


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
    del ws
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "q4_0_gemv_kernel (Q4_0 GEMV 9728x2560, x bf16, y bf16)",
            "bytes_per_launch": GEMV_BYTES, "us_per_launch": round(us, 3),
            "timing": "HIP events over a captured graph of 24 launches on rotating weight sets "
                      "(336 MB), mean per launch including dispatch gaps"}


def attention_roofline(dev, reps: int, splits_list=(4, 8, 16, 32, 64)):
    import torch
    from spark_vllm_ascend_amd.native import torch_ops as ops
    n_q, n_kv, hd, bs = 32, 8, 128, 128
    nblk = ATTN_CTX // bs
    sets = 12
    g = torch.Generator(device=dev).manual_seed(7)
    caches = []
    for _ in range(sets):
        kc = torch.randn((nblk, bs, n_kv, hd), generator=g, device=dev).to(torch.bfloat16)
        vc = torch.randn((nblk, bs, n_kv, hd), generator=g, device=dev).to(torch.bfloat16)
        caches.append((kc, vc))
    table = torch.randperm(nblk, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    table = table.view(1, -1).to(dev)
    q = torch.randn((1, n_q, hd), device=dev).to(torch.bfloat16)
    seq_lens = torch.tensor([ATTN_CTX], dtype=torch.int32, device=dev)
    out = torch.empty((1, n_q, hd), dtype=torch.bfloat16, device=dev)
    algo = 2 * ATTN_CTX * n_kv * hd * 2 + 2 * n_q * hd * 2  # K+V + q + out = 25,182,208
    res = {}
    for S in splits_list:
        po = torch.empty((1, S, n_q, hd), dtype=torch.float32, device=dev)
        pl = torch.empty((1, S, n_q), dtype=torch.float32, device=dev)

        def fn():
            for kc, vc in caches:
                ops.splitkv_decode_merged(q, kc, vc, table, seq_lens, S, hd ** -0.5, po, pl,
                                          out=out)
        us = time_graph(fn, sets, reps)
        gbs = algo / (us * 1e-6) / 1e9
        res[S] = {"us": round(us, 3), "achieved_gbs": round(gbs, 1),
                  "frac": round(gbs / HBM_PEAK_GBS, 4)}
    best = min(res, key=lambda s: res[s]["us"])
    del caches
    return {"ctx": ATTN_CTX, "bytes_per_call": algo, "best_splits": best, **res[best],
            "sweep": res, "timing": "split-KV kernel + LSE merge kernel per call, HIP events "
                                   "over a graph of 12 calls on rotating KV sets (302 MB)"}


COPY_BYTES = 64 << 20


def counter_workload(dev):
    """Eager launches for a hardware-counter run (rocprofv3 --pmc): a plain
    device copy of COPY_BYTES (the calibration kernel: it reads and writes
    exactly COPY_BYTES), then the 9728x2560 GEMV over 24 rotating weight
    sets, then split-KV decode + merge at context 6144 over 12 KV sets."""
    import torch
    from spark_vllm_ascend_amd.integration.weights import synthetic_q4_0
    from spark_vllm_ascend_amd.native import torch_ops as ops
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    ws = [synthetic_q4_0(GEMV_N, GEMV_K, 500 + i, dev) for i in range(24)]
    x = torch.randn(GEMV_K, device=dev).to(torch.bfloat16)
    y = torch.empty((1, GEMV_N), dtype=torch.bfloat16, device=dev)
    for _ in range(2):
        for w in ws:
            ops.q4_0_gemv(x, w, GEMV_N, GEMV_K, out=y)
    torch.cuda.synchronize()
    del ws
    n_q, n_kv, hd, bs = 32, 8, 128, 128
    nblk = ATTN_CTX // bs
    caches = [(torch.randn((nblk, bs, n_kv, hd), device=dev).to(torch.bfloat16),
               torch.randn((nblk, bs, n_kv, hd), device=dev).to(torch.bfloat16))
              for _ in range(12)]
    table = torch.randperm(nblk, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    table = table.view(1, -1).to(dev)
    q = torch.randn((1, n_q, hd), device=dev).to(torch.bfloat16)
    seq_lens = torch.tensor([ATTN_CTX], dtype=torch.int32, device=dev)
    S = 32
    po = torch.empty((1, S, n_q, hd), dtype=torch.float32, device=dev)
    pl = torch.empty((1, S, n_q), dtype=torch.float32, device=dev)
    for kc, vc in caches:
        ops.splitkv_decode_merged(q, kc, vc, table, seq_lens, S, hd ** -0.5, po, pl)
    torch.cuda.synchronize()
    return {"copy_bytes": COPY_BYTES, "gemv_bytes": GEMV_BYTES, "gemv_launches": 48,
            "attn_launches": 12, "attn_splits": S}


def build_model(dev, max_len: int, num_splits: int | None, seed: int = 0):
    from spark_vllm_ascend_amd.integration.model import DecodeModel, DecoderConfig
    return DecodeModel(DecoderConfig(), dev, seed=seed, max_len=max_len, num_splits=num_splits)


def run_decode(model, prompt, warmup: int, steps: int):
    """Feed the prompt, run `warmup` generated steps untimed, time `steps`."""
    import torch
    model.reset(prompt)
    for _ in range(prompt.numel() - 1 + warmup):
        model.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    total = prompt.numel() + warmup + steps
    return (t1 - t0) / steps, model.state.tokens[0, :total].clone().cpu()


def batch_decode(dev, steps: int = 64, warmup: int = 4, batch: int = 8, seed: int = 5):
    """Config-5 style throughput: `batch` sequences at seeded ragged contexts
    ~U[512, 32768] decoded together through the captured step graph (MFMA
    GEMM path, split-KV over per-sequence block tables)."""
    import torch
    from spark_vllm_ascend_amd.integration.model import DecodeModel, DecoderConfig
    ctx = torch.randint(512, 32768, (batch,), generator=torch.Generator().manual_seed(seed))
    max_len = int(ctx.max()) + warmup + steps + 2
    model = DecodeModel(DecoderConfig(), dev, seed=seed, max_len=max_len, batch=batch)
    model.set_context(ctx.tolist())
    model.capture()
    model.set_context(ctx.tolist())
    for _ in range(warmup):
        model.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    c = model.cfg
    rb = lambda n, k: n * k // 32 * 18
    weights = c.n_layers * (rb(c.qkv_rows, c.hidden) + rb(c.hidden, c.n_q * c.head_dim)
                            + rb(2 * c.intermediate, c.hidden) + rb(c.hidden, c.intermediate)) \
        + rb(c.vocab, c.hidden)
    mid = ctx.to(torch.float64) + warmup + steps / 2
    kv = int((mid * 2 * c.n_kv * c.head_dim * 2 * c.n_layers).sum())
    model_items, model_splits = model.num_items, model.num_splits
    del model
    torch.cuda.empty_cache()
    return {"batch": batch, "contexts": ctx.tolist(), "steps": steps, "ms_per_step": round(dt * 1e3, 4),
            "tok_s": round(batch / dt, 2),
            # every sequence advances one token per step: its TPOT is the step time
            "tpot_ms_per_sequence": [round(dt * 1e3, 4)] * batch,
            "plan": {"num_items": model_items, "num_splits": model_splits},
            "bytes_per_step": weights + kv,
            "achieved_gbs": round((weights + kv) / dt / 1e9, 1),
            "note": "8 sequences, contexts ~U[512, 32768] (seeded), random KV contents, greedy; "
                    "split-KV over a per-sequence split plan"}


def step_bytes(cfg, ctx: int) -> int:
    c = cfg
    rb = lambda n, k: n * k // 32 * 18
    layer = (rb(c.qkv_rows, c.hidden) + rb(c.hidden, c.n_q * c.head_dim)
             + rb(2 * c.intermediate, c.hidden) + rb(c.hidden, c.intermediate))
    kv = 2 * ctx * c.n_kv * c.head_dim * 2
    norms = (2 * c.hidden + 2 * c.head_dim) * 2
    return c.n_layers * (layer + kv + norms) + rb(c.vocab, c.hidden) + c.hidden * 2 * 2


def cpu_baseline(model, ctx: int, max_steps: int, budget_s: float):
    """The reference's CPU path on this host: bf16 weights (RNE(d*q), the
    bytes the reference deploys) + F.linear, timed per decode step."""
    import torch
    from oracle.cpu_path import CpuDecoder
    from spark_vllm_ascend_amd.integration.weights import dequantize_bf16
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
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
                     model.cos_sin.cpu(), ctx + max_steps + 1)
    dec.fill_cache(ctx)
    dec.step(1, ctx)  # warm-up (first-touch, thread pool)
    times = []
    t_start = time.perf_counter()
    tok = 1
    for i in range(max_steps):
        t0 = time.perf_counter()
        tok = dec.step(tok, ctx + 1 + i)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    med = statistics.median(times)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "ms_per_token": round(med * 1e3, 2), "cpu": cpu_model,
            "sample": f"{len(times)} decode steps of the 36-layer model at context {ctx + 1}.."
                      f"{ctx + len(times)} (KV cache pre-filled with random bf16), torch "
                      f"{torch.__version__} CPU, bf16 F.linear, {cores} threads, median step"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4095)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--runs", type=int, default=3)
    ap.add_argument("--prompt-len", type=int, default=2048)
    ap.add_argument("--num-splits", type=int, default=0, help="0 = backend default")
    ap.add_argument("--phase", choices=["all", "roofline", "decode", "counters", "batch"],
                    default="all",
                    help="counters: eager launches for a rocprofv3 --pmc run, no timing")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
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
        print(json.dumps(batch_decode(dev)))
        return 0

    if args.phase in ("all", "roofline"):
        log("GEMV roofline (9728x2560, 24 rotating weight sets)")
        result["roofline"] = gemv_roofline(dev, reps=20)
        log(f"  {result['roofline']['us_per_launch']} us/launch, "
            f"{result['roofline']['achieved']} GB/s")
        log("attention roofline (ctx 6144, 12 rotating KV sets)")
        result["attention"] = attention_roofline(dev, reps=20)
        log(f"  best splits {result['attention']['best_splits']}: {result['attention']['us']} us")
        pmc = ROOT / "profiles" / "q4_0_gemv_9728x2560_traffic.json"
        if pmc.exists():
            result["roofline"]["traffic"] = json.loads(pmc.read_text()).get("traffic_bytes")
        torch.cuda.empty_cache()
        if args.phase == "roofline":
            print(json.dumps(result))
            return 0

    max_len = args.prompt_len + args.warmup + args.steps + 1
    log(f"building the 4B model (max_len {max_len})")
    model = build_model(dev, max_len, args.num_splits or None)
    model.capture()
    prompt = torch.randint(0, model.cfg.vocab, (args.prompt_len,),
                           generator=torch.Generator().manual_seed(1234))
    tpots, token_runs = [], []
    for r in range(args.runs):
        tpot, toks = run_decode(model, prompt, args.warmup, args.steps)
        tpots.append(tpot)
        token_runs.append(toks)
        log(f"run {r}: TPOT {tpot * 1e3:.4f} ms ({1 / tpot:.1f} tok/s)")
    tpot = statistics.median(tpots)
    deterministic = all(torch.equal(token_runs[0], t) for t in token_runs[1:])
    gen = token_runs[0][args.prompt_len:]
    valid = bool(((gen >= 0) & (gen < model.cfg.vocab)).all())

    c = model.cfg
    ctx_lo = args.prompt_len + args.warmup + 1
    ctx_hi = args.prompt_len + args.warmup + args.steps
    mean_bytes = statistics.fmean(step_bytes(c, t) for t in (ctx_lo, ctx_hi))
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
        "data": "synthetic (random-init weights, seeded random prompt ids)",
        "config": {"workload": "4B Q4_0 decoder: 36 layers, hidden 2560, 32q/8kv x 128, SwiGLU "
                               "9728, vocab 151936 Q4_0 head, BF16 paged KV block 128; prompt "
                               f"{args.prompt_len}, greedy decode, TPOT over {args.steps} tokens "
                               f"after {args.warmup} warmup, median of {args.runs} runs",
                   "global_batch": 1, "seq_len": ctx_hi, "parallelism": "single GPU",
                   "num_splits": model.num_splits},
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
    if args.phase == "all":
        log("batched decode (8 ragged sequences)")
        out["batch_decode"] = batch_decode(dev)
        log(f"  {out['batch_decode']['tok_s']} tok/s aggregate")
    if not args.skip_cpu:
        log("CPU baseline")
        out["cpu_baseline"] = cpu_baseline(model, ctx=args.prompt_len, max_steps=16,
                                           budget_s=args.cpu_budget)
        log(f"  {out['cpu_baseline']['ms_per_token']} ms/token on "
            f"{out['cpu_baseline']['cores']} cores")
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
