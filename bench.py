#!/usr/bin/env python3
"""Benchmark of the paged f16 decode-attention + append hot path on one MI355X.

Default workload: BASELINE.json config 3, the one the target is quoted on --
a continuous-batching trace with 64 sequence slots, Poisson arrivals (seeded,
1 request per step so the slots stay full), prompts U[32,512], outputs
U[16,256], GPT-2 attention shape (12 layers x 12 heads x 64), f16 KV in
16-token pages from a 3080-page pool (the reference's default pool for 64
full slots), pages freed on completion and reused.  One step = one
ni_kv_step over every layer: append every row of the iteration (decode rows
and budgeted prefill chunks) and run decode attention for every running
sequence (the last prompt row of a finished prefill included).  The first
W steps (the ramp-up) are warmup; K steps are timed.

Prints ONE JSON line.  ``value`` is algorithmic HBM bytes per second over the
timed steps (bytes formula in nanoinfer_amd/workloads.py, each KV byte once
per step); ``roofline`` prices the attention kernel alone, timed by HIP
events the library records around each of its launches on the caller's
stream; ``cpu_baseline`` times the oracle's restatement of the reference's
CPU path (threaded, paged) on a bounded sample of the same trace.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "paged decode-attn+append HBM GB/s (% of peak) and seq-tokens/sec, 1 MI355X"
PEAK_GBS = 8000.0  # MI355X HBM3E, AMD's published figure


def log(*a):
    print(*a, file=sys.stderr, flush=True)


PROFILE_SUMMARY = os.path.join(ROOT, "profiles", "attn_split_fused_config3.md")


def measured_traffic():
    """HBM bytes per launch of the attention kernel from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (scaled by the copy calibration
    it records), with the algorithmic bytes of the same profiled steps."""
    vals = {}
    try:
        for line in open(PROFILE_SUMMARY):
            if "=" in line and line.split("=")[0].strip() in ("traffic_bytes_per_launch",
                                                              "algorithmic_bytes_per_launch_same_steps"):
                k, v = line.split("=")
                vals[k.strip()] = int(float(v))
    except OSError:
        return None
    if len(vals) != 2:
        return None
    return vals


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--workload", default="config3", choices=["config3", "config2", "config4", "config5"])
    ap.add_argument("--split", type=int, default=0, help="split_tokens (0 = automatic)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline sample budget (0 = skip)")
    ap.add_argument("--threads", type=int, default=0, help="CPU baseline threads (0 = min(cpus, 16))")
    ap.add_argument("--no-profile", action="store_true", help="time without the per-launch HIP events")
    ap.add_argument("--seed", type=int, default=7)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only plain 256 MiB device copies (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def calibrate_copy():
    """Ten plain device-to-device copies of 256 MiB: under rocprofv3 --pmc the
    copy kernel's FETCH_SIZE and WRITE_SIZE should each read 262144 KiB; the
    ratio scales the hot kernel's counters to bytes."""
    import torch

    n = 256 * 1024 * 1024 // 4
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(10):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read_per_launch": n * 4, "bytes_written_per_launch": n * 4,
                      "launches": 10}), flush=True)


# ------------------------------------------------------------------ config 3

SPEC_WINDOW = 64  # config 5: rows a sequence may grow past its drawn context before it restarts
CFG3 = dict(max_batch=64, prompt=(32, 512), out=(16, 256), rate=1.0, budget=256, max_rows=512, n_ctx=1024)


def cfg3_pages():
    from nanoinfer_amd.workloads import pages

    # metal_serve.rs:485: max_batch * pages(prompt_max + out_max) + 8
    return CFG3["max_batch"] * pages(CFG3["prompt"][1] + CFG3["out"][1]) + 8


def cfg3_opts(host_only=False):
    import nanoinfer_amd as na
    from nanoinfer_amd import workloads

    return na.BatchOpts(**workloads.GPT2, kv_blocks=cfg3_pages(), max_seqs=CFG3["max_batch"], n_ctx=CFG3["n_ctx"],
                        max_rows=CFG3["max_rows"], host_only=host_only)


def cfg3_trace(n_steps, seed):
    """Plan the whole trace on a host-only handle (the same C++ allocator
    makes the same decisions on the device handle)."""
    import nanoinfer_amd as na
    from nanoinfer_amd import workloads

    host = na.PagedKv(cfg3_opts(host_only=True))
    tr = workloads.ContinuousBatching(host, seed=seed, max_batch=CFG3["max_batch"], prompt=CFG3["prompt"],
                                      out=CFG3["out"], rate=CFG3["rate"], budget=CFG3["budget"],
                                      max_rows=CFG3["max_rows"])
    steps = []
    for _ in range(n_steps):
        st = tr.plan()
        # commit what the device handle's ni_kv_step will commit
        for seq, n_new, _ in st.work:
            host.reserve(int(seq), host.seq_len(int(seq)) + int(n_new))
            host.commit(int(seq), int(n_new))
        tr.commit()
        steps.append(st)
    return steps


def replay_gpu(kv, steps, bufs, split, profile):
    """Run steps on the device handle; returns (seconds, attention ms, attention launches)."""
    import torch

    q, k, v, out = bufs
    if profile:
        kv.profile([1])  # the attention launch only: events around every launch cost time
        for kid in range(3):
            kv.profile_read(kid)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    in_step = 0.0
    for st in steps:
        for s in st.retire:
            kv.free_seq(s)
        for s in st.admit:
            got = kv.add_seq()
            assert got == s, (got, s)
        t1 = time.perf_counter()
        kv.step(st.work, q, k, v, out=out, split_tokens=split)
        in_step += time.perf_counter() - t1
    t_loop = time.perf_counter() - t0
    torch.cuda.synchronize()
    t = time.perf_counter() - t0
    log(f"bench: host loop {t_loop / len(steps) * 1e6:.1f} us/step (inside ni_kv_step {in_step / len(steps) * 1e6:.1f}), "
        f"wall {t / len(steps) * 1e6:.1f} us/step")
    prof = None
    if profile:
        prof = {name: kv.profile_read(i) for i, name in enumerate(["append", "attention", "merge"])}
        kv.profile([])
    return t, prof


def cpu_baseline_cfg3(steps, warmup, seconds, threads):
    """The oracle's restatement of the reference CPU path on the same trace:
    warmup steps append only (untimed), then whole steps until `seconds`."""
    import oracle
    from nanoinfer_amd import workloads

    opts = cfg3_opts(host_only=True)
    alloc = oracle.Alloc(opts.kv_blocks, opts.max_seqs, opts.n_ctx)
    c = opts.n_head * opts.head_dim
    pools = oracle.PagedPools(opts.n_layer, opts.kv_blocks, c)
    runner = oracle.CpuStep(threads)
    rng = np.random.default_rng(1)
    big = CFG3["max_rows"]
    q = rng.standard_normal((opts.n_layer, big, c), dtype=np.float32)
    k = rng.standard_normal((opts.n_layer, big, c), dtype=np.float32)
    v = rng.standard_normal((opts.n_layer, big, c), dtype=np.float32)
    out = np.zeros_like(q)
    done_bytes = 0
    done_tokens = 0
    t_cpu = 0.0
    n_timed = 0
    for i, st in enumerate(steps):
        for s in st.retire:
            alloc.free_seq(s)
        for s in st.admit:
            assert alloc.add_seq() == s
        rows_s, rows_p, qrows = [], [], []
        for seq, n_new, n_q in st.work:
            seq, n_new, n_q = int(seq), int(n_new), int(n_q)
            L = alloc.seq_len(seq)
            assert alloc.ensure(seq, L + n_new) == 0
            for j in range(n_new):
                if j >= n_new - n_q:
                    qrows.append(len(rows_s))
                rows_s.append(seq)
                rows_p.append(L + j)
        n = len(rows_s)
        rs = np.asarray(rows_s, np.uint32)
        rp = np.asarray(rows_p, np.uint32)
        timed = i >= warmup
        qr = np.asarray(qrows if timed else [], np.uint32)
        t0 = time.perf_counter()
        runner.run(pools, alloc.table(), alloc.max_blocks, rs, rp, qr, q, k, v, out, opts.n_head, opts.head_dim)
        dt = time.perf_counter() - t0
        for seq, n_new, _ in st.work:
            alloc.commit(int(seq), int(n_new))
        if timed:
            b = workloads.step_bytes(st.work, st.ctx_after, opts.n_layer, c)
            done_bytes += b["total"]
            done_tokens += b["seq_tokens"]
            t_cpu += dt
            n_timed += 1
            if t_cpu >= seconds:
                break
    return {"seconds": t_cpu, "bytes": done_bytes, "tokens": done_tokens, "steps": n_timed, "threads": runner.threads}


def run_config3(args):
    import torch

    import nanoinfer_amd as na
    from nanoinfer_amd import workloads

    n_total = args.warmup + args.steps
    log(f"bench: planning {n_total} steps of the config-3 trace")
    steps = cfg3_trace(n_total, args.seed)
    opts = cfg3_opts()
    kv = na.PagedKv(opts)
    c = opts.n_head * opts.head_dim
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    shape = (opts.n_layer, CFG3["max_rows"], c)
    q = torch.randn(shape, device="cuda", generator=g)
    k = torch.randn(shape, device="cuda", generator=g)
    v = torch.randn(shape, device="cuda", generator=g)
    out = torch.zeros(shape, device="cuda")
    bufs = (q, k, v, out)
    log(f"bench: warmup {args.warmup} steps")
    replay_gpu(kv, steps[: args.warmup], bufs, args.split, profile=False)
    log(f"bench: timing {args.steps} steps")
    t, prof = replay_gpu(kv, steps[args.warmup:], bufs, args.split, profile=not args.no_profile)
    timed = steps[args.warmup:]
    tot = {"append": 0, "attention": 0, "total": 0, "seq_tokens": 0}
    ctx_sum = 0
    live_sum = 0
    for st in timed:
        b = workloads.step_bytes(st.work, st.ctx_after, opts.n_layer, c)
        for key in tot:
            tot[key] += b[key]
        q_mask = st.work[:, 2] > 0
        ctx_sum += int(st.ctx_after[q_mask].sum())
        live_sum += int(q_mask.sum())
    gbs = tot["total"] / t / 1e9
    res = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "kv_dtype": "f16",
        "data": "synthetic (seeded N(0,1) q/k/v, seeded Poisson trace)",
        "config": {
            "workload": "config3: continuous batching, 64 slots, Poisson arrivals 1/step, prompt U[32,512], "
                        "output U[16,256], GPT-2 12x12x64, 16-token pages, 3080-page pool",
            "n_layer": opts.n_layer, "n_head": opts.n_head, "head_dim": opts.head_dim,
            "kv_pages": opts.kv_blocks, "max_batch": CFG3["max_batch"], "prefill_budget": CFG3["budget"],
            "prefill_attention": "last prompt row only",
            "split_tokens": args.split, "launches_per_step": "append + attention (+ merge when split), all layers",
            "mean_live_seqs": round(live_sum / len(timed), 2),
            "mean_context": round(ctx_sum / max(live_sum, 1), 1),
            "algorithmic_bytes_per_step": int(tot["total"] / len(timed)),
        },
        "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
        "seq_tokens_per_s": round(tot["seq_tokens"] / t, 1),
    }
    if prof:
        ms, n = prof["attention"]
        # ni_kv_step fuses the append into the attention launch whenever every
        # sequence has one query group (always here): its bytes are then the
        # step's append bytes too.
        kbytes = tot["total"]
        ach = kbytes / (ms / 1e3) / 1e9
        res["roofline"] = {
            "bound": "hbm", "achieved": round(ach, 2), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / PEAK_GBS, 4), "traffic": None,
            "kernel": "attn_split_kernel<64,1,4,2,fused>", "avg_launch_us": round(ms / n * 1e3, 3), "launches": n,
            "algorithmic_bytes_per_launch": int(kbytes / n),
        }
        tr = measured_traffic()
        if tr:
            res["roofline"]["traffic"] = tr["traffic_bytes_per_launch"]
            res["roofline"]["traffic_vs_algorithmic"] = round(
                tr["traffic_bytes_per_launch"] / tr["algorithmic_bytes_per_launch_same_steps"], 3)
            res["roofline"]["traffic_source"] = "profiles/attn_split_fused_config3.md (rocprofv3 --pmc, scaled)"
    if args.cpu_seconds > 0:
        threads = args.threads or min(os.cpu_count() or 1, 16)
        log(f"bench: CPU baseline ({threads} threads, ~{args.cpu_seconds:.0f} s)")
        cb = cpu_baseline_cfg3(steps, args.warmup, args.cpu_seconds, threads)
        res["cpu_baseline"] = {
            "value": round(cb["bytes"] / cb["seconds"] / 1e9, 3), "unit": "GB/s",
            "seq_tokens_per_s": round(cb["tokens"] / cb["seconds"], 1), "cores": cb["threads"], "kind": "port",
            "sample": f"steps {args.warmup}..{args.warmup + cb['steps'] - 1} of the same trace "
                      f"({cb['seconds']:.1f} s; the oracle's C restatement of the reference x86 CPU path: "
                      f"narrow + attend_f16_portable + fastops::exp over kv_slot, units on a thread pool)",
        }
    return res


# ------------------------------------------------- secondary configurations

def _fill(kv, seq, length, c, n_layer, std, chunk, gen):
    """Reserve and append positions 0..length-1 of `seq` with random K/V
    (untimed set-up)."""
    import torch

    kv.reserve(seq, length)
    for p0 in range(0, length, chunk):
        n = min(chunk, length - p0)
        kk = torch.randn((n_layer, n, c), device="cuda", generator=gen) * std
        vv = torch.randn((n_layer, n, c), device="cuda", generator=gen) * std
        kv.append([(seq, p) for p in range(p0, p0 + n)], kk, vv)
    kv.commit(seq, length)


def _timed_steps(kv, args, one_step):
    """Warm up, then time args.steps calls of one_step() with the attention
    launch bracketed by the library's events."""
    import torch

    for _ in range(args.warmup):
        one_step()
    kv.profile([1])
    for kid in range(3):
        kv.profile_read(kid)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    torch.cuda.synchronize()
    t = time.perf_counter() - t0
    prof = {name: kv.profile_read(i) for i, name in enumerate(["append", "attention", "merge"])}
    kv.profile([])
    return t, prof


def _result(args, workload, cfg, t, prof, step_bytes, seq_tokens, n_layer):
    gbs = step_bytes * args.steps / t / 1e9
    ms, n = prof["attention"]
    mm, mn = prof["merge"]
    res = {"metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(t / args.steps * 1e3, 5), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "kv_dtype": "f16",
           "data": "synthetic (seeded normal q/k/v)", "config": dict(workload=workload, **cfg),
           "pct_of_peak": round(100 * gbs / PEAK_GBS, 2), "seq_tokens_per_s": round(seq_tokens * args.steps / t, 1)}
    if n:
        kernel_s = (ms + mm) / 1e3
        ach = step_bytes * args.steps / kernel_s / 1e9
        res["roofline"] = {"bound": "hbm", "achieved": round(ach, 2), "peak": PEAK_GBS, "unit": "GB/s",
                           "frac": round(ach / PEAK_GBS, 4), "traffic": None,
                           "kernel": "attn_split_kernel (+ attn_merge_kernel when split)",
                           "avg_launch_us": round(ms / n * 1e3, 3),
                           "avg_merge_us": round(mm / mn * 1e3, 3) if mn else 0.0,
                           "algorithmic_bytes_per_launch": int(step_bytes)}
    return res


def run_config2(args):
    """Config 2: 16 sequences, contexts U[64,1024] (after the append), pages
    from a seeded permutation of a 1024-page pool; one step appends a token
    per sequence and runs attention.  Each timed step is rolled back
    (truncate) so every step sees the same state."""
    import torch

    import nanoinfer_amd as na
    from nanoinfer_amd import workloads

    ctx, order = workloads.config2_contexts()
    kv = na.PagedKv(na.BatchOpts(**workloads.GPT2, kv_blocks=1024, max_seqs=16, n_ctx=1024, page_order=order))
    c = 768
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    seqs = [kv.add_seq() for _ in ctx]
    for s, L in zip(seqs, ctx):
        _fill(kv, s, L - 1, c, 12, 1.0, 512, g)
    n = len(seqs)
    q, k, v = (torch.randn((12, n, c), device="cuda", generator=g) for _ in range(3))
    out = torch.zeros_like(q)
    work = [(s, 1, 1) for s in seqs]

    def one_step():
        kv.step(work, q, k, v, out=out, split_tokens=args.split)
        for s, L in zip(seqs, ctx):
            kv.truncate(s, L - 1)

    t, prof = _timed_steps(kv, args, one_step)
    b = workloads.step_bytes(np.asarray(work), np.asarray(ctx), 12, c)
    return _result(args, "config2: 16 seqs, ctx U[64,1024], 1024-page pool, seeded page permutation, "
                         "append 1 + attention, GPT-2 12x12x64", {"mean_context": float(np.mean(ctx))},
                   t, prof, b["total"], b["seq_tokens"], 12)


def run_config4(args):
    """Config 4: batch 4, 32 heads x 128, context 32768, random page tables,
    512-token partitions + LSE merge; q ~ N(0,1), k/v ~ N(0,0.5).  One step
    appends a token per sequence (rolled back after each step)."""
    import torch

    import nanoinfer_amd as na
    from nanoinfer_amd import workloads

    B, L = 4, 32768
    order = workloads.XorShift.seeded(4).permutation(B * L // 16)
    kv = na.PagedKv(na.BatchOpts(**workloads.LONG, kv_blocks=B * L // 16, max_seqs=B, n_ctx=L, max_rows=4096,
                                 page_order=order))
    c = 4096
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    seqs = [kv.add_seq() for _ in range(B)]
    for s in seqs:
        _fill(kv, s, L - 1, c, 1, 0.5, 4096, g)
    q = torch.randn((1, B, c), device="cuda", generator=g)
    k, v = (torch.randn((1, B, c), device="cuda", generator=g) * 0.5 for _ in range(2))
    out = torch.zeros_like(q)
    work = [(s, 1, 1) for s in seqs]
    split = args.split or 512

    def one_step():
        kv.step(work, q, k, v, out=out, split_tokens=split)
        for s in seqs:
            kv.truncate(s, L - 1)

    t, prof = _timed_steps(kv, args, one_step)
    b = workloads.step_bytes(np.asarray(work), np.full(B, L), 1, c)
    return _result(args, "config4: batch 4, 32 heads x 128, context 32768, random page tables, "
                         "512-token partitions + LSE merge", {"split_tokens": split}, t, prof, b["total"],
                   b["seq_tokens"], 1)


def run_config5(args):
    """Config 5: speculative verify, 32 sequences with contexts U[128,1024];
    each step appends g + 4 drafts (5 rows, 5 causal queries per sequence),
    accepts U[0,4] and truncates to tlen + 1 + accepted.  A sequence that
    has grown SPEC_WINDOW rows past its drawn context goes back to it, so
    any number of steps stays at the drawn contexts."""
    import torch

    import nanoinfer_amd as na
    from nanoinfer_amd import workloads

    ctx, _ = workloads.config5_contexts()
    n_ctx = 2048
    kv = na.PagedKv(na.BatchOpts(**workloads.GPT2, kv_blocks=32 * n_ctx // 16, max_seqs=32, n_ctx=n_ctx))
    c = 768
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    seqs = [kv.add_seq() for _ in ctx]
    for s, L in zip(seqs, ctx):
        _fill(kv, s, L, c, 12, 1.0, 512, g)
    spec = workloads.SpecVerify(kv, seqs, k=4, seed=args.seed, window=SPEC_WINDOW)
    n = 5 * len(seqs)
    q, k, v = (torch.randn((12, n, c), device="cuda", generator=g) for _ in range(3))
    out = torch.zeros_like(q)
    acc_bytes = [0, 0]

    def one_step():
        st = spec.plan()
        kv.step(st.work, q, k, v, out=out, split_tokens=args.split)
        accs = spec.commit()
        b = workloads.step_bytes(st.work, st.ctx_after, 12, c)
        acc_bytes[0] += b["total"]
        acc_bytes[1] += sum(a + 1 for a in accs)

    for _ in range(args.warmup):
        one_step()
    acc_bytes[:] = [0, 0]
    args_w = argparse.Namespace(**vars(args))
    args_w.warmup = 0
    t, prof = _timed_steps(kv, args_w, one_step)
    return _result(args, "config5: spec verify, 32 seqs, ctx U[128,1024], append g + 4 drafts, 5 causal queries, "
                         "accept U[0,4], truncate", {"draft_k": 4, "reset_window": SPEC_WINDOW}, t, prof, acc_bytes[0] / args.steps,
                   acc_bytes[1] / args.steps, 12)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (see DESIGN.md for how the "
                                   "path would shard)"}))
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        log("bench: no GPU visible")
        sys.exit(1)
    if args.calibrate_copy:
        calibrate_copy()
        return
    # The headline line is config 3; the others are secondary measurements.
    res = {"config3": run_config3, "config2": run_config2, "config4": run_config4,
           "config5": run_config5}[args.workload](args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
