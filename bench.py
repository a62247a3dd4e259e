#!/usr/bin/env python3
"""Benchmark of the paged f16 decode-attention + append hot path on one MI355X.

Default workload: benchmark configuration 3, the one the target is quoted on --
a continuous-batching trace with 64 sequence slots, Poisson arrivals (seeded,
1 request per step so the slots stay full), prompts U[32,512], outputs
U[16,256], GPT-2 attention shape (12 layers x 12 heads x 64), f16 KV in
16-token pages from a 3080-page pool (the reference's default pool for 64
full slots), pages freed on completion and reused.  One step = one
ni_kv_step over every layer: append every row of the iteration (decode rows
and budgeted prefill chunks) and run decode attention for every running
sequence (the last prompt row of a finished prefill included).

Whatever --steps/--warmup say, the timed window sits in the trace's steady
state: a fixed untimed ramp of RAMP_STEPS append-only steps (rows reserved,
appended and committed, no attention) comes first, then W warmup steps, then
the K timed steps (trace steps RAMP_STEPS+W .. RAMP_STEPS+W+K-1).

The host loop is the C++ serving driver (ni_drive_run: the scheduler of
metal_serve.rs restated in C++, calling the C ABI), as a compiled caller of
the library runs it.  Prints ONE JSON line.  ``value`` is algorithmic HBM
bytes per second over the timed steps (bytes formula in
nanoinfer_amd/workloads.py, each KV byte once per step), the median of REPS
identical runs without per-launch events (``repetitions`` lists them);
``copy_ceiling`` is a plain device copy timed in the same process;
``roofline`` prices the attention launch alone, timed by HIP events the
library records around each of its launches on the caller's stream in one
more run of the same window, with ``traffic`` from the committed rocprofv3
counter summary only when that summary covers the same window;
``per_layer_launches`` runs the window one layer per launch, as a model's
forward must (the step planned once, ni_kv_step_layer per layer), and
``per_layer_append_attention`` through separate per-layer append and
attention calls; ``cpu_baseline`` times the oracle's restatement of the
reference's CPU path (threaded, paged) on the first steps of the same window.
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
# Workloads whose committed profile holds a PMC traffic section.
TRAFFIC_PROFILES = {
    "config3": PROFILE_SUMMARY,
    "config2": os.path.join(ROOT, "profiles", "attn_split_config2.md"),
    "config4": os.path.join(ROOT, "profiles", "attn_split_merge_config4.md"),
    "config5": os.path.join(ROOT, "profiles", "attn_mfma_config5.md"),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--workload", default="config3",
                    help="config3 (default), config1 (one sequence, prefill 64 + 64 decode steps, with the CPU "
                         "path beside it), config2, config4, config5, configNq8 (the same on the Q8 cache), "
                         "prefill (16 x 512-row prompts, every row queried), prefillq8 (the same on the Q8 cache), or qkv[ROWS][f16|q8|q4] (the QKV "
                         "projection with the append in its epilogue, ROWS rows per layer, default 64, f32 weights or the reference's "
                         "f16 / q8_0 / q4_0 formats)")
    ap.add_argument("--split", type=int, default=0, help="split_tokens (0 = automatic)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline sample budget (0 = skip)")
    ap.add_argument("--threads", type=int, default=0,
                    help="CPU baseline threads (0 = available parallelism, as the reference's thread pools)")
    ap.add_argument("--no-profile", action="store_true", help="skip the run timed by per-launch HIP events")
    ap.add_argument("--skip-per-layer", action="store_true", help="config 3: skip the per-layer launch run")
    ap.add_argument("--skip-secondary", action="store_true",
                    help="config 3: skip the secondary workloads measured beside the headline")
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


def available_parallelism() -> int:
    """std::thread::available_parallelism() on Linux, by which the
    reference's thread pools size themselves when asked for 0 threads
    (crates/core/src/fastpool.rs:148, pool.rs:163): the CPUs of this
    process's affinity mask, capped by a cgroup CPU quota (quota / period,
    at least 1) where one is set."""
    n = len(os.sched_getaffinity(0))
    quotas = []
    try:
        rel = ""
        for line in open("/proc/self/cgroup"):
            if line.startswith("0::"):
                rel = line.strip()[3:]
        # cgroup v2: every level from the process's group up to the root
        path = "/sys/fs/cgroup" + rel
        while True:
            try:
                q, per = open(os.path.join(path, "cpu.max")).read().split()[:2]
                if q != "max":
                    quotas.append(max(1, int(q) // int(per)))
            except (OSError, ValueError):
                pass
            if os.path.normpath(path) == "/sys/fs/cgroup":
                break
            path = os.path.dirname(path)
    except OSError:
        pass
    try:  # cgroup v1
        q = int(open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read())
        per = int(open("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read())
        if q > 0 and per > 0:
            quotas.append(max(1, q // per))
    except (OSError, ValueError):
        pass
    return min([n] + quotas)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_cfg3(args, ramp, threads, reps=5):
    """The oracle's restatement of the reference's x86 CPU path on the bench's
    own window of the config-3 trace.

    The trace comes from the same C++ scheduler the device run uses (ni_serve
    on a host-only handle, so the same admissions, retirements and rows), its
    tables from the oracle's allocator.  The ramp and warmup steps append only
    (untimed; numpy's float16 conversion, bit-identical to the reference's
    f32_to_f16 on these finite inputs, checked below).  Then each step of the
    window runs the CPU step (narrow + attend_f16_portable with fastops::exp
    over kv_slot, (query, head) units on `threads` threads): the first
    repetition records each step's table and rows until it has spent
    seconds / reps (at most the window's `steps` steps), and the other
    repetitions replay the same steps.  Returns the median repetition."""
    import oracle
    import nanoinfer_amd as na
    from nanoinfer_amd import drivers, workloads

    opts = cfg3_opts(host_only=True)
    host = na.PagedKv(opts)
    sv = drivers.Serve(host, seed=args.seed, rate=CFG3["rate"], max_batch=CFG3["max_batch"], prompt=CFG3["prompt"],
                       out=CFG3["out"], budget=CFG3["budget"], max_rows=CFG3["max_rows"])
    alloc = oracle.Alloc(opts.kv_blocks, opts.max_seqs, opts.n_ctx)
    c, L, mb = opts.n_head * opts.head_dim, opts.n_layer, opts.max_rows
    pools = oracle.PagedPools(L, opts.kv_blocks, c)
    kpool = pools.k.reshape(L, -1, c)
    vpool = pools.v.reshape(L, -1, c)
    rng = np.random.default_rng(args.seed)
    q, k, v = (rng.standard_normal((L, mb, c), dtype=np.float32) for _ in range(3))
    out = np.zeros_like(q)
    k16, v16 = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    assert np.array_equal(k16.reshape(-1), oracle.f32_to_f16(k.reshape(-1)))
    assert np.array_equal(v16.reshape(-1), oracle.f32_to_f16(v.reshape(-1)))
    runner = oracle.CpuStep(threads)
    budget = args.cpu_seconds / reps
    recorded, t_first = [], 0.0
    for i in range(ramp + args.warmup + args.steps):
        work, ctx, adm, ret = sv.plan()
        for s in ret:
            alloc.free_seq(s)
        for s in adm:
            assert alloc.add_seq() == s
        rs, rp, qr = [], [], []
        for seq, n_new, n_q in work:
            seq, n_new, n_q = int(seq), int(n_new), int(n_q)
            ln = alloc.seq_len(seq)
            assert alloc.ensure(seq, ln + n_new) == 0
            host.reserve(seq, ln + n_new)
            for j in range(n_new):
                if j >= n_new - n_q:
                    qr.append(len(rs))
                rs.append(seq)
                rp.append(ln + j)
        rs, rp = np.asarray(rs, np.uint32), np.asarray(rp, np.uint32)
        tab = alloc.table()
        if i < ramp + args.warmup:
            slots = tab[rs, rp // 16].astype(np.int64) * 16 + rp % 16
            kpool[:, slots, :] = k16[:, : len(rs), :]
            vpool[:, slots, :] = v16[:, : len(rs), :]
        else:
            qr = np.asarray(qr, np.uint32)
            t0 = time.perf_counter()
            runner.run(pools, tab, alloc.max_blocks, rs, rp, qr, q, k, v, out, opts.n_head, opts.head_dim)
            t_first += time.perf_counter() - t0
            b = workloads.step_bytes(work, ctx, L, c)
            recorded.append((tab, rs, rp, qr, b["total"], b["seq_tokens"]))
        for seq, n_new, _ in work:
            alloc.commit(int(seq), int(n_new))
            host.commit(int(seq), int(n_new))
        sv.commit()
        if recorded and t_first >= budget:
            break
    times = [t_first]
    for _ in range(reps - 1):
        t = 0.0
        for tab, rs, rp, qr, _, _ in recorded:
            t0 = time.perf_counter()
            runner.run(pools, tab, alloc.max_blocks, rs, rp, qr, q, k, v, out, opts.n_head, opts.head_dim)
            t += time.perf_counter() - t0
        times.append(t)
    return {"seconds": float(np.median(times)), "rep_seconds": times, "bytes": sum(r[4] for r in recorded),
            "tokens": sum(r[5] for r in recorded), "steps": len(recorded), "threads": runner.threads}


def _drive(name, args, launch=None, profile_mask=0, ramp=0, all_prompt_rows=False):
    """One ni_drive_run of a preset: the C++ driver's host loop (the
    scheduler, ni_kv_step and its bookkeeping) with inputs resident in HBM."""
    from nanoinfer_amd import drivers

    launch = drivers.NI_DRIVE_STEP if launch is None else launch
    o = drivers.preset(name, args.steps, args.warmup, launch=launch, split=args.split, seed=args.seed,
                       profile_mask=profile_mask, ramp=ramp, query_all_prompt_rows=all_prompt_rows)
    r = drivers.drive(o)
    gbs = r["bytes"] / r["seconds"] / 1e9
    log(f"bench: {name} launch {launch}{' (profiled)' if profile_mask else ''}: {gbs:.1f} GB/s, "
        f"{r['seconds'] / r['steps'] * 1e6:.1f} us/step, host {r['host_us_per_step']:.1f} us/step, "
        f"{r['mean_live']:.2f} live, mean context {r['mean_context']:.1f}")
    return r


def _median_run(name, args, reps, launch=None, ramp=0):
    """`reps` identical runs; the run of median throughput and the spread."""
    runs = [_drive(name, args, launch=launch, ramp=ramp) for _ in range(reps)]
    gbs = [r["bytes"] / r["seconds"] / 1e9 for r in runs]
    order = np.argsort(gbs)
    med = runs[int(order[len(runs) // 2])]
    spread = {"reps": reps, "gbs": [round(g, 2) for g in gbs], "median_gbs": round(float(np.median(gbs)), 2),
              "stdev_gbs": round(float(np.std(gbs, ddof=1)) if reps > 1 else 0.0, 2)}
    return med, spread


def _line(args, r, workload, cfg, data):
    """The JSON fields every workload shares, from an unprofiled run."""
    gbs = r["bytes"] / r["seconds"] / 1e9
    return {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["seconds"] / r["steps"] * 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "kv_dtype": "f16", "data": data,
        "config": dict(workload=workload, **cfg), "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
        "seq_tokens_per_s": round(r["seq_tokens"] / r["seconds"], 1),
    }


def _roofline(rp, kernel, with_merge, with_append=False):
    """Algorithmic bytes of the profiled run / the attention (+ merge, + an
    append launch before it when the step has one) launches' event time."""
    ms, n = rp["kernel_ms"][1], rp["kernel_launches"][1]
    mm, mn = rp["kernel_ms"][2], rp["kernel_launches"][2]
    am, an = rp["kernel_ms"][0], rp["kernel_launches"][0]
    kernel_ms = ms + (mm if with_merge else 0.0) + (am if with_append else 0.0)
    ach = rp["bytes"] / (kernel_ms / 1e3) / 1e9
    out = {"bound": "hbm", "achieved": round(ach, 2), "peak": PEAK_GBS, "unit": "GB/s", "frac": round(ach / PEAK_GBS, 4),
           "traffic": None, "kernel": kernel, "avg_launch_us": round(ms / n * 1e3, 3), "launches": n,
           "algorithmic_bytes_per_launch": int(rp["bytes"] / n)}
    if with_merge:
        out["avg_merge_us"] = round(mm / mn * 1e3, 3) if mn else 0.0
    if with_append and an:
        out["avg_append_us"] = round(am / an * 1e3, 3)
        out["append_launches"] = an
    return out


def copy_ceiling(nbytes=2 << 30, reps=5):
    """A plain device-to-device copy of `nbytes` (torch's copy_, the runtime's
    copy kernel) timed with events on torch's stream: read + write bytes per
    second, median of `reps` copies after one untimed copy."""
    import torch

    x = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    y = torch.empty_like(x)
    y.copy_(x)
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        y.copy_(x)
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / 1e3)
    del x, y
    torch.cuda.empty_cache()
    t = float(np.median(ts))
    return {"value": round(2 * nbytes / t / 1e9, 1), "unit": "GB/s", "bytes_read": nbytes, "bytes_written": nbytes,
            "method": f"torch copy_ of {nbytes >> 20} MiB device to device, HIP events, median of {reps}"}


def hbm_peak_reported():
    """What the device reports of its memory interface (hipDeviceGetAttribute).
    HIP gives the bus width and a memory clock but not the per-pin data rate,
    so the peak is AMD's published figure; the bus width is the check."""
    from nanoinfer_amd import drivers

    clk, bits = drivers.device_memory(0)
    return {"mem_clock_khz": clk, "bus_width_bits": bits,
            "note": f"{bits}-bit bus x 8.0 Gb/s per pin (HBM3E) = {bits * 8 / 8:.0f} GB/s; AMD publishes 8.0 TB/s, "
                    f"the peak used"}


def stream_ceiling(nbytes=2 << 30, reps=5, blocks=(1024, 2048, 4096, 8192)):
    """The library's streaming probe (ni_stream_probe: 16-byte non-temporal
    loads, 4 in flight per thread) over `nbytes`, read and copy, each in a
    grid stride and in one contiguous span per workgroup, for each launch
    size; timed with events on torch's stream, median of `reps` after one
    untimed pass.  The best pattern and size per kind is the ceiling."""
    import torch

    from nanoinfer_amd import _abi

    L = _abi.lib()
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    st = torch.cuda.current_stream().cuda_stream
    out, all_runs = {}, {}
    for copy in (0, 1):
        best = None
        for span in (0, 2):
            for b in blocks:
                ts = []
                for r in range(reps + 1):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    rc = L.ni_stream_probe(copy | span, src.data_ptr(), dst.data_ptr(), nbytes, b, st)
                    e1.record()
                    if rc != 0:
                        raise RuntimeError(f"ni_stream_probe: status {rc}")
                    e1.synchronize()
                    if r:
                        ts.append(e0.elapsed_time(e1) / 1e3)
                gbs = (2 if copy else 1) * nbytes / float(np.median(ts)) / 1e9
                all_runs[f"{'copy' if copy else 'read'}/{'span' if span else 'stride'}/{b}"] = round(gbs, 1)
                if best is None or gbs > best[0]:
                    best = (gbs, b, "span" if span else "stride")
        out["copy" if copy else "read"] = {"value": round(best[0], 1), "unit": "GB/s", "blocks": best[1],
                                           "pattern": best[2]}
    del src, dst
    torch.cuda.empty_cache()
    out["all"] = all_runs
    out["method"] = (f"ni_stream_probe over {nbytes >> 20} MiB (copy: read + write bytes), grid stride and one span "
                     f"per workgroup, {list(blocks)} workgroups of 256 threads, median of {reps}")
    return out


# Config 3's timed window: an untimed append-only ramp of RAMP_STEPS trace
# steps brings the 64 slots to their steady state (slots full from step ~100,
# contexts stationary from ~300; the trace's initial synchronised admissions
# have mixed by ~1000), then W warmup steps and the K timed steps.
RAMP_STEPS = 1000
REPS = 5


def measured_traffic(workload, args, ramp):
    """HBM bytes per launch of the attention kernel (with its merge, where
    the workload splits) from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (scaled by the copy calibration it records), with the
    algorithmic bytes of the same steps -- only when the summary was taken
    over this run's window (the `window` line matches), else None."""
    vals, window = {}, None
    path = TRAFFIC_PROFILES.get(workload)
    if path is None:
        return None
    want = f"{workload} ramp={ramp} warmup={args.warmup} steps={args.steps} seed={args.seed} split={args.split}"
    try:
        for line in open(path):
            if "=" not in line:
                continue
            key, _, val = line.partition("=")
            key = key.strip()
            if key == "window":
                window = val.strip()
            elif key in ("traffic_bytes_per_launch", "algorithmic_bytes_per_launch_same_steps"):
                vals[key] = int(float(val))
    except OSError:
        return None
    if len(vals) != 2 or window != want:
        return None
    return vals


def kv_serving_summary(r, n_iters):
    """The reference's paged-KV serving figures (metal_serve.rs:320-331,
    361, 440-464) for the config-3 run -- blocks in use after each step (peak
    and mean) and the internal fragmentation of the block-table snapshots
    taken every 10 iterations -- and, beside them, the reference's own
    recorded run with every request at t = 0 (bench/serving.json, rate=0,
    via tests/golden/serving_rate0.json) replayed on ni_serve over a
    host-only handle, which must give the reference's figures exactly."""
    import nanoinfer_amd as na
    from nanoinfer_amd import drivers, workloads

    st = r["serve_stats"]
    out = {"window": f"trace steps 0..{n_iters - 1} (ramp, warmup and timed steps)",
           "kv_pages_peak": st["kv_pages_peak"], "kv_pages_total": cfg3_pages(),
           "kv_pages_avg_used": round(st["kv_pages_avg_used"], 1),
           "kv_pages_avg_weighting": "every iteration the same (step clock; the reference weighs by measured GPU time)",
           "snapshots": st["snapshots"], "avg_live_seqs": round(st["avg_live_seqs"], 2),
           "avg_pages_per_seq": round(st["avg_pages_per_seq"], 2),
           "internal_fragmentation": round(st["internal_fragmentation"], 5)}
    g = json.load(open(os.path.join(ROOT, "tests", "golden", "serving_rate0.json")))
    w = g["workload"]
    kv = na.PagedKv(na.BatchOpts(**workloads.GPT2, kv_blocks=w["kv_pages"], max_seqs=w["max_batch"], n_ctx=1024,
                                 max_rows=w["max_rows"], host_only=True))
    sv = drivers.Serve(kv, seed=w["seed"], rate=w["rate"], n_requests=w["requests"], max_batch=w["max_batch"],
                       prompt=tuple(w["prompt"]), out=tuple(w["output"]), budget=w["prefill_budget"],
                       max_rows=w["max_rows"])
    while sv.done() < w["requests"]:
        work, _, _, _ = sv.plan()
        for s, n_new, _ in work:
            kv.reserve(int(s), kv.seq_len(int(s)) + int(n_new))
            kv.commit(int(s), int(n_new))
        sv.commit()
    rs = sv.stats()
    mine = {"iterations": rs["iterations"], "kv_pages_peak": rs["kv_pages_peak"],
            "internal_fragmentation": round(rs["internal_fragmentation"], 5),
            "avg_pages_per_seq": round(rs["avg_pages_per_seq"], 2)}
    ref = {"iterations": g["continuous"]["iterations"], "kv_pages_peak": g["continuous"]["kv_pages_peak"],
           "internal_fragmentation": g["kv_stats"]["internal_fragmentation"],
           "avg_pages_per_seq": g["kv_stats"]["avg_pages_per_seq"]}
    out["reference_record"] = {"workload": "128 requests at t=0, prompt/output U[16,256], 32 slots, 1032 pages "
                                           "(bench/serving.json rate=0, M4)",
                               "reference": ref, "ni_serve_host_replay": mine, "equal": mine == ref}
    return out


def run_config3(args):
    from nanoinfer_amd import drivers

    ramp = RAMP_STEPS
    r, spread = _median_run("config3", args, REPS, ramp=ramp)
    res = _line(args, r, "config3: continuous batching, 64 slots, Poisson arrivals 1/step, prompt U[32,512], "
                         "output U[16,256], GPT-2 12x12x64, 16-token pages, 3080-page pool",
                dict(n_layer=12, n_head=12, head_dim=64, kv_pages=cfg3_pages(), max_batch=CFG3["max_batch"],
                     prefill_budget=CFG3["budget"], prefill_attention="last prompt row only",
                     split_tokens=args.split, host_loop="C++ driver (ni_drive_run: ni_serve + ni_kv_step)",
                     launches_per_step="one ni_kv_step: append fused into the attention launch, all layers",
                     ramp_steps=ramp, ramp="untimed, append only (the steps' rows reserved, appended and "
                                           "committed, no attention), before the warmup",
                     timed_trace_steps=[ramp + args.warmup, ramp + args.warmup + args.steps - 1],
                     mean_live_seqs=round(r["mean_live"], 2), mean_context=round(r["mean_context"], 1),
                     algorithmic_bytes_per_step=int(r["bytes"] / r["steps"])),
                "synthetic (seeded N(0,1) q/k/v resident in HBM, seeded Poisson request trace; one q/k/v/out "
                "buffer serves every step, so its rows, ~2% of a step's bytes, may stay in the last-level cache "
                "between steps, as a model's freshly projected rows would)")
    res["repetitions"] = spread
    res["host_idle_us"] = {"ni_kv_step": round(r["idle_us_plan_call"], 2)}  # per call, device idle
    res["config"]["kv_serving"] = kv_serving_summary(r, ramp + args.warmup + args.steps)
    res["copy_ceiling"] = copy_ceiling()
    res["stream_ceiling"] = stream_ceiling()
    try:
        res["hbm_peak_reported"] = hbm_peak_reported()
    except RuntimeError as e:
        log(f"bench: {e}")
    if not args.no_profile:
        # ni_kv_step fuses the append into the attention launch whenever every
        # sequence has one query group (always here): the launch's bytes are
        # the whole step's.
        rp = _drive("config3", args, profile_mask=(1 << 1) | (1 << 2), ramp=ramp)
        if rp["kernel_launches"][1] != rp["steps"] or rp["kernel_launches"][2] != 0:
            raise RuntimeError(f"expected one fused launch per step and no merge, got {rp['kernel_launches']}")
        res["roofline"] = _roofline(rp, "attn_split_kernel<64,1,4,2,fused>", with_merge=False)
        tr = measured_traffic("config3", args, ramp)
        if tr:
            res["roofline"]["traffic"] = tr["traffic_bytes_per_launch"]
            res["roofline"]["traffic_vs_algorithmic"] = round(
                tr["traffic_bytes_per_launch"] / tr["algorithmic_bytes_per_launch_same_steps"], 3)
            res["roofline"]["traffic_source"] = ("profiles/attn_split_fused_config3.md (rocprofv3 --pmc over the "
                                                 "same trace steps, scaled by a plain copy's counters)")
    # A model's forward runs a step's layers one at a time (layer l+1's q/k/v
    # come from layer l's output); the reference encodes the step once and
    # dispatches each layer's KV write and attention (batch.rs:280-306,
    # 390-416).  The same window with the step planned once and one fused
    # append + attention launch per layer (ni_kv_step_layer), and through
    # separate ni_kv_append + ni_paged_decode_attention calls per layer.
    if not args.skip_per_layer:
        for key, mode in (("per_layer_launches", drivers.NI_DRIVE_STEP_LAYERS),
                          ("per_layer_append_attention", drivers.NI_DRIVE_PER_LAYER)):
            rl, sp = _median_run("config3", args, 3, launch=mode, ramp=ramp)
            gbs = rl["bytes"] / rl["seconds"] / 1e9
            res[key] = {"value": round(gbs, 2), "unit": "GB/s", "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
                        "ms_per_step": round(rl["seconds"] / rl["steps"] * 1e3, 5),
                        "host_us_per_step": round(rl["host_us_per_step"], 1),
                        "abi_calls_per_step": round(rl["launches"] / rl["steps"], 1), "repetitions": sp}
            if mode == drivers.NI_DRIVE_STEP_LAYERS:
                # host_us_per_step above is paced by the device's queue; the
                # calls' own cost with the device idle:
                res[key]["host_idle_us"] = {"ni_kv_step_begin": round(rl["idle_us_plan_call"], 2),
                                            "ni_kv_step_layer": round(rl["idle_us_layer_call"], 2)}
    if not args.skip_secondary:
        res["secondary"] = secondary_lines(args)
    if args.cpu_seconds > 0:
        threads = args.threads or available_parallelism()
        log(f"bench: CPU baseline ({threads} threads, ~{args.cpu_seconds:.0f} s)")
        cb = cpu_baseline_cfg3(args, ramp, threads)
        w0 = ramp + args.warmup
        res["cpu_baseline"] = {
            "value": round(cb["bytes"] / cb["seconds"] / 1e9, 3), "unit": "GB/s",
            "seq_tokens_per_s": round(cb["tokens"] / cb["seconds"], 1), "cores": cb["threads"], "kind": "port",
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
            "threads_rule": "available_parallelism (affinity mask, cgroup quota), as the reference's pools",
            "repetitions": {"reps": len(cb["rep_seconds"]), "seconds": [round(t, 3) for t in cb["rep_seconds"]]},
            "sample": f"trace steps {w0}..{w0 + cb['steps'] - 1} (the first {cb['steps']} of the GPU's timed steps), "
                      f"median of {len(cb['rep_seconds'])} repetitions ({cb['seconds']:.2f} s each): the oracle's C "
                      f"restatement of the reference x86 CPU path (narrow + attend_f16_portable + fastops::exp over "
                      f"kv_slot, (query, head) units on a thread pool)",
        }
    return res


# ------------------------------------------------- secondary configurations

# Workloads measured beside the headline in the default run, each over a fixed
# window (their own steps, not the caller's), so that the driver's run records
# them too: line -> (preset, steps, warmup, kernel(s) the roofline prices,
# launch form, every prompt row queried).  "step": one ni_kv_step per step
# (all layers per launch); "layers": ni_kv_step_begin, one ni_kv_step_layer
# per layer (the form a model's forward runs, batch.rs:390-416), ni_kv_step_end.
# Lines without a ramp warm up for ~100 ms of their own steps: from idle the
# GPU's first ~50 ms of work run slower (16 x 512 prefill launches 290 ->
# 230 us over the first ~100 launches; config 2 and the prefill kernel measured
# 2.5% and 3% slower after 20 and 10 warmup steps than after 2000 and 200).
SECONDARY_LINES = {
    "config2": ("config2", 200, 2000, "attn_split_kernel (fused append)", "step", False),
    "config4": ("config4", 100, 300, "attn_split_kernel + attn_merge_kernel", "step", False),
    "config5": ("config5", 200, 800, "kv_append_kernel + attn_mfma_kernel", "step", False),
    "config3q8": ("config3q8", 200, 20, "kv_append_kernel + attn_q8_kernel, Q8 cache", "step", False),
    "prefill": ("prefill", 100, 250, "attn_prefill_kernel (after its append launch)", "step", False),
    "qkv64": ("qkv64", 200, 1000, "qkv_mid_kernel (append in the epilogue)", "step", False),
    # every prompt row queried (the reference's attention covers every row of a
    # step, batch.rs:577-600): decode rows fused, prompt chunks appended by the
    # same launch's extra blocks, then their prefill launch
    "config3_all_prompt_rows": ("config3", 200, 20, "attn_split_kernel (fused) + attn_prefill_kernel", "step", True),
    "config3_per_layer_q8": ("config3q8", 200, 20, "attn_q8_kernel (wide, fused), per layer", "layers", False),
    "config5_per_layer": ("config5", 200, 500, "attn_mfma_kernel (wide, fused), per layer", "layers", False),
    "config5_per_layer_q8": ("config5q8", 200, 600, "attn_mfma_kernel (wide, fused), per layer, Q8 cache", "layers",
                             False),
    "prefill_per_layer": ("prefill", 50, 200, "kv_append_kernel + attn_prefill_kernel, per layer", "layers", False),
}


def secondary_lines(args, reps=3):
    """Each of SECONDARY_LINES through the C++ driver: the median of `reps`
    unprofiled runs (algorithmic GB/s, as the headline) and one run timing its
    kernels with per-launch events.  config3q8 runs the headline's trace after
    the same append-only ramp."""
    import argparse as _ap
    from nanoinfer_amd import drivers

    out = {}
    for name, (preset, steps, warmup, kernel, form, all_rows) in SECONDARY_LINES.items():
        a = _ap.Namespace(steps=steps, warmup=warmup, split=0, seed=args.seed)
        ramp = RAMP_STEPS if preset.startswith("config3") else 0
        launch = drivers.NI_DRIVE_STEP_LAYERS if form == "layers" else drivers.NI_DRIVE_STEP
        runs = [_drive(preset, a, launch=launch, ramp=ramp, all_prompt_rows=all_rows) for _ in range(reps)]
        gbs = sorted(r["bytes"] / r["seconds"] / 1e9 for r in runs)
        med = gbs[len(gbs) // 2]
        r = runs[[round(r["bytes"] / r["seconds"] / 1e9, 6) for r in runs].index(round(med, 6))]
        line = {"value": round(med, 2), "unit": "GB/s", "pct_of_peak": round(100 * med / PEAK_GBS, 2),
                "ms_per_step": round(r["seconds"] / r["steps"] * 1e3, 5),
                "seq_tokens_per_s": round(r["seq_tokens"] / r["seconds"], 1),
                "algorithmic_bytes_per_step": int(r["bytes"] / r["steps"]), "steps": steps, "warmup": warmup,
                "ramp_steps": ramp, "reps_gbs": [round(g, 1) for g in gbs],
                "launch": "one ni_kv_step_layer launch per layer" if form == "layers" else "all layers per launch"}
        if all_rows:
            line["prefill_attention"] = "every prompt row queried"
        if name.startswith("qkv"):
            line["tflops"] = round(r["flops"] / r["seconds"] / 1e12, 2)
            mask, ids = 1 << 3, (3,)
        else:
            # every launch of the step (config 5's append launch too); the
            # prefill line below takes its attention launch alone
            mask = (1 << 0) | (1 << 1) | (1 << 2)
            ids = (1, 2) if name == "prefill" else (0, 1, 2)
        rp = _drive(preset, a, launch=launch, profile_mask=mask, ramp=ramp, all_prompt_rows=all_rows)
        kms = sum(rp["kernel_ms"][i] for i in ids)
        if name == "prefill" and rp["kernel_launches"][0]:
            # the attention launch alone: the step's bytes less its append launch's
            c, L = 768, 12
            app = drivers_prefill_append_bytes(c, L)
            kb = rp["bytes"] / rp["steps"] - app
            kgbs = kb * rp["steps"] / (kms / 1e3) / 1e9
        else:
            kgbs = rp["bytes"] / (kms / 1e3) / 1e9
        line["kernel"] = {"name": kernel, "us_per_step": round(kms / rp["steps"] * 1e3, 3),
                          "achieved_gbs": round(kgbs, 1), "frac": round(kgbs / PEAK_GBS, 4)}
        out[name] = line
    return out


def drivers_prefill_append_bytes(c, L):
    """Algorithmic bytes of the prefill step's append (f32 K/V read, f16
    written), per step."""
    from nanoinfer_amd import drivers

    return drivers.PREFILL_SEQS * drivers.PREFILL_ROWS * L * (8 * c + 4 * c)

SECONDARY = {
    "config2": ("config2: 16 seqs, ctx U[64,1024], 1024-page pool, seeded page permutation, append 1 + attention, "
                "GPT-2 12x12x64; each step rolled back", {}),
    "config4": ("config4: batch 4, 32 heads x 128, context 32768, random page tables, 512-token partitions + LSE "
                "merge, k/v ~ N(0, 0.5); each step rolled back", {"split_tokens": 512}),
    "config5": ("config5: spec verify, 32 seqs, ctx U[128,1024], append g + 4 drafts, 5 causal queries, accept U[0,4], "
                "truncate", {"draft_k": 4, "reset_window": SPEC_WINDOW}),
}
# The same workloads on a Q8 cache (NI_KV_Q8: int8 + an f32 scale per position and head); algorithmic
# bytes count the Q8 bytes, so compare formats by seq_tokens_per_s.
for _name in list(SECONDARY):
    SECONDARY[_name + "q8"] = (SECONDARY[_name][0] + "; Q8 KV cache", dict(SECONDARY[_name][1], kv_format="q8"))
SECONDARY["config3q8"] = ("config3: continuous batching (bench default trace); Q8 KV cache",
                          {"kv_format": "q8", "prefill_attention": "last prompt row only"})


def run_secondary(args):
    desc, cfg = SECONDARY[args.workload]
    r, spread = _median_run(args.workload, args, REPS)
    res = _line(args, r, desc, dict(cfg, mean_context=round(r["mean_context"], 1),
                                    algorithmic_bytes_per_step=int(r["bytes"] / r["steps"]),
                                    host_loop="C++ driver (ni_drive_run)"),
                "synthetic (seeded normal q/k/v resident in HBM)")
    res["repetitions"] = spread
    if not args.no_profile:
        rp = _drive(args.workload, args, profile_mask=(1 << 0) | (1 << 1) | (1 << 2))
        res["roofline"] = _roofline(rp, "attn_q8_kernel (+ attn_merge_kernel when split)" if args.workload.endswith("q8")
                                    else "attn_split_kernel / attn_mfma_kernel (+ attn_merge_kernel when split, "
                                         "+ kv_append_kernel before a step of query groups)",
                                    with_merge=True, with_append=True)
        tr = measured_traffic(args.workload, args, 0)
        if tr:
            res["roofline"]["traffic"] = tr["traffic_bytes_per_launch"]
            res["roofline"]["traffic_vs_algorithmic"] = round(
                tr["traffic_bytes_per_launch"] / tr["algorithmic_bytes_per_launch_same_steps"], 3)
            res["roofline"]["traffic_source"] = os.path.relpath(TRAFFIC_PROFILES[args.workload], ROOT) + \
                " (rocprofv3 --pmc, scaled; attention + merge per step)"
    if args.workload.endswith("q8"):
        res["kv_dtype"] = "int8 + f32 scale per (position, head)"
    return res


PEAK_F32_TFLOPS = 157.3  # MI355X dense f32 matrix throughput, AMD's published figure


def run_qkv(args):
    """The QKV projection of GPT-2 (d_in 768 -> 3C = 2304) per layer with K/V
    appended to pages in its epilogue (ni_kv_qkv_append, the reference's
    BEPI_QKV path), against the unfused path (f32 projection, then
    ni_kv_append).  Both are timed on the same algorithmic bytes: W, bias,
    x, q out and the f16 K/V stores."""
    from nanoinfer_amd import drivers

    spec, wname = args.workload[3:], "f32"
    for suffix, nm in (("f16", "f16"), ("q8", "q8_0"), ("q4", "q4_0")):
        if spec.endswith(suffix):
            spec, wname = spec[: -len(suffix)], nm
    rows = int(spec or 64)
    r = _drive(args.workload, args)
    # the unfused comparison: f32 projection + append (f32 weights)
    ru = _drive(f"qkv{rows}", args, launch=drivers.NI_DRIVE_PER_LAYER)
    res = _line(args, r, f"qkv: GPT-2 QKV projection, {rows} rows x 12 layers (768 -> 2304, {wname} weights) with "
                         f"K/V appended as f16 in the epilogue",
                {"rows": rows, "d_in": 768, "n_feat": 2304, "weights": wname},
                "synthetic (seeded normal x, W ~ N(0, 1/768) quantised as the reference uploads it, bias, "
                "resident in HBM)")
    res["metric"] = "fused QKV projection + KV append, algorithmic GB/s, 1 MI355X"
    res["tflops"] = round(r["flops"] / r["seconds"] / 1e12, 2)
    gu = ru["bytes"] / ru["seconds"] / 1e9
    res["unfused"] = {"value": round(gu, 2), "unit": "GB/s", "ms_per_step": round(ru["seconds"] / ru["steps"] * 1e3, 5),
                      "path": "ni_kv_qkv_project (f32 [n][3C]) + ni_kv_append per layer"}
    if not args.no_profile:
        rp = _drive(args.workload, args, profile_mask=1 << 3)
        ms, n = rp["kernel_ms"][3], rp["kernel_launches"][3]
        t = ms / 1e3
        gbs, tfl = rp["bytes"] / t / 1e9, rp["flops"] / t / 1e12
        mfma_bound = rp["flops"] / (PEAK_F32_TFLOPS * 1e12) > rp["bytes"] / (PEAK_GBS * 1e9)
        res["roofline"] = {"bound": "mfma" if mfma_bound else "hbm",
                           "achieved": round(tfl if mfma_bound else gbs, 2),
                           "peak": PEAK_F32_TFLOPS if mfma_bound else PEAK_GBS,
                           "unit": "TFLOP/s" if mfma_bound else "GB/s",
                           "frac": round(tfl / PEAK_F32_TFLOPS if mfma_bound else gbs / PEAK_GBS, 4), "traffic": None,
                           "kernel": "qkv_kernel (fused epilogue)", "avg_launch_us": round(ms / n * 1e3, 3),
                           "launches": n, "algorithmic_bytes_per_launch": int(rp["bytes"] / n),
                           "flops_per_launch": int(rp["flops"] / n), "achieved_gbs": round(gbs, 2),
                           "achieved_tflops": round(tfl, 2)}
    return res


PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16 matrix throughput, AMD's published figure


def run_prefill(args):
    """Prefill: 16 sequences each append a 512-row prompt from empty and
    attend every row causally (groups of up to 64 rows on the prefill
    kernel, whose workgroups append each sequence's rows before its groups
    read them), rolled back each step.  The roofline prices the prefill
    launch: its algorithmic bytes (the rows' f32 K/V read and stored, q
    read, out written, each sequence's K/V read once; without the rows'
    bytes when a separate append launch stored them) against HBM, with its
    useful flops (4 per query, visible key and element of C) against the f16
    matrix peak beside them."""
    from nanoinfer_amd import drivers, workloads

    B, P = drivers.PREFILL_SEQS, drivers.PREFILL_ROWS
    c, L, H = 768, workloads.GPT2["n_layer"], workloads.GPT2["n_head"]
    q8 = args.workload.endswith("q8")
    kvb = c + 4 * H if q8 else 2 * c  # stored bytes of one position's K (or V) in one layer
    r = _drive(args.workload, args)
    res = _line(args, r, f"prefill: {B} sequences x {P}-row prompt from empty, every row queried (causal), GPT-2 "
                         f"12x12x64, 16-token pages, rolled back each step{'; Q8 KV cache' if q8 else ''}",
                {"seqs": B, "rows": P, "algorithmic_bytes_per_step": int(r["bytes"] / r["steps"]),
                 "host_loop": "C++ driver (ni_drive_run)"},
                "synthetic (seeded N(0,1) q/k/v resident in HBM)")
    res["metric"] = "paged prefill attention + append, algorithmic GB/s, 1 MI355X"
    if q8:
        res["kv_dtype"] = "q8"
    res["attention_tflops_whole_step"] = round(r["flops"] / r["seconds"] / 1e12, 2)
    if not args.no_profile:
        rp = _drive(args.workload, args, profile_mask=(1 << 0) | (1 << 1) | (1 << 2))
        steps = rp["steps"]
        attn_ms = rp["kernel_ms"][1] + rp["kernel_ms"][2]
        append_bytes = B * P * L * (8 * c + 2 * kvb)
        fused = rp["kernel_launches"][0] == 0  # the prefill launch appends the rows
        attn_bytes = rp["bytes"] / steps - (0 if fused else append_bytes)
        t = attn_ms / 1e3 / steps
        gbs = attn_bytes / t / 1e9
        tfl = rp["flops"] / steps / t / 1e12
        res["roofline"] = {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_GBS, "unit": "GB/s",
                           "frac": round(gbs / PEAK_GBS, 4), "traffic": None,
                           "kernel": "attn_prefill_q8_kernel" if q8 else "attn_prefill_kernel<64,2>",
                           "avg_launch_us": round(t * 1e6, 3), "launches": rp["kernel_launches"][1],
                           "algorithmic_bytes_per_launch": int(attn_bytes),
                           "flops_per_launch": int(rp["flops"] / steps), "achieved_tflops": round(tfl, 2),
                           "frac_of_f16_matrix_peak": round(tfl / PEAK_F16_TFLOPS, 4),
                           "append": "in the prefill launch" if fused else
                           f"its own launch, {rp['kernel_ms'][0] / steps * 1e3:.3f} us per step"}
    return res


CFG1 = dict(prompt=64, decode=64)  # GPT-2 shape, one sequence: prefill 64 positions, then 64 decode steps


def _cfg1_bytes(c, L, P, T):
    """Algorithmic bytes of config 1 (the step formula summed): the prefill
    appends and queries P rows over contexts 1..P (each K/V byte once), then
    decode step t appends and queries one row over P + t + 1 keys."""
    from nanoinfer_amd.workloads import step_bytes

    total = step_bytes([(0, P, P)], [P], L, c)["total"]
    for t in range(T):
        total += step_bytes([(0, 1, 1)], [P + t + 1], L, c)["total"]
    return total


def run_config1(args, reps=REPS):
    """Benchmark configuration 1, the reference's CPU-runnable case: one GPT-2
    sequence (12 layers x 12 heads x 64, f16 KV in 16-token pages) prefills
    64 positions (every row queried, as the CPU forward attends every prompt
    row) and decodes 64 steps, one K/V row appended and attended per layer
    and step.  On the device: one ni_kv_step for the prefill, then
    ni_kv_decode_steps for the 64 decode steps (Batch::decode_resident: all
    enqueued at once), timed with events around both; `reps` runs, the
    sequence truncated to 0 between them, median.  Beside it: the contiguous
    f32 form of the same attention through ni_attention (the CPU engine's
    Kernels::attention, stage 0/1 caches), and the reference's CPU path (the
    oracle's restatement of kv16::attention with attend_f16_portable on a
    thread pool) on the same inputs."""
    import torch

    import nanoinfer_amd as na
    from nanoinfer_amd import workloads

    sh = workloads.GPT2
    L, H, D = sh["n_layer"], sh["n_head"], sh["head_dim"]
    c, P, T = H * D, CFG1["prompt"], CFG1["decode"]
    n = P + T
    kv = na.PagedKv(na.BatchOpts(**sh, kv_blocks=n // 16, max_seqs=1, n_ctx=1024, max_rows=P))
    s = kv.add_seq()
    rng = np.random.default_rng(args.seed)
    q, k, v = (rng.standard_normal((L, n, c), dtype=np.float32) for _ in range(3))
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
    # decode_steps layout [step][layer][row][C]: views of the same rows
    qs, ks, vs = (x[:, P:, :].permute(1, 0, 2).unsqueeze(2) for x in (qd, kd, vd))
    out_p = torch.empty((L, P, c), device="cuda")
    out_d = torch.empty((T, L, 1, c), device="cuda")

    def one():
        kv.truncate(s, 0)
        kv.step([(s, P, P)], qd[:, :P], kd[:, :P], vd[:, :P], out=out_p)
        kv.decode_steps([s], qs, ks, vs, out=out_d)

    one()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        one()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1) / 1e3)
    t = float(np.median(times))
    nbytes = _cfg1_bytes(c, L, P, T)
    res = {"metric": METRIC, "value": round(nbytes / t / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": T + 1,
           "warmup": 1, "ms_per_step": round(t / (T + 1) * 1e3, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32", "kv_dtype": "f16",
           "data": "synthetic (seeded N(0,1) q/k/v resident in HBM)",
           "config": {"workload": "config1: one GPT-2 sequence (12x12x64), f16 KV in 16-token pages, prefill 64 "
                                  "positions (every row queried) then 64 decode steps", "n_layer": L, "n_head": H,
                      "head_dim": D, "prompt": P, "decode_steps": T, "algorithmic_bytes": int(nbytes),
                      "calls": "ni_kv_step (prefill) + ni_kv_decode_steps (64 steps, one enqueue)"},
           "pct_of_peak": round(100 * nbytes / t / 1e9 / PEAK_GBS, 3),
           "seq_tokens_per_s": round(n / t, 1), "seconds_per_run": round(t, 6),
           "repetitions": {"reps": reps, "seconds": [round(x, 6) for x in times]},
           "note": "latency-bound: 65 dependent steps of ~0.8 MB each; the figure is tokens/s, not bandwidth"}

    # The contiguous f32 form (Kernels::attention over [pos][C] caches): per
    # layer the prefill's 64 queries, then one query per decode step.
    att_out = torch.empty((L, n, c), device="cuda")

    def contiguous():
        for l in range(L):
            na.attention(qd[l, :P], kd[l], vd[l], P, 0, H, D, out=att_out[l, :P])
        for tt in range(T):
            for l in range(L):
                na.attention(qd[l, P + tt:P + tt + 1], kd[l], vd[l], 1, P + tt, H, D, out=att_out[l, P + tt:P + tt + 1])

    contiguous()
    torch.cuda.synchronize()
    ct = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        contiguous()
        e1.record()
        e1.synchronize()
        ct.append(e0.elapsed_time(e1) / 1e3)
    res["contiguous_attention"] = {
        "seconds_per_run": round(float(np.median(ct)), 6), "seq_tokens_per_s": round(n / float(np.median(ct)), 1),
        "calls": f"ni_attention per layer and step ({L * (T + 1)} calls), f32 K/V rows", "reps": reps}

    if args.cpu_seconds > 0:
        import oracle

        threads = args.threads or available_parallelism()
        pools = oracle.PagedPools(L, n // 16, c)
        table = np.arange(n // 16, dtype=np.uint32).reshape(1, -1)
        runner = oracle.CpuStep(threads)
        outc = np.zeros((L, P, c), np.float32)
        outd = np.zeros((T, L, 1, c), np.float32)
        # decode step t's inputs: row P + t of each layer, as [L][1][C]
        qkv_d = [tuple(np.ascontiguousarray(x[:, P + tt:P + tt + 1]) for x in (q, k, v)) for tt in range(T)]
        qp, kp, vp = (np.ascontiguousarray(x[:, :P]) for x in (q, k, v))

        def cpu_run():
            rows = np.arange(P, dtype=np.uint32)
            runner.run(pools, table, n // 16, np.zeros(P, np.uint32), rows, rows, qp, kp, vp, outc, H, D)
            for tt in range(T):
                runner.run(pools, table, n // 16, np.zeros(1, np.uint32), np.array([P + tt], np.uint32),
                           np.zeros(1, np.uint32), *qkv_d[tt], outd[tt], H, D)

        cts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            cpu_run()
            cts.append(time.perf_counter() - t0)
        tc = float(np.median(cts))
        # the device result against the CPU path on the same inputs (a check, not timed)
        dev = torch.cat([out_p.cpu(), out_d[:, :, 0].permute(1, 0, 2).cpu()], dim=1).numpy()
        want = np.concatenate([outc, outd[:, :, 0].transpose(1, 0, 2)], axis=1)
        cp = {"value": round(nbytes / tc / 1e9, 3), "unit": "GB/s", "seq_tokens_per_s": round(n / tc, 1),
              "seconds_per_run": round(tc, 6), "cores": runner.threads, "kind": "port", "cpu_model": cpu_model(),
              "repetitions": {"reps": reps, "seconds": [round(x, 6) for x in cts]},
              "sample": "the whole of config 1 (prefill 64 + 64 decode steps, 12 layers): the oracle's C restatement "
                        "of the reference x86 CPU path (narrow + attend_f16_portable + fastops::exp, (query, head) "
                        "units on a thread pool), per step as the device runs it",
              "max_abs_diff_vs_device": float(np.abs(dev - want).max())}
        res["cpu_baseline"] = cp
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (the path would shard by "
                                   "sequence, one page pool per GPU, with no exchange)"}))
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        log("bench: no GPU visible")
        sys.exit(1)
    if args.calibrate_copy:
        calibrate_copy()
        return
    # The headline line is config 3; the others are secondary measurements.
    if args.workload == "config3":
        res = run_config3(args)
    elif args.workload == "config1":
        res = run_config1(args)
    elif args.workload.startswith("qkv"):
        res = run_qkv(args)
    elif args.workload in ("prefill", "prefillq8"):
        res = run_prefill(args)
    elif args.workload in SECONDARY:
        res = run_secondary(args)
    else:
        log(f"bench: unknown workload {args.workload}")
        sys.exit(2)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
