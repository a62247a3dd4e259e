"""The C++ drivers and the multi-step decode entry point on the device.

* ni_drive_run runs the config-3 trace and the config-5 verify loop with
  all-layer steps and with per-layer launches; both see the same trace, so
  their algorithmic bytes and tokens agree.
* Per-layer launches (ni_kv_append + ni_paged_decode_attention per layer,
  the reference's dispatch) store the same f16 K/V as ni_kv_step and attend
  within f32 rounding of it.
* ni_kv_decode_steps (decode_resident's KV part, batch.rs:322-363) equals
  the same steps made one ni_kv_step at a time, bit for bit, and fails as
  the reference does (not live, context full) before enqueueing anything.
"""
import sys

import numpy as np
import pytest
import torch

import oracle

import nanoinfer_amd as na
from nanoinfer_amd import drivers, workloads

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def drive_opts(workload, launch, steps=60, warmup=20):
    o = drivers.ni_drive_opts()
    o.workload, o.launch, o.steps, o.warmup, o.data_seed = workload, launch, steps, warmup, 7
    o.kv.n_layer, o.kv.n_head, o.kv.head_dim = 12, 12, 64
    if workload == drivers.NI_DRIVE_SERVE:
        o.serve = drivers.ni_serve_opts(7, 1.0, 100000, 64, 32, 512, 16, 256, 256, 512, 0)
        o.kv.kv_pages, o.kv.max_seqs, o.kv.max_ctx, o.kv.max_rows = 3080, 64, 1024, 512
    else:
        o.spec_seqs, o.spec_ctx_min, o.spec_ctx_max, o.spec_k, o.spec_seed, o.spec_window = 32, 128, 1024, 4, 5, 64
        o.kv.kv_pages, o.kv.max_seqs, o.kv.max_ctx, o.kv.max_rows = 32 * 128, 32, 2048, 512
    return o


@pytest.mark.parametrize("workload", [drivers.NI_DRIVE_SERVE, drivers.NI_DRIVE_SPEC], ids=["serve", "spec"])
def test_drive_launch_modes_agree(gpu, workload):
    res = {}
    for launch in (drivers.NI_DRIVE_STEP, drivers.NI_DRIVE_PER_LAYER):
        say(f"ni_drive_run workload {workload} launch {launch}")
        r = drivers.drive(drive_opts(workload, launch))
        say(f"  {r['bytes'] / r['seconds'] / 1e9:.0f} GB/s, {r['seconds'] / r['steps'] * 1e6:.1f} us/step, "
            f"host {r['host_us_per_step']:.1f} us/step")
        assert r["steps"] == 60 and r["seconds"] > 0 and r["gpu_seconds"] > 0
        res[launch] = r
    a, b = res[drivers.NI_DRIVE_STEP], res[drivers.NI_DRIVE_PER_LAYER]
    assert a["bytes"] == b["bytes"] and a["seq_tokens"] == b["seq_tokens"]
    assert a["launches"] == 60 and b["launches"] >= 12 * 60


def test_drive_prefill_accounting(gpu):
    """The prefill preset (fixed contexts with every appended row queried):
    both launch paths run, and bytes, flops and tokens per step follow the
    closed forms of the workload."""
    B, P, c, L = drivers.PREFILL_SEQS, drivers.PREFILL_ROWS, 768, 12
    want_bytes = L * B * (P * c * 12 + P * c * 8 + 2 * P * c * 2 + (P + 15) // 16 * 4)
    want_flops = 4.0 * c * L * B * P * (P + 1) / 2
    for launch in (drivers.NI_DRIVE_STEP, drivers.NI_DRIVE_PER_LAYER):
        say(f"ni_drive_run prefill launch {launch}")
        r = drivers.drive(drivers.preset("prefill", 4, 1, launch=launch))
        say(f"  {r['seconds'] / r['steps'] * 1e6:.1f} us/step")
        assert r["steps"] == 4
        assert r["bytes"] == 4 * want_bytes
        assert r["flops"] == pytest.approx(4 * want_flops, rel=1e-12)
        assert r["seq_tokens"] == 4 * B * P


def test_per_layer_launches_match_step(gpu):
    """A config-3 trace through both ABI paths on twin handles."""
    opts = na.BatchOpts(**workloads.GPT2, kv_blocks=3080, max_seqs=64, n_ctx=1024, max_rows=512)
    a, b = na.PagedKv(opts), na.PagedKv(opts)
    sa, sb = drivers.Serve(a), drivers.Serve(b)
    g = torch.Generator(device="cuda").manual_seed(3)
    C = 768
    worst = 0.0
    for i in range(40):
        work, _, adm, _ = sa.plan()
        work_b, _, _, _ = sb.plan()
        assert np.array_equal(work, work_b)
        n = int(work[:, 1].sum())
        q, k, v = (torch.randn((12, n, C), device="cuda", generator=g) for _ in range(3))
        out_a = a.step(work, q, k, v)
        # per layer: reserve, append every row, attend the queried rows, commit
        rows, qrows, qidx = [], [], []
        for seq, n_new, n_q in work.tolist():
            L = b.seq_len(seq)
            b.reserve(seq, L + n_new)
            for j in range(n_new):
                if j >= n_new - n_q:
                    qrows.append((seq, L + j))
                    qidx.append(len(rows))
                rows.append((seq, L + j))
        out_b = torch.zeros_like(q)
        qi = torch.tensor(qidx, device="cuda", dtype=torch.long)
        for l in range(12):
            b.append(rows, k[l], v[l], layer=l)
            if qidx:
                ob = b.attention(q[l].index_select(0, qi).contiguous(), qrows, layer=l)
                out_b[l].index_copy_(0, qi, ob)
        for seq, n_new, _ in work.tolist():
            b.commit(seq, n_new)
        torch.cuda.synchronize()
        if qidx:
            d = (out_a[:, qi] - out_b[:, qi]).abs().max().item()
            worst = max(worst, d)
            assert d < 1e-5, f"step {i}: {d}"
        sa.commit()
        sb.commit()
    for s in range(64):
        if a.is_live(s):
            L = a.seq_len(s)
            assert a.block_table(s) == b.block_table(s)
            ka, va = a.gather([(s, p) for p in range(min(L, 512))])
            kb, vb = b.gather([(s, p) for p in range(min(L, 512))])
            assert torch.equal(ka, kb) and torch.equal(va, vb)
    say(f"per-layer vs step: max abs difference {worst:.2e}")


def test_decode_steps_equal_single_steps(gpu):
    opts = na.BatchOpts(**workloads.GPT2, kv_blocks=256, max_seqs=8, n_ctx=1024, max_rows=512)
    a, b = na.PagedKv(opts), na.PagedKv(opts)
    g = torch.Generator(device="cuda").manual_seed(5)
    C, T = 768, 9
    lens = [15, 16, 100, 511]
    seqs = []
    for L in lens:
        s = a.add_seq()
        assert b.add_seq() == s
        k, v = (torch.randn((12, L, C), device="cuda", generator=g) for _ in range(2))
        for kv in (a, b):
            kv.reserve(s, L)
            kv.append([(s, p) for p in range(L)], k, v)
            kv.commit(s, L)
        seqs.append(s)
    n = len(seqs)
    q, k, v = (torch.randn((T, 12, n, C), device="cuda", generator=g) for _ in range(3))
    out_a = a.decode_steps(seqs, q, k, v)
    out_b = torch.zeros_like(q)
    for t in range(T):
        out_b[t] = b.step([(s, 1, 1) for s in seqs], q[t], k[t], v[t])
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    # decode_resident reserves every sequence's pages for all steps first
    # (batch.rs:341-349), so its page ids follow that order, not the order
    # in which one-step-at-a-time growth asks for pages.
    h = na.PagedKv(na.BatchOpts(**{**opts.__dict__, "host_only": True}))
    for s, L in zip(seqs, lens):
        assert h.add_seq() == s
        h.reserve(s, L)
    for s, L in zip(seqs, lens):
        h.reserve(s, L + T)
    # The same order on the oracle's allocator (batch.rs:159-254 restated):
    # fill, then every sequence's pages for all steps, then the commits.
    al = oracle.Alloc(opts.kv_blocks, opts.max_seqs, opts.n_ctx)
    for s, L in zip(seqs, lens):
        assert al.add_seq() == s
        assert al.ensure(s, L) == 0
        al.commit(s, L)
    for s, L in zip(seqs, lens):
        assert al.ensure(s, L + T) == 0
    for s in seqs:
        al.commit(s, T)
    assert a.free_block_count() == al.free_block_count() and a.blocks_used() == al.blocks_used()
    for s, L in zip(seqs, lens):
        assert a.seq_len(s) == b.seq_len(s) == al.seq_len(s) == L + T
        assert a.block_table(s) == h.block_table(s) == al.block_table(s)
        rows = [(s, p) for p in range(max(0, L + T - 64), L + T)]
        ka, va = a.gather(rows)
        kb, vb = b.gather(rows)
        assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_decode_steps_errors(gpu):
    opts = na.BatchOpts(n_layer=1, n_head=2, head_dim=64, kv_blocks=8, max_seqs=2, n_ctx=64, max_rows=8)
    kv = na.PagedKv(opts)
    s = kv.add_seq()
    q = torch.zeros((4, 1, 1, 128), device="cuda")
    with pytest.raises(na.KvError) as e:
        kv.decode_steps([1], q, q, q)
    assert "sequence 1 is not live" in str(e.value)
    kv.reserve(s, 62)
    kv.commit(s, 62)
    with pytest.raises(na.KvError) as e:
        kv.decode_steps([s], q, q, q)
    assert "context full (66 > 64)" in str(e.value)
    assert kv.seq_len(s) == 62
    with pytest.raises(na.KvError) as e:
        kv.decode_steps([s, s], torch.zeros((1, 1, 2, 128), device="cuda"), *(torch.zeros((1, 1, 2, 128),
                                                                                           device="cuda"),) * 2)
    assert "twice" in str(e.value)
    out = kv.decode_steps([s], q[:2], q[:2], q[:2])
    torch.cuda.synchronize()
    assert kv.seq_len(s) == 64 and torch.isfinite(out).all()


def test_decode_steps_against_the_oracle(gpu, oracle_lib):
    """decode_resident's KV part (batch.rs:322-363) checked directly against
    the oracle: every step's appended rows bit for bit and every step's
    attention output within 1e-3, for steps enqueued at once, including a
    sequence that crosses a page boundary during the run and 64-token
    partitions (split partials and merges on every step)."""
    from paged_mirror import Mirror, assert_close

    rng = np.random.default_rng(41)
    m = Mirror(na.BatchOpts(**workloads.GPT2, kv_blocks=256, max_seqs=8, n_ctx=1024, max_rows=512))
    lens = [1, 15, 16, 100, 511, 300]
    seqs = [m.kv.add_seq() for _ in lens]
    for s, L in zip(seqs, lens):
        m.fill(s, L, rng)
    T, n, C = 7, len(seqs), m.c
    q, k, v = (rng.standard_normal((T, 12, n, C)).astype(np.float32) for _ in range(3))
    for split in (0, 64):
        say(f"decode_steps vs oracle: {n} sequences x {T} steps, split {split}")
        base = {s: m.kv.seq_len(s) for s in seqs}
        qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
        got = m.kv.decode_steps(seqs, qd, kd, vd, split_tokens=split)
        torch.cuda.synchronize()
        got = got.cpu().numpy()
        t = m.table()
        worst = 0.0
        for step in range(T):
            rows = np.asarray([(s, base[s] + step) for s in seqs], np.uint32)
            want = np.zeros((12, n, C), np.float32)
            for l in range(12):
                oracle.paged_append(m.pools, l, t, m.kv.max_blocks, rows[:, 0], rows[:, 1], k[step, l], v[step, l])
                want[l] = oracle.paged_attention(m.pools, l, t, m.kv.max_blocks, rows[:, 0], rows[:, 1], q[step, l],
                                                 12, 64)
            worst = max(worst, assert_close(got[step], want, f"step {step}"))
        rows = np.asarray([(s, p) for s in seqs for p in range(base[s], base[s] + T)], np.uint32)
        (kg, vg), (kw, vw) = m.gather(rows)
        assert np.array_equal(kg, kw) and np.array_equal(vg, vw)
        say(f"decode_steps vs oracle: max abs err {worst:.2e}")
