"""Configs 3 (f16 and Q8) and 5 at the sizes the benchmark measures, every step
against the oracle.

Config 3 is the continuous-batching trace of metal_serve.rs:255-363 with 64
slots and the reference's 3080-page pool (metal_serve.rs:485); config 5 is the
speculative-verify loop of metal_spec.rs:118-169 over 32 sequences with
contexts U[128, 1024].  test_gpu_lifecycle.py runs both scaled down for many
more steps; here the sizes are the real ones (GPT-2 12 x 12 x 64, 16-token
pages), so every launch shape the benchmark uses -- all layers in one fused
launch, 768+ workgroups, prompt chunks appended by the launch's extra blocks,
5-row groups on the matrix cores -- is checked row by row.
"""
import sys

import numpy as np
import pytest
import torch

import oracle
import nanoinfer_amd as na
from nanoinfer_amd import workloads
from paged_mirror import Mirror, assert_close, mirror_step, step_rows

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def test_config3_full_size_trace(gpu, oracle_lib):
    """Config 3 from an empty cache into its steady state: Poisson arrivals
    at 1 per step, prompts U[32,512], outputs U[16,256], prefill budget 256
    rows per step, 64 slots, 3080 pages; every decode row and the last row
    of each prompt queried (the benchmark's setting), the append fused into
    the attention launch.  Every step's appends go to the oracle too; the
    attention of every queried row is checked on the first 30 steps (the
    ramp-up) and on steps 300..319, where all 64 slots are live, sequences
    have retired and their pages have gone to new arrivals (the reference's
    page-reuse test, crates/metal/tests/batch.rs:112-143, at full size).
    Then every live sequence's K/V is gathered bit for bit."""
    rng = np.random.default_rng(41)
    m = Mirror(na.BatchOpts(**workloads.GPT2, kv_blocks=3080, max_seqs=64, n_ctx=1024, max_rows=512))
    trace = workloads.ContinuousBatching(m.kv)  # config 3's parameters are the defaults
    # Inputs: windows of one resident random buffer (a fresh window per step).
    R = 2048
    qa, ka, va = (rng.standard_normal((12, R, m.c), dtype=np.float32) for _ in range(3))
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (qa, ka, va))
    worst, queried, retired, readmitted = 0.0, 0, 0, 0
    checked = list(range(30)) + list(range(300, 320))
    for step in range(320):
        st = trace.plan()
        retired += len(st.retire)
        if retired:
            readmitted += len(st.admit)
        n = int(st.work[:, 1].sum())
        off = (step * 389) % (R - 512)
        rows, qrows = step_rows(m.kv, st.work)
        out = m.kv.step(st.work, qd[:, off:off + n], kd[:, off:off + n], vd[:, off:off + n])
        t = m.table()
        for l in range(12):
            oracle.paged_append(m.pools, l, t, m.kv.max_blocks, rows[:, 0], rows[:, 1], ka[l, off:off + n],
                                va[l, off:off + n])
        if step in checked:
            if step >= 300:
                assert sum(m.kv.is_live(s) for s in range(64)) == 64
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            for l in range(12):
                want = oracle.paged_attention(m.pools, l, t, m.kv.max_blocks, rows[qrows, 0], rows[qrows, 1],
                                              qa[l, off:off + n][qrows], 12, 64)
                worst = max(worst, assert_close(got[l][qrows], want, f"config 3 step {step} layer {l}"))
            queried += len(qrows)
        trace.commit()
        if step % 40 == 39:
            torch.cuda.synchronize()
            live = sum(m.kv.is_live(s) for s in range(64))
            say(f"config 3 step {step}: {live} live, {n} rows this step, {retired} retired, max abs err {worst:.2e}")
    assert retired > 0 and readmitted > 0 and queried >= 20 * 64
    live = [s for s in range(64) if m.kv.is_live(s)]
    assert len(live) == 64
    used = sum(-(-m.kv.seq_len(s) // 16) for s in live)
    assert 3080 - m.kv.free_block_count() == used
    rows = [(s, p) for s in live for p in range(m.kv.seq_len(s))]
    (kg, vg), (kw, vw) = m.gather(rows)
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)
    say(f"config 3: {len(live)} live after {retired} retirements and {readmitted} later admissions, "
        f"{len(rows)} rows gathered bit for bit, {queried} rows queried, max abs err {worst:.2e}")


def test_config3_q8_full_size_steady_state(gpu, oracle_lib):
    """Config 3 on a Q8 cache (kv8.metal:15-95), the same trace from an empty
    3080-page pool: every step's appends mirrored into the Q8 oracle
    (quantised by the oracle from the same f32 inputs), the attention of
    every queried row checked on steps 300..309 with all 64 slots live after
    retirements and page reuse, then every live row's int8 values and
    scales compared bit for bit."""
    from test_gpu_q8 import MirrorQ8

    rng = np.random.default_rng(43)
    m = MirrorQ8(na.BatchOpts(**workloads.GPT2, kv_blocks=3080, max_seqs=64, n_ctx=1024, max_rows=512, q8=True))
    trace = workloads.ContinuousBatching(m.kv)
    R = 2048
    qa, ka, va = (rng.standard_normal((12, R, m.c), dtype=np.float32) for _ in range(3))
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (qa, ka, va))
    worst, queried, retired = 0.0, 0, 0
    for step in range(310):
        st = trace.plan()
        retired += len(st.retire)
        n = int(st.work[:, 1].sum())
        off = (step * 389) % (R - 512)
        rows, qrows = step_rows(m.kv, st.work)
        out = m.kv.step(st.work, qd[:, off:off + n], kd[:, off:off + n], vd[:, off:off + n])
        m.append_oracle(rows, ka[:, off:off + n], va[:, off:off + n])
        if step >= 300:
            assert sum(m.kv.is_live(s) for s in range(64)) == 64
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            want = m.attention_oracle(rows[qrows], qa[:, off:off + n][:, qrows])
            worst = max(worst, assert_close(got[:, qrows], want, f"Q8 config 3 step {step}"))
            queried += len(qrows)
        trace.commit()
        if step % 40 == 39:
            say(f"Q8 config 3 step {step}: {retired} retired, max abs err {worst:.2e}")
    assert retired > 0 and queried >= 10 * 56  # (a sequence mid-prompt has no query that step)
    live = [s for s in range(64) if m.kv.is_live(s)]
    rows = [(s, p) for s in live for p in range(m.kv.seq_len(s))]
    for i in range(0, len(rows), 512):  # one gather holds at most max_rows rows
        m.check_bytes(rows[i:i + 512])
    say(f"Q8 config 3: {retired} retirements, {len(rows)} rows' int8 values and scales bit for bit, "
        f"{queried} rows queried, max abs err {worst:.2e}")


@pytest.mark.parametrize("per_layer", [False, True], ids=["all_layers", "per_layer"])
def test_config5_full_size_trace(gpu, oracle_lib, per_layer):
    """Config 5: 32 sequences with contexts U[128, 1024] (the benchmark's
    seed), each step appending g + 4 drafts and querying them as one causal
    5-row group, accepting U[0,4] and truncating the rest.  5 steps against
    the oracle.  per_layer: one launch per layer, whose 384 (item, head)
    units run on 8-wave workgroups sharing each item's pages."""
    rng = np.random.default_rng(42)
    ctx, _ = workloads.config5_contexts()
    m = Mirror(na.BatchOpts(**workloads.GPT2, kv_blocks=2400, max_seqs=32, n_ctx=1104, max_rows=512))
    seqs = [m.kv.add_seq() for _ in ctx]
    for s, L in zip(seqs, ctx):
        m.fill(s, L, rng, chunk=512)
    spec = workloads.SpecVerify(m.kv, seqs, k=4, seed=9)
    worst = 0.0
    for step in range(5):
        st = spec.plan()
        n = int(st.work[:, 1].sum())
        assert n == 5 * len(seqs)
        q, k, v = (rng.standard_normal((12, n, m.c)).astype(np.float32) for _ in range(3))
        got, want, qrows = mirror_step(m, st.work, q, k, v, per_layer=per_layer)
        worst = max(worst, assert_close(got[:, qrows], want[:, qrows], f"config 5 step {step}"))
        spec.commit()
        say(f"config 5 step {step}: max abs err {worst:.2e}")
    for s in seqs:
        assert len(m.kv.block_table(s)) == -(-m.kv.seq_len(s) // 16)
