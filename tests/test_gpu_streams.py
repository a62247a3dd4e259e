"""Calls of one handle on two streams run in call order.

The reference cannot interleave its work: Batch::step waits for the GPU
before it commits (crates/metal/src/batch.rs:259-273, gpu.rs:200-209).  Here
data-path calls return at once, and they share the handle's split partials;
a page that truncate returns may go to the very next append.  So a call on a
stream other than the one holding the handle's previous work makes its
stream wait for that work first.  These tests issue the calls back to back on
two streams with no host wait between them (heavy work first, so that an
unordered second call would overlap it) and check every output against the
oracle and every stored row bit for bit.
"""
import sys

import numpy as np
import pytest
import torch

import oracle
import nanoinfer_amd as na
from nanoinfer_amd import workloads
from paged_mirror import Mirror, assert_close

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def oracle_step(m, rows, qrows, q, k, v):
    """The oracle's append and attention of one step, in call order."""
    t = m.table()
    want = np.zeros_like(q)
    for l in range(m.opts.n_layer):
        oracle.paged_append(m.pools, l, t, m.kv.max_blocks, rows[:, 0], rows[:, 1], k[l], v[l])
        if len(qrows):
            want[l][qrows] = oracle.paged_attention(m.pools, l, t, m.kv.max_blocks, rows[qrows, 0], rows[qrows, 1],
                                                    q[l][qrows], m.opts.n_head, m.opts.head_dim)
    return want


def test_split_steps_alternating_streams(gpu, oracle_lib):
    """Steps with 64-token partitions (split partials and a merge launch
    each, all in the handle's one partials buffer) and one step run one
    layer per launch, alternating between two streams with no wait."""
    rng = np.random.default_rng(201)
    m = Mirror(na.BatchOpts(**workloads.GPT2, kv_blocks=2400, max_seqs=48, n_ctx=1024, max_rows=512))
    seqs = [m.kv.add_seq() for _ in range(48)]
    for s in seqs:
        m.fill(s, int(rng.integers(300, 900)), rng)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    plans = [  # (work, stream, per_layer)
        ([(s, 1, 1) for s in seqs], sa, False),             # heavy: 48 rows of 300..900 keys
        ([(s, 1, 1) for s in seqs[::7]], sb, False),        # light, on the other stream
        ([(s, 2, 2) for s in seqs[::3]], sa, False),        # verify-style groups
        ([(s, 1, 1) for s in seqs[1::5]], sb, True),        # one launch per layer
        ([(s, 1, 1) for s in seqs[::2]], sa, False),
    ]
    launched = []
    lens = {s: m.kv.seq_len(s) for s in seqs}  # the lengths each step will see
    for i, (work, stream, per_layer) in enumerate(plans):
        rows, qrows = [], []
        for seq, n_new, n_q in work:
            for j in range(n_new):
                if j >= n_new - n_q:
                    qrows.append(len(rows))
                rows.append((seq, lens[seq] + j))
            lens[seq] += n_new
        rows, qrows = np.asarray(rows, np.uint32), np.asarray(qrows, np.int64)
        n = len(rows)
        q, k, v = (rng.standard_normal((m.opts.n_layer, n, m.c)).astype(np.float32) for _ in range(3))
        qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
        out = torch.full_like(qd, float("nan"))
        torch.cuda.synchronize()  # inputs ready; from here no host wait until every step is enqueued
        launched.append((rows, qrows, q, k, v, qd, kd, vd, out))
    for i, ((work, stream, per_layer), (rows, qrows, q, k, v, qd, kd, vd, out)) in enumerate(zip(plans, launched)):
        say(f"streams: step {i} on stream {'A' if stream is sa else 'B'}, {len(rows)} rows, per_layer={per_layer}")
        if per_layer:
            m.kv.step_begin(work, split_tokens=64)
            for l in range(m.opts.n_layer):
                m.kv.step_layer(l, qd[l], kd[l], vd[l], out=out[l], stream=stream)
            m.kv.step_end()
        else:
            m.kv.step(work, qd, kd, vd, out=out, split_tokens=64, stream=stream)
    torch.cuda.synchronize()
    for i, (rows, qrows, q, k, v, qd, kd, vd, out) in enumerate(launched):
        want = oracle_step(m, rows, qrows, q, k, v)
        got = out.cpu().numpy()
        err = assert_close(got[:, qrows], want[:, qrows], f"step {i}")
        say(f"streams: step {i} max abs err {err:.2e}")
    (kg, vg), (kw, vw) = m.gather(np.concatenate([r for r, *_ in launched]))
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)


def test_truncate_then_reuse_on_another_stream(gpu, oracle_lib):
    """Attention over a long sequence on stream A; at once, with no wait,
    the sequence is truncated, a new sequence takes its freed pages and
    appends new rows on stream B.  A's outputs must be those of the old
    rows, and the new sequence's rows must be stored bit for bit."""
    rng = np.random.default_rng(202)
    m = Mirror(na.BatchOpts(**workloads.GPT2, kv_blocks=2400, max_seqs=40, n_ctx=1024, max_rows=512))
    seqs = [m.kv.add_seq() for _ in range(32)]
    for s in seqs:
        m.fill(s, int(rng.integers(600, 1000)), rng)
    x = seqs[0]
    # A: every sequence's last row, all layers, 128-token partitions
    rows = np.asarray([(s, m.kv.seq_len(s) - 1) for s in seqs], np.uint32)
    q = rng.standard_normal((m.opts.n_layer, len(rows), m.c)).astype(np.float32)
    want = np.zeros_like(q)
    t = m.table()
    for l in range(m.opts.n_layer):
        want[l] = oracle.paged_attention(m.pools, l, t, m.kv.max_blocks, rows[:, 0], rows[:, 1], q[l],
                                         m.opts.n_head, m.opts.head_dim)
    # B's new rows: a fresh sequence on x's freed pages
    keep = 16
    n_new = m.kv.seq_len(x) - keep
    k_new, v_new = (rng.standard_normal((m.opts.n_layer, n_new, m.c)).astype(np.float32) for _ in range(2))
    qd = torch.from_numpy(q).cuda()
    kd, vd = torch.from_numpy(k_new).cuda(), torch.from_numpy(v_new).cuda()
    out = torch.full_like(qd, float("nan"))
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    freed = m.kv.block_table(x)[1:]
    m.kv.attention(qd, rows, out=out, split_tokens=128, stream=sa)
    m.kv.truncate(x, keep)
    y = m.kv.add_seq()
    m.kv.reserve(y, n_new)
    reused = set(m.kv.block_table(y)) & set(freed)
    assert len(reused) >= len(freed) - 1, "the new sequence should take the freed pages"
    new_rows = np.stack([np.full(n_new, y), np.arange(n_new)], 1).astype(np.uint32)
    for p0 in range(0, n_new, 512):
        p1 = min(n_new, p0 + 512)
        m.kv.append(new_rows[p0:p1], kd[:, p0:p1], vd[:, p0:p1], stream=sb)
    m.kv.commit(y, n_new)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    err = assert_close(got, want, "attention over the old rows")
    say(f"truncate/reuse: {len(reused)} pages reused, attention max abs err {err:.2e}")
    # the oracle takes the same truncate and appends
    t = m.table()
    for l in range(m.opts.n_layer):
        oracle.paged_append(m.pools, l, t, m.kv.max_blocks, new_rows[:, 0], new_rows[:, 1], k_new[l], v_new[l])
    (kg, vg), (kw, vw) = m.gather(new_rows)
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)
    m.kv.sync(sb)
    m.kv.sync(sa)
