"""The Q8 cache (NI_KV_Q8; kv8.metal:15-95) on the device against the
oracle: appends bit-exact (int8 values and f32 scales, through
ni_kv_gather_q8), attention within the north star's 1e-3 of the oracle's
double-precision Q8 attention over the same stored bytes, fused steps,
rollback, and the calls a Q8 cache refuses."""
import sys

import numpy as np
import pytest
import torch

import oracle
import nanoinfer_amd as na
from nanoinfer_amd import workloads
from paged_mirror import assert_close, step_rows

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


class MirrorQ8:
    def __init__(self, opts):
        self.opts = opts
        self.kv = na.PagedKv(opts)
        self.c = opts.n_head * opts.head_dim
        self.pools = oracle.PagedPoolsQ8(opts.n_layer, opts.kv_blocks, opts.n_head, opts.head_dim)

    def table(self):
        t = np.zeros((self.opts.max_seqs, self.kv.max_blocks), np.uint32)
        for s in range(self.opts.max_seqs):
            bt = self.kv.block_table(s)
            t[s, :len(bt)] = bt
        return t

    def append_oracle(self, rows, k, v):
        rows = np.asarray(rows, np.uint32).reshape(-1, 2)
        t = self.table()
        for l in range(self.opts.n_layer):
            oracle.paged_q8_append(self.pools, l, t, self.kv.max_blocks, rows[:, 0], rows[:, 1], k[l], v[l])

    def fill(self, seq, length, rng, chunk=256, vstd=1.0):
        start = self.kv.seq_len(seq)
        self.kv.reserve(seq, length)
        for p0 in range(start, length, chunk):
            p1 = min(length, p0 + chunk)
            rows = [(seq, p) for p in range(p0, p1)]
            shape = (self.opts.n_layer, p1 - p0, self.c)
            k = rng.standard_normal(shape, dtype=np.float32)
            v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(vstd)).astype(np.float32)
            self.kv.append(rows, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
            self.append_oracle(rows, k, v)
        self.kv.commit(seq, length - start)

    def attention_oracle(self, rows, q):
        rows = np.asarray(rows, np.uint32).reshape(-1, 2)
        t = self.table()
        return np.stack([oracle.paged_q8_attention(self.pools, l, t, self.kv.max_blocks, rows[:, 0], rows[:, 1], q[l])
                         for l in range(self.opts.n_layer)])

    def check_bytes(self, rows):
        rows = np.asarray(rows, np.uint32).reshape(-1, 2)
        t = self.table()
        (kq, vq), (ks, vs) = self.kv.gather_q8(rows)
        kq, vq, ks, vs = (x.cpu().numpy() for x in (kq, vq, ks, vs))
        for l in range(self.opts.n_layer):
            (wk, wv), (wks, wvs) = oracle.paged_q8_gather(self.pools, l, t, self.kv.max_blocks, rows[:, 0], rows[:, 1])
            assert np.array_equal(kq[l], wk) and np.array_equal(vq[l], wv), f"layer {l}: int8 values"
            assert np.array_equal(ks[l].view(np.uint32), wks.view(np.uint32)), f"layer {l}: k scales"
            assert np.array_equal(vs[l].view(np.uint32), wvs.view(np.uint32)), f"layer {l}: v scales"


def opts(shape, **kw):
    base = dict(**shape, kv_blocks=256, max_seqs=8, n_ctx=2048, max_rows=512, q8=True)
    base.update(kw)
    return na.BatchOpts(**base)


@pytest.mark.parametrize("shape", [workloads.GPT2, dict(n_layer=2, n_head=4, head_dim=128)], ids=["hd64", "hd128"])
def test_q8_append_bit_exact(gpu, oracle_lib, shape):
    rng = np.random.default_rng(90)
    m = MirrorQ8(opts(shape))
    s = m.kv.add_seq()
    L = 77
    m.kv.reserve(s, L)
    rows = [(s, p) for p in range(L)]
    shape3 = (shape["n_layer"], L, m.c)
    k = (rng.standard_normal(shape3) * rng.choice([1e-4, 1.0, 1e3], size=(1, L, 1))).astype(np.float32)
    v = rng.standard_normal(shape3).astype(np.float32)
    d = shape["head_dim"]
    k[:, 3, :d] = 0.0                  # an all-zero (position, head): scale 0, values 0
    k[:, 4, :d] = 0.0
    k[:, 4, 5] = -7.25                 # one spike: it alone sets amax
    v[:, 5, :] = np.float32(2.5) * np.sign(v[:, 5, :])  # ties of rint at amax/127 steps
    m.kv.append(rows, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    m.append_oracle(rows, k, v)
    torch.cuda.synchronize()
    m.check_bytes(rows)


@pytest.mark.parametrize("shape", [workloads.GPT2, dict(n_layer=2, n_head=4, head_dim=128)], ids=["hd64", "hd128"])
@pytest.mark.parametrize("split", [0, 64, 512])
def test_q8_decode_contexts(gpu, oracle_lib, shape, split):
    rng = np.random.default_rng(91)
    m = MirrorQ8(opts(shape, page_order=rng.permutation(256).tolist()))
    lens = [1, 15, 16, 17, 300, 1023]
    seqs = [m.kv.add_seq() for _ in lens]
    for s, L in zip(seqs, lens):
        m.fill(s, L, rng)
    rows = [(s, L - 1) for s, L in zip(seqs, lens)]
    q = rng.standard_normal((shape["n_layer"], len(rows), m.c)).astype(np.float32)
    got = m.kv.attention(torch.from_numpy(q).cuda(), rows, split_tokens=split).cpu().numpy()
    want = m.attention_oracle(rows, q)
    err = assert_close(got, want, f"q8 split {split}")
    say(f"q8 {shape} split {split}: max abs err {err:.2e}")


@pytest.mark.parametrize("nq", [2, 5, 16, 20, 64, 100])
def test_q8_causal_groups(gpu, oracle_lib, nq):
    """Consecutive rows of one sequence share their K/V reads on the matrix
    cores (int8 converted to f16 exactly, scales applied to scores and p):
    up to 16 rows on the group kernel, 17..64 on the prefill kernel (int8
    tiles by DMA, V^T through the 8-bit transposing read), longer runs cut
    into groups of 64."""
    rng = np.random.default_rng(93 + nq)
    m = MirrorQ8(opts(workloads.GPT2, n_layer=2))
    for split in (0, 64):
        for L in sorted({nq, nq + 1, 17 + nq, 130, 700}):
            s = m.kv.add_seq()
            m.fill(s, L, rng)
            rows = [(s, p) for p in range(L - nq, L)]
            q = rng.standard_normal((2, nq, m.c)).astype(np.float32)
            got = m.kv.attention(torch.from_numpy(q).cuda(), rows, split_tokens=split).cpu().numpy()
            assert_close(got, m.attention_oracle(rows, q), f"q8 nq {nq} L {L} split {split}")
            m.kv.free_seq(s)


def test_q8_long_groups_head_dim_128(gpu, oracle_lib):
    """head_dim 128 on a Q8 cache keeps runs over 16 rows in groups of 16 on
    the group kernel (the Q8 prefill tiles are for head_dim 64)."""
    rng = np.random.default_rng(97)
    m = MirrorQ8(opts(workloads.LONG, n_head=4))
    s = m.kv.add_seq()
    m.fill(s, 300, rng)
    rows = [(s, p) for p in range(260, 300)]
    q = rng.standard_normal((1, len(rows), m.c)).astype(np.float32)
    for split in (0, 128):
        got = m.kv.attention(torch.from_numpy(q).cuda(), rows, split_tokens=split).cpu().numpy()
        assert_close(got, m.attention_oracle(rows, q), f"q8 hd128 40 rows split {split}")


@pytest.mark.parametrize("nq", [1, 5, 16, 64])
def test_q8_large_values(gpu, oracle_lib, nq):
    """Value scales far above 1 (|v| in the thousands) after a prefix of
    ordinary values: on the matrix cores p * scale would overflow f16 without
    the value-scale reference, which here must also move in mid-stream."""
    rng = np.random.default_rng(95 + nq)
    m = MirrorQ8(opts(workloads.GPT2, n_layer=2))
    s = m.kv.add_seq()
    m.fill(s, 300, rng)
    m.fill(s, 600, rng, vstd=3000.0)
    rows = [(s, p) for p in range(600 - nq, 600)]
    q = rng.standard_normal((2, nq, m.c)).astype(np.float32)
    for split in (0, 128):
        got = m.kv.attention(torch.from_numpy(q).cuda(), rows, split_tokens=split).cpu().numpy()
        err = assert_close(got, m.attention_oracle(rows, q), f"q8 large values nq {nq} split {split}")
        say(f"q8 large values nq {nq} split {split}: max abs err {err:.3e}")


@pytest.mark.parametrize("per_layer", [False, True], ids=["all_layers", "per_layer"])
def test_q8_step_fused_rollback_and_reuse(gpu, oracle_lib, per_layer):
    """ni_kv_step on a Q8 cache: decode rows, a prompt chunk queried at its
    last row, a 5-row verify group and a mid-prompt chunk (no query) in one
    step -- one fused launch, or, all layers with the 37-row chunk queried,
    an append launch and then the attention launch (per_layer: one fused
    launch per layer over one plan); then truncate, free and reuse pages."""
    rng = np.random.default_rng(92)
    m = MirrorQ8(opts(workloads.GPT2, n_layer=3))
    a, b, c, d = (m.kv.add_seq() for _ in range(4))
    for s, L in zip((a, b, c), (100, 40, 333)):
        m.fill(s, L, rng)
    for rnd in range(3):
        work = [(a, 1, 1), (b, 5, 5), (c, 1, 1), (d, 37, 1 if rnd else 0)]
        rows, qrows = step_rows(m.kv, work)
        n = len(rows)
        q, k, v = (rng.standard_normal((3, n, m.c)).astype(np.float32) for _ in range(3))
        qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
        if per_layer:
            out = torch.zeros_like(qd)
            m.kv.step_begin(work)
            for l in (2, 0, 1):  # any order
                m.kv.step_layer(l, qd[l], kd[l], vd[l], out=out[l])
            m.kv.step_end()
            got = out.cpu().numpy()
        else:
            got = m.kv.step(work, qd, kd, vd).cpu().numpy()
        # the oracle appends with the tables the step reserved
        m.append_oracle(rows, k, v)
        want = m.attention_oracle(rows[qrows], q[:, qrows])
        assert_close(got[:, qrows], want, f"round {rnd}")
        m.check_bytes(rows)
        # verify rollback: keep 2 of b's 5 rows
        m.kv.truncate(b, m.kv.seq_len(b) - 3)
    m.kv.free_seq(c)
    e = m.kv.add_seq()
    m.fill(e, 50, rng)  # reuses c's pages
    rows = [(e, 49), (a, m.kv.seq_len(a) - 1)]
    q = rng.standard_normal((3, 2, m.c)).astype(np.float32)
    got = m.kv.attention(torch.from_numpy(q).cuda(), rows).cpu().numpy()
    assert_close(got, m.attention_oracle(rows, q), "after reuse")


def test_q8_verify_groups_per_layer_wide(gpu, oracle_lib):
    """A verify step on a Q8 cache one launch per layer: 24 sequences x 12
    heads = 288 units of 5-row groups, enough for 8-wave workgroups sharing
    each item's pages (no partitions); every layer against the oracle, then
    the appended bytes."""
    rng = np.random.default_rng(93)
    m = MirrorQ8(opts(workloads.GPT2, n_layer=2, max_seqs=24, kv_blocks=800))
    seqs = [m.kv.add_seq() for _ in range(24)]
    for s in seqs:
        m.fill(s, int(rng.integers(20, 400)), rng)
    work = [(s, 5, 5) for s in seqs]
    rows, qrows = step_rows(m.kv, work)
    q, k, v = (rng.standard_normal((2, len(rows), m.c)).astype(np.float32) for _ in range(3))
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
    out = torch.zeros_like(qd)
    m.kv.step_begin(work)
    for l in range(2):
        m.kv.step_layer(l, qd[l], kd[l], vd[l], out=out[l])
    m.kv.step_end()
    got = out.cpu().numpy()
    m.append_oracle(rows, k, v)
    assert_close(got[:, qrows], m.attention_oracle(rows[qrows], q[:, qrows]), "wide Q8 groups")
    m.check_bytes(rows)


def test_q8_rows_per_layer_wide_with_orphans(gpu, oracle_lib):
    """One launch per layer on a Q8 cache with 48 sequences x 12 heads = 576
    units of single rows (wide workgroups sharing each item's pages): decode
    rows, prompt chunks queried at their last row, and chunks of sequences
    without a query (appended by the launch's extra blocks); every layer
    against the oracle, then the stored bytes of every appended row."""
    rng = np.random.default_rng(94)
    m = MirrorQ8(opts(workloads.GPT2, n_layer=2, max_seqs=48, kv_blocks=1600))
    seqs = [m.kv.add_seq() for _ in range(48)]
    for i, s in enumerate(seqs):
        if i % 6:
            m.fill(s, int(rng.integers(16, 500)), rng)
    for rnd in range(2):
        work = []
        for i, s in enumerate(seqs):
            if i % 6 == 0:
                work.append((s, 37, 1 if i % 12 else 0))  # a prompt chunk: queried at its last row, or not at all
            else:
                work.append((s, 1, 1))
        rows, qrows = step_rows(m.kv, work)
        q, k, v = (rng.standard_normal((2, len(rows), m.c)).astype(np.float32) for _ in range(3))
        qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
        out = torch.zeros_like(qd)
        m.kv.step_begin(work)
        for l in range(2):
            m.kv.step_layer(l, qd[l], kd[l], vd[l], out=out[l])
        m.kv.step_end()
        got = out.cpu().numpy()
        m.append_oracle(rows, k, v)
        assert_close(got[:, qrows], m.attention_oracle(rows[qrows], q[:, qrows]), f"wide Q8 rows round {rnd}")
        m.check_bytes(rows)


def test_q8_refusals(gpu):
    kv = na.PagedKv(na.BatchOpts(n_layer=1, n_head=2, head_dim=64, kv_blocks=8, max_seqs=2, n_ctx=64, q8=True))
    s = kv.add_seq()
    kv.reserve(s, 4)
    with pytest.raises(na.KvError, match="ni_kv_gather_q8"):
        kv.gather([(s, 0)])
    w = torch.zeros((384, 64), device="cuda")
    with pytest.raises(na.KvError, match="Q8 cache"):
        kv.qkv_append([(s, 0)], torch.zeros((1, 64), device="cuda"), w)
    f16 = na.PagedKv(na.BatchOpts(n_layer=1, n_head=2, head_dim=64, kv_blocks=8, max_seqs=2, n_ctx=64))
    t = f16.add_seq()
    f16.reserve(t, 4)
    with pytest.raises(na.KvError, match="not a Q8 cache"):
        f16.gather_q8([(t, 0)])
    assert kv.kv_block_bytes() * 2 < f16.kv_block_bytes() * 1.1


def test_q8_prompt_chunk_steps(gpu, oracle_lib):
    """A Q8 step of prompt chunks only, every sequence queried at more than
    16 rows, over at least 1536 (sequence, layer, head) units: the prefill
    launch quantises and appends each sequence's rows before its groups read
    them (no append launch); int8 values and scales bit for bit."""
    rng = np.random.default_rng(95)
    n_fill = 61
    m = MirrorQ8(opts(workloads.GPT2, n_layer=2, max_rows=2100, kv_blocks=600, max_seqs=3 + n_fill))
    a, b, c = (m.kv.add_seq() for _ in range(3))
    fill = [m.kv.add_seq() for _ in range(n_fill)]
    m.fill(b, 90, rng)
    work = [(a, 512, 512), (b, 200, 100), (c, 50, 20)] + [(s, 17 + i % 9, 17 + i % 9) for i, s in enumerate(fill)]
    assert len(work) * 2 * 12 >= 1536
    rows, qrows = step_rows(m.kv, work)
    q, k, v = (rng.standard_normal((2, len(rows), m.c)).astype(np.float32) for _ in range(3))
    m.kv.profile([0])
    got = m.kv.step(work, *(torch.from_numpy(x).cuda() for x in (q, k, v))).cpu().numpy()
    _, n_app = m.kv.profile_read(0)
    m.kv.profile([])
    assert n_app == 0
    m.append_oracle(rows, k, v)
    want = m.attention_oracle(rows[qrows], q[:, qrows])
    err = assert_close(got[:, qrows], want, "q8 prompt chunks")
    m.check_bytes(rows)
    say(f"q8 prompt chunks: max abs err {err:.2e}")
    # Three sequences (72 units): an append launch, then the groups.
    work = [(a, 40, 40), (b, 30, 20), (c, 18, 18)]
    rows, qrows = step_rows(m.kv, work)
    q, k, v = (rng.standard_normal((2, len(rows), m.c)).astype(np.float32) for _ in range(3))
    m.kv.profile([0])
    got = m.kv.step(work, *(torch.from_numpy(x).cuda() for x in (q, k, v))).cpu().numpy()
    _, n_app = m.kv.profile_read(0)
    m.kv.profile([])
    assert n_app == 1
    m.append_oracle(rows, k, v)
    assert_close(got[:, qrows], m.attention_oracle(rows[qrows], q[:, qrows]), "q8 prompt chunks, 3 sequences")
    m.check_bytes(rows)
