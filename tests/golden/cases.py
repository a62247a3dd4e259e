"""Golden cases: seeded inputs and results for config 1 (the reference's
CPU-runnable case), config 2 and a small speculative-verify trace with page
reuse.

Each case is written once, against a small backend interface (add_seq,
free_seq, truncate, fill, step, block tables, gathers).  ``make_golden.py``
runs the cases on the oracle backends below and writes the records as JSON
beside this file; ``tests/test_golden.py`` checks that the oracle still
reproduces them bit for bit, and ``tests/test_gpu_golden.py`` runs the same
cases on the device through the C ABI and checks block tables, free counts
and gathered f16 K/V bit for bit, attention outputs within the 1e-3 bound.

Record fields: ``exact`` entries must match bit for bit on every backend;
``approx`` entries hold attention outputs -- ``out_sha256`` (exact on the
oracle only), per-layer ``sum`` with ``bound`` = sum over the values of
1e-3 + 1e-3*|want| (a device within the bound everywhere is within it in
total), and a ``slice``: the first 8 dims of the first, middle and last
queried rows of the first and last layer.

Config 1's oracle is the reference's own CPU cache (contiguous
[layer][head][pos][dim] f16, ``kv16.rs:33-58,168-204``); the device runs it
through paged block tables, so the case also pins "paged through any table
= contiguous cache".
"""
from __future__ import annotations

import hashlib

import numpy as np

import oracle
from nanoinfer_amd import workloads

ATOL = 1e-3
RTOL = 1e-3
KV_BLOCK = 16


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


class InputLog:
    """Seeded f32 N(0,1) draws, hashed in draw order (pins the generator)."""

    def __init__(self, seed: int):
        self.rng = np.random.default_rng(seed)
        self.h = hashlib.sha256()

    def normal(self, shape) -> np.ndarray:
        a = self.rng.standard_normal(shape, dtype=np.float32)
        self.h.update(a.tobytes())
        return a

    def digest(self) -> str:
        return self.h.hexdigest()


def step_rows(seq_len, work):
    """(seq, pos) of every row of a step in work order, and the queried row
    indices (the last n_query rows of each item), batch.rs:259-315."""
    rows, qrows = [], []
    for seq, n_new, n_q in work:
        L = seq_len(seq)
        for i in range(n_new):
            if i >= n_new - n_q:
                qrows.append(len(rows))
            rows.append((seq, L + i))
    return rows, qrows


def slice_index(n_layer: int, n_rows: int):
    """(layers, rows) of the values a record keeps verbatim."""
    return [0, n_layer - 1], sorted({0, n_rows // 2, n_rows - 1})


def out_summary(out: np.ndarray, qrows) -> dict:
    """out [n_layer][rows][C]; only queried rows carry attention."""
    o = np.ascontiguousarray(out[:, qrows, :])
    d = o.astype(np.float64)
    sl = o[np.ix_(*slice_index(o.shape[0], len(qrows)))][:, :, :8]
    return {
        "out_sha256": sha(o),
        "sum": [float(x) for x in d.sum(axis=(1, 2))],
        "bound": [float(x) for x in (ATOL + RTOL * np.abs(d)).sum(axis=(1, 2))],
        "slice": [[[float(x) for x in r] for r in lay] for lay in sl],
    }


# ------------------------------------------------------------ oracle backends

class PagedOracle:
    """The oracle allocator (batch.rs:129-254) and paged pools
    (batch.rs:166, batch.metal:24-26,329-424)."""

    def __init__(self, shape, kv_blocks, max_seqs, n_ctx, order=None):
        self.L, self.H, self.D = shape["n_layer"], shape["n_head"], shape["head_dim"]
        self.C = self.H * self.D
        self.alloc = oracle.Alloc(kv_blocks, max_seqs, n_ctx, order)
        self.pools = oracle.PagedPools(self.L, kv_blocks, self.C)
        self.mb = self.alloc.max_blocks

    def add_seq(self):
        return self.alloc.add_seq()

    def free_seq(self, s):
        self.alloc.free_seq(s)

    def truncate(self, s, n):
        self.alloc.truncate(s, n)

    def seq_len(self, s):
        return self.alloc.seq_len(s)

    def block_table(self, s):
        return self.alloc.block_table(s)

    def free_block_count(self):
        return self.alloc.free_block_count()

    def _append(self, rows, k, v):
        rows = np.asarray(rows, np.uint32).reshape(-1, 2)
        t = self.alloc.table()
        for l in range(self.L):
            oracle.paged_append(self.pools, l, t, self.mb, rows[:, 0], rows[:, 1], k[l], v[l])

    def fill(self, s, k, v):
        """Append positions seq_len.. (k/v [n_layer][n][C]) and commit."""
        n = k.shape[1]
        L0 = self.seq_len(s)
        assert self.alloc.ensure(s, L0 + n) == 0
        self._append([(s, L0 + i) for i in range(n)], k, v)
        self.alloc.commit(s, n)

    def step(self, work, q, k, v):
        rows, qrows = step_rows(self.seq_len, work)
        for seq, n_new, _ in work:
            assert self.alloc.ensure(seq, self.seq_len(seq) + n_new) == 0
        self._append(rows, k, v)
        out = np.zeros_like(q)
        r = np.asarray(rows, np.uint32).reshape(-1, 2)
        if qrows:
            t = self.alloc.table()
            for l in range(self.L):
                out[l][qrows] = oracle.paged_attention(self.pools, l, t, self.mb, r[qrows, 0], r[qrows, 1],
                                                       q[l][qrows], self.H, self.D)
        for seq, n_new, _ in work:
            self.alloc.commit(seq, n_new)
        return out, qrows

    def kv_sha(self, seqs) -> str:
        """Hash of every stored K/V row of the sequences, per seq, per layer,
        K then V, in the reference's row layout [pos][C]."""
        h = hashlib.sha256()
        t = self.alloc.table()
        for s in seqs:
            n = self.seq_len(s)
            for l in range(self.L):
                kg, vg = oracle.paged_gather(self.pools, l, t, self.mb, np.full(n, s), np.arange(n))
                h.update(kg.tobytes())
                h.update(vg.tobytes())
        return h.hexdigest()


class ContiguousOracle:
    """The reference's CPU cache, one sequence: k/v [layer][head][cap][dim]
    f16 (kv16.rs:33-58), append by narrow (kv16.rs:61-82,246-258), attention
    by kv16::attention (kv16.rs:168-204).  No pages: tables are empty."""

    def __init__(self, shape, capacity):
        self.L, self.H, self.D = shape["n_layer"], shape["n_head"], shape["head_dim"]
        self.C = self.H * self.D
        self.cap = capacity
        self.k = np.zeros((self.L, self.H, capacity, self.D), np.uint16)
        self.v = np.zeros_like(self.k)
        self.n = 0

    def add_seq(self):
        return 0

    def seq_len(self, s):
        return self.n

    def step(self, work, q, k, v):
        (seq, n_new, n_q), = work
        assert n_q == n_new
        p0 = self.n
        qrows = list(range(n_new))
        out = np.zeros_like(q)
        for l in range(self.L):
            self.k[l][:, p0:p0 + n_new] = oracle.f32_to_f16(k[l]).reshape(n_new, self.H, self.D).transpose(1, 0, 2)
            self.v[l][:, p0:p0 + n_new] = oracle.f32_to_f16(v[l]).reshape(n_new, self.H, self.D).transpose(1, 0, 2)
            qkv = np.concatenate([q[l], k[l], v[l]], axis=1)
            out[l] = oracle.kv16_attention(qkv, self.k[l], self.v[l], self.cap, n_new, p0, self.H, self.D)
        self.n += n_new
        return out, qrows

    def kv_sha(self, seqs) -> str:
        h = hashlib.sha256()
        for _ in seqs:
            for l in range(self.L):
                h.update(np.ascontiguousarray(self.k[l][:, :self.n].transpose(1, 0, 2)).tobytes())
                h.update(np.ascontiguousarray(self.v[l][:, :self.n].transpose(1, 0, 2)).tobytes())
        return h.hexdigest()


# ---------------------------------------------------------------------- cases
# Each case takes a backend factory make(shape, kv_blocks, max_seqs, n_ctx,
# order) and returns its record.

CONFIG1 = dict(seed=1, prefill=64, decode=64)


def config1(make) -> dict:
    """Benchmark configuration 1: one sequence, prefill 64 positions (all queried,
    causal), then 64 decode steps of one row each; qkv f32 N(0,1) from seed 1
    drawn as [layer][rows][3C] per step (the reference's fused QKV rows)."""
    shape = workloads.GPT2
    C = shape["n_head"] * shape["head_dim"]
    n_ctx = CONFIG1["prefill"] + CONFIG1["decode"]
    kv = make(shape, kv_blocks=n_ctx // KV_BLOCK, max_seqs=1, n_ctx=n_ctx, order=None)
    inp = InputLog(CONFIG1["seed"])
    s = kv.add_seq()
    steps = []
    for n in [CONFIG1["prefill"]] + [1] * CONFIG1["decode"]:
        qkv = inp.normal((shape["n_layer"], n, 3 * C))
        q, k, v = qkv[:, :, :C], qkv[:, :, C:2 * C], qkv[:, :, 2 * C:]
        out, qrows = kv.step([(s, n, n)], q, k, v)
        steps.append({"approx": out_summary(out, qrows)})
    return {"case": "config1", "inputs_sha256": inp.digest(), "steps": steps,
            "exact": {"seq_len": kv.seq_len(s), "kv_sha256": kv.kv_sha([s])}}


def config2(make) -> dict:
    """Benchmark configuration 2: 16 sequences, context U[64,1024] after the step
    (XorShift seed 2), pages from a seeded permutation of a 1024-page pool;
    fill ctx-1 positions per sequence, then one step appending one row per
    sequence and querying it.  k/v/q f32 N(0,1), seed 2."""
    shape = workloads.GPT2
    ctx, order = workloads.config2_contexts()
    kv = make(shape, kv_blocks=1024, max_seqs=16, n_ctx=1024, order=order)
    inp = InputLog(2)
    seqs = [kv.add_seq() for _ in ctx]
    L, C = shape["n_layer"], shape["n_head"] * shape["head_dim"]
    for s, n in zip(seqs, ctx):
        k = inp.normal((L, n - 1, C))
        v = inp.normal((L, n - 1, C))
        kv.fill(s, k, v)
    q, k, v = (inp.normal((L, len(seqs), C)) for _ in range(3))
    out, qrows = kv.step([(s, 1, 1) for s in seqs], q, k, v)
    return {"case": "config2", "inputs_sha256": inp.digest(), "ctx": list(ctx),
            "order_sha256": sha(np.asarray(order, np.uint32)),
            "steps": [{"approx": out_summary(out, qrows)}],
            "exact": {"tables": [kv.block_table(s) for s in seqs], "free": kv.free_block_count(),
                      "seq_len": [kv.seq_len(s) for s in seqs], "kv_sha256": kv.kv_sha(seqs)}}


SPEC = dict(seed=9, n_seqs=4, ctx=(128, 256), pool=80, drafts=4, rounds=3)


def spec_verify(make) -> dict:
    """A small config-5 trace: 4 sequences, context U[128,256] (XorShift seed
    9), an 80-page pool handed out in a seeded permutation; 3 verify rounds
    (append g + 4 drafts, 5 causal queries each, accept U[0,4] with
    SpecVerify's seed, truncate, metal_spec.rs:118-169); then sequence 1
    retires, a new sequence reuses its slot and freed pages with a 37-row
    prompt chunk whose last row is queried, beside one decode row for each
    other sequence (metal_serve.rs:255-363)."""
    shape = workloads.GPT2
    L, C = shape["n_layer"], shape["n_head"] * shape["head_dim"]
    rng = workloads.XorShift.seeded(SPEC["seed"])
    ctx = [rng.range(*SPEC["ctx"]) for _ in range(SPEC["n_seqs"])]
    order = rng.permutation(SPEC["pool"])
    kv = make(shape, kv_blocks=SPEC["pool"], max_seqs=SPEC["n_seqs"], n_ctx=512, order=order)
    inp = InputLog(SPEC["seed"])
    seqs = [kv.add_seq() for _ in ctx]
    for s, n in zip(seqs, ctx):
        kv.fill(s, inp.normal((L, n, C)), inp.normal((L, n, C)))
    sv = workloads.SpecVerify(kv, seqs, k=SPEC["drafts"], seed=55)
    steps = []
    for _ in range(SPEC["rounds"]):
        st = sv.plan()
        work = [tuple(int(x) for x in w) for w in st.work]
        n = sum(w[1] for w in work)
        q, k, v = (inp.normal((L, n, C)) for _ in range(3))
        out, qrows = kv.step(work, q, k, v)
        accs = sv.commit()
        steps.append({"approx": out_summary(out, qrows),
                      "exact": {"accepted": accs, "seq_len": [kv.seq_len(s) for s in seqs],
                                "tables": [kv.block_table(s) for s in seqs], "free": kv.free_block_count()}})
    kv.free_seq(seqs[1])
    s_new = kv.add_seq()
    work = [(s_new, 37, 1)] + [(s, 1, 1) for s in seqs if s != seqs[1]]
    n = sum(w[1] for w in work)
    q, k, v = (inp.normal((L, n, C)) for _ in range(3))
    out, qrows = kv.step(work, q, k, v)
    live = [s_new] + [s for s in seqs if s != seqs[1]]
    steps.append({"approx": out_summary(out, qrows),
                  "exact": {"new_seq": s_new, "seq_len": [kv.seq_len(s) for s in live],
                            "tables": [kv.block_table(s) for s in live], "free": kv.free_block_count()}})
    return {"case": "spec_verify", "inputs_sha256": inp.digest(), "ctx": ctx, "steps": steps,
            "exact": {"kv_sha256": kv.kv_sha(live)}}


CASES = {"config1": config1, "config2": config2, "spec_verify": spec_verify}


def oracle_backend(case: str):
    """The backend factory each case's fixture was generated with."""
    if case == "config1":
        return lambda shape, kv_blocks, max_seqs, n_ctx, order: ContiguousOracle(shape, n_ctx)
    return lambda shape, kv_blocks, max_seqs, n_ctx, order: PagedOracle(shape, kv_blocks, max_seqs, n_ctx, order)
