"""Pins the oracle's paged pieces: kv_slot, append/gather, paged attention and
the page allocator (batch.metal:24-26,329-344; batch.rs:129-254).

* identity tables reduce paging to the contiguous cache (kv_write_h,
  attn.metal:225-236);
* any permuted table gathers back exactly the narrowed rows;
* paged attention equals the contiguous kv16 path on the same values, bit
  for bit (same arithmetic, only the addressing differs);
* the allocator is compared with a brute-force Python model written from the
  reference's behaviour, on random operation sequences, plus invariants.
"""
import numpy as np
import pytest

import oracle

KB = 16


def test_kv_slot_identity_table_is_contiguous(oracle_lib):
    max_blocks, n_seq = 8, 3
    table = np.arange(n_seq * max_blocks, dtype=np.uint32).reshape(n_seq, max_blocks)
    for s in range(n_seq):
        for pos in range(max_blocks * KB):
            assert oracle.kv_slot(table, s, pos, max_blocks) == s * max_blocks * KB + pos


def test_append_gather_any_table(oracle_lib):
    rng = np.random.default_rng(0)
    n_layer, n_head, hd, kv_blocks, max_blocks = 2, 3, 8, 40, 6
    c = n_head * hd
    for trial in range(3):
        table = rng.permutation(kv_blocks)[: 4 * max_blocks].astype(np.uint32).reshape(4, max_blocks)
        pools = oracle.PagedPools(n_layer, kv_blocks, c)
        seqs = rng.integers(0, 4, 50).astype(np.uint32)
        poss = rng.integers(0, max_blocks * KB, 50).astype(np.uint32)
        # unique (seq, pos) so later writes do not overwrite earlier ones
        _, idx = np.unique(seqs.astype(np.int64) * 1000 + poss, return_index=True)
        seqs, poss = seqs[idx], poss[idx]
        k = rng.standard_normal((len(seqs), c)).astype(np.float32)
        v = rng.standard_normal((len(seqs), c)).astype(np.float32)
        for l in range(n_layer):
            oracle.paged_append(pools, l, table, max_blocks, seqs, poss, k + l, v - l)
        for l in range(n_layer):
            kg, vg = oracle.paged_gather(pools, l, table, max_blocks, seqs, poss)
            assert np.array_equal(kg, oracle.f32_to_f16(k + l))
            assert np.array_equal(vg, oracle.f32_to_f16(v - l))


def test_paged_attention_equals_contiguous_kv16(oracle_lib):
    rng = np.random.default_rng(1)
    n_head, hd, kv_blocks = 4, 64, 64
    c = n_head * hd
    n_kv = 150
    max_blocks = 16
    table = rng.permutation(kv_blocks)[:max_blocks].astype(np.uint32)[None]
    pools = oracle.PagedPools(1, kv_blocks, c)
    k = rng.standard_normal((n_kv, c)).astype(np.float32)
    v = rng.standard_normal((n_kv, c)).astype(np.float32)
    oracle.paged_append(pools, 0, table, max_blocks, np.zeros(n_kv, np.uint32), np.arange(n_kv, dtype=np.uint32), k, v)
    n_q, pos0 = 5, n_kv - 5
    q = rng.standard_normal((n_q, c)).astype(np.float32)
    got = oracle.paged_attention(pools, 0, table, max_blocks, np.zeros(n_q, np.uint32),
                                 np.arange(pos0, pos0 + n_q, dtype=np.uint32), q, n_head, hd)
    k16, v16 = oracle.f32_to_f16(k), oracle.f32_to_f16(v)
    kc = np.ascontiguousarray(k16.reshape(n_kv, n_head, hd).transpose(1, 0, 2))
    vc = np.ascontiguousarray(v16.reshape(n_kv, n_head, hd).transpose(1, 0, 2))
    qkv = np.zeros((n_q, 3 * c), np.float32)
    qkv[:, :c] = q
    want = oracle.kv16_attention(qkv, kc, vc, n_kv, n_q, pos0, n_head, hd)
    assert np.array_equal(got, want)


def test_cpu_step_equals_serial_composition(oracle_lib):
    """The threaded baseline computes what the serial pieces compute."""
    rng = np.random.default_rng(2)
    n_layer, n_head, hd, kv_blocks = 2, 3, 64, 32
    c = n_head * hd
    a = oracle.Alloc(kv_blocks, 4, 128)
    seqs, lens = [], [40, 17, 64]
    for L in lens:
        s = a.add_seq()
        assert a.ensure(s, L) == 0
        seqs.append(s)
    rows_s = np.concatenate([np.full(L, s) for s, L in zip(seqs, lens)]).astype(np.uint32)
    rows_p = np.concatenate([np.arange(L) for L in lens]).astype(np.uint32)
    n = len(rows_s)
    q = rng.standard_normal((n_layer, n, c)).astype(np.float32)
    k = rng.standard_normal((n_layer, n, c)).astype(np.float32)
    v = rng.standard_normal((n_layer, n, c)).astype(np.float32)
    qrows = np.array([39, 40 + 16, n - 2, n - 1], np.uint32)
    p1 = oracle.PagedPools(n_layer, kv_blocks, c)
    out1 = np.zeros_like(q)
    oracle.CpuStep(4).run(p1, a.table(), a.max_blocks, rows_s, rows_p, qrows, q, k, v, out1, n_head, hd)
    p2 = oracle.PagedPools(n_layer, kv_blocks, c)
    for l in range(n_layer):
        oracle.paged_append(p2, l, a.table(), a.max_blocks, rows_s, rows_p, k[l], v[l])
        want = oracle.paged_attention(p2, l, a.table(), a.max_blocks, rows_s[qrows], rows_p[qrows], q[l][qrows],
                                      n_head, hd)
        assert np.array_equal(out1[l][qrows], want)
    assert np.array_equal(p1.k, p2.k) and np.array_equal(p1.v, p2.v)


class ModelAlloc:
    """Brute-force model of batch.rs:129-254 written from the reference's
    behaviour, independent of the C restatement."""

    def __init__(self, kv_blocks, max_seqs, n_ctx, order=None):
        self.free = list(reversed(order)) if order is not None else list(range(kv_blocks))[::-1]
        self.blocks = [[] for _ in range(max_seqs)]
        self.len = [0] * max_seqs
        self.live = [False] * max_seqs
        self.n_ctx, self.kv_blocks = n_ctx, kv_blocks

    def add_seq(self):
        for s, l in enumerate(self.live):
            if not l:
                self.live[s] = True
                self.len[s] = 0
                return s
        return None

    def truncate(self, s, n):
        assert n <= self.len[s]
        self.len[s] = n
        keep = -(-n // KB)
        while len(self.blocks[s]) > keep:
            self.free.append(self.blocks[s].pop())

    def free_seq(self, s):
        self.truncate(s, 0)
        self.live[s] = False

    def ensure(self, s, n):
        if n > self.n_ctx:
            return 1
        while len(self.blocks[s]) * KB < n:
            if not self.free:
                return 2
            self.blocks[s].append(self.free.pop())
        return 0


def random_ops(rng, n_ops, max_seqs, n_ctx):
    ops = []
    for _ in range(n_ops):
        r = rng.random()
        s = int(rng.integers(0, max_seqs))
        if r < 0.2:
            ops.append(("add",))
        elif r < 0.3:
            ops.append(("free", s))
        elif r < 0.65:
            ops.append(("grow", s, int(rng.integers(1, 40))))
        elif r < 0.9:
            ops.append(("trunc", s, float(rng.random())))
        else:
            ops.append(("big", s, max(0, int(n_ctx + rng.integers(-20, 20)))))
    return ops


def apply(alloc_ops, a, op):
    """Run one op on an allocator exposing add_seq/free_seq/ensure/truncate/
    seq_len/commit; returns an observable result."""
    kind = op[0]
    if kind == "add":
        return a.add_seq()
    s = op[1]
    if kind == "free":
        a.free_seq(s)
        return None
    if kind in ("grow", "big"):
        if not alloc_ops["live"](a, s):
            return "dead"
        n = alloc_ops["len"](a, s) + op[2] if kind == "grow" else op[2]
        rc = a.ensure(s, n)
        if rc == 0 and n > alloc_ops["len"](a, s):
            alloc_ops["commit"](a, s, n - alloc_ops["len"](a, s))
        return rc
    if kind == "trunc":
        n = int(alloc_ops["len"](a, s) * op[2])
        a.truncate(s, n)
        return None


ORACLE_OPS = {"live": lambda a, s: a.live(s), "len": lambda a, s: a.seq_len(s),
              "commit": lambda a, s, n: a.commit(s, n)}


def model_commit(a, s, n):
    a.len[s] += n


MODEL_OPS = {"live": lambda a, s: a.live[s], "len": lambda a, s: a.len[s], "commit": model_commit}


@pytest.mark.parametrize("seed", range(6))
def test_allocator_matches_model(oracle_lib, seed):
    rng = np.random.default_rng(seed)
    kv_blocks, max_seqs, n_ctx = int(rng.integers(4, 12)), int(rng.integers(1, 5)), int(rng.integers(16, 100))
    order = rng.permutation(kv_blocks).tolist() if seed % 2 else None
    a = oracle.Alloc(kv_blocks, max_seqs, n_ctx, order)
    m = ModelAlloc(kv_blocks, max_seqs, n_ctx, order)
    for op in random_ops(rng, 400, max_seqs, n_ctx):
        assert apply(ORACLE_OPS, a, op) == apply(MODEL_OPS, m, op), op
        tables = [a.block_table(s) for s in range(max_seqs)]
        assert tables == m.blocks
        assert a.free_block_count() == len(m.free)
        # invariants: used + free = pool; no page twice; pages cover the length
        used = [p for t in tables for p in t]
        assert len(used) == len(set(used)) and a.blocks_used() + a.free_block_count() == kv_blocks
        for s in range(max_seqs):
            assert len(tables[s]) * KB >= a.seq_len(s)


def test_truncate_then_regrow_returns_same_pages(oracle_lib):
    a = oracle.Alloc(32, 2, 512, oracle_perm := list(np.random.default_rng(7).permutation(32)))
    s = a.add_seq()
    assert a.ensure(s, 100) == 0
    a.commit(s, 100)
    before = a.block_table(s)
    a.truncate(s, 33)  # keeps ceil(33/16) = 3 pages
    assert a.block_table(s) == before[:3]
    assert a.ensure(s, 100) == 0
    assert a.block_table(s) == before  # LIFO: freed last-first, re-popped in order
    assert len(oracle_perm) == 32
