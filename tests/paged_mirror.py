"""Test helper: drive the GPU library and the CPU oracle side by side.

``Mirror`` owns a device ``PagedKv`` and oracle pools in the reference's
layout ([layer][page][16][C], batch.rs:166).  Every append goes to both (same
f32 inputs, same pages: the oracle reads the product's block tables); every
attention call returns the device result and the oracle's
(kv16.rs:144-164 over the keys kv_slot finds).
"""
from __future__ import annotations

import numpy as np
import torch

import oracle
import nanoinfer_amd as na

ATOL = 1e-3  # the north star's bound: 1e-3 max-abs / 1e-3 relative
RTOL = 1e-3


def assert_close(got: np.ndarray, want: np.ndarray, what: str = ""):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = ATOL + RTOL * np.abs(want.astype(np.float64))
    bad = err > bound
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert not bad.any(), f"{what}: {bad.sum()} values off, max abs err {err.max():.3e}"
    return float(err.max()) if err.size else 0.0


class Mirror:
    def __init__(self, opts: na.BatchOpts):
        self.opts = opts
        self.kv = na.PagedKv(opts)
        self.c = opts.n_head * opts.head_dim
        self.pools = oracle.PagedPools(opts.n_layer, opts.kv_blocks, self.c)

    def table(self) -> np.ndarray:
        mb = self.kv.max_blocks
        t = np.zeros((self.opts.max_seqs, mb), np.uint32)
        for s in range(self.opts.max_seqs):
            bt = self.kv.block_table(s)
            t[s, : len(bt)] = bt
        return t

    # ------------------------------------------------------------- appends
    def append(self, rows, k: np.ndarray, v: np.ndarray, layer=na.ALL_LAYERS):
        """rows [(seq, pos)]; k/v [n_layer][n][C] (or [n][C] for one layer)."""
        rows = np.asarray(rows, np.uint32).reshape(-1, 2)
        kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
        self.kv.append(rows, kd, vd, layer=layer)
        t = self.table()
        layers = range(self.opts.n_layer) if layer == na.ALL_LAYERS else [layer]
        for i, l in enumerate(layers):
            kl = k[i] if layer == na.ALL_LAYERS else k
            vl = v[i] if layer == na.ALL_LAYERS else v
            oracle.paged_append(self.pools, l, t, self.kv.max_blocks, rows[:, 0], rows[:, 1], kl, vl)

    def fill(self, seq: int, length: int, rng: np.random.Generator, std: float = 1.0, chunk: int = 256):
        """Reserve and append positions seq_len .. length-1 with random K/V."""
        start = self.kv.seq_len(seq)
        self.kv.reserve(seq, length)
        for p0 in range(start, length, chunk):
            p1 = min(length, p0 + chunk)
            n = p1 - p0
            rows = np.stack([np.full(n, seq), np.arange(p0, p1)], 1)
            shape = (self.opts.n_layer, n, self.c)
            k = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)
            v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)
            self.append(rows, k, v)
        self.kv.commit(seq, length - start)

    # ----------------------------------------------------------- attention
    def attention(self, rows, q: np.ndarray, split_tokens: int = 0, layer=na.ALL_LAYERS):
        """Device and oracle outputs ([n_layer][n][C] or [n][C])."""
        rows = np.asarray(rows, np.uint32).reshape(-1, 2)
        qd = torch.from_numpy(q).cuda()
        got = self.kv.attention(qd, rows, layer=layer, split_tokens=split_tokens)
        torch.cuda.synchronize()
        got = got.cpu().numpy()
        t = self.table()
        want = np.zeros_like(q)
        layers = range(self.opts.n_layer) if layer == na.ALL_LAYERS else [layer]
        for i, l in enumerate(layers):
            ql = q[i] if layer == na.ALL_LAYERS else q
            w = oracle.paged_attention(self.pools, l, t, self.kv.max_blocks, rows[:, 0], rows[:, 1], ql,
                                       self.opts.n_head, self.opts.head_dim)
            if layer == na.ALL_LAYERS:
                want[i] = w
            else:
                want[:] = w
        return got, want

    def gather(self, rows, layer=na.ALL_LAYERS):
        """Device gather (f16 bits as uint16) and the oracle's."""
        rows = np.asarray(rows, np.uint32).reshape(-1, 2)
        ks, vs = [], []
        step = self.opts.max_rows
        for i in range(0, len(rows), step):  # one call holds at most max_rows rows
            kd, vd = self.kv.gather(rows[i:i + step], layer=layer)
            ks.append(kd.cpu().numpy().view(np.uint16))
            vs.append(vd.cpu().numpy().view(np.uint16))
        axis = 1 if layer == na.ALL_LAYERS else 0
        kg = np.concatenate(ks, axis)
        vg = np.concatenate(vs, axis)
        t = self.table()
        layers = range(self.opts.n_layer) if layer == na.ALL_LAYERS else [layer]
        kw = np.zeros_like(kg)
        vw = np.zeros_like(vg)
        for i, l in enumerate(layers):
            a, b = oracle.paged_gather(self.pools, l, t, self.kv.max_blocks, rows[:, 0], rows[:, 1])
            if layer == na.ALL_LAYERS:
                kw[i], vw[i] = a, b
            else:
                kw[:], vw[:] = a, b
        return (kg, vg), (kw, vw)


def step_rows(kv, work):
    """Rows (seq, pos) of a ni_kv_step work list in row order, the queried
    row indices, from the sequences' lengths before the step."""
    rows, qrows = [], []
    for seq, n_new, n_q in np.asarray(work, np.int64).reshape(-1, 3):
        L = kv.seq_len(int(seq))
        for i in range(int(n_new)):
            if i >= n_new - n_q:
                qrows.append(len(rows))
            rows.append((int(seq), L + i))
    return np.asarray(rows, np.uint32).reshape(-1, 2), np.asarray(qrows, np.int64)


def mirror_step(m: "Mirror", work, q: np.ndarray, k: np.ndarray, v: np.ndarray, split_tokens: int = 0,
                per_layer: bool = False):
    """ni_kv_step on the device (per_layer: ni_kv_step_begin, one
    ni_kv_step_layer per layer, ni_kv_step_end) and the same step on the
    oracle; returns (device out, oracle out, queried rows)."""
    rows, qrows = step_rows(m.kv, work)
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
    if per_layer:
        out = torch.zeros_like(qd)
        m.kv.step_begin(work, split_tokens=split_tokens)
        for l in range(m.opts.n_layer):
            m.kv.step_layer(l, qd[l], kd[l], vd[l], out=out[l])
        m.kv.step_end()
    else:
        out = m.kv.step(work, qd, kd, vd, split_tokens=split_tokens)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    t = m.table()
    want = np.zeros_like(q)
    for l in range(m.opts.n_layer):
        oracle.paged_append(m.pools, l, t, m.kv.max_blocks, rows[:, 0], rows[:, 1], k[l], v[l])
        if len(qrows):
            want[l][qrows] = oracle.paged_attention(m.pools, l, t, m.kv.max_blocks, rows[qrows, 0], rows[qrows, 1],
                                                    q[l][qrows], m.opts.n_head, m.opts.head_dim)
    return got, want, qrows
