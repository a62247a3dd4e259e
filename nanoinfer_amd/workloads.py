"""Synthetic workloads of the benchmark configurations and their byte counts.

The drivers restate the reference's serving harnesses on a step clock (one
tick per iteration instead of measured seconds) so that a trace is the same on
every machine:

* ``XorShift`` -- the seeded RNG of ``crates/cli/src/metal_serve.rs:97-111``.
* ``requests`` -- ``metal_serve.rs:113-126`` (Poisson gaps ``-ln(u)/rate``,
  uniform prompt/output lengths).
* ``ContinuousBatching`` -- the admission / iteration / retirement policy of
  ``metal_serve.rs:255-363``: admit while a slot is free and
  ``free_pages >= pages(prompt+1) + live``; one decode row per running
  sequence plus prefill chunks (oldest first) under the token budget; retire
  when ``generated == out_len`` with ``swap_remove``.
* ``SpecVerify`` -- the verify/rollback of ``crates/cli/src/metal_spec.rs:118-169``:
  append ``[g, d1..dk]`` (k+1 rows, causal queries at every row), accept a
  prefix, ``truncate(seq, tlen + 1 + acc)``.

Bulk f32 inputs (q/k/v) come from numpy's seeded PCG64 normal generator: the
reference has no normal sampler, and only the fact that the GPU and the
oracle see the same numbers matters.

``step_bytes`` is the algorithmic byte count the roofline uses (each KV byte
once per step; partials and re-reads are not algorithmic):

    per layer, per sequence s with n_s rows appended and q_s of them queried,
    L_s = context after the append:
        n_s * C * 12            append: read K,V f32, write K,V f16
      + q_s * C * 8             read q f32, write out f32
      + [q_s > 0] * (2 * L_s * C * 2 + ceil(L_s / 16) * 4)
                                read K and V f16 and the page-table entries
"""
from __future__ import annotations

import math
from collections import deque
from dataclasses import dataclass, field

import numpy as np

KV_BLOCK = 16
MASK64 = (1 << 64) - 1


class XorShift:
    """metal_serve.rs:97-111."""

    def __init__(self, state: int):
        self.s = state & MASK64

    @classmethod
    def seeded(cls, seed: int) -> "XorShift":
        """metal_serve.rs:114: Rng(seed * 0x9e3779b97f4a7c15 | 1)."""
        return cls(((seed * 0x9E3779B97F4A7C15) & MASK64) | 1)

    def next(self) -> int:
        s = self.s
        s ^= (s << 13) & MASK64
        s ^= s >> 7
        s ^= (s << 17) & MASK64
        self.s = s
        return s

    def unif(self) -> float:
        return (self.next() >> 11) / float(1 << 53)

    def range(self, lo: int, hi: int) -> int:
        return lo + self.next() % (hi - lo + 1)

    def permutation(self, n: int) -> list:
        """Fisher-Yates shuffle of 0..n-1 (used for seeded page orders)."""
        p = list(range(n))
        for i in range(n - 1, 0, -1):
            j = self.next() % (i + 1)
            p[i], p[j] = p[j], p[i]
        return p


def pages(n: int) -> int:
    return -(-n // KV_BLOCK)


@dataclass
class Req:
    id: int
    arrival: float
    prompt_len: int
    out_len: int


def requests(seed: int, n: int, rate: float, prompt=(32, 512), out=(16, 256), text_len=None):
    """metal_serve.rs:113-126.  The reference also draws a text offset per
    request; the draw is kept (its value is unused) so the stream of random
    numbers is the reference's."""
    rng = XorShift.seeded(seed)
    text_len = text_len or (4 * prompt[1] + 64)
    t = 0.0
    reqs = []
    for i in range(n):
        if rate > 0:
            t += -math.log(max(rng.unif(), 1e-12)) / rate
        pl = rng.range(prompt[0], prompt[1])
        rng.range(0, text_len - pl - 1)
        reqs.append(Req(i, t, pl, rng.range(out[0], out[1])))
    return reqs


@dataclass
class _Live:
    req: int
    seq: int
    prefilled: int = 0
    generated: int = 0


@dataclass
class Step:
    """One iteration: pages freed before it, sequences added, the work."""
    retire: list = field(default_factory=list)   # seqs freed before this step
    admit: list = field(default_factory=list)    # seqs added before this step (expected ids)
    work: np.ndarray = None                      # [n][3] uint32 (seq, n_new, n_query)
    ctx_after: np.ndarray = None                 # [n] context of each work item after the append


class ContinuousBatching:
    """metal_serve.rs:255-363 on a step clock, driving any allocator with
    ``add_seq / free_seq / free_block_count / seq_len`` (the GPU handle, a
    host-only handle or the oracle)."""

    def __init__(self, kv, seed=7, max_batch=64, prompt=(32, 512), out=(16, 256), rate=1.0, budget=256,
                 max_rows=512, n_requests=100000, prefill_queries="last"):
        self.kv = kv
        self.reqs = requests(seed, n_requests, rate, prompt, out)
        self.max_batch, self.budget, self.max_rows = max_batch, budget, max_rows
        self.prefill_queries = prefill_queries
        self.clock = 0.0
        self.next = 0
        self.waiting = deque()
        self.live: list[_Live] = []
        self.done = 0
        self._kinds = None
        self._pending_retire: list = []

    def plan(self) -> Step:
        st = Step(retire=self._pending_retire)
        self._pending_retire = []
        reqs = self.reqs
        while True:
            while self.next < len(reqs) and reqs[self.next].arrival <= self.clock:
                self.waiting.append(self.next)
                self.next += 1
            if not self.live and not self.waiting:
                self.clock = reqs[self.next].arrival
                continue
            break
        while len(self.live) < self.max_batch and self.waiting:
            i = self.waiting[0]
            need = pages(reqs[i].prompt_len + 1) + len(self.live)
            if self.kv.free_block_count() < need:
                break
            self.waiting.popleft()
            seq = self.kv.add_seq()
            if seq is None:
                raise RuntimeError("no sequence slot")
            st.admit.append(seq)
            self.live.append(_Live(i, seq))
        work, kinds = [], []
        decode_rows = 0
        for j, l in enumerate(self.live):
            if l.prefilled == reqs[l.req].prompt_len:
                work.append((l.seq, 1, 1))
                kinds.append((j, False, 1))
                decode_rows += 1
        budget_left = min(self.budget, self.max_rows - decode_rows)
        for j, l in enumerate(self.live):
            p = reqs[l.req].prompt_len
            if l.prefilled < p and budget_left > 0:
                n = min(p - l.prefilled, budget_left)
                last = l.prefilled + n == p
                nq = n if self.prefill_queries == "all" else (1 if last else 0)
                work.append((l.seq, n, nq))
                kinds.append((j, True, n))
                budget_left -= n
        self._kinds = kinds
        st.work = np.asarray(work, dtype=np.uint32).reshape(-1, 3)
        st.ctx_after = np.asarray([self.kv.seq_len(s) + n for s, n, _ in work], dtype=np.int64)
        return st

    def commit(self):
        """After the step ran: advance prompts/outputs, retire finished ones
        (freed before the next step, as the reference does at the end of its
        iteration)."""
        reqs = self.reqs
        for j, is_prefill, n in self._kinds:
            l = self.live[j]
            if is_prefill:
                l.prefilled += n
                if l.prefilled < reqs[l.req].prompt_len:
                    continue
            l.generated += 1
        self.clock += 1.0
        k = 0
        while k < len(self.live):
            l = self.live[k]
            if l.generated == reqs[l.req].out_len:
                self.kv.free_seq(l.seq)
                self._pending_retire.append(l.seq)
                self.live[k] = self.live[-1]
                self.live.pop()
                self.done += 1
            else:
                k += 1


def step_bytes(work: np.ndarray, ctx_after: np.ndarray, n_layer: int, c: int) -> dict:
    """Algorithmic bytes of one step (module docstring), split per kernel."""
    work = np.asarray(work, dtype=np.int64).reshape(-1, 3)
    ctx = np.asarray(ctx_after, dtype=np.int64)
    n_new, n_q = work[:, 1], work[:, 2]
    queried = n_q > 0
    append = int(n_new.sum()) * c * 12
    attn = int(n_q.sum()) * c * 8 + int((2 * ctx[queried] * c * 2).sum() + (((ctx[queried] + 15) // 16) * 4).sum())
    return {"append": append * n_layer, "attention": attn * n_layer, "total": (append + attn) * n_layer,
            "seq_tokens": int(queried.sum())}


def normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


# Shapes of the benchmark configurations.
GPT2 = dict(n_layer=12, n_head=12, head_dim=64)
LONG = dict(n_layer=1, n_head=32, head_dim=128)


def config2_contexts(seed: int = 2, n_seqs: int = 16, lo: int = 64, hi: int = 1024):
    """Config 2: context lengths uniform in [lo, hi] (after the step's
    append) and a seeded permutation of the 1024-page pool."""
    rng = XorShift.seeded(seed)
    ctx = [rng.range(lo, hi) for _ in range(n_seqs)]
    order = rng.permutation(1024)
    return ctx, order


def config5_contexts(seed: int = 5, n_seqs: int = 32, lo: int = 128, hi: int = 1024):
    """Config 5: per-sequence context before the verify step, uniform in
    [lo, hi]."""
    rng = XorShift.seeded(seed)
    return [rng.range(lo, hi) for _ in range(n_seqs)], rng


class SpecVerify:
    """metal_spec.rs:118-169, verify side only: each round appends
    [g, d1..dk] (k+1 rows, all queried) to every sequence, then keeps
    g + acc accepted drafts with acc ~ U[0, k] (seeded) and truncates."""

    def __init__(self, kv, seqs, k: int = 4, seed: int = 55, window=None):
        """``window``: once a sequence has grown more than ``window`` rows
        past its context at construction, it is truncated back to that
        context after the round (a request ends and the next one with the
        same prompt length takes its slot), so a long run stays at the
        drawn contexts.  None: sequences grow without bound."""
        self.kv, self.seqs, self.k = kv, list(seqs), k
        self.rng = XorShift.seeded(seed)
        self.window = window
        self._base = [kv.seq_len(s) for s in self.seqs]
        self._tlen = None

    def plan(self) -> Step:
        self._tlen = [self.kv.seq_len(s) for s in self.seqs]
        work = np.asarray([(s, self.k + 1, self.k + 1) for s in self.seqs], dtype=np.uint32).reshape(-1, 3)
        ctx = np.asarray([t + self.k + 1 for t in self._tlen], dtype=np.int64)
        return Step(work=work, ctx_after=ctx)

    def commit(self) -> list:
        """Roll back the rejected drafts: truncate(seq, tlen + 1 + acc).
        Returns the accepted counts."""
        accs = []
        for s, t, b in zip(self.seqs, self._tlen, self._base):
            acc = self.rng.range(0, self.k)
            self.kv.truncate(s, t + 1 + acc)
            if self.window is not None and t + 1 + acc > b + self.window:
                self.kv.truncate(s, b)
            accs.append(acc)
        return accs
