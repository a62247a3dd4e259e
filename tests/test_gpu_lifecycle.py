"""Page free/reuse, rollback and whole steps on the device.

Restates, at kernel level, the reference's batch tests
(crates/metal/tests/batch.rs:82-143: page reuse after free_seq, truncate then
continue) and runs scaled-down continuous-batching (metal_serve.rs:255-363)
and speculative-verify (metal_spec.rs:118-169) traces through ni_kv_step,
checking every step against the oracle.
"""
import sys

import numpy as np
import pytest
import torch

import oracle
import nanoinfer_amd as na
from nanoinfer_amd import _abi, workloads
from paged_mirror import Mirror, assert_close, mirror_step

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def gpt2(**kw):
    base = dict(**workloads.GPT2, kv_blocks=128, max_seqs=8, n_ctx=1024, max_rows=512)
    base.update(kw)
    return na.BatchOpts(**base)


def fill_with(kv, seq, k, v):
    """Reserve, append and commit given K/V [n_layer][L][C] to a fresh seq."""
    L = k.shape[1]
    kv.reserve(seq, L)
    kv.append([(seq, p) for p in range(L)], torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    kv.commit(seq, L)


def test_page_reuse_matches_fresh_cache(gpu):
    """batch.rs:112-120: free two sequences, start a new one on their pages;
    its attention equals the same K/V in a fresh cache, bit for bit."""
    rng = np.random.default_rng(30)
    kv = na.PagedKv(gpt2())
    seqs = [kv.add_seq() for _ in range(4)]
    for s in seqs:
        L = int(rng.integers(50, 200))
        fill_with(kv, s, rng.standard_normal((12, L, 768)).astype(np.float32),
                  rng.standard_normal((12, L, 768)).astype(np.float32))
    freed = set(kv.block_table(seqs[0])) | set(kv.block_table(seqs[2]))
    kv.free_seq(seqs[0])
    kv.free_seq(seqs[2])
    L = 150
    k = rng.standard_normal((12, L, 768)).astype(np.float32)
    v = rng.standard_normal((12, L, 768)).astype(np.float32)
    s = kv.add_seq()
    fill_with(kv, s, k, v)
    assert set(kv.block_table(s)) <= freed  # it really runs on recycled pages
    q = torch.from_numpy(rng.standard_normal((12, 3, 768)).astype(np.float32)).cuda()
    rows = [(s, 49), (s, 148), (s, 149)]
    reused = kv.attention(q, rows, split_tokens=64).cpu().numpy()
    fresh_kv = na.PagedKv(gpt2())
    t = fresh_kv.add_seq()
    fill_with(fresh_kv, t, k, v)
    fresh = fresh_kv.attention(q, [(t, p) for _, p in rows], split_tokens=64).cpu().numpy()
    assert np.array_equal(reused, fresh)


def test_truncate_rollback_matches_sequential(gpu):
    """batch.rs:127-143: append drafts, roll back with truncate, continue; the
    result equals a cache that never saw the rejected drafts."""
    rng = np.random.default_rng(31)
    kv = na.PagedKv(gpt2())
    s = kv.add_seq()
    base_k = rng.standard_normal((12, 100, 768)).astype(np.float32)
    base_v = rng.standard_normal((12, 100, 768)).astype(np.float32)
    fill_with(kv, s, base_k, base_v)
    drafts_k = rng.standard_normal((12, 5, 768)).astype(np.float32)
    drafts_v = rng.standard_normal((12, 5, 768)).astype(np.float32)
    q5 = torch.from_numpy(rng.standard_normal((12, 5, 768)).astype(np.float32)).cuda()
    kv.step([(s, 5, 5)], q5, torch.from_numpy(drafts_k).cuda(), torch.from_numpy(drafts_v).cuda())
    assert kv.seq_len(s) == 105
    kv.truncate(s, 102)  # keep g + 1 accepted draft
    assert len(kv.block_table(s)) == 7
    new_k = rng.standard_normal((12, 5, 768)).astype(np.float32)
    new_v = rng.standard_normal((12, 5, 768)).astype(np.float32)
    out = kv.step([(s, 5, 5)], q5, torch.from_numpy(new_k).cuda(), torch.from_numpy(new_v).cuda(),
                  split_tokens=64).cpu().numpy()
    ref = na.PagedKv(gpt2())
    t = ref.add_seq()
    fill_with(ref, t, np.concatenate([base_k, drafts_k[:, :2]], 1), np.concatenate([base_v, drafts_v[:, :2]], 1))
    want = ref.step([(t, 5, 5)], q5, torch.from_numpy(new_k).cuda(), torch.from_numpy(new_v).cuda(),
                    split_tokens=64).cpu().numpy()
    assert np.array_equal(out, want)


@pytest.mark.parametrize("per_layer", [False, True], ids=["all_layers", "per_layer"])
@pytest.mark.parametrize("prefill_queries", ["all", "last"])
def test_continuous_batching_trace(gpu, oracle_lib, prefill_queries, per_layer):
    """Scaled config 3: Poisson arrivals, admission by free pages, decode rows
    plus budgeted prefill chunks, retire and reuse pages; every step checked
    against the oracle.  "all": attention at every prefill row (many query
    groups per sequence, separate append launch); "last": only the row that
    ends a prompt (the append fused into the attention launch, mid-prompt
    chunks appended by the launch's extra blocks).  per_layer: each step
    planned once and run one launch per layer (ni_kv_step_layer)."""
    rng = np.random.default_rng(32)
    opts = gpt2(kv_blocks=160, max_seqs=8, max_rows=128)
    m = Mirror(opts)
    trace = workloads.ContinuousBatching(m.kv, seed=3, max_batch=8, prompt=(20, 100), out=(3, 12), rate=0.7,
                                         budget=64, max_rows=128, prefill_queries=prefill_queries)
    worst = 0.0
    for step in range(40):
        st = trace.plan()
        n = int(st.work[:, 1].sum())
        q, k, v = (rng.standard_normal((12, n, 768)).astype(np.float32) for _ in range(3))
        got, want, qrows = mirror_step(m, st.work, q, k, v, per_layer=per_layer)
        worst = max(worst, assert_close(got[:, qrows], want[:, qrows], f"step {step}"))
        trace.commit()
    say(f"continuous trace: {trace.done} retired, max abs err {worst:.2e}")
    assert trace.done > 3
    live = [s for s in range(8) if m.kv.is_live(s)]
    rows = [(s, p) for s in live for p in range(m.kv.seq_len(s))]
    (kg, vg), (kw, vw) = m.gather(rows)
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)


@pytest.mark.parametrize("per_layer", [False, True], ids=["all_layers", "per_layer"])
def test_spec_verify_trace(gpu, oracle_lib, per_layer):
    """Scaled config 5: append g + 4 drafts, 5 causal queries, accept
    U[0,4], truncate; pages freed by rollback are reused.  per_layer: each
    step planned once and run one launch per layer."""
    rng = np.random.default_rng(33)
    ctx, _ = workloads.config5_contexts(n_seqs=6, lo=20, hi=300)
    m = Mirror(gpt2(kv_blocks=200, max_seqs=6, n_ctx=1024))
    seqs = [m.kv.add_seq() for _ in ctx]
    for s, L in zip(seqs, ctx):
        m.fill(s, L, rng)
    spec = workloads.SpecVerify(m.kv, seqs, k=4, seed=9)
    for step in range(12):
        st = spec.plan()
        n = int(st.work[:, 1].sum())
        q, k, v = (rng.standard_normal((12, n, 768)).astype(np.float32) for _ in range(3))
        got, want, qrows = mirror_step(m, st.work, q, k, v, per_layer=per_layer)
        assert_close(got[:, qrows], want[:, qrows], f"spec step {step}")
        spec.commit()
    for s in seqs:
        assert len(m.kv.block_table(s)) == -(-m.kv.seq_len(s) // 16)


def test_step_errors_match_reference(gpu):
    kv = na.PagedKv(gpt2(kv_blocks=4, max_seqs=3, n_ctx=40, max_rows=8))
    a, b = kv.add_seq(), kv.add_seq()
    z = torch.zeros((12, 64, 768), device=gpu)

    def step(work):
        n = sum(w[1] for w in work)
        t = z[:, :max(n, 1)].contiguous()
        return kv.step(work, t, t, t)

    with pytest.raises(na.KvError) as e:
        step([(2, 1, 1)])
    assert str(e.value) == "sequence 2 is not live"
    with pytest.raises(na.KvError) as e:
        step([(a, 0, 0)])
    assert str(e.value) == "empty work item"
    with pytest.raises(na.KvError) as e:
        step([(a, 41, 1)])
    assert str(e.value) == "sequence 0: context full (41 > 40)"
    with pytest.raises(na.KvError) as e:
        step([(a, 9, 1)])
    assert str(e.value) == "9 rows > max_rows 8"
    assert kv.seq_len(a) == 0  # nothing committed on error
    step([(a, 8, 1)])
    assert kv.seq_len(a) == 8
    with pytest.raises(na.KvError) as e:
        step([(b, 1, 1), (b, 1, 1)])
    assert e.value.code == _abi.NI_ERR_BAD_ARG  # one sequence twice in a step
    kv.sync()

    small = na.PagedKv(gpt2(kv_blocks=2, max_seqs=3, n_ctx=64, max_rows=64))
    a, b = small.add_seq(), small.add_seq()
    t16 = z[:, :16].contiguous()
    small.step([(a, 16, 1)], t16, t16, t16)
    small.step([(b, 16, 1)], t16, t16, t16)
    t1 = z[:, :1].contiguous()
    with pytest.raises(na.KvError) as e:
        small.step([(a, 1, 1)], t1, t1, t1)
    assert str(e.value) == "KV cache pool exhausted"
    small.free_seq(b)
    small.step([(a, 1, 1)], t1, t1, t1)  # b's page is reused
    assert small.seq_len(a) == 17
    small.sync()


def test_per_layer_step_head_dim_128(gpu, oracle_lib):
    """One launch per layer at head_dim 128 (config 4's head shape): decode
    rows, a 5-row verify group, a queried 40-row prompt chunk (its own launch
    on the prefill path) and a chunk with no query, over contexts that need
    split-K partitions; every layer's output against the oracle and the
    appended rows gathered bit for bit."""
    rng = np.random.default_rng(51)
    opts = na.BatchOpts(n_layer=3, n_head=4, head_dim=128, kv_blocks=400, max_seqs=6, n_ctx=4096, max_rows=256)
    m = Mirror(opts)
    seqs = [m.kv.add_seq() for _ in range(5)]
    for s, L in zip(seqs, (1500, 700, 33, 0, 2100)):
        if L:
            m.fill(s, L, rng)
    for rnd in range(2):
        work = [(seqs[0], 1, 1), (seqs[1], 5, 5), (seqs[2], 40, 40), (seqs[3], 23, 0), (seqs[4], 1, 1)]
        n = sum(w[1] for w in work)
        q, k, v = (rng.standard_normal((3, n, m.c)).astype(np.float32) for _ in range(3))
        got, want, qrows = mirror_step(m, work, q, k, v, split_tokens=512 if rnd else 0, per_layer=True)
        assert_close(got[:, qrows], want[:, qrows], f"head_dim 128 per-layer round {rnd}")
    rows = [(s, p) for s in seqs for p in range(m.kv.seq_len(s))]
    (kg, vg), (kw, vw) = m.gather(rows)
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)
