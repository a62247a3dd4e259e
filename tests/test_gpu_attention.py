"""Paged split-K decode attention on the device against the oracle
(kv16.rs:144-164 over kv_slot, batch.metal:349-424), within the north
star's 1e-3 max-abs / 1e-3 relative; closed forms and invariances exactly."""
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


def opts(shape, **kw):
    base = dict(**shape, kv_blocks=256, max_seqs=8, n_ctx=2048, max_rows=512)
    base.update(kw)
    return na.BatchOpts(**base)


@pytest.mark.parametrize("shape", [workloads.GPT2, dict(n_layer=2, n_head=4, head_dim=128)], ids=["hd64", "hd128"])
@pytest.mark.parametrize("split", [0, 64, 128, 512])
def test_decode_contexts(gpu, oracle_lib, shape, split):
    rng = np.random.default_rng(20)
    m = Mirror(opts(shape, page_order=rng.permutation(256).tolist()))
    lens = [1, 15, 16, 17, 65, 300, 1023, 1024]
    seqs = [m.kv.add_seq() for _ in lens]
    for s, L in zip(seqs, lens):
        m.fill(s, L, rng)
    rows = [(s, L - 1) for s, L in zip(seqs, lens)]
    q = rng.standard_normal((shape["n_layer"], len(rows), m.c)).astype(np.float32)
    got, want = m.attention(rows, q, split_tokens=split)
    err = assert_close(got, want, f"split {split}")
    say(f"{shape} split {split}: max abs err {err:.2e}")


@pytest.mark.parametrize("shape", [workloads.GPT2, dict(n_layer=2, n_head=4, head_dim=128)], ids=["hd64", "hd128"])
@pytest.mark.parametrize("nq", [2, 5, 8, 13, 16, 17, 20, 33, 64, 65, 100, 200])
def test_causal_groups(gpu, oracle_lib, shape, nq):
    """nq consecutive rows of one sequence (g + drafts, prefill chunks) attend
    causally and share their K/V reads; rows straddle page and partition
    edges.  Up to 16 rows run as one matrix-core group, 17..64 as one
    prefill group (attn_prefill_kernel), longer runs as several prefill
    groups."""
    rng = np.random.default_rng(21 + nq)
    m = Mirror(opts(shape))
    for split in (0, 64, 128):
        for L in sorted({nq, nq + 1, 14 + nq, 16, 62, 127, 130, 512}):
            if L < nq:
                continue
            s = m.kv.add_seq()
            m.fill(s, L, rng)
            rows = [(s, p) for p in range(L - nq, L)]
            q = rng.standard_normal((shape["n_layer"], nq, m.c)).astype(np.float32)
            got, want = m.attention(rows, q, split_tokens=split)
            assert_close(got, want, f"nq {nq} L {L} split {split}")
            m.kv.free_seq(s)


@pytest.mark.parametrize("shape", [dict(n_layer=1, n_head=12, head_dim=64), dict(n_layer=1, n_head=4, head_dim=128)],
                         ids=["hd64", "hd128"])
@pytest.mark.parametrize("sharp", [1.0, 8.0])
@pytest.mark.parametrize("nq", [16, 64])
def test_group_precision(gpu, oracle_lib, shape, sharp, nq):
    """Query groups keep f32-level accuracy on the matrix cores (q and p are
    split into f16 hi + scaled lo parts), also with sharply peaked scores
    where most weights are tiny: max error well under the 1e-3 bound.  16
    rows run on attn_mfma_kernel, 64 on attn_prefill_kernel."""
    rng = np.random.default_rng(41)
    m = Mirror(opts(shape))
    s = m.kv.add_seq()
    L = 900
    m.fill(s, L, rng)
    rows = [(s, p) for p in range(L - nq, L)]
    q = (rng.standard_normal((1, nq, m.c)) * sharp).astype(np.float32)
    got, want = m.attention(rows, q, split_tokens=0)
    err = float(np.abs(got - want).max())
    # The same queries one row at a time run on the vector kernel (f32
    # throughout): the group may differ from the oracle by f32 summation
    # order only, like the vector kernel does.
    qd = torch.from_numpy(q).cuda()
    single = np.concatenate([m.kv.attention(qd[:, i:i + 1].contiguous(), [rows[i]], split_tokens=0).cpu().numpy()
                             for i in range(nq)], axis=1)
    err1 = float(np.abs(single - want).max())
    say(f"{shape} sharp {sharp} nq {nq}: group max abs err {err:.2e}, one row at a time {err1:.2e}")
    assert_close(got, want, "group")
    assert err <= 4 * err1 + 2e-6


def test_mixed_rows_and_long_groups(gpu, oracle_lib):
    """Decode rows, a 5-row group (matrix-core group kernel) and a 20-row
    group (prefill kernel, a second launch) in one call, rows interleaved."""
    rng = np.random.default_rng(22)
    m = Mirror(opts(workloads.GPT2))
    a, b, c = m.kv.add_seq(), m.kv.add_seq(), m.kv.add_seq()
    m.fill(a, 200, rng)
    m.fill(b, 77, rng)
    m.fill(c, 900, rng)
    rows = [(a, 199)] + [(b, p) for p in range(72, 77)] + [(c, p) for p in range(880, 900)] + [(a, 150)]
    q = rng.standard_normal((12, len(rows), m.c)).astype(np.float32)
    for split in (0, 128):
        got, want = m.attention(rows, q, split_tokens=split)
        assert_close(got, want, f"split {split}")


def test_single_key_copies_value(gpu, oracle_lib):
    """reference.rs:188-199 on the device: one key -> out == v exactly."""
    rng = np.random.default_rng(23)
    m = Mirror(opts(workloads.GPT2))
    s = m.kv.add_seq()
    m.fill(s, 1, rng)
    q = rng.standard_normal((12, 1, m.c)).astype(np.float32)
    got, want = m.attention([(s, 0)], q)
    (kg, vg), _ = m.gather([(s, 0)])
    assert np.array_equal(got, vg.view(np.float16).astype(np.float32))
    assert np.array_equal(got, want)


def test_identical_keys_give_mean(gpu, oracle_lib):
    rng = np.random.default_rng(24)
    m = Mirror(opts(workloads.GPT2, n_layer=1))
    s = m.kv.add_seq()
    L = 333
    m.kv.reserve(s, L)
    k = np.tile(rng.standard_normal((1, 1, m.c)).astype(np.float32), (1, L, 1))
    v = rng.standard_normal((1, L, m.c)).astype(np.float32)
    m.append([(s, p) for p in range(L)], k, v)
    m.kv.commit(s, L)
    q = rng.standard_normal((1, 1, m.c)).astype(np.float32)
    got, _ = m.attention([(s, L - 1)], q, split_tokens=64)
    mean = oracle.f16_to_f32(oracle.f32_to_f16(v[0])).astype(np.float64).mean(0)
    assert np.abs(got[0, 0] - mean).max() < 1e-5


def test_split_size_invariance(gpu, oracle_lib):
    """The log-sum-exp merge: every partition size gives the same output
    (to f32 rounding)."""
    rng = np.random.default_rng(25)
    m = Mirror(opts(dict(n_layer=1, n_head=4, head_dim=128), n_ctx=4096, kv_blocks=300))
    s = m.kv.add_seq()
    m.fill(s, 4000, rng, chunk=512)
    q = rng.standard_normal((1, 1, m.c)).astype(np.float32)
    outs = []
    for split in (64, 128, 512, 1024, 4096):
        outs.append(m.kv.attention(torch.from_numpy(q).cuda(), [(s, 3999)], split_tokens=split).cpu().numpy())
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() < 1e-5


def test_batch_invariance(gpu, oracle_lib):
    """A sequence's output is bit-identical alone or batched with others
    (fixed partition size), as the reference's batch tests require of its
    kernels (crates/metal/tests/batch.rs:82-111)."""
    rng = np.random.default_rng(26)
    m = Mirror(opts(workloads.GPT2))
    seqs = [m.kv.add_seq() for _ in range(5)]
    lens = [100, 513, 64, 999, 7]
    for s, L in zip(seqs, lens):
        m.fill(s, L, rng)
    rows = [(s, L - 1) for s, L in zip(seqs, lens)]
    q = rng.standard_normal((12, len(rows), m.c)).astype(np.float32)
    qd = torch.from_numpy(q).cuda()
    together = m.kv.attention(qd, rows, split_tokens=128).cpu().numpy()
    for i, r in enumerate(rows):
        alone = m.kv.attention(qd[:, i:i + 1].contiguous(), [r], split_tokens=128).cpu().numpy()
        assert np.array_equal(alone[:, 0], together[:, i])


def test_config2_full_size(gpu, oracle_lib):
    """Config 2: 16 sequences, contexts U[64,1024], pages from a seeded
    permutation of a 1024-page pool; append 1 token each, then attention."""
    ctx, order = workloads.config2_contexts()
    m = Mirror(na.BatchOpts(**workloads.GPT2, kv_blocks=1024, max_seqs=16, n_ctx=1024, page_order=order))
    rng = np.random.default_rng(27)
    seqs = [m.kv.add_seq() for _ in ctx]
    for s, L in zip(seqs, ctx):
        m.fill(s, L - 1, rng, chunk=512)
    from paged_mirror import mirror_step

    work = [(s, 1, 1) for s in seqs]
    n = len(work)
    q, k, v = (rng.standard_normal((12, n, m.c)).astype(np.float32) for _ in range(3))
    got, want, qrows = mirror_step(m, work, q, k, v)
    err = assert_close(got[:, qrows], want[:, qrows], "config 2")
    say(f"config 2: max abs err {err:.2e}")
    assert [m.kv.seq_len(s) for s in seqs] == ctx


def test_config4_full_size(gpu, oracle_lib):
    """Config 4: batch 4, 32 heads x 128, context 32768, random page tables,
    512-token partitions + LSE merge; k/v ~ N(0, 0.5), q ~ N(0, 1)."""
    B, L = 4, 32768
    order = workloads.XorShift.seeded(4).permutation(B * L // 16)
    m = Mirror(na.BatchOpts(**workloads.LONG, kv_blocks=B * L // 16, max_seqs=B, n_ctx=L, max_rows=4096,
                            page_order=order))
    rng = np.random.default_rng(28)
    seqs = [m.kv.add_seq() for _ in range(B)]
    for s in seqs:
        m.fill(s, L, rng, std=0.5, chunk=4096)
        say(f"config 4: filled seq {s}")
    rows = [(s, L - 1) for s in seqs]
    q = rng.standard_normal((1, B, m.c)).astype(np.float32)
    got, want = m.attention(rows, q, split_tokens=512)
    err = assert_close(got, want, "config 4")
    say(f"config 4: max abs err {err:.2e}")


def test_wide_workgroups(gpu, oracle_lib):
    """Launches of single rows with 512..2047 (item, layer, head) units run
    wide workgroups (kWideWaves waves) sharing each item's pages (no
    partitions, no merge launch): per-layer decode of 48 sequences (576 units), all layers of 30
    sequences (720) and a fused step of 30 decode rows plus a mid-prompt
    chunk (orphan rows), against the oracle."""
    rng = np.random.default_rng(31)
    shape = dict(n_layer=2, n_head=12, head_dim=64)
    m = Mirror(opts(shape, kv_blocks=1400, max_seqs=48, n_ctx=1024))
    seqs = [m.kv.add_seq() for _ in range(48)]
    lens = np.concatenate([[1, 2, 16, 17, 33, 400], rng.integers(3, 401, 42)])
    for s, L in zip(seqs, lens):
        m.fill(s, int(L), rng)
    m.kv.profile([1, 2])
    rows = [(s, int(L) - 1) for s, L in zip(seqs, lens)]
    for layer in (0, 1):
        q = rng.standard_normal((len(rows), m.c)).astype(np.float32)
        got, want = m.attention(rows, q, layer=layer)
        assert_close(got, want, f"per-layer {layer}")
    q = rng.standard_normal((2, 30, m.c)).astype(np.float32)
    got, want = m.attention(rows[:30], q)
    assert_close(got, want, "all layers, 30 sequences")
    # fused step: decode rows of 30 sequences, 40 rows of a prompt without a query
    work = [(s, 1, 1) for s in seqs[:30]] + [(seqs[40], 40, 0)]
    srows, _ = step_rows(m.kv, work)
    n = len(srows)
    q, k, v = (rng.standard_normal((2, n, m.c)).astype(np.float32) for _ in range(3))
    got, want, qr = mirror_step(m, work, q, k, v)
    assert_close(got[:, qr], want[:, qr], "fused step")
    (kg, vg), (kw, vw) = m.gather(srows)
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)
    _, n_attn = m.kv.profile_read(1)
    _, n_merge = m.kv.profile_read(2)
    m.kv.profile([])
    assert n_attn == 4 and n_merge == 0, (n_attn, n_merge)
    say("wide workgroups: per-layer, all-layer and fused launches within bounds, no merge launches")




@pytest.mark.parametrize("shape", [dict(n_layer=3, n_head=12, head_dim=64), dict(n_layer=2, n_head=4, head_dim=128)],
                         ids=["hd64", "hd128"])
@pytest.mark.parametrize("per_layer", [False, True], ids=["all_layers", "per_layer"])
def test_prompt_chunk_steps(gpu, oracle_lib, shape, per_layer):
    """Steps whose every sequence is queried at more than 16 rows (prompt
    chunks, the reference's all_logits) on an f16 pool: an append launch,
    then the groups of 17..64 rows on the prefill kernel (a last group of up
    to 16 rows on the group kernel).  Chunks from empty and after existing context, queried
    at every row or at the last rows only, 17..512 queried rows, plus 39
    short prompts of 17..24 rows; every row gathered bit for bit; then a
    step with a decode row mixed in and automatic partitions.  (On Q8 pools
    the prefill launch appends the rows itself: test_gpu_q8.)"""
    rng = np.random.default_rng(33)
    n_fill = 39
    m = Mirror(opts(shape, kv_blocks=600, n_ctx=1024, max_rows=2048, max_seqs=4 + n_fill))
    a, b, c, d = (m.kv.add_seq() for _ in range(4))
    fill = [m.kv.add_seq() for _ in range(n_fill)]
    m.fill(b, 100, rng)
    m.fill(d, 40, rng)
    L = shape["n_layer"]
    m.kv.profile([0, 1])
    for work in ([(a, 512, 512), (b, 300, 150), (c, 70, 17), (d, 64, 64)] +
                 [(s, 17 + i % 8, 17 + i % 8) for i, s in enumerate(fill)],
                 [(a, 33, 33), (b, 20, 17), (c, 100, 80), (d, 20, 17)] + [(s, 20, 17) for s in fill]):
        srows, _ = step_rows(m.kv, work)
        q, k, v = (rng.standard_normal((L, len(srows), m.c)).astype(np.float32) for _ in range(3))
        # the automatic split: prefill groups are not split to fill the GPU
        # (a last group of up to 16 rows may be, in the group kernel's launch)
        got, want, qr = mirror_step(m, work, q, k, v, per_layer=per_layer)
        err = assert_close(got[:, qr], want[:, qr], f"{len(work)} sequences")
        (kg, vg), (kw, vw) = m.gather(srows)
        assert np.array_equal(kg, kw) and np.array_equal(vg, vw)
        _, n_app = m.kv.profile_read(0)
        _, n_attn = m.kv.profile_read(1)
        launches = L if per_layer else 1
        # (a last group of up to 16 rows runs in a group-kernel launch of its own)
        assert n_app == launches and n_attn in (launches, 2 * launches), (n_app, n_attn)
        say(f"{shape} per_layer {per_layer} {len(work)} sequences: max abs err {err:.2e}")
    work = [(a, 1, 1), (c, 40, 40)]
    srows, _ = step_rows(m.kv, work)
    q, k, v = (rng.standard_normal((L, len(srows), m.c)).astype(np.float32) for _ in range(3))
    got, want, qr = mirror_step(m, work, q, k, v, per_layer=per_layer)
    assert_close(got[:, qr], want[:, qr], "mixed")
    (kg, vg), (kw, vw) = m.gather(srows)
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)
    m.kv.profile([])
