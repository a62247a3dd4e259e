"""The oracle's Q8 cache (kv8.metal:15-95 restated in C) pinned without
the reference: known answers of the rounding rule, invariants a wrong scale,
sign or rounding breaks, numpy's float32 arithmetic as an independent
restatement, and Q8 attention reducing to the pinned f16 attention when the
scales are 1."""
import numpy as np

import oracle


def test_q8_known_answers(oracle_lib):
    x = np.zeros(64, np.float32)
    x[:7] = [127, -127, 0.5, 1.5, 2.5, -0.5, 63.5]
    q, s = oracle.q8_quantize(x)
    assert s == np.float32(1.0)
    assert q[:7].tolist() == [127, -127, 0, 2, 2, 0, 64]  # rint: half to even
    assert not q[7:].any()
    q, s = oracle.q8_quantize(np.zeros(64, np.float32))
    assert s == 0 and not q.any()  # amax 0: inverse 0, all zero


def test_q8_invariants(oracle_lib):
    rng = np.random.default_rng(80)
    for it in range(200):
        x = (rng.standard_normal(64) * rng.choice([1e-3, 1.0, 300.0])).astype(np.float32)
        q, s = oracle.q8_quantize(x)
        amax = np.abs(x).max()
        assert s == np.float32(amax / np.float32(127))
        assert np.abs(q).max() == 127 and abs(int(q[np.abs(x).argmax()])) == 127
        assert (np.abs(x - q.astype(np.float64) * s) <= 0.5 * s * (1 + 1e-5)).all()
        qn, sn = oracle.q8_quantize(-x)
        assert sn == s and np.array_equal(qn, -q)
        # numpy's float32 arithmetic, independently
        inv = np.float32(1) / np.float32(s)
        want = np.clip(np.rint(x * inv), -127, 127).astype(np.int8)
        assert np.array_equal(q, want)


def test_q8_attention_reduces_to_f16_attention(oracle_lib):
    """Integer-valued K/V with amax 127 quantise exactly (scale 1): Q8
    attention equals the f16 attention oracle over the same values."""
    rng = np.random.default_rng(81)
    H, D, L = 2, 64, 40
    C = H * D
    pools8 = oracle.PagedPoolsQ8(1, 8, H, D)
    pools16 = oracle.PagedPools(1, 8, C)
    table = np.zeros((1, 8), np.uint32)
    table[0, :3] = [5, 2, 7]
    k = rng.integers(-126, 127, (L, C)).astype(np.float32)
    v = rng.integers(-126, 127, (L, C)).astype(np.float32)
    k[:, ::D] = 127  # amax 127 in every (position, head)
    v[:, ::D] = -127
    seqs = np.zeros(L, np.uint32)
    poss = np.arange(L, dtype=np.uint32)
    oracle.paged_q8_append(pools8, 0, table, 8, seqs, poss, k, v)
    oracle.paged_append(pools16, 0, table, 8, seqs, poss, k, v)
    (kq, vq), (ks, vs) = oracle.paged_q8_gather(pools8, 0, table, 8, seqs, poss)
    assert (ks == 1).all() and (vs == 1).all() and np.array_equal(kq, k.astype(np.int8))
    q = (rng.standard_normal((3, C)) * 0.01).astype(np.float32)
    rows_p = np.array([0, 17, 39], np.uint32)
    got = oracle.paged_q8_attention(pools8, 0, table, 8, np.zeros(3, np.uint32), rows_p, q)
    want = oracle.paged_attention(pools16, 0, table, 8, np.zeros(3, np.uint32), rows_p, q, H, D)
    assert np.abs(got - want).max() < 1e-3 * np.abs(want).max()


def _np_attention_f64(q, k, v, n_kv, n_head, hd):
    """Softmax attention of one row over keys 0..n_kv-1 in float64 (the
    mathematics kv8.metal:50-95 computes: scores (q.k)/sqrt(hd), then the
    probability-weighted sum of V)."""
    out = np.zeros(n_head * hd)
    for h in range(n_head):
        sl = slice(h * hd, (h + 1) * hd)
        s = (k[:n_kv, sl] @ q[sl].astype(np.float64)) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[sl] = (p / p.sum()) @ v[:n_kv, sl]
    return out


def test_q8_attention_matches_float64_with_spread_scales(oracle_lib):
    """Scales spread over 1e-3..30 per (position, head), different for K and
    V: the oracle's Q8 attention equals a float64 closed form over the
    dequantised values kq*ks and vq*vs.  Two planted mistakes (on the CPU,
    in the pools the oracle reads): key scales dropped, value scales
    dropped -- each must move the result far outside the tolerance."""
    rng = np.random.default_rng(82)
    H, D, L, P = 3, 64, 150, 16
    C = H * D
    pages = -(-L // 16)
    pools = oracle.PagedPoolsQ8(1, 32, H, D)
    table = np.zeros((1, 32), np.uint32)
    table[0, :pages] = rng.permutation(32)[:pages]
    # per (position, head) target scales log-uniform in [1e-3, 30]
    sk = np.exp(rng.uniform(np.log(1e-3), np.log(30), (L, H)))
    sv = np.exp(rng.uniform(np.log(1e-3), np.log(30), (L, H)))
    k = (rng.uniform(-1, 1, (L, H, D)) * 127 * sk[:, :, None]).astype(np.float32).reshape(L, C)
    v = (rng.uniform(-1, 1, (L, H, D)) * 127 * sv[:, :, None]).astype(np.float32).reshape(L, C)
    seqs = np.zeros(L, np.uint32)
    poss = np.arange(L, dtype=np.uint32)
    oracle.paged_q8_append(pools, 0, table, 32, seqs, poss, k, v)
    (kq, vq), (ks, vs) = oracle.paged_q8_gather(pools, 0, table, 32, seqs, poss)
    assert ks.min() < 3e-3 and ks.max() > 10 and vs.min() < 3e-3 and vs.max() > 10
    kd = (kq.reshape(L, H, D).astype(np.float64) * ks[:, :, None]).reshape(L, C)
    vd = (vq.reshape(L, H, D).astype(np.float64) * vs[:, :, None]).reshape(L, C)
    # dequantised values are within half a step of the inputs (the scales are real)
    assert (np.abs(kd - k).reshape(L, H, D) <= 0.5 * ks[:, :, None] * (1 + 1e-5)).all()
    rows_p = np.array([0, 15, 16, 77, L - 1], np.uint32)
    q = (rng.standard_normal((len(rows_p), C)) * 0.02).astype(np.float32)
    want = np.stack([_np_attention_f64(q[i], kd, vd, int(p) + 1, H, D) for i, p in enumerate(rows_p)])
    tol = lambda w: 1e-6 * np.abs(w).max() + 1e-6 * np.abs(w)  # noqa: E731
    got = oracle.paged_q8_attention(pools, 0, table, 32, np.zeros(len(rows_p), np.uint32), rows_p, q)
    assert (np.abs(got - want) <= tol(want)).all(), np.abs(got - want).max()
    # planted: the oracle reading every key scale as 1
    ks_saved, vs_saved = pools.ks.copy(), pools.vs.copy()
    pools.ks[:] = 1.0
    bad = oracle.paged_q8_attention(pools, 0, table, 32, np.zeros(len(rows_p), np.uint32), rows_p, q)
    assert np.abs(bad - want).max() > 100 * tol(want).max()
    # planted: the oracle reading every value scale as 1
    pools.ks[:], pools.vs[:] = ks_saved, 1.0
    bad = oracle.paged_q8_attention(pools, 0, table, 32, np.zeros(len(rows_p), np.uint32), rows_p, q)
    assert np.abs(bad - want).max() > 100 * tol(want).max()
    pools.vs[:] = vs_saved
    again = oracle.paged_q8_attention(pools, 0, table, 32, np.zeros(len(rows_p), np.uint32), rows_p, q)
    assert np.array_equal(again, got)
