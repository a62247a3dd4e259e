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
