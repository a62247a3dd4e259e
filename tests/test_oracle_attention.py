"""Pins the oracle's exp and attention functions.

Sources of truth, none of them the oracle's own formula retyped:
* the reference's tests: fastops.rs:219-236 (exp vs std), fastops.rs:238-253
  (fast attention vs ground truth), attn_neon.rs:149-166 (head_dim 64 path vs
  ground truth), reference.rs:170-176 (softmax sums to 1), reference.rs:188-199
  (one key -> out == v);
* closed forms: identical keys give mean(V); a float64 numpy softmax-attention
  on tiny inputs;
* the log-sum-exp identity: the split/merge of batch.metal:349-424 with any
  partition size equals the unsplit softmax.
"""
import math

import numpy as np
import pytest

import oracle


def det(i):
    """The reference tests' deterministic vectors: ((i*7919) % 13)/6 - 1."""
    i = np.asarray(i, dtype=np.int64)
    return (((i * 7919) % 13).astype(np.float32) / np.float32(6.0) - np.float32(1.0)).astype(np.float32)


def np_attention(q, k, v, n_q, q_pos0, n_head, hd):
    """float64 closed form: softmax(q k^T / sqrt(hd)) v, causal."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    c = n_head * hd
    out = np.zeros((n_q, c))
    for i in range(n_q):
        n_kv = q_pos0 + i + 1
        for h in range(n_head):
            sl = slice(h * hd, (h + 1) * hd)
            s = k[:n_kv, sl] @ q[i, sl] / math.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[i, sl] = p @ v[:n_kv, sl]
    return out


def test_fast_exp_matches_std(oracle_lib):
    # fastops.rs:219-236 (the reference compares with Rust's f32 exp; here with
    # the correctly rounded double exp, a stricter reference).
    worst = 0.0
    for i in range(-20000, 20001):
        x = np.float32(i / 1000.0)
        e = math.exp(float(x))
        worst = max(worst, abs(oracle.fast_exp(float(x)) - e) / e)
    for i in range(-860, 1):
        x = np.float32(i / 10.0)
        e = math.exp(float(x))
        worst = max(worst, abs(oracle.fast_exp(float(x)) - e) / max(e, 1.1754944e-38))
    assert worst < 2e-6, worst
    assert oracle.fast_exp(0.0) == 1.0


def test_softmax_sums_to_one(oracle_lib):
    # reference.rs:170-176.
    x = oracle.softmax([1.0, 2.0, 3.0, 1000.0])
    assert abs(float(x.sum()) - 1.0) < 1e-6
    assert x[3] > 0.999


def test_single_key_copies_value(oracle_lib):
    # reference.rs:188-199.
    out = oracle.reference_attention(np.array([[0.3, -0.2]]), np.array([[0.5, 0.5]]), np.array([[7.0, 8.0]]), 1, 0,
                                     1, 2)
    assert np.array_equal(out[0], np.array([7.0, 8.0], np.float32))
    # The f16 unit: fast_exp(0) == 1 and p/total == 1, so out == v exactly.
    rng = np.random.default_rng(1)
    for hd in (8, 64, 128):
        q = rng.standard_normal(hd).astype(np.float32)
        k16 = oracle.f32_to_f16(rng.standard_normal(hd))
        v16 = oracle.f32_to_f16(rng.standard_normal(hd))
        out = oracle.attend_f16_portable(q, k16, v16, 1)
        assert np.array_equal(out, oracle.f16_to_f32(v16))


def test_fastops_attention_matches_reference(oracle_lib):
    # fastops.rs:238-253.
    n_head, hd, n_q, pos0 = 3, 8, 5, 7
    c = n_head * hd
    n_kv = pos0 + n_q
    q = det(np.arange(n_q * c)).reshape(n_q, c)
    k = det(np.arange(n_kv * c) + 3).reshape(n_kv, c)
    v = det(np.arange(n_kv * c) + 11).reshape(n_kv, c)
    a = oracle.reference_attention(q, k, v, n_q, pos0, n_head, hd)
    b = oracle.fastops_attention(q, k, v, n_q, pos0, n_head, hd)
    assert np.abs(a - b).max() < 1e-5
    assert np.abs(a - np_attention(q, k, v, n_q, pos0, n_head, hd)).max() < 1e-5


@pytest.mark.parametrize("n_q,pos0", [(1, 0), (1, 37), (3, 10)])
def test_f16_path_matches_reference_hd64(oracle_lib, n_q, pos0):
    # attn_neon.rs:149-166, for the f16 CPU path of kv16.rs:144-204: K/V go
    # through the f16 cache; the ground truth sees the same f16 values.
    n_head, hd = 3, 64
    c = n_head * hd
    n_kv = pos0 + n_q
    q = det(np.arange(n_q * c)).reshape(n_q, c)
    k = det(np.arange(n_kv * c) + 3).reshape(n_kv, c)
    v = det(np.arange(n_kv * c) + 11).reshape(n_kv, c)
    k16, v16 = oracle.f32_to_f16(k), oracle.f32_to_f16(v)
    kw, vw = oracle.f16_to_f32(k16), oracle.f16_to_f32(v16)
    a = oracle.reference_attention(q, kw, vw, n_q, pos0, n_head, hd)
    # head-major cache [n_head][cap][hd] (kv16.rs:33-58), qkv rows of 3C
    cap = n_kv
    kc = np.ascontiguousarray(k16.reshape(n_kv, n_head, hd).transpose(1, 0, 2))
    vc = np.ascontiguousarray(v16.reshape(n_kv, n_head, hd).transpose(1, 0, 2))
    qkv = np.zeros((n_q, 3 * c), np.float32)
    qkv[:, :c] = q
    b = oracle.kv16_attention(qkv, kc, vc, cap, n_q, pos0, n_head, hd)
    assert np.abs(a - b).max() < 1e-5


def test_identical_keys_give_mean_value(oracle_lib):
    rng = np.random.default_rng(2)
    hd, n = 64, 37
    q = rng.standard_normal(hd).astype(np.float32)
    k16 = np.tile(oracle.f32_to_f16(rng.standard_normal(hd)), (n, 1))
    v16 = oracle.f32_to_f16(rng.standard_normal((n, hd)))
    out = oracle.attend_f16_portable(q, k16, v16, n)
    want = oracle.f16_to_f32(v16).astype(np.float64).mean(0)
    assert np.abs(out - want).max() < 1e-5


def test_f16_unit_matches_float64_closed_form(oracle_lib):
    rng = np.random.default_rng(3)
    for hd, n in [(8, 1), (8, 5), (64, 100), (128, 300)]:
        q = rng.standard_normal(hd).astype(np.float32)
        k16 = oracle.f32_to_f16(rng.standard_normal((n, hd)))
        v16 = oracle.f32_to_f16(rng.standard_normal((n, hd)))
        out = oracle.attend_f16_portable(q, k16, v16, n)
        want = np_attention(q[None], oracle.f16_to_f32(k16), oracle.f16_to_f32(v16), 1, n - 1, 1, hd)[0]
        assert np.abs(out - want).max() < 1e-5, (hd, n)


def test_split_merge_identity(oracle_lib):
    # batch.metal:349-424: split-K with any partition size == unsplit softmax.
    rng = np.random.default_rng(4)
    for hd, n in [(64, 1), (64, 63), (64, 65), (64, 1000), (128, 2049)]:
        q = rng.standard_normal(hd).astype(np.float32)
        k = rng.standard_normal((n, hd)).astype(np.float32)
        v = rng.standard_normal((n, hd)).astype(np.float32)
        whole = oracle.split_attention_f64(q, k, v, 0)
        closed = np_attention(q[None], k, v, 1, n - 1, 1, hd)[0]
        assert np.abs(whole - closed).max() < 1e-12
        for part in (16, 64, 100, 512):
            got = oracle.split_attention_f64(q, k, v, part)
            assert np.abs(got - whole).max() <= 1e-12 * max(1.0, np.abs(whole).max()), (hd, n, part)


def test_closed_form_catches_a_dropped_scale(oracle_lib):
    # The closed-form check is strong enough to see a plausible mistake: the
    # same attention without the 1/sqrt(hd) scale (planted here, on the CPU).
    rng = np.random.default_rng(5)
    hd, n = 64, 50
    q = rng.standard_normal(hd).astype(np.float32)
    k16 = oracle.f32_to_f16(rng.standard_normal((n, hd)))
    v16 = oracle.f32_to_f16(rng.standard_normal((n, hd)))
    good = oracle.attend_f16_portable(q, k16, v16, n)
    wrong = oracle.attend_f16_portable(q * np.float32(math.sqrt(hd)), k16, v16, n)
    want = np_attention(q[None], oracle.f16_to_f32(k16), oracle.f16_to_f32(v16), 1, n - 1, 1, hd)[0]
    assert np.abs(good - want).max() < 1e-5
    assert np.abs(wrong - want).max() > 1e-2
