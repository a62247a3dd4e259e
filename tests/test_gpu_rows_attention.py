"""Contiguous causal attention over f32 K/V rows on the device (ni_attention,
the CPU engine's Kernels::attention, crates/core/src/kernels/mod.rs:86-98)
against the oracle's restatement of reference::attention
(kernels/reference.rs:109-142), within the north star's 1e-3 max-abs /
1e-3 relative; the closed forms of reference.rs:188-199 exactly or to f32
rounding."""
import sys

import numpy as np
import pytest
import torch

import oracle
import nanoinfer_amd as na
from paged_mirror import assert_close

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


@pytest.mark.parametrize("n_head,head_dim", [(12, 64), (4, 128)], ids=["hd64", "hd128"])
@pytest.mark.parametrize("n_q,q_pos0", [(1, 0), (1, 15), (1, 16), (3, 14), (64, 0), (1, 127), (5, 300), (1, 2047)])
def test_matches_reference(gpu, oracle_lib, n_head, head_dim, n_q, q_pos0):
    rng = np.random.default_rng(1000 + n_q * 7 + q_pos0)
    c = n_head * head_dim
    n_kv = q_pos0 + n_q
    q = rng.standard_normal((n_q, c)).astype(np.float32)
    k = rng.standard_normal((n_kv, c)).astype(np.float32)
    v = rng.standard_normal((n_kv, c)).astype(np.float32)
    got = na.attention(*(torch.from_numpy(x).cuda() for x in (q, k, v)), n_q, q_pos0, n_head, head_dim)
    torch.cuda.synchronize()
    want = oracle.reference_attention(q, k, v, n_q, q_pos0, n_head, head_dim)
    err = assert_close(got.cpu().numpy(), want, f"n_q {n_q} q_pos0 {q_pos0}")
    say(f"hd {head_dim} n_q {n_q} q_pos0 {q_pos0}: max abs err {err:.2e}")


def test_fused_qkv_rows(gpu, oracle_lib):
    """q, k and v as views of one fused [n][3C] buffer (the reference's stage
    0 layout, kernels/mod.rs:46-49), out written into a wider buffer."""
    rng = np.random.default_rng(7)
    n_head, hd, n = 12, 64, 64
    c = n_head * hd
    qkv = rng.standard_normal((n, 3 * c)).astype(np.float32)
    d = torch.from_numpy(qkv).cuda()
    out = torch.full((n, 2 * c), 7.0, device="cuda")
    na.attention(d[:, :c], d[:, c:2 * c], d[:, 2 * c:], n, 0, n_head, hd, out=out[:, :c])
    torch.cuda.synchronize()
    want = oracle.reference_attention(qkv[:, :c], qkv[:, c:2 * c], qkv[:, 2 * c:], n, 0, n_head, hd)
    o = out.cpu().numpy()
    assert_close(o[:, :c], want, "fused")
    assert (o[:, c:] == 7.0).all(), "wrote past the output rows' C columns"


def test_closed_forms(gpu, oracle_lib):
    """reference.rs:188-199: one key gives out == v (exactly: its weight is
    exp(0) = 1); identical keys give the mean of V."""
    rng = np.random.default_rng(8)
    n_head, hd = 12, 64
    c = n_head * hd
    q = rng.standard_normal((1, c)).astype(np.float32)
    v = rng.standard_normal((1, c)).astype(np.float32)
    k = rng.standard_normal((1, c)).astype(np.float32)
    got = na.attention(*(torch.from_numpy(x).cuda() for x in (q, k, v)), 1, 0, n_head, hd).cpu().numpy()
    assert np.array_equal(got, v)
    n_kv = 100
    k = np.repeat(rng.standard_normal((1, c)).astype(np.float32), n_kv, axis=0)
    v = rng.standard_normal((n_kv, c)).astype(np.float32)
    got = na.attention(*(torch.from_numpy(x).cuda() for x in (q, k, v)), 1, n_kv - 1, n_head, hd).cpu().numpy()
    np.testing.assert_allclose(got[0], v.astype(np.float64).mean(axis=0), rtol=0, atol=2e-6)


def test_keys_past_the_last_query_unread(gpu, oracle_lib):
    """K/V hold exactly q_pos0 + n_q rows at the end of an allocation whose
    next bytes are NaN: nothing past them may reach the result."""
    rng = np.random.default_rng(9)
    n_head, hd, n_q, q_pos0 = 4, 128, 3, 61
    c = n_head * hd
    n_kv = q_pos0 + n_q
    bk = torch.full((n_kv + 16, c), float("nan"), device="cuda")
    bv = torch.full((n_kv + 16, c), float("nan"), device="cuda")
    k = rng.standard_normal((n_kv, c)).astype(np.float32)
    v = rng.standard_normal((n_kv, c)).astype(np.float32)
    q = rng.standard_normal((n_q, c)).astype(np.float32)
    bk[:n_kv].copy_(torch.from_numpy(k))
    bv[:n_kv].copy_(torch.from_numpy(v))
    got = na.attention(torch.from_numpy(q).cuda(), bk[:n_kv], bv[:n_kv], n_q, q_pos0, n_head, hd).cpu().numpy()
    assert np.isfinite(got).all()
    assert_close(got, oracle.reference_attention(q, k, v, n_q, q_pos0, n_head, hd), "tail")


def test_errors(gpu):
    x = torch.zeros((4, 96 * 2), device="cuda")
    with pytest.raises(na.KvError, match="head_dim 96"):
        na.attention(x, x, x, 1, 0, 2, 96)
    with pytest.raises(ValueError):
        na.attention(x, x[:1], x, 1, 3, 2, 64)  # k too short for q_pos0 + n_q rows
