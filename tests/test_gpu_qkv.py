"""The QKV projection with the append in its epilogue (ni_kv_qkv_append,
the reference's BEPI_QKV epilogue, batch.metal:94-165) on the device.

* ni_kv_qkv_project (the same kernel, every column to f32) is within f32
  rounding of the oracle's double-precision matvec.
* ni_kv_qkv_append stores exactly f32_to_f16 of those f32 k/v columns in the
  rows' page slots (bit for bit, through the gather), returns the same q
  columns bit for bit, and attention over the stored K/V matches the oracle.
"""
import sys

import numpy as np
import pytest
import torch

import oracle
import nanoinfer_amd as na
from nanoinfer_amd import workloads
from paged_mirror import assert_close

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def make(shape, n_ctx=1024, kv_blocks=256, max_rows=512):
    return na.PagedKv(na.BatchOpts(**shape, kv_blocks=kv_blocks, max_seqs=8, n_ctx=n_ctx, max_rows=max_rows))


def weights(rng, c, d_in, bias=True):
    # GPT-2-like scale: W ~ N(0, 0.02^2) would make q/k tiny; 1/sqrt(d_in)
    # keeps outputs ~N(0,1) so f16 rounding is exercised at full range.
    w = (rng.standard_normal((3 * c, d_in)) / np.sqrt(d_in)).astype(np.float32)
    b = (rng.standard_normal(3 * c) * 0.1).astype(np.float32) if bias else None
    return w, b


@pytest.mark.parametrize("shape", [workloads.GPT2, dict(n_layer=2, n_head=4, head_dim=128)], ids=["hd64", "hd128"])
@pytest.mark.parametrize("n", [1, 37, 512])
def test_project_matches_f64(gpu, oracle_lib, shape, n):
    rng = np.random.default_rng(60 + n)
    kv = make(shape)
    c = kv.opts.n_embd
    d_in = 768
    x = rng.standard_normal((n, d_in)).astype(np.float32)
    w, b = weights(rng, c, d_in)
    got = kv.qkv_project(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda())
    torch.cuda.synchronize()
    got = got.cpu().numpy().astype(np.float64)
    want = oracle.matvec_f64(x, w, b)
    err = np.abs(got - want)
    # f32 sums of 768 products of N(0,1/768)-scaled terms: ~1e-6 absolute
    assert err.max() < 2e-5, err.max()
    say(f"{shape} n {n}: max abs err vs f64 {err.max():.2e}")


@pytest.mark.parametrize("shape", [workloads.GPT2, dict(n_layer=2, n_head=4, head_dim=128)], ids=["hd64", "hd128"])
@pytest.mark.parametrize("d_in", [64, 400, 768])
def test_project_batch_invariant(gpu, oracle_lib, shape, d_in):
    """Each output is accumulated in an order that does not depend on the
    row count (row tiles are independent, d_in is summed in 8 fixed parts
    and a fixed tree), so a row's outputs have the same bits in a batch of
    any size -- the property the reference's matvec_batch keeps
    (batch.metal:60-66) and speculative verification relies on.  Batches of
    up to 16 rows run on the small-batch kernel, 17..64 on the mid-size
    kernel and larger ones on the LDS-staged kernel -- 16-feature tiles at 100
    and 384 rows, 48-feature tiles for the 512-row batch of head_dim 64 (its
    768 workgroups fill a round of the GPU) -- so this also checks that they
    all give the same bits."""
    rng = np.random.default_rng(80 + d_in)
    kv = make(shape)
    c = kv.opts.n_embd
    x = rng.standard_normal((512, d_in)).astype(np.float32)
    w, b = weights(rng, c, d_in)
    xd, wd, bd = (torch.from_numpy(t).cuda() for t in (x, w, b))
    big = kv.qkv_project(xd, wd, bd).cpu().numpy()
    want = oracle.matvec_f64(x, w, b)
    assert np.abs(big - want).max() < 2e-5
    for n in (1, 9, 16, 17, 64, 100, 384):
        small = kv.qkv_project(xd[:n].contiguous(), wd, bd).cpu().numpy()
        assert np.array_equal(small.view(np.uint32), big[:n].view(np.uint32)), f"n={n}"
    # the same rows at an offset inside the big batch, through a strided view
    small = kv.qkv_project(xd[100:130], wd, bd).cpu().numpy()
    assert np.array_equal(small.view(np.uint32), big[100:130].view(np.uint32))
    say(f"{shape} d_in {d_in}: batches of 1/9/16/17/64/100/384/30 rows bit-identical to the 512-row batch")


@pytest.mark.parametrize("bias", [True, False])
def test_fused_append_is_f16_of_projection(gpu, oracle_lib, bias):
    shape = workloads.GPT2
    rng = np.random.default_rng(70)
    kv = make(shape)
    c = kv.opts.n_embd
    d_in = 768
    # two sequences, rows at arbitrary positions spanning pages
    a, b_ = kv.add_seq(), kv.add_seq()
    kv.reserve(a, 300)
    kv.reserve(b_, 40)
    rows = [(a, p) for p in (0, 15, 16, 17, 255, 299)] + [(b_, p) for p in range(3, 40, 4)]
    n = len(rows)
    x = rng.standard_normal((n, d_in)).astype(np.float32)
    w, bb = weights(rng, c, d_in, bias)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    bd = torch.from_numpy(bb).cuda() if bias else None
    for layer in (0, 11):
        y = kv.qkv_project(xd, wd, bd)
        q = kv.qkv_append(rows, xd, wd, bd, layer=layer)
        torch.cuda.synchronize()
        y = y.cpu().numpy()
        assert np.array_equal(q.cpu().numpy(), y[:, :c])
        kg, vg = kv.gather(rows, layer=layer)
        assert np.array_equal(kg.cpu().numpy().view(np.uint16), oracle.f32_to_f16(y[:, c:2 * c]))
        assert np.array_equal(vg.cpu().numpy().view(np.uint16), oracle.f32_to_f16(y[:, 2 * c:]))


def test_attention_over_projected_kv(gpu, oracle_lib):
    """Prefill a sequence through the fused projection (per layer), then
    decode-attend its last row: within the north star's bound of the oracle
    over the same f16 K/V."""
    shape = dict(n_layer=2, n_head=12, head_dim=64)
    rng = np.random.default_rng(71)
    kv = make(shape)
    c, d_in, L = 768, 768, 200
    s = kv.add_seq()
    kv.reserve(s, L)
    rows = [(s, p) for p in range(L)]
    pools = oracle.PagedPools(2, 256, c)
    qs = []
    for layer in range(2):
        x = rng.standard_normal((L, d_in)).astype(np.float32)
        w, b = weights(rng, c, d_in)
        xd, wd, bd = (torch.from_numpy(t).cuda() for t in (x, w, b))
        y = kv.qkv_project(xd, wd, bd).cpu().numpy()
        qs.append(kv.qkv_append(rows, xd, wd, bd, layer=layer).cpu().numpy())
        table = np.zeros((8, kv.max_blocks), np.uint32)
        bt = kv.block_table(s)
        table[s, :len(bt)] = bt
        r = np.asarray(rows, np.uint32)
        oracle.paged_append(pools, layer, table, kv.max_blocks, r[:, 0], r[:, 1], y[:, c:2 * c], y[:, 2 * c:])
    kv.commit(s, L)
    q = np.stack([qs[l][-1:] for l in range(2)])
    got = kv.attention(torch.from_numpy(q).cuda(), [(s, L - 1)]).cpu().numpy()
    table = np.zeros((8, kv.max_blocks), np.uint32)
    bt = kv.block_table(s)
    table[s, :len(bt)] = bt
    want = np.stack([oracle.paged_attention(pools, l, table, kv.max_blocks, np.array([s], np.uint32),
                                            np.array([L - 1], np.uint32), q[l], 12, 64) for l in range(2)])
    err = assert_close(got, want, "attention over projected K/V")
    say(f"attention over projected K/V: max abs err {err:.2e}")


def test_qkv_errors(gpu):
    kv = make(dict(n_layer=2, n_head=2, head_dim=64), kv_blocks=8, n_ctx=64, max_rows=16)
    s = kv.add_seq()
    kv.reserve(s, 4)
    c = 128
    w = torch.zeros((3 * c, 64), device="cuda")
    x = torch.zeros((2, 64), device="cuda")
    with pytest.raises(na.KvError, match="layer 2 out of range"):
        kv.qkv_append([(s, 0), (s, 1)], x, w, layer=2)
    with pytest.raises(na.KvError, match="has no page"):
        kv.qkv_append([(s, 0), (s, 16)], x, w)
    w40 = torch.zeros((3 * c, 40), device="cuda")
    with pytest.raises(na.KvError, match="multiple of 16"):
        kv.qkv_project(torch.zeros((2, 40), device="cuda"), w40)
    with pytest.raises(na.KvError, match="max_rows"):
        kv.qkv_project(torch.zeros((17, 64), device="cuda"), w)


@pytest.mark.parametrize("fmt", ["f16", "q8_0", "q4_0"])
def test_weight_formats_equal_the_dequantised_projection(gpu, oracle_lib, fmt):
    """The reference's weight formats (DType, weights.rs:12-86, loaded by
    batch.metal:45-90's BF16/BQ8/BQ4): each weight is dequantised exactly into
    f32 on load, so the projection with the quantised bytes has the bits of
    the f32 projection with the dequantised matrix, at every row count (all
    three kernels), and is within f32 rounding of the f64 product."""
    shape = workloads.GPT2
    rng = np.random.default_rng(90)
    kv = make(shape)
    c, d_in = kv.opts.n_embd, 768
    w, b = weights(rng, c, d_in)
    wq = oracle.quantize(w, fmt)
    wdq = oracle.dequantize(wq, w.size, fmt).reshape(w.shape)
    x = rng.standard_normal((512, d_in)).astype(np.float32)
    xd, wqd, wdd, bd = (torch.from_numpy(t).cuda() for t in (x, wq, wdq, b))
    for n in (1, 9, 16, 17, 40, 64, 100, 512):
        got = kv.qkv_project(xd[:n].contiguous(), wqd, bd, w_format=fmt).cpu().numpy()
        ref = kv.qkv_project(xd[:n].contiguous(), wdd, bd).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"{fmt} n={n}"
    err = np.abs(got.astype(np.float64) - oracle.matvec_f64(x, wdq, b)).max()
    assert err < 2e-5, err
    say(f"{fmt}: bit-identical to the dequantised f32 projection at 1..512 rows; max err vs f64 {err:.2e}")


@pytest.mark.parametrize("fmt", ["f16", "q4_0"])
def test_weight_formats_fused_append(gpu, oracle_lib, fmt):
    """ni_kv_qkv_append_w stores f32_to_f16 of ni_kv_qkv_project_w's k/v
    columns and returns its q columns, bit for bit."""
    rng = np.random.default_rng(91)
    kv = make(workloads.GPT2)
    c, d_in = kv.opts.n_embd, 768
    s = kv.add_seq()
    kv.reserve(s, 100)
    rows = [(s, p) for p in range(3, 100, 3)]
    w, b = weights(rng, c, d_in)
    wq = torch.from_numpy(oracle.quantize(w, fmt)).cuda()
    x = torch.from_numpy(rng.standard_normal((len(rows), d_in)).astype(np.float32)).cuda()
    bd = torch.from_numpy(b).cuda()
    y = kv.qkv_project(x, wq, bd, w_format=fmt).cpu().numpy()
    q = kv.qkv_append(rows, x, wq, bd, layer=5, w_format=fmt).cpu().numpy()
    assert np.array_equal(q, y[:, :c])
    kg, vg = kv.gather(rows, layer=5)
    assert np.array_equal(kg.cpu().numpy().view(np.uint16), oracle.f32_to_f16(y[:, c:2 * c]))
    assert np.array_equal(vg.cpu().numpy().view(np.uint16), oracle.f32_to_f16(y[:, 2 * c:]))


def test_weight_format_errors(gpu):
    kv = make(dict(n_layer=2, n_head=2, head_dim=64), kv_blocks=8, n_ctx=64, max_rows=16)
    c = 128
    x = torch.zeros((2, 48), device="cuda")
    with pytest.raises(ValueError, match="multiple of 32"):
        kv.qkv_project(x, torch.zeros(3 * c * 48 // 2 + 3 * c * 48 // 16, dtype=torch.uint8, device="cuda"),
                       w_format="q4_0")
    with pytest.raises(ValueError, match="bytes"):
        kv.qkv_project(torch.zeros((2, 64), device="cuda"), torch.zeros(100, dtype=torch.uint8, device="cuda"),
                       w_format="q8_0")
    with pytest.raises(ValueError, match="unknown weight format"):
        kv.qkv_project(torch.zeros((2, 64), device="cuda"), torch.zeros(1, device="cuda"), w_format="bf16")
    L = kv._L
    w = torch.zeros(3 * c * 48, dtype=torch.uint8, device="cuda")  # the library's own check, past the wrapper
    rc = L.ni_kv_qkv_project_w(kv.handle, x.data_ptr(), 48, 2, 48, w.data_ptr(), 2, None,
                               torch.zeros((2, 3 * c), device="cuda").data_ptr(), 3 * c, None)
    assert rc == na._abi.NI_ERR_BAD_ARG and "multiple of 32" in L.ni_kv_last_error(kv.handle).decode()
    rc = L.ni_kv_qkv_project_w(kv.handle, x.data_ptr(), 48, 2, 48, w.data_ptr(), 7, None,
                               torch.zeros((2, 3 * c), device="cuda").data_ptr(), 3 * c, None)
    assert rc == na._abi.NI_ERR_BAD_ARG and "unknown weight format" in L.ni_kv_last_error(kv.handle).decode()
