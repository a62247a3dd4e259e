"""ni_kv_step_noalloc, the step entry point that allocates nothing, against
ni_kv_step through the C ABI.

Two handles with identical options see the same calls; one makes them
through ni_kv_step, the other through ni_kv_step_noalloc (split-K partials
in the library's file-scope device array, plans inline).  The same kernels
run over the same plans, so outputs, stored K/V and block tables must be
bit-identical -- on two calls in a row, the second smaller (the array keeps
the first call's contents).  The no-allocation call must not lower the
device's free memory, and steps beyond its limits (a plan over 32 KB, split
partials over 32 MiB) are refused with a clear error, launching nothing.
Captured in a HIP graph, the call replays bit-identically.  The array
belongs to the first handle that calls the entry point on the GPU until that
handle is destroyed (each test closes its caller); other handles are
refused meanwhile.
"""
import ctypes as C
import sys

import numpy as np
import pytest
import torch

import nanoinfer_amd as na
from nanoinfer_amd import _abi

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, file=sys.stderr, flush=True)


def call(kv, fn, work, q, k, v, out, split):
    w = np.ascontiguousarray(np.asarray(work, np.uint32).reshape(-1, 3))
    return fn(kv.handle, w.ctypes.data_as(C.POINTER(_abi.ni_work)), w.shape[0], q.data_ptr(), k.data_ptr(),
              v.data_ptr(), q.stride(1), q.stride(0), out.data_ptr(), out.stride(1), out.stride(0), split,
              torch.cuda.current_stream().cuda_stream)


def fill(kvs, seqs, lens, g, C_):
    for s, L in zip(seqs, lens):
        k, v = (torch.randn((kvs[0].opts.n_layer, L, C_), device="cuda", generator=g) for _ in range(2))
        for kv in kvs:
            assert kv.add_seq() == s
            kv.reserve(s, L)
            step = kv.opts.max_rows
            for p0 in range(0, L, step):
                p1 = min(L, p0 + step)
                kv.append([(s, p) for p in range(p0, p1)], k[:, p0:p1], v[:, p0:p1])
            kv.commit(s, L)


def same_state(a, b, seqs):
    for s in seqs:
        assert a.seq_len(s) == b.seq_len(s)
        assert a.block_table(s) == b.block_table(s)
        n = a.seq_len(s)
        for p0 in range(0, n, a.opts.max_rows):
            rows = [(s, p) for p in range(p0, min(n, p0 + a.opts.max_rows))]
            ka, va = a.gather(rows)
            kb, vb = b.gather(rows)
            assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_noalloc_equals_step_on_two_calls(gpu):
    L, H, D = 12, 12, 64
    C_ = H * D
    opts = na.BatchOpts(n_layer=L, n_head=H, head_dim=D, kv_blocks=512, max_seqs=16, n_ctx=1024, max_rows=512)
    a, b = na.PagedKv(opts), na.PagedKv(opts)
    g = torch.Generator(device="cuda").manual_seed(71)
    seqs = list(range(8))
    fill([a, b], seqs, [1, 15, 16, 100, 300, 511, 700, 64], g, C_)
    lib = _abi.lib()
    # Call 1: decode rows, a 5-row verify group, a prompt chunk queried at its
    # last row, and a 24-row chunk queried at every row (the prefill launch);
    # 64-token partitions, so every kind of launch writes split partials.
    work1 = [(0, 1, 1), (1, 1, 1), (2, 5, 5), (3, 40, 1), (4, 24, 24), (5, 1, 1), (6, 1, 1), (7, 3, 0)]
    # Call 2: fewer, smaller rows, another partition size.
    work2 = [(1, 1, 1), (6, 2, 2), (4, 1, 1)]
    # Call 3: prompt chunks only, every sequence queried at more than 16 rows
    # and no partitions (on this f16 pool: an append launch, then the prefill
    # launch; the Q8 test below covers the prefill launch that appends).
    work3 = [(4, 40, 40), (7, 30, 20)]
    for i, (work, split) in enumerate(((work1, 64), (work2, 128), (work3, 1024))):
        n = sum(w[1] for w in work)
        q, k, v = (torch.randn((L, n, C_), device="cuda", generator=g) for _ in range(3))
        out_a = torch.full((L, n, C_), float("nan"), device="cuda")
        out_b = torch.full((L, n, C_), float("nan"), device="cuda")
        say(f"no-alloc call {i + 1}: {len(work)} items, {n} rows, split {split}")
        rc = call(a, lib.ni_kv_step, work, q, k, v, out_a, split)
        assert rc == 0, lib.ni_kv_last_error(a.handle).decode()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        rc = call(b, lib.ni_kv_step_noalloc, work, q, k, v, out_b, split)
        assert rc == 0, lib.ni_kv_last_error(b.handle).decode()
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] >= free0
        queried = [r for w, r0 in zip(work, np.cumsum([0] + [w[1] for w in work])) for r in
                   range(r0 + w[1] - w[2], r0 + w[1])]
        qi = torch.tensor(queried, device="cuda")
        assert torch.isfinite(out_a[:, qi]).all()
        assert torch.equal(out_a[:, qi], out_b[:, qi])
        same_state(a, b, seqs)
    b.close()  # (the GPU's scratch array goes back with its holder)


def test_noalloc_q8_prompt_chunks_appended_by_the_prefill_launch(gpu):
    """A Q8 step of prompt chunks only with 64 x 2 x 12 = 1536 (sequence,
    layer, head) units: its prefill launch appends each sequence's rows
    itself (no append launch, checked on the ni_kv_step twin's launch
    counts); outputs and the stored int8 values and scales bit-identical."""
    L, H, D = 2, 12, 64
    C_ = H * D
    opts = na.BatchOpts(n_layer=L, n_head=H, head_dim=D, kv_blocks=200, max_seqs=64, n_ctx=256, max_rows=2048,
                        q8=True)
    a, b = na.PagedKv(opts), na.PagedKv(opts)
    g = torch.Generator(device="cuda").manual_seed(77)
    for kv in (a, b):
        assert [kv.add_seq() for _ in range(64)] == list(range(64))
    lib = _abi.lib()
    work = [(s, 17 + (s % 3), 17 + (s % 3)) for s in range(64)]
    n = sum(w[1] for w in work)
    q, k, v = (torch.randn((L, n, C_), device="cuda", generator=g) for _ in range(3))
    out_a = torch.full((L, n, C_), float("nan"), device="cuda")
    out_b = torch.full((L, n, C_), float("nan"), device="cuda")
    say(f"no-alloc Q8 prompt chunks: 64 sequences, {n} rows")
    a.profile([_abi.NI_K_APPEND, _abi.NI_K_ATTN])
    rc = call(a, lib.ni_kv_step, work, q, k, v, out_a, 0)
    assert rc == 0, lib.ni_kv_last_error(a.handle).decode()
    torch.cuda.synchronize()
    _, n_append = a.profile_read(_abi.NI_K_APPEND)
    _, n_attn = a.profile_read(_abi.NI_K_ATTN)
    a.profile([])
    assert n_append == 0 and n_attn == 1, (n_append, n_attn)
    free0 = torch.cuda.mem_get_info()[0]
    rc = call(b, lib.ni_kv_step_noalloc, work, q, k, v, out_b, 0)
    assert rc == 0, lib.ni_kv_last_error(b.handle).decode()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] >= free0
    assert torch.isfinite(out_a).all()
    assert torch.equal(out_a, out_b)
    for s in range(64):
        assert a.seq_len(s) == b.seq_len(s) and a.block_table(s) == b.block_table(s)
    rows = [(s, p) for s in range(64) for p in range(a.seq_len(s))]
    for i in range(0, len(rows), 1024):
        ga, gb = a.gather_q8(rows[i:i + 1024]), b.gather_q8(rows[i:i + 1024])
        for x, y in zip(ga, gb):
            for xx, yy in zip(x, y):
                assert torch.equal(xx, yy)
    b.close()


def test_noalloc_limits(gpu):
    lib = _abi.lib()
    # A plan over 32 KB: 64 sequences of 2048 positions list 64 x 129 page ids.
    opts = na.BatchOpts(n_layer=1, n_head=1, head_dim=64, kv_blocks=64 * 129, max_seqs=64, n_ctx=2064, max_rows=64)
    kv = na.PagedKv(opts)
    for s in range(64):
        assert kv.add_seq() == s
        kv.reserve(s, 2048)
        kv.commit(s, 2048)  # pages hold zeros: never written
    work = [(s, 1, 1) for s in range(64)]
    q, k, v = (torch.randn((1, 64, 64), device="cuda") for _ in range(3))
    out = torch.zeros_like(q)
    say("no-alloc limits: 64 x 2049-key decode rows (plan over 32 KB)")
    rc = call(kv, lib.ni_kv_step_noalloc, work, q, k, v, out, 0)
    assert rc == _abi.NI_ERR_BAD_ARG
    msg = lib.ni_kv_last_error(kv.handle).decode()
    assert "ni_kv_step_noalloc passes plans of at most 32768 bytes" in msg, msg
    assert all(kv.seq_len(s) == 2048 for s in range(64))
    rc = call(kv, lib.ni_kv_step, work, q, k, v, out, 0)  # the allocating entry point takes it
    assert rc == 0, lib.ni_kv_last_error(kv.handle).decode()
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    kv.close()
    # Split partials over 32 MiB: 4 rows of 3073 keys in 64-key partitions
    # (49 each) x 12 layers x 32 heads x 130 floats.
    opts = na.BatchOpts(n_layer=12, n_head=32, head_dim=128, kv_blocks=4 * 193, max_seqs=4, n_ctx=3088, max_rows=8)
    kv = na.PagedKv(opts)
    for s in range(4):
        assert kv.add_seq() == s
        kv.reserve(s, 3072)
        kv.commit(s, 3072)
    work = [(s, 1, 1) for s in range(4)]
    q, k, v = (torch.randn((12, 4, 4096), device="cuda") for _ in range(3))
    out = torch.zeros_like(q)
    say("no-alloc limits: 4 x 3073-key rows in 64-key partitions (partials over 32 MiB)")
    rc = call(kv, lib.ni_kv_step_noalloc, work, q, k, v, out, 64)
    assert rc == _abi.NI_ERR_BAD_ARG
    msg = lib.ni_kv_last_error(kv.handle).decode()
    assert "bytes of split partials; ni_kv_step_noalloc holds at most 33554432" in msg, msg
    # at 512-key partitions the same step fits
    out2 = torch.zeros_like(q)
    rc = call(kv, lib.ni_kv_step_noalloc, work, q, k, v, out2, 512)
    assert rc == 0, lib.ni_kv_last_error(kv.handle).decode()
    torch.cuda.synchronize()
    assert torch.isfinite(out2).all()
    kv.close()


def test_noalloc_step_replayed_from_a_graph(gpu):
    """The callers it is for: ni_kv_step_noalloc captured in a HIP graph
    (through torch.cuda.graph) and replayed three times, with eager work and
    gathers between the replays; every replay's outputs and stored K/V equal
    the eager ni_kv_step of a twin handle."""
    L, H, D = 12, 12, 64
    C_ = H * D
    opts = na.BatchOpts(n_layer=L, n_head=H, head_dim=D, kv_blocks=512, max_seqs=16, n_ctx=1024, max_rows=512)
    a, b = na.PagedKv(opts), na.PagedKv(opts)
    g = torch.Generator(device="cuda").manual_seed(73)
    seqs = list(range(6))
    fill([a, b], seqs, [1, 17, 100, 300, 511, 64], g, C_)
    lib = _abi.lib()
    # decode rows, a 5-row verify group, a chunk without a query (orphan
    # rows), 64-token partitions (split partials in the library's array)
    work = [(0, 1, 1), (1, 1, 1), (2, 5, 5), (3, 1, 1), (4, 1, 1), (5, 7, 0)]
    n = sum(w[1] for w in work)
    q, k, v = (torch.randn((L, n, C_), device="cuda", generator=g) for _ in range(3))
    out_a = torch.full((L, n, C_), float("nan"), device="cuda")
    out_b = torch.full((L, n, C_), float("nan"), device="cuda")
    rc = call(a, lib.ni_kv_step, work, q, k, v, out_a, 64)
    assert rc == 0, lib.ni_kv_last_error(a.handle).decode()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    say("graph: capturing ni_kv_step_noalloc")
    with torch.cuda.graph(graph):
        rc = call(b, lib.ni_kv_step_noalloc, work, q, k, v, out_b, 64)
    assert rc == 0, lib.ni_kv_last_error(b.handle).decode()
    queried = [r for w, r0 in zip(work, np.cumsum([0] + [w[1] for w in work])) for r in
               range(r0 + w[1] - w[2], r0 + w[1])]
    qi = torch.tensor(queried, device="cuda")
    for rep in range(3):
        say(f"graph: replay {rep + 1}")
        out_b.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_a[:, qi], out_b[:, qi]), f"replay {rep + 1}"
        same_state(a, b, seqs)  # eager gathers between the replays
        x = torch.randn((1024, 1024), device="cuda", generator=g)
        (x @ x).sum().item()  # unrelated eager work
    del graph
    b.close()


def test_noalloc_scratch_held_by_one_handle(gpu):
    """The GPU's one scratch array belongs to the first handle that calls
    ni_kv_step_noalloc: another handle's call is refused (nothing launched,
    its pages and lengths unchanged) until the holder is destroyed, and
    then succeeds with the holder's results."""
    L, H, D = 2, 4, 64
    C_ = H * D
    opts = na.BatchOpts(n_layer=L, n_head=H, head_dim=D, kv_blocks=64, max_seqs=4, n_ctx=512, max_rows=64)
    a, b = na.PagedKv(opts), na.PagedKv(opts)
    g = torch.Generator(device="cuda").manual_seed(79)
    fill([a, b], [0, 1], [40, 200], g, C_)
    lib = _abi.lib()
    work = [(0, 1, 1), (1, 1, 1)]
    q, k, v = (torch.randn((L, 2, C_), device="cuda", generator=g) for _ in range(3))
    out_a = torch.full((L, 2, C_), float("nan"), device="cuda")
    out_b = torch.full((L, 2, C_), float("nan"), device="cuda")
    say("no-alloc scratch: two handles")
    rc = call(a, lib.ni_kv_step_noalloc, work, q, k, v, out_a, 0)
    assert rc == 0, lib.ni_kv_last_error(a.handle).decode()
    rc = call(b, lib.ni_kv_step_noalloc, work, q, k, v, out_b, 0)
    assert rc == _abi.NI_ERR_BAD_ARG
    msg = lib.ni_kv_last_error(b.handle).decode()
    assert "scratch array is held by another handle" in msg, msg
    assert b.seq_len(0) == 40 and b.seq_len(1) == 200
    torch.cuda.synchronize()
    assert torch.isnan(out_b).all()
    a.close()  # releases the array
    rc = call(b, lib.ni_kv_step_noalloc, work, q, k, v, out_b, 0)
    assert rc == 0, lib.ni_kv_last_error(b.handle).decode()
    torch.cuda.synchronize()
    assert torch.isfinite(out_b).all() and torch.equal(out_a, out_b)
    assert b.seq_len(0) == 41 and b.seq_len(1) == 201
    b.close()
