"""The C++ drivers (include/nanoinfer_drivers.h) on host-only handles: they
export what the header declares, and their traces equal the Python
restatements of metal_serve.rs:255-363 and metal_spec.rs:118-169 decision
for decision (work lists, admissions, retirements, accepted counts, and the
block tables and free pages those leave behind)."""
import subprocess

import numpy as np
import pytest

import nanoinfer_amd as na
from nanoinfer_amd import build, drivers, workloads


def test_drivers_export_every_declared_function():
    L = drivers.lib()
    declared = drivers.declared_functions()
    assert len(declared) >= 10
    assert not [f for f in declared if not hasattr(L, f)]
    out = subprocess.run(["nm", "-D", "--defined-only", build.DRIVERS_LIB], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert set(declared) <= exported


def host(kv_blocks, max_seqs, n_ctx=1024, max_rows=512):
    return na.PagedKv(na.BatchOpts(**workloads.GPT2, kv_blocks=kv_blocks, max_seqs=max_seqs, n_ctx=n_ctx,
                                   max_rows=max_rows, host_only=True))


def run_step(kv, work):
    """What ni_kv_step does to the bookkeeping."""
    for seq, n_new, _ in work:
        kv.reserve(int(seq), kv.seq_len(int(seq)) + int(n_new))
        kv.commit(int(seq), int(n_new))


def same_state(a, b, max_seqs):
    assert a.free_block_count() == b.free_block_count()
    for s in range(max_seqs):
        assert a.is_live(s) == b.is_live(s)
        if a.is_live(s):
            assert a.seq_len(s) == b.seq_len(s)
            assert a.block_table(s) == b.block_table(s)


@pytest.mark.parametrize("all_rows", [False, True])
@pytest.mark.parametrize("cfg", [dict(max_batch=64, budget=256, pool=3080, rate=1.0, out=(16, 256), steps=700),
                                 dict(max_batch=8, budget=64, pool=200, rate=0.5, out=(16, 32), steps=900)],
                         ids=["config3", "tight-pool"])
def test_serve_trace_equals_python(cfg, all_rows):
    """Same seed, same policy: identical iterations on both drivers."""
    a = host(cfg["pool"], cfg["max_batch"])
    b = host(cfg["pool"], cfg["max_batch"])
    cxx = drivers.Serve(a, seed=7, rate=cfg["rate"], max_batch=cfg["max_batch"], budget=cfg["budget"], out=cfg["out"],
                        query_all_prompt_rows=all_rows)
    py = workloads.ContinuousBatching(b, seed=7, rate=cfg["rate"], max_batch=cfg["max_batch"], budget=cfg["budget"],
                                      out=cfg["out"], prefill_queries="all" if all_rows else "last")
    for i in range(cfg["steps"]):
        work, ctx, adm, ret = cxx.plan()
        st = py.plan()
        assert np.array_equal(work, st.work), f"step {i}"
        assert np.array_equal(ctx, st.ctx_after), f"step {i}"
        assert adm == st.admit and ret == st.retire, f"step {i}"
        run_step(a, work)
        run_step(b, st.work)
        cxx.commit()
        py.commit()
        if i % 50 == 0:
            same_state(a, b, cfg["max_batch"])
    assert cxx.done() == py.done > 0
    same_state(a, b, cfg["max_batch"])


@pytest.mark.parametrize("window", [0, 64])
def test_spec_trace_equals_python(window):
    ctx, _ = workloads.config5_contexts()
    a = host(32 * 128, 32, n_ctx=2048)
    b = host(32 * 128, 32, n_ctx=2048)
    seqs = []
    for L in ctx:
        s, t = a.add_seq(), b.add_seq()
        assert s == t
        for kv in (a, b):
            kv.reserve(s, L)
            kv.commit(s, L)
        seqs.append(s)
    cxx = drivers.Spec(a, seqs, k=4, seed=55, window=window)
    py = workloads.SpecVerify(b, seqs, k=4, seed=55, window=window or None)
    for i in range(300):
        work, ctx_after = cxx.plan()
        st = py.plan()
        assert np.array_equal(work, st.work) and np.array_equal(ctx_after, st.ctx_after), f"round {i}"
        run_step(a, work)
        run_step(b, st.work)
        assert cxx.commit() == py.commit(), f"round {i}"
    same_state(a, b, 32)
    if window:
        for s, L in zip(seqs, ctx):
            assert L <= a.seq_len(s) <= L + window


def test_drive_refuses_host_only_and_bad_modes():
    o = drivers.ni_drive_opts()
    o.kv.n_layer, o.kv.n_head, o.kv.head_dim, o.kv.kv_pages, o.kv.max_seqs = 1, 1, 64, 8, 1
    o.kv.max_ctx, o.kv.max_rows, o.kv.flags = 64, 16, na._abi.NI_KV_HOST_ONLY
    with pytest.raises(RuntimeError, match="device handle"):
        drivers.drive(o)
    o.kv.flags = 0
    o.launch = 7
    with pytest.raises(RuntimeError, match="launch mode"):
        drivers.drive(o)


def test_serve_plan_errors_when_trace_is_exhausted():
    a = host(64, 2)
    cxx = drivers.Serve(a, seed=3, n_requests=1, max_batch=2, prompt=(4, 4), out=(1, 1))
    work, _, adm, _ = cxx.plan()
    assert adm == [0] and work.tolist() == [[0, 4, 1]]
    run_step(a, work)
    cxx.commit()
    assert cxx.done() == 1 and not a.is_live(0)
    with pytest.raises(RuntimeError, match="every request has finished"):
        cxx.plan()


@pytest.mark.parametrize("name,fmt,q8", [("qkv64", 0, False), ("qkv64f16", 1, False), ("qkv64q8", 2, False),
                                         ("qkv16q4", 3, False), ("config3q8", 0, True), ("config3", 0, False)])
def test_preset_weight_format_and_q8_suffix(name, fmt, q8):
    """After "qkv<rows>" a trailing q8 names the q8_0 weight format, not the
    Q8 KV cache (whose pages the fused QKV epilogue cannot write); elsewhere
    it names the Q8 cache."""
    from nanoinfer_amd import _abi

    o = drivers.preset(name, 1, 0)
    assert bool(o.kv.flags & _abi.NI_KV_Q8) == q8
    if name.startswith("qkv"):
        assert o.qkv_wformat == fmt
        assert o.workload == drivers.NI_DRIVE_QKV
