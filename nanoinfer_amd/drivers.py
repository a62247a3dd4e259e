"""ctypes binding of ``include/nanoinfer_drivers.h``: the C++ restatements
of the reference's serving harnesses (``metal_serve.rs:255-363``,
``metal_spec.rs:118-169``) over the KV C ABI, and ``ni_drive_run``.

``Serve`` and ``Spec`` drive a :class:`~nanoinfer_amd.batch.PagedKv` (a
device handle or a host-only one); :func:`drive` runs a whole synthetic
workload on the device with the C++ host loop.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import _abi
from . import build as _build

_lib = None
_vp = C.c_void_p
_u32 = C.c_uint32


class ni_serve_opts(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("rate", C.c_double), ("n_requests", _u32), ("max_batch", _u32),
                ("prompt_min", _u32), ("prompt_max", _u32), ("out_min", _u32), ("out_max", _u32),
                ("budget", _u32), ("max_rows", _u32), ("query_all_prompt_rows", _u32)]


class ni_serve_iter(C.Structure):
    _fields_ = [("work", C.POINTER(_abi.ni_work)), ("n_work", _u32), ("ctx_after", C.POINTER(_u32)),
                ("admitted", C.POINTER(_u32)), ("n_admitted", _u32), ("retired", C.POINTER(_u32)),
                ("n_retired", _u32)]


class ni_drive_opts(C.Structure):
    _fields_ = [("workload", _u32), ("launch", _u32), ("kv", _abi.ni_kv_opts), ("serve", ni_serve_opts),
                ("spec_seqs", _u32), ("spec_ctx_min", _u32), ("spec_ctx_max", _u32), ("spec_k", _u32),
                ("spec_seed", C.c_uint64), ("spec_window", _u32), ("ramp", _u32), ("warmup", _u32), ("steps", _u32),
                ("split_tokens", _u32), ("data_seed", C.c_uint64), ("fixed_ctx", C.POINTER(_u32)),
                ("fixed_n", _u32), ("kv_std", C.c_float), ("profile_mask", _u32), ("qkv_rows", _u32),
                ("fixed_rows", _u32), ("qkv_wformat", _u32)]


class ni_serve_stats(C.Structure):
    _fields_ = [("iterations", _u32), ("rows", C.c_uint64), ("generated", C.c_uint64), ("kv_pages_peak", _u32),
                ("kv_pages_avg_used", C.c_double), ("snapshots", _u32), ("avg_live_seqs", C.c_double),
                ("avg_pages_per_seq", C.c_double), ("internal_fragmentation", C.c_double)]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


class ni_drive_result(C.Structure):
    _fields_ = [("seconds", C.c_double), ("gpu_seconds", C.c_double), ("bytes", C.c_double),
                ("seq_tokens", C.c_double), ("host_us_per_step", C.c_double), ("steps", _u32),
                ("launches", C.c_uint64), ("mean_live", C.c_double), ("mean_context", C.c_double),
                ("flops", C.c_double),
                ("kernel_ms", C.c_double * _abi.NI_K_COUNT), ("kernel_launches", C.c_uint64 * _abi.NI_K_COUNT),
                ("idle_us_plan_call", C.c_double), ("idle_us_layer_call", C.c_double),
                ("serve_stats", ni_serve_stats)]


NI_DRIVE_SERVE, NI_DRIVE_SPEC, NI_DRIVE_FIXED, NI_DRIVE_QKV = 0, 1, 2, 3
NI_DRIVE_STEP, NI_DRIVE_PER_LAYER, NI_DRIVE_STEP_LAYERS = 0, 1, 2


def lib():
    global _lib
    if _lib is not None:
        return _lib
    _abi.lib()  # the KV library first (the drivers link against it)
    if not os.path.exists(_build.DRIVERS_LIB):
        _build.build()
    L = C.CDLL(_build.DRIVERS_LIB)
    L.ni_serve_create.argtypes = [_vp, C.POINTER(ni_serve_opts), C.POINTER(_vp)]
    L.ni_serve_destroy.argtypes = [_vp]
    L.ni_serve_destroy.restype = None
    L.ni_serve_plan.argtypes = [_vp, C.POINTER(ni_serve_iter)]
    L.ni_serve_commit.argtypes = [_vp]
    L.ni_serve_done.argtypes = [_vp]
    L.ni_serve_done.restype = _u32
    L.ni_serve_get_stats.argtypes = [_vp, C.POINTER(ni_serve_stats)]
    L.ni_serve_reset_stats.argtypes = [_vp]
    L.ni_spec_create.argtypes = [_vp, C.POINTER(_u32), _u32, _u32, C.c_uint64, C.POINTER(_vp)]
    L.ni_spec_destroy.argtypes = [_vp]
    L.ni_spec_destroy.restype = None
    L.ni_spec_plan.argtypes = [_vp, C.POINTER(C.POINTER(_abi.ni_work)), C.POINTER(_u32), C.POINTER(C.POINTER(_u32))]
    L.ni_spec_commit.argtypes = [_vp, C.POINTER(C.POINTER(_u32))]
    L.ni_spec_set_window.argtypes = [_vp, _u32]
    L.ni_drive_run.argtypes = [C.POINTER(ni_drive_opts), C.POINTER(ni_drive_result)]
    L.ni_drive_last_error.restype = C.c_char_p
    L.ni_drive_last_error.argtypes = []
    L.ni_drive_device_memory.argtypes = [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
    _lib = L
    return L


def declared_functions() -> list[str]:
    import re

    text = open(os.path.join(_build.INCLUDE, "nanoinfer_drivers.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ni_[a-z0-9_]+)\s*\(", text)))


def _work(ptr, n) -> np.ndarray:
    return np.asarray([(ptr[i].seq, ptr[i].n_new, ptr[i].n_query) for i in range(n)], np.uint32).reshape(-1, 3)


def _check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: {lib().ni_drive_last_error().decode()} (status {rc})")


class Serve:
    """ni_serve over a PagedKv handle: plan() -> (work, ctx_after, admitted,
    retired); commit() after the step ran."""

    def __init__(self, kv, seed=7, rate=1.0, n_requests=100000, max_batch=64, prompt=(32, 512), out=(16, 256),
                 budget=256, max_rows=512, query_all_prompt_rows=False):
        L = lib()
        o = ni_serve_opts(seed, rate, n_requests, max_batch, prompt[0], prompt[1], out[0], out[1], budget, max_rows,
                          int(query_all_prompt_rows))
        h = _vp()
        _check(L.ni_serve_create(kv.handle, C.byref(o), C.byref(h)), "ni_serve_create")
        self._h, self._L, self.kv = h, L, kv

    def plan(self):
        it = ni_serve_iter()
        _check(self._L.ni_serve_plan(self._h, C.byref(it)), "ni_serve_plan")
        work = _work(it.work, it.n_work)
        ctx = np.asarray([it.ctx_after[i] for i in range(it.n_work)], np.int64)
        adm = [int(it.admitted[i]) for i in range(it.n_admitted)]
        ret = [int(it.retired[i]) for i in range(it.n_retired)]
        return work, ctx, adm, ret

    def commit(self):
        _check(self._L.ni_serve_commit(self._h), "ni_serve_commit")

    def done(self) -> int:
        return int(self._L.ni_serve_done(self._h))

    def stats(self) -> dict:
        """The KV summary of metal_serve.rs:320-331,440-464 over the current
        window (ni_serve_get_stats)."""
        st = ni_serve_stats()
        _check(self._L.ni_serve_get_stats(self._h, C.byref(st)), "ni_serve_get_stats")
        return st.as_dict()

    def reset_stats(self):
        _check(self._L.ni_serve_reset_stats(self._h), "ni_serve_reset_stats")

    def __del__(self):
        if getattr(self, "_h", None):
            self._L.ni_serve_destroy(self._h)
            self._h = None


class Spec:
    """ni_spec over a PagedKv handle."""

    def __init__(self, kv, seqs, k=4, seed=55, window=0):
        L = lib()
        s = np.ascontiguousarray(np.asarray(seqs, np.uint32))
        h = _vp()
        _check(L.ni_spec_create(kv.handle, s.ctypes.data_as(C.POINTER(_u32)), s.size, k, seed, C.byref(h)),
               "ni_spec_create")
        self._h, self._L, self.kv, self.n = h, L, kv, s.size
        _check(L.ni_spec_set_window(h, window), "ni_spec_set_window")

    def plan(self):
        w = C.POINTER(_abi.ni_work)()
        n = _u32()
        ctx = C.POINTER(_u32)()
        _check(self._L.ni_spec_plan(self._h, C.byref(w), C.byref(n), C.byref(ctx)), "ni_spec_plan")
        return _work(w, n.value), np.asarray([ctx[i] for i in range(n.value)], np.int64)

    def commit(self):
        acc = C.POINTER(_u32)()
        _check(self._L.ni_spec_commit(self._h, C.byref(acc)), "ni_spec_commit")
        return [int(acc[i]) for i in range(self.n)]

    def __del__(self):
        if getattr(self, "_h", None):
            self._L.ni_spec_destroy(self._h)
            self._h = None


def device_memory(device: int = 0) -> tuple[int, int]:
    """(peak memory clock in kHz, bus width in bits) as HIP reports them."""
    clk, bits = C.c_int(), C.c_int()
    _check(lib().ni_drive_device_memory(device, C.byref(clk), C.byref(bits)), "ni_drive_device_memory")
    return clk.value, bits.value


def drive(opts: ni_drive_opts) -> dict:
    """ni_drive_run: a whole synthetic run on the device (C++ host loop)."""
    r = ni_drive_result()
    _check(lib().ni_drive_run(C.byref(opts), C.byref(r)), "ni_drive_run")
    out = {f: getattr(r, f) for f, _ in ni_drive_result._fields_}
    out["serve_stats"] = r.serve_stats.as_dict()
    out["kernel_ms"] = list(r.kernel_ms)
    out["kernel_launches"] = list(r.kernel_launches)
    return out


# ------------------------------------------------------- configuration presets
# The benchmark configurations as ni_drive_opts; contexts and page orders come
# from nanoinfer_amd.workloads, the same definitions the tests use.

def _kv(o, shape, kv_pages, max_seqs, max_ctx, max_rows, order=None):
    o.kv.n_layer, o.kv.n_head, o.kv.head_dim = shape["n_layer"], shape["n_head"], shape["head_dim"]
    o.kv.kv_pages, o.kv.max_seqs, o.kv.max_ctx, o.kv.max_rows = kv_pages, max_seqs, max_ctx, max_rows
    if order is not None:
        arr = np.ascontiguousarray(np.asarray(order, np.uint32))
        o._keep.append(arr)
        o.kv.page_order = arr.ctypes.data_as(C.POINTER(_u32))


PREFILL_SEQS, PREFILL_ROWS = 16, 512


def preset(name: str, steps: int, warmup: int, launch: int = NI_DRIVE_STEP, split: int = 0, seed: int = 7,
           profile_mask: int = 0, query_all_prompt_rows: bool = False, ramp: int = 0) -> ni_drive_opts:
    """ni_drive_opts of benchmark configuration 2, 3, 4 or 5, the QKV projection (qkvN) or the prefill workload.
    `ramp` untimed append-only iterations precede the `warmup` full ones."""
    from . import workloads

    o = ni_drive_opts()
    o._keep = []  # arrays the struct points into
    o.launch, o.steps, o.warmup, o.split_tokens, o.data_seed, o.profile_mask = launch, steps, warmup, split, seed, \
        profile_mask
    o.ramp = ramp
    # A trailing "q8" names the same workload on a Q8 cache -- except after
    # "qkv<rows>", where it names the q8_0 weight format (the fused QKV epilogue
    # writes f16 pages only).
    q8 = name.endswith("q8") and not name.startswith("qkv")
    if q8:
        name = name[:-2]
    if name == "config3":
        o.workload = NI_DRIVE_SERVE
        o.serve = ni_serve_opts(seed, 1.0, 100000, 64, 32, 512, 16, 256, 256, 512, int(query_all_prompt_rows))
        # metal_serve.rs:485: max_batch * pages(prompt_max + out_max) + 8
        _kv(o, workloads.GPT2, 64 * workloads.pages(512 + 256) + 8, 64, 1024, 512)
    elif name == "config5":
        o.workload = NI_DRIVE_SPEC
        o.spec_seqs, o.spec_ctx_min, o.spec_ctx_max, o.spec_k, o.spec_seed = 32, 128, 1024, 4, 5
        o.spec_window = 64
        _kv(o, workloads.GPT2, 32 * 2048 // 16, 32, 2048, 512)
    elif name == "config2":
        ctx, order = workloads.config2_contexts()
        o.workload = NI_DRIVE_FIXED
        arr = np.ascontiguousarray(np.asarray(ctx, np.uint32))
        o._keep.append(arr)
        o.fixed_ctx, o.fixed_n = arr.ctypes.data_as(C.POINTER(_u32)), arr.size
        _kv(o, workloads.GPT2, 1024, 16, 1024, 512, order)
    elif name == "config4":
        B, L = 4, 32768
        o.workload = NI_DRIVE_FIXED
        arr = np.full(B, L, np.uint32)
        o._keep.append(arr)
        o.fixed_ctx, o.fixed_n = arr.ctypes.data_as(C.POINTER(_u32)), B
        o.kv_std = 0.5
        o.split_tokens = split or 512
        _kv(o, workloads.LONG, B * L // 16, B, L, 4096, workloads.XorShift.seeded(4).permutation(B * L // 16))
    elif name == "prefill":
        # Prefill (every row of a prompt queried): 16 sequences each
        # append and query a 512-row prompt from empty, rolled back each step.
        B, P = PREFILL_SEQS, PREFILL_ROWS
        o.workload = NI_DRIVE_FIXED
        arr = np.full(B, P, np.uint32)
        o._keep.append(arr)
        o.fixed_ctx, o.fixed_n, o.fixed_rows = arr.ctypes.data_as(C.POINTER(_u32)), B, P
        _kv(o, workloads.GPT2, B * workloads.pages(P) + 8, B, 1024, B * P)
    elif name.startswith("qkv"):
        # qkv<rows>[f16|q8|q4]: the projection of <rows> rows per layer, GPT-2
        # shape, with f32 weights or in one of the reference's weight formats
        o.workload = NI_DRIVE_QKV
        spec = name[3:]
        fmt = 0
        for suffix, f in (("f16", 1), ("q8", 2), ("q4", 3)):
            if spec.endswith(suffix):
                spec, fmt = spec[: -len(suffix)], f
                break
        o.qkv_rows = int(spec or 64)
        o.qkv_wformat = fmt
        _kv(o, workloads.GPT2, 64 * 64, 64, 1024, 512)
    else:
        raise ValueError(name)
    if q8:
        o.kv.flags |= _abi.NI_KV_Q8
    return o
