"""CPU oracle for the paged f16 KV-cache path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's CPU code (joshuaramkissoon/nanoinfer,
Rust) in C (``oracle/oracle.c``) and wraps it with ctypes + numpy.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it, and only as the checker or the timed CPU baseline.  The
product (``nanoinfer_amd``) never imports it.

Functions and the reference code they restate:

* ``f32_to_f16`` / ``f16_to_f32`` -- ``crates/core/src/quant.rs:25-73``
* ``fast_exp`` -- ``crates/core/src/kernels/fastops.rs:55-63``
* ``reference_attention`` -- ``crates/core/src/kernels/reference.rs:109-142``
* ``fastops_attention`` -- ``crates/core/src/kernels/fastops.rs:130-213``
* ``attend_f16_portable`` -- ``crates/core/src/stages/kv16.rs:144-164``
* ``kv16_attention`` -- ``crates/core/src/stages/kv16.rs:168-204``
* ``paged_append`` / ``paged_gather`` / ``paged_attention`` --
  ``crates/metal/src/shaders/batch.metal:24-26,329-344`` composed with the
  kv16 CPU arithmetic
* ``split_attention_f64`` -- ``batch.metal:349-424`` split/merge in float64
* ``Alloc`` -- ``crates/metal/src/batch.rs:129-254``
* ``CpuStep`` -- ``kv16.rs:214-263`` + ``lowlat.rs:21,35-40`` per layer,
  threaded (the reported CPU baseline)
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")
_lib = None

KV_BLOCK = 16

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build(force: bool = False) -> str:
    """Compile ``oracle.c`` into ``liboracle.so`` (gcc, via the Makefile)."""
    if force or not os.path.exists(_SO) or os.path.getmtime(_SO) < os.path.getmtime(os.path.join(_HERE, "oracle.c")):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", _HERE], check=True)
    return _SO


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_SO):
        build()
    L = C.CDLL(_SO)
    L.or_f32_to_f16.restype = C.c_uint16
    L.or_f32_to_f16.argtypes = [C.c_float]
    L.or_f16_to_f32.restype = C.c_float
    L.or_f16_to_f32.argtypes = [C.c_uint16]
    L.or_narrow.argtypes = [_f32p, _u16p, _sz]
    L.or_widen.argtypes = [_u16p, _f32p, _sz]
    L.or_f16_check_f16c.restype = C.c_uint64
    L.or_f16_check_f16c.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64)]
    L.or_f16_compare_range.restype = C.c_uint64
    L.or_f16_compare_range.argtypes = [C.c_uint64, C.c_uint64, _u16p, C.POINTER(C.c_uint64)]
    L.or_fast_exp.restype = C.c_float
    L.or_fast_exp.argtypes = [C.c_float]
    L.or_softmax.argtypes = [_f32p, _sz]
    att = [_f32p, _f32p, _sz, _f32p, _sz, _f32p, _sz, _sz, _sz, _sz, _sz, _f32p]
    L.or_reference_attention.argtypes = att
    L.or_fastops_attention.argtypes = att
    L.or_attend_f16_portable.argtypes = [_f32p, _f32p, _u16p, _u16p, _sz, _sz, _f32p]
    L.or_kv16_attention.argtypes = [_f32p, _f32p, _u16p, _u16p, _sz, _sz, _sz, _sz, _sz, _f32p]
    L.or_kv_slot.restype = C.c_uint32
    L.or_kv_slot.argtypes = [_u32p, C.c_uint32, C.c_uint32, C.c_uint32]
    L.or_paged_append.argtypes = [_u16p, _u16p, _u32p, C.c_uint32, _u32p, _u32p, _sz, _f32p, _f32p, _sz, _sz]
    L.or_paged_gather.argtypes = [_u16p, _u16p, _u16p, _u16p, _u32p, C.c_uint32, _u32p, _u32p, _sz, _sz]
    L.or_paged_attention.argtypes = [_f32p, _sz, _f32p, _sz, _u16p, _u16p, _u32p, C.c_uint32, _u32p, _u32p, _sz,
                                     _sz, _sz, _f32p]
    L.or_split_attention_f64.argtypes = [_f64p, _f32p, _f32p, _f32p, _sz, _sz, _sz]
    L.or_matvec_f64.argtypes = [_f64p, _f32p, _sz, _f32p, C.c_void_p, _sz, _sz, _sz]
    _u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
    L.or_quantize_q8_0.restype = _sz
    L.or_quantize_q8_0.argtypes = [_f32p, _sz, _u8p]
    L.or_quantize_q4_0.restype = _sz
    L.or_quantize_q4_0.argtypes = [_f32p, _sz, _u8p]
    L.or_dequantize.argtypes = [_u8p, _sz, C.c_int, _f32p]
    _i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
    L.or_q8_quantize.restype = C.c_float
    L.or_q8_quantize.argtypes = [_f32p, _sz, _i8p]
    L.or_paged_q8_append.argtypes = [_i8p, _i8p, _f32p, _f32p, _u32p, C.c_uint32, _u32p, _u32p, _sz, _f32p, _f32p,
                                     _sz, _sz, _sz]
    L.or_paged_q8_attention.argtypes = [_f32p, _sz, _f32p, _sz, _i8p, _i8p, _f32p, _f32p, _u32p, C.c_uint32, _u32p,
                                        _u32p, _sz, _sz, _sz, _f64p]
    L.or_alloc_new.restype = C.c_void_p
    L.or_alloc_new.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p]
    L.or_alloc_free.argtypes = [C.c_void_p]
    L.or_alloc_add_seq.restype = C.c_int64
    L.or_alloc_add_seq.argtypes = [C.c_void_p]
    L.or_alloc_truncate.restype = C.c_int
    L.or_alloc_truncate.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
    L.or_alloc_free_seq.argtypes = [C.c_void_p, C.c_uint32]
    L.or_alloc_ensure.restype = C.c_int
    L.or_alloc_ensure.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
    L.or_alloc_commit.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
    L.or_alloc_seq_len.restype = C.c_uint32
    L.or_alloc_seq_len.argtypes = [C.c_void_p, C.c_uint32]
    L.or_alloc_live.restype = C.c_int
    L.or_alloc_live.argtypes = [C.c_void_p, C.c_uint32]
    L.or_alloc_blocks_used.restype = C.c_uint32
    L.or_alloc_blocks_used.argtypes = [C.c_void_p]
    L.or_alloc_free_block_count.restype = C.c_uint32
    L.or_alloc_free_block_count.argtypes = [C.c_void_p]
    L.or_alloc_block_table.restype = C.c_uint32
    L.or_alloc_block_table.argtypes = [C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32)]
    L.or_alloc_table.restype = C.POINTER(C.c_uint32)
    L.or_alloc_table.argtypes = [C.c_void_p]
    L.or_alloc_max_blocks.restype = C.c_uint32
    L.or_alloc_max_blocks.argtypes = [C.c_void_p]
    L.or_pool_new.restype = C.c_void_p
    L.or_pool_new.argtypes = [C.c_int]
    L.or_pool_free.argtypes = [C.c_void_p]
    L.or_pool_threads.restype = C.c_int
    L.or_pool_threads.argtypes = [C.c_void_p]
    L.or_cpu_step.argtypes = [C.c_void_p, _u16p, _u16p, _sz, _u32p, C.c_uint32, _u32p, _u32p, _sz, _u32p, _sz,
                              _f32p, _f32p, _f32p, _sz, _sz, _f32p, _sz, _sz, _sz, _sz, _sz]
    _lib = L
    return L


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- f16, exp

def f32_to_f16(x) -> np.ndarray:
    """quant.rs:25-54 elementwise: float32 array -> uint16 f16 bits."""
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_narrow(x.reshape(-1), out.reshape(-1), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    """quant.rs:57-73 elementwise: uint16 f16 bits -> float32."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_widen(h.reshape(-1), out.reshape(-1), h.size)
    return out


def f32_to_f16_scalar(x: float) -> int:
    return int(lib().or_f32_to_f16(C.c_float(x)))


def f16_check_f16c(start: int, count: int):
    """Compare quant.rs:25-54 with x86 F16C over f32 bit patterns
    [start, start+count); returns (mismatches, NaN patterns seen)."""
    nan = C.c_uint64(0)
    bad = lib().or_f16_check_f16c(start, count, C.byref(nan))
    return int(bad), int(nan.value)


def f16_compare_range(start: int, got: np.ndarray):
    """Compare device f16 bits for bit patterns [start, start+len(got))."""
    got = np.ascontiguousarray(got, dtype=np.uint16)
    first = C.c_uint64(0)
    bad = lib().or_f16_compare_range(start, got.size, got, C.byref(first))
    return int(bad), int(first.value)


def fast_exp(x: float) -> float:
    return float(lib().or_fast_exp(C.c_float(x)))


def softmax(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().or_softmax(x, x.size)
    return x


# --------------------------------------------------------------- attention

def _attention(fn, q, k, v, n_q, q_pos0, n_head, head_dim):
    q, k, v = _f32(q), _f32(k), _f32(v)
    c = n_head * head_dim
    out = np.zeros(n_q * c, np.float32)
    scores = np.zeros(q_pos0 + n_q, np.float32)
    fn(out, q.reshape(-1), c if q.ndim == 1 else q.shape[-1], k.reshape(-1), c if k.ndim == 1 else k.shape[-1],
       v.reshape(-1), c if v.ndim == 1 else v.shape[-1], n_q, q_pos0, n_head, head_dim, scores)
    return out.reshape(n_q, c)


def reference_attention(q, k, v, n_q, q_pos0, n_head, head_dim):
    """reference.rs:109-142 on [rows][C] float32 arrays."""
    return _attention(lib().or_reference_attention, q, k, v, n_q, q_pos0, n_head, head_dim)


def fastops_attention(q, k, v, n_q, q_pos0, n_head, head_dim):
    """fastops.rs:130-213 (attend_one, 16-lane dot, fast exp)."""
    return _attention(lib().or_fastops_attention, q, k, v, n_q, q_pos0, n_head, head_dim)


def attend_f16_portable(q, k16, v16, n_kv):
    """kv16.rs:144-164: q [hd] f32, k16/v16 [n_kv][hd] f16 bits."""
    q = _f32(q)
    hd = q.size
    out = np.zeros(hd, np.float32)
    scores = np.zeros(max(n_kv, 1), np.float32)
    lib().or_attend_f16_portable(out, q, np.ascontiguousarray(k16, np.uint16).reshape(-1),
                                 np.ascontiguousarray(v16, np.uint16).reshape(-1), hd, n_kv, scores)
    return out


def kv16_attention(qkv, k16, v16, capacity, n, pos0, n_head, hd):
    """kv16.rs:168-204 for one layer: qkv [n][3C]; k16/v16 [n_head][cap][hd]."""
    c = n_head * hd
    out = np.zeros(n * c, np.float32)
    scores = np.zeros(pos0 + n, np.float32)
    lib().or_kv16_attention(out, _f32(qkv).reshape(-1), np.ascontiguousarray(k16, np.uint16).reshape(-1),
                            np.ascontiguousarray(v16, np.uint16).reshape(-1), capacity, n, pos0, n_head, hd, scores)
    return out.reshape(n, c)


def split_attention_f64(q, k, v, part):
    """batch.metal:349-424 split + LSE merge in float64; part=0 -> unsplit."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    hd = q.size
    n_kv = k.size // hd
    out = np.zeros(hd, np.float64)
    lib().or_split_attention_f64(out, q, k.reshape(-1), v.reshape(-1), hd, n_kv, part)
    return out


def matvec_f64(x, w, bias=None):
    """batch.metal:94-165 in double: x [n][d_in] f32, w [d_out][d_in] f32,
    bias [d_out] or None -> [n][d_out] float64."""
    x, w = _f32(x), _f32(w)
    n, d_in = x.shape
    d_out = w.shape[0]
    assert w.shape[1] == d_in
    out = np.zeros((n, d_out), np.float64)
    b = None if bias is None else _f32(bias)
    lib().or_matvec_f64(out, x.reshape(-1), d_in, w.reshape(-1), None if b is None else b.ctypes.data, n, d_in, d_out)
    return out


# ------------------------------------------------------------ weight formats

W_FORMAT_IDS = {"f32": 0, "f16": 1, "q8_0": 2, "q4_0": 3}


def quantize(w, fmt: str) -> np.ndarray:
    """The reference's weight upload (weights.rs:12-27, 54-72, 115-118) of a
    row-major matrix w in format fmt, as bytes (uint8)."""
    w = _f32(w).reshape(-1)
    n = w.size
    if fmt == "f32":
        return w.view(np.uint8).copy()
    if fmt == "f16":
        return f32_to_f16(w).view(np.uint8).copy()
    assert n % 32 == 0, "block formats need whole blocks of 32"
    if fmt == "q8_0":
        out = np.zeros(n + n // 16, np.uint8)
        assert lib().or_quantize_q8_0(w, n, out) == out.size
        return out
    if fmt == "q4_0":
        out = np.zeros(n // 2 + n // 16, np.uint8)
        assert lib().or_quantize_q4_0(w, n, out) == out.size
        return out
    raise ValueError(fmt)


def dequantize(q, n: int, fmt: str) -> np.ndarray:
    """weights.rs:29-52 (and the f16/f32 formats): n weights from bytes q."""
    q = np.ascontiguousarray(q, dtype=np.uint8).reshape(-1)
    out = np.zeros(n, np.float32)
    lib().or_dequantize(q, n, W_FORMAT_IDS[fmt], out)
    return out


# ------------------------------------------------------------- paged (CPU)

class PagedPools:
    """The reference's pool layout: k/v [n_layer][kv_blocks][16][C] f16 bits
    (batch.rs:166)."""

    def __init__(self, n_layer, kv_blocks, c):
        self.n_layer, self.kv_blocks, self.c = n_layer, kv_blocks, c
        self.k = np.zeros((n_layer, kv_blocks * KV_BLOCK * c), np.uint16)
        self.v = np.zeros((n_layer, kv_blocks * KV_BLOCK * c), np.uint16)


def kv_slot(table, seq, pos, max_blocks) -> int:
    """batch.metal:24-26."""
    return int(lib().or_kv_slot(np.ascontiguousarray(table, np.uint32).reshape(-1), seq, pos, max_blocks))


def paged_append(pools: PagedPools, layer, table, max_blocks, seqs, poss, k, v):
    """batch.metal:329-344 for one layer; k/v [n][C] float32."""
    k, v = _f32(k), _f32(v)
    n = len(seqs)
    lib().or_paged_append(pools.k[layer], pools.v[layer], np.ascontiguousarray(table, np.uint32).reshape(-1),
                          max_blocks, np.ascontiguousarray(seqs, np.uint32), np.ascontiguousarray(poss, np.uint32), n,
                          k.reshape(-1), v.reshape(-1), k.shape[-1] if k.ndim > 1 else pools.c, pools.c)


def paged_gather(pools: PagedPools, layer, table, max_blocks, seqs, poss):
    """K/V f16 bits [n][C] of (seq, pos) rows through kv_slot."""
    n = len(seqs)
    ko = np.zeros((n, pools.c), np.uint16)
    vo = np.zeros((n, pools.c), np.uint16)
    lib().or_paged_gather(ko, vo, pools.k[layer], pools.v[layer], np.ascontiguousarray(table, np.uint32).reshape(-1),
                          max_blocks, np.ascontiguousarray(seqs, np.uint32), np.ascontiguousarray(poss, np.uint32), n, pools.c)
    return ko, vo


def paged_attention(pools: PagedPools, layer, table, max_blocks, seqs, poss, q, n_head, hd):
    """Per row (seq, pos): kv16.rs:144-164 over keys 0..=pos found by kv_slot.
    q [n][C] float32 -> out [n][C] float32."""
    q = _f32(q)
    n = len(seqs)
    c = n_head * hd
    out = np.zeros((n, c), np.float32)
    max_kv = int(max(poss)) + 1 if n else 1
    scores = np.zeros(max_kv, np.float32)
    lib().or_paged_attention(out, c, q.reshape(-1), q.shape[-1] if q.ndim > 1 else c, pools.k[layer],
                             pools.v[layer], np.ascontiguousarray(table, np.uint32).reshape(-1), max_blocks,
                             np.ascontiguousarray(seqs, np.uint32), np.ascontiguousarray(poss, np.uint32), n, n_head, hd, scores)
    return out


# ------------------------------------------------------------ Q8 cache (CPU)

def q8_quantize(x):
    """kv8.metal:15-48 for one (position, head): (int8 values, f32 scale)."""
    x = _f32(x).reshape(-1)
    q = np.zeros(x.size, np.int8)
    scale = lib().or_q8_quantize(x, x.size, q)
    return q, np.float32(scale)


class PagedPoolsQ8:
    """Q8 pools in the reference's row layout: values [n_layer][kv_blocks*16][C]
    int8, scales [n_layer][kv_blocks*16][n_head] f32."""

    def __init__(self, n_layer, kv_blocks, n_head, hd):
        self.n_layer, self.kv_blocks, self.n_head, self.hd = n_layer, kv_blocks, n_head, hd
        c = n_head * hd
        self.kq = np.zeros((n_layer, kv_blocks * KV_BLOCK * c), np.int8)
        self.vq = np.zeros_like(self.kq)
        self.ks = np.zeros((n_layer, kv_blocks * KV_BLOCK * n_head), np.float32)
        self.vs = np.zeros_like(self.ks)


def paged_q8_append(pools: PagedPoolsQ8, layer, table, max_blocks, seqs, poss, k, v):
    k, v = _f32(k), _f32(v)
    n = len(seqs)
    lib().or_paged_q8_append(pools.kq[layer], pools.vq[layer], pools.ks[layer], pools.vs[layer],
                             np.ascontiguousarray(table, np.uint32).reshape(-1), max_blocks,
                             np.ascontiguousarray(seqs, np.uint32), np.ascontiguousarray(poss, np.uint32), n,
                             k.reshape(-1), v.reshape(-1), k.shape[-1], pools.n_head, pools.hd)


def paged_q8_gather(pools: PagedPoolsQ8, layer, table, max_blocks, seqs, poss):
    """(k, v) int8 [n][C] and (ks, vs) f32 [n][n_head] of (seq, pos) rows."""
    c, h = pools.n_head * pools.hd, pools.n_head
    slots = [kv_slot(table, s, p, max_blocks) for s, p in zip(seqs, poss)]
    kq = pools.kq[layer].reshape(-1, c)[slots]
    vq = pools.vq[layer].reshape(-1, c)[slots]
    ks = pools.ks[layer].reshape(-1, h)[slots]
    vs = pools.vs[layer].reshape(-1, h)[slots]
    return (kq, vq), (ks, vs)


def paged_q8_attention(pools: PagedPoolsQ8, layer, table, max_blocks, seqs, poss, q):
    q = _f32(q)
    n = len(seqs)
    c = pools.n_head * pools.hd
    out = np.zeros((n, c), np.float32)
    scores = np.zeros(int(max(poss)) + 1 if n else 1, np.float64)
    lib().or_paged_q8_attention(out, c, q.reshape(-1), q.shape[-1] if q.ndim > 1 else c, pools.kq[layer],
                                pools.vq[layer], pools.ks[layer], pools.vs[layer],
                                np.ascontiguousarray(table, np.uint32).reshape(-1), max_blocks,
                                np.ascontiguousarray(seqs, np.uint32), np.ascontiguousarray(poss, np.uint32), n,
                                pools.n_head, pools.hd, scores)
    return out


# --------------------------------------------------------------- allocator

class Alloc:
    """batch.rs:129-254 page allocator, restated in C."""

    def __init__(self, kv_blocks, max_seqs, n_ctx, order=None):
        self.kv_blocks, self.max_seqs, self.n_ctx = kv_blocks, max_seqs, n_ctx
        self._order = None if order is None else np.ascontiguousarray(order, np.uint32)
        ptr = None if self._order is None else self._order.ctypes.data
        self._a = lib().or_alloc_new(kv_blocks, max_seqs, n_ctx, ptr)
        self.max_blocks = int(lib().or_alloc_max_blocks(self._a))

    def __del__(self):
        if getattr(self, "_a", None):
            lib().or_alloc_free(self._a)
            self._a = None

    def add_seq(self):
        s = lib().or_alloc_add_seq(self._a)
        return None if s < 0 else int(s)

    def free_seq(self, s):
        lib().or_alloc_free_seq(self._a, s)

    def truncate(self, s, n):
        if lib().or_alloc_truncate(self._a, s, n) != 0:
            raise AssertionError("assertion failed: len <= self.seq_len[s]")

    def ensure(self, s, n):
        """0 ok, 1 context full, 2 pool exhausted."""
        return int(lib().or_alloc_ensure(self._a, s, n))

    def commit(self, s, n):
        lib().or_alloc_commit(self._a, s, n)

    def seq_len(self, s):
        return int(lib().or_alloc_seq_len(self._a, s))

    def live(self, s):
        return bool(lib().or_alloc_live(self._a, s))

    def blocks_used(self):
        return int(lib().or_alloc_blocks_used(self._a))

    def free_block_count(self):
        return int(lib().or_alloc_free_block_count(self._a))

    def block_table(self, s):
        buf = (C.c_uint32 * self.max_blocks)()
        n = lib().or_alloc_block_table(self._a, s, buf)
        return [int(buf[i]) for i in range(n)]

    def table(self) -> np.ndarray:
        """Dense [max_seqs][max_blocks] table (unused entries 0), a copy."""
        p = lib().or_alloc_table(self._a)
        return np.ctypeslib.as_array(p, shape=(self.max_seqs * self.max_blocks,)).copy().reshape(
            self.max_seqs, self.max_blocks)


# -------------------------------------------------------- threaded CPU step

class CpuStep:
    """The reported CPU baseline: the reference's x86 CPU path per layer
    (append, then attention units on a thread pool), over paged pools."""

    def __init__(self, threads=None):
        self.threads = int(threads or os.cpu_count() or 1)
        self._p = lib().or_pool_new(self.threads)

    def __del__(self):
        if getattr(self, "_p", None):
            lib().or_pool_free(self._p)
            self._p = None

    def run(self, pools: PagedPools, table, max_blocks, seqs, poss, qrows, q, k, v, out, n_head, hd):
        """q/k/v/out: contiguous [n_layer][rows][C] float32 with rows >= the
        step's rows (row t of layer l at l*rows*C + t*C)."""
        n_layer = pools.n_layer
        n = len(seqs)
        c = n_head * hd
        for a in (q, k, v, out):
            assert a.dtype == np.float32 and a.flags.c_contiguous and a.shape[0] == n_layer and a.shape[1] >= n
        ls = q.shape[1] * c
        assert k.shape[1] * c == ls and v.shape[1] * c == ls
        lib().or_cpu_step(self._p, pools.k.reshape(-1), pools.v.reshape(-1), pools.kv_blocks,
                          np.ascontiguousarray(table, np.uint32).reshape(-1), max_blocks,
                          np.ascontiguousarray(seqs, np.uint32), np.ascontiguousarray(poss, np.uint32), n,
                          np.ascontiguousarray(qrows, np.uint32), len(qrows), q.reshape(-1), k.reshape(-1), v.reshape(-1),
                          c, ls, out.reshape(-1), c, out.shape[1] * c, n_layer, n_head, hd)
