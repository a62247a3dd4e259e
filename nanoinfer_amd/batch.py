"""Host-side mirror of the reference's paged-KV ``Batch`` API over the C ABI.

``PagedKv`` keeps the names, argument meanings and error behaviour of the KV
part of ``Batch`` (``crates/metal/src/batch.rs:128-363``):

=====================  ==========================================  ==================
reference              here                                        batch.rs
=====================  ==========================================  ==================
``add_seq``            ``add_seq() -> int | None``                 :201-206
``free_seq``           ``free_seq(s)``                             :209-212
``seq_len``            ``seq_len(s)``                              :214-216
``truncate``           ``truncate(s, len)`` (AssertionError)       :220-227
``block_table``        ``block_table(s) -> list[int]``             :230-232
``blocks_used``        ``blocks_used()``                           :235-237
``free_block_count``   ``free_block_count()``                      :238-240
``ensure_blocks``      ``reserve(s, len)``                         :243-254
``step``               ``step(work, q, k, v, out)``                :259-315
``decode_resident``    ``decode_steps(seqs, q, k, v, out)``        :322-363
``kv_block_bytes``     ``kv_block_bytes()``                        :107-109
=====================  ==========================================  ==================

``Err(String)`` results raise :class:`KvError` carrying the reference's text;
the reference's panics (``truncate`` past the length) raise
``AssertionError``.  Device buffers are torch tensors on the GPU (float32 for
q/k/v/out, int16 for gathered f16 bits); work is enqueued on the current torch
stream.  Nothing here computes on the CPU: every data call goes to the gfx950
library and fails if it cannot.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _abi
from ._abi import NI_ALL_LAYERS, NI_KV_BLOCK

ALL_LAYERS = NI_ALL_LAYERS
KV_BLOCK = NI_KV_BLOCK


class KvError(RuntimeError):
    """A failed call; ``code`` is the NI_ERR_* status, ``str()`` the message."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


@dataclass
class BatchOpts:
    """Sizes of a :class:`PagedKv` (the KV fields of ``BatchOpts``,
    batch.rs:44-76, plus the model shape of ``Config``)."""

    n_layer: int = 12
    n_head: int = 12
    head_dim: int = 64
    kv_blocks: int = 1024
    max_seqs: int = 64
    n_ctx: int = 1024
    max_rows: int = 512
    host_only: bool = False
    page_order: Optional[Sequence[int]] = None  # order in which pages are handed out
    q8: bool = False  # int8 K/V + f32 scale per (position, head) (kv8.metal)

    @property
    def n_embd(self) -> int:
        return self.n_head * self.head_dim


def _stream_ptr(stream) -> int:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _rows(rows) -> tuple:
    arr = np.ascontiguousarray(np.asarray(rows, dtype=np.uint32).reshape(-1, 2))
    n = arr.shape[0]
    return arr, arr.ctypes.data_as(C.POINTER(_abi.ni_row)), n


def _f32_arg(t, name, layered, rows, c, n_layer):
    """(row_stride, layer_stride) of a float32 tensor laid out
    [n_layer][>= rows][c] (layered) or [>= rows][c], unit stride in its last
    dimension.  The C ABI sees only pointers and strides, so a short tensor is
    refused here, before any device access (`_on_device` checks placement
    once every layout has passed)."""
    import torch

    if not isinstance(t, torch.Tensor) or t.dtype != torch.float32:
        raise TypeError(f"{name} must be a float32 CUDA tensor")
    if layered:
        if t.dim() != 3 or t.stride(2) != 1:
            raise ValueError(f"{name} must be [n_layer, rows, C] with unit stride in C")
        if t.shape[0] != n_layer or t.shape[1] < rows or t.shape[2] != c:
            raise ValueError(f"{name} is {list(t.shape)}: needs [{n_layer}, >= {rows}, {c}]")
        return t.stride(1), t.stride(0)
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be [rows, C] with unit stride in C")
    if t.shape[0] < rows or t.shape[1] != c:
        raise ValueError(f"{name} is {list(t.shape)}: needs [>= {rows}, {c}]")
    return t.stride(0), 0


def _on_device(device, **tensors):
    """Every tensor on the GPU, on the cache's device."""
    for name, t in tensors.items():
        if t is None:
            continue
        if not t.is_cuda:
            raise TypeError(f"{name} must be a float32 CUDA tensor")
        if device is not None and t.device.index != device:
            raise ValueError(f"{name} is on cuda:{t.device.index}, the cache on cuda:{device}")


# Weight formats of the QKV projection (the reference's DType, crates/metal/src/lib.rs:36-43).
W_FORMATS = {"f32": _abi.NI_W_F32, "f16": _abi.NI_W_F16, "q8_0": _abi.NI_W_Q8_0, "q4_0": _abi.NI_W_Q4_0}


def w_bytes(fmt: str, n: int) -> int:
    """Bytes of n weights in format fmt (weights.rs:12-86: quants, then one
    f16 scale per block of 32)."""
    return {"f32": 4 * n, "f16": 2 * n, "q8_0": n + n // 16, "q4_0": n // 2 + n // 16}[fmt]


def _weights(w, bias, c, d_in, fmt="f32"):
    """Check the layout of W [3C, d_in] in format fmt (f32: a contiguous
    float32 [3C, d_in] tensor; otherwise a contiguous uint8 tensor of the
    format's bytes) and bias."""
    import torch

    if fmt not in W_FORMATS:
        raise ValueError(f"unknown weight format {fmt!r} (one of {sorted(W_FORMATS)})")
    if fmt == "f32":
        if not isinstance(w, torch.Tensor) or w.dtype != torch.float32 or not w.is_contiguous() \
                or tuple(w.shape) != (3 * c, d_in):
            raise ValueError(f"w must be a contiguous float32 CUDA tensor [{3 * c}, {d_in}]")
    else:
        if fmt != "f16" and d_in % 32:
            raise ValueError(f"d_in {d_in} must be a multiple of 32 for {fmt}")
        need = w_bytes(fmt, 3 * c * d_in)
        if not isinstance(w, torch.Tensor) or not w.is_contiguous() or w.numel() * w.element_size() != need:
            raise ValueError(f"w must be a contiguous tensor of the {need} bytes of a [{3 * c}, {d_in}] {fmt} matrix")
    if bias is not None and (not isinstance(bias, torch.Tensor) or bias.dtype != torch.float32
                             or not bias.is_contiguous() or bias.numel() != 3 * c):
        raise ValueError(f"bias must be a contiguous float32 CUDA tensor of {3 * c} values")


def _work(work) -> np.ndarray:
    w = np.ascontiguousarray(np.asarray(work, dtype=np.uint32).reshape(-1, 3))
    return w


def _work_rows(w: np.ndarray) -> int:
    """Rows a step's work numbers (sum of n_new)."""
    return int(w[:, 1].astype(np.int64).sum())


class PagedKv:
    """The KV cache and block tables of a batch of sequences on one MI355X."""

    def __init__(self, opts: BatchOpts):
        self.opts = opts
        self._L = _abi.lib()
        o = _abi.ni_kv_opts()
        o.n_layer, o.n_head, o.head_dim = opts.n_layer, opts.n_head, opts.head_dim
        o.kv_pages, o.max_seqs, o.max_ctx, o.max_rows = opts.kv_blocks, opts.max_seqs, opts.n_ctx, opts.max_rows
        o.flags = (_abi.NI_KV_HOST_ONLY if opts.host_only else 0) | (_abi.NI_KV_Q8 if opts.q8 else 0)
        self._order = None
        if opts.page_order is not None:
            self._order = np.ascontiguousarray(np.asarray(opts.page_order, dtype=np.uint32))
            o.page_order = self._order.ctypes.data_as(C.POINTER(C.c_uint32))
        # The device a handle lives on is the current one at creation.
        self.device = None
        if not opts.host_only:
            import torch

            self.device = torch.cuda.current_device()
        self._open_rows = None  # rows of the step opened by step_begin
        h = C.c_void_p()
        rc = self._L.ni_kv_create(C.byref(o), C.byref(h))
        if rc != 0:
            raise KvError(rc, self._L.ni_kv_last_error(None).decode())
        self._h = h

    # -------------------------------------------------------------- plumbing
    def close(self):
        if getattr(self, "_h", None):
            self._L.ni_kv_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    def _check(self, rc):
        if rc != 0:
            raise KvError(rc, self._L.ni_kv_last_error(self._h).decode())

    def _f32(self, t, name, layered, rows, c=None):
        return _f32_arg(t, name, layered, rows, self.opts.n_embd if c is None else c, self.opts.n_layer)

    def _on_device(self, **tensors):
        _on_device(self.device, **tensors)

    @property
    def max_blocks(self) -> int:
        """Pages per sequence at most: ceil(n_ctx / 16) (batch.rs:164)."""
        return -(-self.opts.n_ctx // KV_BLOCK)

    # ------------------------------------------------------------ bookkeeping
    def add_seq(self) -> Optional[int]:
        s = C.c_uint32()
        rc = self._L.ni_kv_add_seq(self._h, C.byref(s))
        if rc == _abi.NI_ERR_NO_SLOT:
            return None
        self._check(rc)
        return int(s.value)

    def free_seq(self, s: int):
        self._check(self._L.ni_kv_free_seq(self._h, s))

    def seq_len(self, s: int) -> int:
        n = C.c_uint32()
        self._check(self._L.ni_kv_seq_len(self._h, s, C.byref(n)))
        return int(n.value)

    def is_live(self, s: int) -> bool:
        v = C.c_int()
        self._check(self._L.ni_kv_is_live(self._h, s, C.byref(v)))
        return bool(v.value)

    def truncate(self, s: int, length: int):
        rc = self._L.ni_kv_truncate(self._h, s, length)
        if rc == _abi.NI_ERR_BAD_LEN:
            raise AssertionError(self._L.ni_kv_last_error(self._h).decode())
        self._check(rc)

    def reserve(self, s: int, length: int):
        self._check(self._L.ni_kv_reserve(self._h, s, length))

    def commit(self, s: int, n: int):
        self._check(self._L.ni_kv_commit(self._h, s, n))

    def block_table(self, s: int) -> list:
        p = C.POINTER(C.c_uint32)()
        n = C.c_uint32()
        self._check(self._L.ni_kv_block_table(self._h, s, C.byref(p), C.byref(n)))
        return [int(p[i]) for i in range(n.value)]

    def blocks_used(self) -> int:
        return int(self._L.ni_kv_blocks_used(self._h))

    def free_block_count(self) -> int:
        return int(self._L.ni_kv_free_block_count(self._h))

    def kv_block_bytes(self) -> int:
        return int(self._L.ni_kv_page_bytes(self._h))

    # -------------------------------------------------------------- data path
    def append(self, rows, k, v, layer: int = ALL_LAYERS, stream=None):
        """Write f32 K/V rows as f16 into their pages (b_kv_write)."""
        arr, rp, n = _rows(rows)
        layered = layer == ALL_LAYERS
        rs, ls = self._f32(k, "k", layered, n)
        rs2, ls2 = self._f32(v, "v", layered, n)
        if (rs, ls) != (rs2, ls2):
            raise ValueError("k and v must share strides")
        self._on_device(k=k, v=v)
        self._check(self._L.ni_kv_append(self._h, layer, rp, n, k.data_ptr(), v.data_ptr(), rs, ls,
                                         _stream_ptr(stream)))

    def qkv_append(self, rows, x, w, bias=None, q_out=None, layer: int = 0, stream=None, w_format: str = "f32"):
        """The QKV projection with the append in its epilogue (BEPI_QKV):
        x [n, d_in], w [3C, d_in], bias [3C] float32 CUDA tensors; k/v go to
        the rows' page slots of `layer` as f16, q is returned [n, C].
        w_format "f16", "q8_0" or "q4_0": w holds the matrix in the
        reference's format (weights.rs:12-86), any dtype, contiguous."""
        import torch

        arr, rp, n = _rows(rows)
        if not isinstance(x, torch.Tensor) or x.dim() != 2:
            raise ValueError("x must be a [rows, d_in] tensor")
        xs, _ = self._f32(x, "x", False, n, c=x.shape[1])
        _weights(w, bias, self.opts.n_embd, x.shape[1], w_format)
        if q_out is not None:
            self._f32(q_out, "q_out", False, n)
        self._on_device(x=x, w=w, bias=bias, q_out=q_out)
        if q_out is None:
            q_out = torch.zeros((n, self.opts.n_embd), dtype=torch.float32, device=x.device)
        qs, _ = self._f32(q_out, "q_out", False, n)
        self._check(self._L.ni_kv_qkv_append_w(self._h, layer, rp, n, x.data_ptr(), xs, x.shape[1], w.data_ptr(),
                                               W_FORMATS[w_format], None if bias is None else bias.data_ptr(),
                                               q_out.data_ptr(), qs, _stream_ptr(stream)))
        return q_out

    def qkv_project(self, x, w, bias=None, out=None, stream=None, w_format: str = "f32"):
        """The same projection, every output column to out [n, 3C] (f32)."""
        import torch

        if not isinstance(x, torch.Tensor) or x.dim() != 2:
            raise ValueError("x must be a [rows, d_in] tensor")
        xs, _ = self._f32(x, "x", False, x.shape[0], c=x.shape[1])
        _weights(w, bias, self.opts.n_embd, x.shape[1], w_format)
        if out is not None:
            self._f32(out, "out", False, x.shape[0], c=3 * self.opts.n_embd)
        self._on_device(x=x, w=w, bias=bias, out=out)
        if out is None:
            out = torch.zeros((x.shape[0], 3 * self.opts.n_embd), dtype=torch.float32, device=x.device)
        os_, _ = self._f32(out, "out", False, x.shape[0], c=3 * self.opts.n_embd)
        self._check(self._L.ni_kv_qkv_project_w(self._h, x.data_ptr(), xs, x.shape[0], x.shape[1], w.data_ptr(),
                                                W_FORMATS[w_format], None if bias is None else bias.data_ptr(),
                                                out.data_ptr(), os_, _stream_ptr(stream)))
        return out

    def gather(self, rows, layer: int = ALL_LAYERS, stream=None):
        """f16 bits (int16 tensors) of K and V at each (seq, pos) row."""
        import torch

        arr, rp, n = _rows(rows)
        c = self.opts.n_embd
        shape = (self.opts.n_layer, n, c) if layer == ALL_LAYERS else (n, c)
        ko = torch.empty(shape, dtype=torch.int16, device="cuda")
        vo = torch.empty(shape, dtype=torch.int16, device="cuda")
        ls = n * c if layer == ALL_LAYERS else 0
        self._check(self._L.ni_kv_gather(self._h, layer, rp, n, ko.data_ptr(), vo.data_ptr(), c, ls,
                                         _stream_ptr(stream)))
        return ko, vo

    def gather_q8(self, rows, layer: int = ALL_LAYERS, stream=None):
        """Q8 handles: (k int8, v int8) [n_lay, n, C] and (k scale, v scale)
        float32 [n_lay, n, n_head] of each (seq, pos) row."""
        import torch

        arr, rp, n = _rows(rows)
        n_lay = self.opts.n_layer if layer == ALL_LAYERS else 1
        c, h = self.opts.n_embd, self.opts.n_head
        ko = torch.empty((n_lay, n, c), dtype=torch.int8, device="cuda")
        vo = torch.empty_like(ko)
        ks = torch.empty((n_lay, n, h), dtype=torch.float32, device="cuda")
        vs = torch.empty_like(ks)
        self._check(self._L.ni_kv_gather_q8(self._h, layer, rp, n, ko.data_ptr(), vo.data_ptr(), ks.data_ptr(),
                                            vs.data_ptr(), _stream_ptr(stream)))
        return (ko, vo), (ks, vs)

    def attention(self, q, rows, out=None, layer: int = ALL_LAYERS, split_tokens: int = 0, stream=None):
        """Paged decode attention of each row over keys 0..pos of its sequence."""
        import torch

        arr, rp, n = _rows(rows)
        layered = layer == ALL_LAYERS
        qrs, qls = self._f32(q, "q", layered, n)
        if out is not None:
            self._f32(out, "out", layered, n)
        self._on_device(q=q, out=out)
        if out is None:
            out = torch.zeros_like(q)
        ors, ols = self._f32(out, "out", layered, n)
        self._check(self._L.ni_paged_decode_attention(self._h, layer, q.data_ptr(), qrs, qls, rp, n, out.data_ptr(),
                                                      ors, ols, split_tokens, _stream_ptr(stream)))
        return out

    def step(self, work, q, k, v, out=None, split_tokens: int = 0, stream=None):
        """One step over every layer (Batch::step's KV part).  ``work`` lists
        ``(seq, n_new, n_query)``; rows are numbered in work order; q/k/v/out
        are [n_layer, rows, C]."""
        import torch

        w = _work(work)
        wp = w.ctypes.data_as(C.POINTER(_abi.ni_work))
        n = _work_rows(w)
        rs3, ls3 = self._f32(q, "q", True, n)
        rs, ls = self._f32(k, "k", True, n)
        rs2, ls2 = self._f32(v, "v", True, n)
        if not (rs == rs2 == rs3 and ls == ls2 == ls3):
            raise ValueError("q, k and v must share strides")
        if out is not None:
            self._f32(out, "out", True, n)
        self._on_device(q=q, k=k, v=v, out=out)
        if out is None:
            out = torch.zeros_like(q)
        ors, ols = self._f32(out, "out", True, n)
        self._check(self._L.ni_kv_step(self._h, wp, w.shape[0], q.data_ptr(), k.data_ptr(), v.data_ptr(), rs, ls,
                                       out.data_ptr(), ors, ols, split_tokens, _stream_ptr(stream)))
        return out

    def step_begin(self, work, split_tokens: int = 0):
        """Check, reserve and plan one step (``work`` as in :meth:`step`) whose
        layers then run one :meth:`step_layer` call each, as a model's forward
        does (batch.rs:280-306 encodes once, batch.rs:390-416 dispatches per
        layer); :meth:`step_end` commits it."""
        w = _work(work)
        self._check(self._L.ni_kv_step_begin(self._h, w.ctypes.data_as(C.POINTER(_abi.ni_work)), w.shape[0],
                                             split_tokens))
        self._open_rows = _work_rows(w)

    def step_layer(self, layer: int, q, k, v, out=None, stream=None):
        """Layer ``layer`` of the open step: its new rows appended and its
        queried rows attended in one launch; q/k/v/out are [rows, C]."""
        import torch

        n = self._open_rows or 0
        rs3, _ = self._f32(q, "q", False, n)
        rs, _ = self._f32(k, "k", False, n)
        rs2, _ = self._f32(v, "v", False, n)
        if not rs == rs2 == rs3:
            raise ValueError("q, k and v must share a row stride")
        if out is not None:
            self._f32(out, "out", False, n)
        self._on_device(q=q, k=k, v=v, out=out)
        if out is None:
            out = torch.zeros_like(q)
        ors, _ = self._f32(out, "out", False, n)
        self._check(self._L.ni_kv_step_layer(self._h, layer, q.data_ptr(), k.data_ptr(), v.data_ptr(), rs,
                                             out.data_ptr(), ors, _stream_ptr(stream)))
        return out

    def step_end(self):
        """Commit the open step: every work item's sequence grows by n_new."""
        self._open_rows = None
        self._check(self._L.ni_kv_step_end(self._h))

    def decode_steps(self, seqs, q, k, v, out=None, split_tokens: int = 0, stream=None):
        """decode_resident's KV part: q/k/v are [steps, n_layer, len(seqs), C];
        step t appends and attends position seq_len + t of every sequence."""
        import torch

        s = np.ascontiguousarray(np.asarray(seqs, dtype=np.uint32).reshape(-1))
        sp = s.ctypes.data_as(C.POINTER(C.c_uint32))
        if out is None and isinstance(q, torch.Tensor):
            out = torch.zeros_like(q)
        for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
            if not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or t.dim() != 4 or t.stride(3) != 1:
                raise ValueError(f"{name} must be a float32 CUDA tensor [steps, n_layer, rows, C] with unit stride in C")
            if t.shape[1] != self.opts.n_layer or t.shape[2] < s.size or t.shape[3] != self.opts.n_embd:
                raise ValueError(f"{name} is {list(t.shape)}: needs [steps, {self.opts.n_layer}, >= {s.size}, "
                                 f"{self.opts.n_embd}]")
        if not (q.stride() == k.stride() == v.stride()) or not (q.shape == k.shape == v.shape):
            raise ValueError("q, k and v must share shapes and strides")
        if out.shape[0] < q.shape[0]:
            raise ValueError(f"out holds {out.shape[0]} steps, q {q.shape[0]}")
        self._on_device(q=q, k=k, v=v, out=out)
        self._check(self._L.ni_kv_decode_steps(self._h, sp, s.size, q.shape[0], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                               q.stride(2), q.stride(1), q.stride(0), out.data_ptr(), out.stride(2),
                                               out.stride(1), out.stride(0), split_tokens, _stream_ptr(stream)))
        return out

    def sync(self, stream=None):
        self._check(self._L.ni_kv_sync(self._h, _stream_ptr(stream)))

    def pools(self):
        kp, vp, nb = C.c_void_p(), C.c_void_p(), C.c_size_t()
        self._check(self._L.ni_kv_pools(self._h, C.byref(kp), C.byref(vp), C.byref(nb)))
        return kp.value, vp.value, nb.value

    # ------------------------------------------------------------ measurement
    def profile(self, kernels=(0, 1, 2)):
        """Bracket launches of the listed kernels (0 append, 1 attention,
        2 merge) with HIP events; an empty list stops."""
        mask = 0
        for k in kernels:
            mask |= 1 << int(k)
        self._check(self._L.ni_kv_profile(self._h, mask))

    def profile_read(self, kernel: int):
        """(total ms, launches) of one kernel since the last read."""
        ms, n = C.c_double(), C.c_uint64()
        self._check(self._L.ni_kv_profile_read(self._h, kernel, C.byref(ms), C.byref(n)))
        return float(ms.value), int(n.value)


def attention(q, k, v, n_q: int, q_pos0: int, n_head: int, head_dim: int, out=None, stream=None):
    """``Kernels::attention`` (crates/core/src/kernels/mod.rs:86-98; the math
    of ``reference::attention``, kernels/reference.rs:109-142) on the GPU
    through ``ni_attention``: causal multi-head attention of the ``n_q``
    queries at positions ``q_pos0 ..`` over f32 K/V rows ``0 .. q_pos0+n_q-1``.

    q, k and v are 2-D float32 CUDA tensors whose rows are positions (the
    reference's ``Rows``: any row stride, e.g. views of a fused ``[n][3C]``
    buffer); q holds ``n_q`` rows, k and v at least ``q_pos0 + n_q``, each at
    least ``C = n_head * head_dim`` wide.  Returns ``out`` ([n_q][C] float32,
    allocated if not given).  No scores buffer is needed."""
    import torch

    c = n_head * head_dim
    if n_q < 0 or q_pos0 < 0:
        raise ValueError("n_q and q_pos0 must be >= 0")
    args = (("q", q, n_q), ("k", k, q_pos0 + n_q), ("v", v, q_pos0 + n_q))
    for name, t, rows in args:  # layout first, then the device
        if not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or t.dim() != 2:
            raise TypeError(f"{name} must be a 2-D float32 tensor")
        if t.stride(1) != 1:
            raise ValueError(f"{name} rows must be contiguous")
        if t.shape[0] < rows or t.shape[1] < c:
            raise ValueError(f"{name} is {tuple(t.shape)}; needs at least {rows} rows of {c}")
    for name, t, _ in args:
        if not t.is_cuda:
            raise TypeError(f"{name} must be a CUDA tensor")
        if t.device != q.device:
            raise ValueError(f"{name} is on {t.device}, q on {q.device}")
    if out is None:
        out = torch.empty((n_q, c), dtype=torch.float32, device=q.device)
    if (not isinstance(out, torch.Tensor) or out.dtype != torch.float32 or out.dim() != 2 or out.stride(1) != 1
            or out.shape[0] < n_q or out.shape[1] < c or out.device != q.device):
        raise ValueError(f"out must be a float32 [{n_q}][{c}] tensor on {q.device} with contiguous rows")
    L = _abi.lib()
    rc = L.ni_attention(out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0),
                        v.data_ptr(), v.stride(0), n_q, q_pos0, n_head, head_dim, _stream_ptr(stream))
    if rc != 0:
        raise KvError(rc, (L.ni_kv_last_error(None) or b"").decode())
    return out


def f32_to_f16_device(x, out=None, stream=None):
    """quant.rs:25-54 on the GPU, elementwise, through the library's device
    conversion (the one the append uses).  Returns int16 bits."""
    import torch

    if not x.is_cuda or x.dtype != torch.float32 or not x.is_contiguous():
        raise TypeError("x must be a contiguous float32 CUDA tensor")
    if out is None:
        out = torch.empty(x.shape, dtype=torch.int16, device=x.device)
    rc = _abi.lib().ni_f32_to_f16(x.data_ptr(), out.data_ptr(), x.numel(), _stream_ptr(stream))
    if rc != 0:
        raise KvError(rc, "ni_f32_to_f16 failed")
    return out
