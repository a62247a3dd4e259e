"""nanoinfer_amd -- MI355X (gfx950) paged f16 KV-cache hot path of nanoinfer.

The product is the C-ABI library ``libnanoinfer_kv.so`` (``include/nanoinfer_kv.h``):
HIP kernels for the f16 append, the block-table gather and paged
flash-decoding attention with split-K and a log-sum-exp merge, plus the C++
page allocator.  This package holds its sources (``csrc/``), its build recipe
(``build.py``), the ctypes binding (``_abi.py``), the host mirror of the
reference's ``Batch`` API (``batch.py``) and the synthetic workloads of the
benchmark configurations (``workloads.py``).
"""
from .batch import ALL_LAYERS, KV_BLOCK, BatchOpts, KvError, PagedKv, attention, f32_to_f16_device

__all__ = ["ALL_LAYERS", "KV_BLOCK", "BatchOpts", "KvError", "PagedKv", "attention", "f32_to_f16_device"]
