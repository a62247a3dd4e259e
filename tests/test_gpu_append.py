"""Device f16 conversion, append and gather: bit-exact against the oracle
(quant.rs:25-54, batch.metal:24-26,329-344)."""
import concurrent.futures as cf
import sys

import numpy as np
import pytest
import torch

import oracle
import nanoinfer_amd as na
from nanoinfer_amd import _abi
from paged_mirror import Mirror

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def test_device_conversion_all_f32_patterns(gpu, oracle_lib):
    """All 2^32 f32 bit patterns through the device conversion the append
    uses, compared with the oracle (NaNs included: canonical sign|0x7e00)."""
    chunk = 1 << 27
    bad_total = 0
    pool = cf.ThreadPoolExecutor(8)
    for start in range(0, 1 << 32, chunk):
        idx = torch.arange(start, start + chunk, dtype=torch.int64, device=gpu)
        bits = torch.where(idx >= (1 << 31), idx - (1 << 32), idx).to(torch.int32)
        x = bits.view(torch.float32)
        h = na.f32_to_f16_device(x)
        got = h.cpu().numpy().view(np.uint16)
        del idx, bits, x, h
        sub = chunk // 8
        res = list(pool.map(lambda i: oracle.f16_compare_range(start + i * sub, got[i * sub:(i + 1) * sub]),
                            range(8)))
        bad = sum(r[0] for r in res)
        if bad:
            first = min(r[1] for r in res if r[0])
            say(f"chunk {start:#x}: {bad} mismatches, first pattern {first:#010x}")
        bad_total += bad
    pool.shutdown()
    assert bad_total == 0


def gpt2_opts(**kw):
    base = dict(n_layer=12, n_head=12, head_dim=64, kv_blocks=96, max_seqs=4, n_ctx=1024, max_rows=512)
    base.update(kw)
    return na.BatchOpts(**base)


def test_append_gather_bit_exact_all_layers(gpu, oracle_lib):
    rng = np.random.default_rng(10)
    order = rng.permutation(96).tolist()
    m = Mirror(gpt2_opts(page_order=order))
    seqs = [m.kv.add_seq() for _ in range(3)]
    for s, L in zip(seqs, [1, 17, 300]):
        m.fill(s, L, rng, chunk=97)  # ragged chunks across page boundaries
    rows = [(s, p) for s, L in zip(seqs, [1, 17, 300]) for p in range(L)]
    (kg, vg), (kw, vw) = m.gather(rows)
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)
    # single-layer gather of layer 7 equals its slice
    (k7, v7), _ = m.gather(rows, layer=7)
    assert np.array_equal(k7, kg[7]) and np.array_equal(v7, vg[7])


def test_append_values_are_the_reference_rounding(gpu, oracle_lib):
    """The gathered bits are exactly quant.rs:25-54 of the inputs, including
    ties, subnormals, overflow to inf and NaN."""
    m = Mirror(gpt2_opts(n_layer=1, kv_blocks=4, max_seqs=1))
    s = m.kv.add_seq()
    m.kv.reserve(s, 4)
    c = m.c
    special = np.array([1.0 + 1 / 2048, 1.0 + 3 / 2048, 65519.0, 65520.0, -65520.0, 6.0e-8, 3.0e-8, 2.9e-8,
                        5.9604645e-8, 1e-45, -1e-45, np.inf, -np.inf, np.nan, -np.nan, 0.0, -0.0], np.float32)
    rng = np.random.default_rng(11)
    k = rng.standard_normal((4, c)).astype(np.float32) * np.float32(1000)
    v = rng.standard_normal((4, c)).astype(np.float32) * np.float32(1e-5)
    k[0, : special.size] = special
    v[1, : special.size] = special[::-1]
    rows = [(s, p) for p in range(4)]
    m.append(rows, k, v, layer=0)
    (kg, vg), (kw, vw) = m.gather(rows, layer=0)
    assert np.array_equal(kg, oracle.f32_to_f16(k)) and np.array_equal(vg, oracle.f32_to_f16(v))
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)


def test_overwrite_after_truncate(gpu, oracle_lib):
    rng = np.random.default_rng(12)
    m = Mirror(gpt2_opts())
    s = m.kv.add_seq()
    m.fill(s, 40, rng)
    m.kv.truncate(s, 33)  # keeps 3 pages, positions 33.. are rewritten
    m.fill(s, 45, rng)
    rows = [(s, p) for p in range(45)]
    (kg, vg), (kw, vw) = m.gather(rows)
    assert np.array_equal(kg, kw) and np.array_equal(vg, vw)


def test_append_refuses_unreserved_rows(gpu):
    kv = na.PagedKv(gpt2_opts())
    s = kv.add_seq()
    kv.reserve(s, 16)
    k = torch.zeros((12, 1, 768), device=gpu)
    with pytest.raises(na.KvError) as e:
        kv.append([(s, 16)], k, k)
    assert e.value.code == _abi.NI_ERR_NOT_RESERVED
    with pytest.raises(na.KvError) as e:
        kv.append([(s + 1, 0)], k, k)
    assert e.value.code == _abi.NI_ERR_NOT_LIVE
    kv.append([(s, 15)], k, k)
    kv.sync()
