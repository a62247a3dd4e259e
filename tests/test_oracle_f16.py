"""Pins the oracle's f16 conversion (crates/core/src/quant.rs:25-73).

* the reference's own known answers (quant.rs:148-166);
* every f16 survives f16 -> f32 -> f16 (quant.rs:160-165);
* all 2^32 f32 bit patterns against an independent library routine, x86 F16C
  (vcvtps2ph, round to nearest even); NaN inputs, where F16C keeps payload
  bits and the reference canonicalises to sign|0x7e00, are checked against
  the canonical value instead;
* a random sample against numpy's float16 cast (a third implementation).
"""
import concurrent.futures as cf
import os

import numpy as np
import pytest

import oracle


def test_reference_known_answers(oracle_lib):
    # quant.rs:150-154: every value round-trips within 1e-3 relative.
    for v in [0.0, -0.0, 1.0, -2.5, 65504.0, 6.1035156e-5, 5.9604645e-8, 1e-3, 1.234_567]:
        h = oracle.f32_to_f16_scalar(v)
        back = float(oracle.f16_to_f32(np.array([h], np.uint16))[0])
        assert abs(back - v) <= abs(v) * 1e-3 + 6e-8, (v, hex(h), back)
    # quant.rs:155-158.
    assert oracle.f32_to_f16_scalar(1.0) == 0x3C00
    assert oracle.f32_to_f16_scalar(65520.0) == 0x7C00  # rounds up to inf
    assert oracle.f32_to_f16_scalar(1.0 + 1.0 / 2048.0) == 0x3C00  # tie -> even
    assert oracle.f32_to_f16_scalar(1.0 + 3.0 / 2048.0) == 0x3C02  # tie -> even (up)


def test_every_f16_round_trips(oracle_lib):
    # quant.rs:160-165.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.f16_to_f32(h)
    keep = ~np.isnan(f)
    assert np.array_equal(oracle.f32_to_f16(f[keep]), h[keep])
    # f16_to_f32 is exact: numpy's float16 widening agrees on every pattern.
    want = h.view(np.float16).astype(np.float32)
    assert np.array_equal(f.view(np.uint32)[keep], want.view(np.uint32)[keep])


def test_all_f32_patterns_match_f16c(oracle_lib):
    chunk = 1 << 26
    starts = range(0, 1 << 32, chunk)
    workers = min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(workers) as ex:  # ctypes drops the GIL
        res = list(ex.map(lambda s: oracle.f16_check_f16c(s, chunk), starts))
    bad = sum(r[0] for r in res)
    nans = sum(r[1] for r in res)
    assert nans == 2 * ((1 << 23) - 1)  # every NaN pattern was seen (and checked canonical)
    assert bad == 0


def test_sample_matches_numpy(oracle_lib):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    # plus the interesting neighbourhoods: subnormal boundary, overflow, ties
    special = np.array([0x33000000, 0x33000001, 0x387FC000, 0x387FE000, 0x38800000, 0x477FE000, 0x477FEFFF,
                        0x477FF000, 0x3F801000, 0x3F803000, 0x00000001, 0x80000001, 0x7F800000, 0xFF800000],
                       np.uint32)
    bits = np.concatenate([bits, special])
    f = bits.view(np.float32)
    ok = ~np.isnan(f)
    with np.errstate(over="ignore"):
        want = f[ok].astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(f[ok]), want)
    got_nan = oracle.f32_to_f16(f[~ok])
    sign = ((bits[~ok] >> 16) & 0x8000).astype(np.uint16)
    assert np.array_equal(got_nan, sign | 0x7E00)
