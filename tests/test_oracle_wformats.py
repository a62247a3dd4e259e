"""The oracle's restatement of the reference's weight formats
(crates/metal/src/weights.rs:12-86: quantize_q8_0, quantize_q4_0,
dequantize), pinned by known answers of the layouts and rounding rules, an
independent numpy dequantiser written from the documented layout, and the
quantisation error bounds.  (The reference's own check of its kernels against
these, crates/metal/tests/kernels.rs:38-42, needs Metal.)"""
import numpy as np
import pytest

import oracle


def np_dequantize(q, n, fmt):
    """weights.rs:29-52 in numpy: quants then one f16 scale per 32 weights."""
    q = np.asarray(q, np.uint8)
    nb = n // 32
    if fmt == "q8_0":
        vals = q[:n].view(np.int8).astype(np.float32)
        scales = q[n:n + 2 * nb].view(np.float16).astype(np.float32)
    else:
        b = q[: n // 2].reshape(nb, 16)
        vals = np.concatenate([b & 15, b >> 4], axis=1).astype(np.float32).reshape(-1) - np.float32(8)
        scales = q[n // 2:n // 2 + 2 * nb].view(np.float16).astype(np.float32)
    return (vals.reshape(nb, 32) * scales[:, None]).astype(np.float32).reshape(-1)


def test_q4_layout_known_answer():
    """A block whose largest-magnitude value is -4 (first) gives d = 0.5,
    id = 2 and q(v) = v * 2 + 8: element i in byte i's low nibble, i + 16 in
    its high nibble; the f16 scale follows the quants."""
    w = np.array([(j % 16 - 8) * 0.5 for j in range(32)], np.float32)
    q = oracle.quantize(w, "q4_0")
    assert q.size == 16 + 2
    assert list(q[:16]) == [i | (i << 4) for i in range(16)]
    assert q[16:18].view(np.uint16)[0] == 0x3800  # f16 0.5
    assert np.array_equal(oracle.dequantize(q, 32, "q4_0"), w)


def test_q4_rounding_and_sign():
    """d = max / -8 keeps the sign of the largest value: a positive maximum
    gives a negative scale; q = trunc(v * id + 8.5) clamped to [0, 15]."""
    w = np.zeros(32, np.float32)
    w[3] = 8.0    # largest magnitude, positive: d = -1, id = -1, q = trunc(-8 + 8.5) = 0
    w[4] = -7.5   # q = trunc(7.5 + 8.5) = 16 -> clamped to 15
    w[5] = 0.49   # q = trunc(-0.49 + 8.5) = 8
    w[6] = -0.5   # q = trunc(0.5 + 8.5) = 9
    q = oracle.quantize(w, "q4_0")
    assert q[16:18].view(np.float16)[0] == np.float16(-1.0)
    nib = np.concatenate([q[:16] & 15, q[:16] >> 4])
    assert (nib[3], nib[4], nib[5], nib[6]) == (0, 15, 8, 9)
    assert nib[0] == 8  # zero
    d = oracle.dequantize(q, 32, "q4_0")
    assert (d[3], d[4], d[5], d[6]) == (8.0, -7.0, 0.0, -1.0)


def test_q8_rounding_known_answer():
    """amax 127 gives d = 1: q = round(w) with halves away from zero (Rust's
    f32::round), not to even."""
    w = np.zeros(32, np.float32)
    w[:6] = [127.0, 0.5, -0.5, 1.5, -2.5, 126.5]
    q = oracle.quantize(w, "q8_0")
    assert q.size == 32 + 2
    assert list(q[:6].view(np.int8)) == [127, 1, -1, 2, -3, 127]
    assert q[32:34].view(np.float16)[0] == np.float16(1.0)


def test_zero_block():
    for fmt in ("q8_0", "q4_0"):
        q = oracle.quantize(np.zeros(64, np.float32), fmt)
        assert np.array_equal(oracle.dequantize(q, 64, fmt), np.zeros(64, np.float32))


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0"])
def test_dequantize_matches_numpy_on_any_bytes(fmt):
    rng = np.random.default_rng(11)
    n = 32 * 40
    qb = n if fmt == "q8_0" else n // 2
    q = rng.integers(0, 256, qb + n // 16, dtype=np.uint8)
    scales = (rng.standard_normal(n // 32) * 0.05).astype(np.float16)  # finite scales, both signs
    q[qb:] = scales.view(np.uint8)
    assert np.array_equal(oracle.dequantize(q, n, fmt), np_dequantize(q, n, fmt))


@pytest.mark.parametrize("fmt,bound", [("q8_0", 0.6), ("q4_0", 1.1)])
def test_round_trip_error_bound(fmt, bound):
    """|dequant(quant(w)) - w| stays within a fraction of the block's step
    |d| (half a step from rounding, a little more from the f16 scale, a whole
    step where Q4_0 clamps at +8)."""
    rng = np.random.default_rng(12)
    w = (rng.standard_normal(32 * 200) * 0.03).astype(np.float32)
    q = oracle.quantize(w, fmt)
    back = oracle.dequantize(q, w.size, fmt)
    nb = w.size // 32
    if fmt == "q8_0":
        step = np.abs(w.reshape(nb, 32)).max(axis=1) / 127
    else:
        step = np.abs(w.reshape(nb, 32)).max(axis=1) / 8
    err = np.abs(back - w).reshape(nb, 32).max(axis=1)
    assert (err <= bound * step + 1e-12).all()
    assert np.array_equal(back, np_dequantize(q, w.size, fmt))


def test_f16_format_is_the_append_rounding():
    rng = np.random.default_rng(13)
    w = rng.standard_normal(256).astype(np.float32)
    q = oracle.quantize(w, "f16")
    assert np.array_equal(q.view(np.uint16), oracle.f32_to_f16(w))
    assert np.array_equal(oracle.dequantize(q, 256, "f16"), w.astype(np.float16).astype(np.float32))
