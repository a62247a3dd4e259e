"""The oracle's QKV matvec (batch.metal:94-165 restated in double) against
numpy's float64 matrix product, an independent routine; a transposed weight
operand (a plausible layout mistake) must fail the same check."""
import numpy as np

import oracle


def test_matvec_f64_matches_numpy(oracle_lib):
    rng = np.random.default_rng(3)
    n, d_in, d_out = 7, 96, 48
    x = rng.standard_normal((n, d_in)).astype(np.float32)
    w = (rng.standard_normal((d_out, d_in)) * 0.05).astype(np.float32)
    b = rng.standard_normal(d_out).astype(np.float32)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b.astype(np.float64)
    got = oracle.matvec_f64(x, w, b)
    assert np.abs(got - want).max() < 1e-12
    assert np.abs(oracle.matvec_f64(x, w) - (want - b)).max() < 1e-12


def test_matvec_f64_planted_transpose_fails(oracle_lib):
    rng = np.random.default_rng(4)
    d = 64
    x = rng.standard_normal((3, d)).astype(np.float32)
    w = rng.standard_normal((d, d)).astype(np.float32)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    wrong = oracle.matvec_f64(x, np.ascontiguousarray(w.T))
    assert np.abs(wrong - want).max() > 1.0
