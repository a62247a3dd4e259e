"""Where a step's rows are appended, all layers per launch: by the attention
workgroups themselves (one fused launch) or by an append launch before the
attention launch, the planner's choice.  Launch counts pin the choice for each
kind of step; every step is checked against the oracle either way (f16:
attention within tolerance and every row gathered bit for bit; Q8: attention
and the stored int8 values and scales).

The choice (kv_host.cpp, build_step_plan): f16 steps whose queried sequences
are all verify-style groups of 2..16 rows take the append launch, mixed
steps and single rows stay fused, and so does one launch per layer; Q8 steps
take it when a queried sequence appends more than 16 rows or when the queried
(sequence, layer, head) units reach 8192."""
import sys

import numpy as np
import pytest
import torch

import nanoinfer_amd as na
from nanoinfer_amd import workloads
from paged_mirror import Mirror, assert_close, mirror_step, step_rows
from test_gpu_q8 import MirrorQ8

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def launches(kv):
    """(append launches, attention launches) since profiling started."""
    return kv.profile_read(0)[1], kv.profile_read(1)[1]


@pytest.mark.parametrize("per_layer", [False, True], ids=["all_layers", "per_layer"])
def test_f16_append_launch_choice(gpu, oracle_lib, per_layer):
    rng = np.random.default_rng(71)
    L = 3
    m = Mirror(na.BatchOpts(**dict(workloads.GPT2, n_layer=L), kv_blocks=128, max_seqs=4, n_ctx=1024, max_rows=256))
    a, b, c = (m.kv.add_seq() for _ in range(3))
    for s, n in zip((a, b, c), (70, 33, 150)):
        m.fill(s, n, rng)
    cases = [
        ("groups only", [(a, 5, 5), (b, 5, 5), (c, 3, 3)], 0 if per_layer else 1),
        ("groups and a single row", [(a, 5, 5), (b, 1, 1), (c, 4, 4)], 0),
        ("single rows and a mid-prompt chunk", [(a, 1, 1), (b, 20, 0), (c, 1, 1)], 0),
    ]
    for what, work, want_app in cases:
        srows, _ = step_rows(m.kv, work)
        q, k, v = (rng.standard_normal((L, len(srows), m.c)).astype(np.float32) for _ in range(3))
        m.kv.profile([0, 1])
        got, want, qr = mirror_step(m, work, q, k, v, per_layer=per_layer)
        n_app, n_attn = launches(m.kv)
        m.kv.profile([])
        err = assert_close(got[:, qr], want[:, qr], what)
        (kg, vg), (kw, vw) = m.gather(srows)
        assert np.array_equal(kg, kw) and np.array_equal(vg, vw), what
        say(f"f16 {what}, per_layer {per_layer}: {n_app} append + {n_attn} attention launches, err {err:.2e}")
        assert n_app == want_app, (what, n_app)
        assert n_attn == (L if per_layer else 1), (what, n_attn)


def q8_step(m, work, rng):
    rows, qrows = step_rows(m.kv, work)
    L = m.opts.n_layer
    q, k, v = (rng.standard_normal((L, len(rows), m.c)).astype(np.float32) for _ in range(3))
    m.kv.profile([0, 1])
    got = m.kv.step(work, *(torch.from_numpy(x).cuda() for x in (q, k, v))).cpu().numpy()
    n_app, n_attn = launches(m.kv)
    m.kv.profile([])
    m.append_oracle(rows, k, v)
    err = assert_close(got[:, qrows], m.attention_oracle(rows[qrows], q[:, qrows]), f"{len(work)} sequences")
    m.check_bytes(rows)
    return n_app, n_attn, err


def test_q8_append_launch_choice(gpu, oracle_lib):
    rng = np.random.default_rng(72)
    L, n_seq = 12, 57  # 57 x 12 x 12 = 8208 units: the threshold is 8192
    m = MirrorQ8(na.BatchOpts(**dict(workloads.GPT2, n_layer=L), kv_blocks=4 * n_seq + 8, max_seqs=n_seq,
                              n_ctx=1024, max_rows=256, q8=True))
    seqs = [m.kv.add_seq() for _ in range(n_seq)]
    for i, s in enumerate(seqs):
        m.fill(s, 20 + (7 * i) % 23, rng)
    a, b, c = seqs[:3]
    cases = [
        ("a group and a single row", [(a, 5, 5), (b, 1, 1)], 0),
        ("a 37-row chunk queried at its last row", [(a, 1, 1), (b, 37, 1), (c, 5, 5)], 1),
        ("a mid-prompt chunk (no query) and single rows", [(a, 1, 1), (b, 37, 0), (c, 1, 1)], 0),
        ("56 single rows (8064 units)", [(s, 1, 1) for s in seqs[:56]], 0),
        ("57 single rows (8208 units)", [(s, 1, 1) for s in seqs], 1),
    ]
    for what, work, want_app in cases:
        n_app, n_attn, err = q8_step(m, work, rng)
        say(f"q8 {what}: {n_app} append + {n_attn} attention launches, err {err:.2e}")
        assert (n_app, n_attn) == (want_app, 1), (what, n_app, n_attn)
