"""The golden cases (config 1, config 2, a speculative-verify trace with page
reuse) on the device through the C ABI, checked against the committed
fixtures alone: inputs regenerated from their seeds (hash-checked), block
tables, free counts, sequence lengths and every stored f16 K/V row bit for
bit; attention outputs within 1e-3 max-abs / 1e-3 relative (sliced values
elementwise, per-layer sums within the summed bound)."""
import hashlib
import json
import os
import sys

import numpy as np
import pytest
import torch

import nanoinfer_amd as na
from golden import cases

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


class Device:
    """The cases' backend interface over PagedKv (ni_kv_* calls)."""

    def __init__(self, shape, kv_blocks, max_seqs, n_ctx, order):
        self.rows_max = 512
        self.kv = na.PagedKv(na.BatchOpts(**shape, kv_blocks=kv_blocks, max_seqs=max_seqs, n_ctx=n_ctx,
                                          max_rows=self.rows_max, page_order=order))
        self.L = shape["n_layer"]

    def add_seq(self):
        return self.kv.add_seq()

    def free_seq(self, s):
        self.kv.free_seq(s)

    def truncate(self, s, n):
        self.kv.truncate(s, n)

    def seq_len(self, s):
        return self.kv.seq_len(s)

    def block_table(self, s):
        return self.kv.block_table(s)

    def free_block_count(self):
        return self.kv.free_block_count()

    def fill(self, s, k, v):
        n = k.shape[1]
        L0 = self.seq_len(s)
        self.kv.reserve(s, L0 + n)
        kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
        for a in range(0, n, self.rows_max):
            b = min(n, a + self.rows_max)
            rows = [(s, L0 + i) for i in range(a, b)]
            self.kv.append(rows, kd[:, a:b], vd[:, a:b])
        self.kv.commit(s, n)

    @staticmethod
    def _upload(q, k, v):
        """Device views of q/k/v; views of one fused [L][n][3C] array stay
        views of one device buffer (the QKV-epilogue strides)."""
        base = q.base
        if base is not None and k.base is base and v.base is base and base.flags.c_contiguous:
            dev = torch.from_numpy(base).cuda()
            flat = dev.reshape(-1)

            def view(a):
                off = (a.ctypes.data - base.ctypes.data) // 4
                return flat.as_strided(a.shape, [s // 4 for s in a.strides], off)

            return view(q), view(k), view(v)
        return (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (q, k, v))

    def step(self, work, q, k, v):
        rows, qrows = cases.step_rows(self.seq_len, work)
        qd, kd, vd = self._upload(q, k, v)
        out = self.kv.step(work, qd, kd, vd)
        torch.cuda.synchronize()
        return out.cpu().numpy(), qrows

    def kv_sha(self, seqs) -> str:
        h = hashlib.sha256()
        for s in seqs:
            n = self.seq_len(s)
            ks, vs = [], []
            for a in range(0, n, self.rows_max):
                kg, vg = self.kv.gather([(s, p) for p in range(a, min(n, a + self.rows_max))])
                ks.append(kg.cpu().numpy().view(np.uint16))
                vs.append(vg.cpu().numpy().view(np.uint16))
            kg, vg = np.concatenate(ks, 1), np.concatenate(vs, 1)
            for l in range(self.L):
                h.update(np.ascontiguousarray(kg[l]).tobytes())
                h.update(np.ascontiguousarray(vg[l]).tobytes())
        return h.hexdigest()


def device_backend(shape, kv_blocks, max_seqs, n_ctx, order):
    return Device(shape, kv_blocks, max_seqs, n_ctx, order)


@pytest.mark.parametrize("name", list(cases.CASES))
def test_device_matches_fixture(gpu, name):
    with open(os.path.join(HERE, f"{name}.json")) as f:
        want = json.load(f)
    print(f"golden case {name}", file=sys.stderr, flush=True)
    got = json.loads(json.dumps(cases.CASES[name](device_backend)))
    assert got["inputs_sha256"] == want["inputs_sha256"], "seeded inputs differ from the fixture's"
    for key in want:
        if key != "steps":
            assert got[key] == want[key], key
    assert len(got["steps"]) == len(want["steps"])
    worst = 0.0
    for i, (g, w) in enumerate(zip(got["steps"], want["steps"])):
        if "exact" in w:
            assert g["exact"] == w["exact"], f"step {i}"
        ga, wa = g["approx"], w["approx"]
        gs, ws = np.asarray(ga["slice"]), np.asarray(wa["slice"])
        err = np.abs(gs - ws)
        assert np.isfinite(gs).all() and (err <= cases.ATOL + cases.RTOL * np.abs(ws)).all(), \
            f"step {i}: slice off by {err.max():.3e}"
        dsum = np.abs(np.asarray(ga["sum"]) - np.asarray(wa["sum"]))
        assert (dsum <= np.asarray(wa["bound"])).all(), f"step {i}: layer sums off by {dsum.max():.3e}"
        worst = max(worst, float(err.max()))
    print(f"golden case {name}: {len(want['steps'])} steps, max slice error {worst:.2e}", file=sys.stderr, flush=True)
