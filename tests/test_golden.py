"""The oracle reproduces the committed golden fixtures bit for bit (inputs,
block tables, f16 K/V, attention outputs), so a change to the oracle or to
the seeded generators cannot pass unnoticed."""
import json
import os

import pytest

from golden import cases

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(HERE, f"{name}.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", list(cases.CASES))
def test_oracle_reproduces_fixture(oracle_lib, name):
    want = load(name)
    got = json.loads(json.dumps(cases.CASES[name](cases.oracle_backend(name))))
    assert got["inputs_sha256"] == want["inputs_sha256"], "seeded inputs changed"
    assert got == want


def test_config1_contiguous_equals_paged(oracle_lib):
    """The reference's contiguous CPU cache and the paged oracle give the
    same f16 K/V and bit-identical attention on config 1 (identity of the
    kv_slot map with any table)."""
    paged = lambda shape, kv_blocks, max_seqs, n_ctx, order: cases.PagedOracle(  # noqa: E731
        shape, kv_blocks * 2, max_seqs, n_ctx, list(reversed(range(kv_blocks * 2))))
    got = cases.config1(paged)
    want = load("config1")
    assert got["exact"] == want["exact"]
    for g, w in zip(got["steps"], want["steps"]):
        assert g["approx"]["out_sha256"] == w["approx"]["out_sha256"]
