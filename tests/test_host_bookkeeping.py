"""The product's page allocator and block tables (C++, through the C ABI on
a host-only handle) against the oracle's restatement of batch.rs:129-254 and
the reference's error texts."""
import numpy as np
import pytest

import oracle
import nanoinfer_amd as na
from nanoinfer_amd import _abi

KB = 16


def make(kv_blocks, max_seqs, n_ctx, order=None):
    kv = na.PagedKv(na.BatchOpts(kv_blocks=kv_blocks, max_seqs=max_seqs, n_ctx=n_ctx, host_only=True,
                                 page_order=order))
    ref = oracle.Alloc(kv_blocks, max_seqs, n_ctx, order)
    return kv, ref


def ensure_product(kv, s, n):
    """0 / 1 / 2 like the oracle's ensure."""
    try:
        kv.reserve(s, n)
        return 0
    except na.KvError as e:
        return {_abi.NI_ERR_CONTEXT_FULL: 1, _abi.NI_ERR_POOL_EXHAUSTED: 2}[e.code]


@pytest.mark.parametrize("seed", range(8))
def test_random_ops_match_oracle(seed):
    rng = np.random.default_rng(100 + seed)
    kv_blocks, max_seqs, n_ctx = int(rng.integers(4, 40)), int(rng.integers(1, 6)), int(rng.integers(16, 300))
    order = rng.permutation(kv_blocks).tolist() if seed % 2 else None
    kv, ref = make(kv_blocks, max_seqs, n_ctx, order)
    for _ in range(600):
        r = rng.random()
        s = int(rng.integers(0, max_seqs))
        if r < 0.2:
            assert kv.add_seq() == ref.add_seq()
        elif r < 0.3:
            kv.free_seq(s)
            ref.free_seq(s)
        elif r < 0.7:
            if not ref.live(s):
                with pytest.raises(na.KvError) as e:
                    kv.reserve(s, 1)
                assert str(e.value) == f"sequence {s} is not live"
                continue
            n = ref.seq_len(s) + int(rng.integers(1, 60)) if rng.random() < 0.9 else n_ctx + 1
            got, want = ensure_product(kv, s, n), ref.ensure(s, n)
            assert got == want
            if got == 0:
                kv.commit(s, n - kv.seq_len(s))
                ref.commit(s, n - ref.seq_len(s))
        else:
            n = int(ref.seq_len(s) * rng.random())
            kv.truncate(s, n)
            ref.truncate(s, n)
        for t in range(max_seqs):
            assert kv.block_table(t) == ref.block_table(t)
            assert kv.seq_len(t) == ref.seq_len(t)
            assert kv.is_live(t) == ref.live(t)
        assert kv.free_block_count() == ref.free_block_count()
        assert kv.blocks_used() == ref.blocks_used()


def test_reference_error_texts():
    kv, _ = make(4, 2, 40)
    s = kv.add_seq()
    with pytest.raises(na.KvError) as e:
        kv.reserve(s, 41)
    assert e.value.code == _abi.NI_ERR_CONTEXT_FULL
    assert str(e.value) == "sequence 0: context full (41 > 40)"  # batch.rs:245
    kv.reserve(s, 40)  # 3 pages
    t = kv.add_seq()
    kv.reserve(t, 16)  # the 4th page
    with pytest.raises(na.KvError) as e:
        kv.reserve(t, 17)
    assert e.value.code == _abi.NI_ERR_POOL_EXHAUSTED
    assert str(e.value) == "KV cache pool exhausted"  # batch.rs:248
    assert kv.add_seq() is None  # batch.rs:201-202: None when every slot is live
    with pytest.raises(AssertionError) as e:
        kv.truncate(s, 1)  # seq_len is still 0 (nothing committed)
    assert str(e.value) == "assertion failed: len <= self.seq_len[s]"  # batch.rs:221
    kv.free_seq(s)
    with pytest.raises(na.KvError) as e:
        kv.reserve(s, 1)
    assert str(e.value) == "sequence 0 is not live"


def test_default_order_and_lifo_reuse():
    kv, _ = make(16, 3, 1024)
    a, b = kv.add_seq(), kv.add_seq()
    kv.reserve(a, 40)
    kv.reserve(b, 20)
    assert kv.block_table(a) == [0, 1, 2]  # batch.rs:174: pop() yields 0, 1, 2, ...
    assert kv.block_table(b) == [3, 4]
    kv.commit(a, 40)
    kv.truncate(a, 17)  # frees page 2
    kv.free_seq(b)      # frees 4 then 3
    c = kv.add_seq()
    assert c == 1       # first non-live slot (batch.rs:202)
    kv.reserve(c, 48)
    assert kv.block_table(c) == [3, 4, 2]


def test_page_order_permutation():
    order = list(np.random.default_rng(3).permutation(32))
    kv, ref = make(32, 4, 512, order)
    s = kv.add_seq()
    ref.add_seq()
    kv.reserve(s, 100)
    assert ref.ensure(s, 100) == 0
    assert kv.block_table(s) == order[:7] == ref.block_table(s)


def test_commit_past_reserve_is_refused():
    kv, _ = make(8, 1, 128)
    s = kv.add_seq()
    kv.reserve(s, 10)
    with pytest.raises(na.KvError) as e:
        kv.commit(s, 17)
    assert e.value.code == _abi.NI_ERR_NOT_RESERVED
    kv.commit(s, 16)
    assert kv.seq_len(s) == 16


def test_per_layer_step_bookkeeping():
    """ni_kv_step_begin / _end on a host-only handle: begin reserves like
    ni_kv_step (the same errors, nothing open after one), end commits
    seq_len += n_new, and while a step is open the calls that free pages or
    move seq_len are refused, as is a second begin; a layer call needs the
    device."""
    kv, ref = make(16, 4, 160)
    a, b = kv.add_seq(), kv.add_seq()
    kv.reserve(a, 20)
    kv.commit(a, 20)
    with pytest.raises(na.KvError) as e:
        kv.step_end()
    assert "no step is open" in str(e.value)
    kv.step_begin([(a, 1, 1), (b, 37, 37)])
    assert kv.seq_len(a) == 20 and kv.seq_len(b) == 0
    assert len(kv.block_table(a)) == 2 and len(kv.block_table(b)) == 3
    for call in (lambda: kv.step_begin([(a, 1, 1)]), lambda: kv.truncate(a, 0), lambda: kv.free_seq(b),
                 lambda: kv.commit(a, 1)):
        with pytest.raises(na.KvError) as e:
            call()
        assert e.value.code == _abi.NI_ERR_BAD_ARG and "open" in str(e.value)
    with pytest.raises(na.KvError) as e:
        kv._check(kv._L.ni_kv_step_layer(kv._h, 0, None, None, None, 0, None, 0, None))
    assert e.value.code == _abi.NI_ERR_NO_DEVICE
    kv.step_end()
    assert kv.seq_len(a) == 21 and kv.seq_len(b) == 37
    # The reference's errors on begin; nothing stays open after them.
    with pytest.raises(na.KvError) as e:
        kv.step_begin([(a, 200, 1)])
    assert e.value.code == _abi.NI_ERR_CONTEXT_FULL
    with pytest.raises(na.KvError) as e:
        kv.step_begin([(3, 1, 1)])
    assert e.value.code == _abi.NI_ERR_NOT_LIVE
    kv.truncate(a, 5)
    assert kv.seq_len(a) == 5 and len(kv.block_table(a)) == 1
