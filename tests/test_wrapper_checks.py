"""The Python wrappers refuse mis-shaped buffers before the C ABI sees them.

The C ABI takes plain pointers and strides, so a q/k/v/out tensor with too
few rows, the wrong width or the wrong layer count would become out-of-bounds
device reads or writes.  These run on the CPU: the layout checks come before
the device checks, so CPU tensors of the wrong shape raise ValueError, and
CPU tensors of the right shape raise TypeError (not on the GPU) -- no call
reaches the library.
"""
import pytest
import torch

import nanoinfer_amd as na

L, H, D = 2, 2, 64
C = H * D


@pytest.fixture
def kv():
    h = na.PagedKv(na.BatchOpts(n_layer=L, n_head=H, head_dim=D, kv_blocks=16, max_seqs=4, n_ctx=128, max_rows=64,
                                host_only=True))
    s = h.add_seq()
    yield h, s
    h.close()


def f(*shape):
    return torch.zeros(shape, dtype=torch.float32)


def test_step_rows_width_layers(kv):
    h, s = kv
    work = [(s, 5, 1)]
    ok = f(L, 5, C)
    with pytest.raises(ValueError, match="needs"):
        h.step(work, f(L, 4, C), ok, ok)  # q one row short of sum(n_new)
    with pytest.raises(ValueError, match="needs"):
        h.step(work, ok, f(L, 5, C - 8), ok)  # k narrower than n_embd
    with pytest.raises(ValueError, match="needs"):
        h.step(work, ok, ok, f(L + 1, 5, C))  # v with a layer too many
    with pytest.raises(ValueError, match="needs"):
        h.step(work, ok, ok, ok, out=f(L, 3, C))  # caller's out too short
    with pytest.raises(ValueError, match="unit stride"):
        h.step(work, f(L, C, 5).transpose(1, 2), ok, ok)
    with pytest.raises(TypeError, match="CUDA"):
        h.step(work, ok, ok, ok)  # the right shape, but not on the GPU


def test_append_and_attention(kv):
    h, s = kv
    rows = [(s, 0), (s, 1), (s, 2)]
    with pytest.raises(ValueError, match="needs"):
        h.append(rows, f(L, 2, C), f(L, 2, C))
    with pytest.raises(ValueError, match="needs"):
        h.append(rows, f(2, C), f(2, C), layer=0)
    with pytest.raises(ValueError, match="needs"):
        h.attention(f(L, 3, C), rows, out=f(L, 2, C))
    with pytest.raises(ValueError, match="needs"):
        h.attention(f(3, C + 1), rows, layer=1)
    with pytest.raises(TypeError, match="CUDA"):
        h.attention(f(L, 3, C), rows, out=f(L, 3, C))


def test_step_layer_uses_the_open_steps_rows(kv):
    h, s = kv
    h.step_begin([(s, 4, 4)])
    try:
        with pytest.raises(ValueError, match="needs"):
            h.step_layer(0, f(3, C), f(4, C), f(4, C))
        with pytest.raises(ValueError, match="needs"):
            h.step_layer(0, f(4, C), f(4, C), f(4, C), out=f(4, 2 * C))
    finally:
        h.step_end()


def test_projection_and_decode_steps(kv):
    h, s = kv
    rows = [(s, 0), (s, 1)]
    with pytest.raises(ValueError, match="needs"):
        h.qkv_append(rows, f(1, C), f(3 * C, C))  # x has one row for two appended rows
    with pytest.raises(ValueError, match="needs"):
        h.qkv_project(f(2, C), f(3 * C, C), out=f(2, 2 * C))
    with pytest.raises(ValueError, match="needs"):
        h.decode_steps([s], f(3, L, 1, C), f(3, L, 1, C), f(3, L, 1, C), out=f(3, L + 1, 1, C))
    with pytest.raises(ValueError, match="needs"):
        h.decode_steps([s, s], f(3, L, 1, C), f(3, L, 1, C), f(3, L, 1, C))
    with pytest.raises(ValueError, match="steps"):
        h.decode_steps([s], f(3, L, 1, C), f(3, L, 1, C), f(3, L, 1, C), out=f(2, L, 1, C))


def test_contiguous_attention_shapes():
    """na.attention (Kernels::attention): k/v need q_pos0 + n_q rows of C."""
    ok_q, ok_kv = f(2, C), f(5, C)
    with pytest.raises(ValueError, match="needs"):
        na.attention(ok_q, f(4, C), ok_kv, 2, 3, H, D)  # k one row short
    with pytest.raises(ValueError, match="needs"):
        na.attention(ok_q, ok_kv, f(5, C - 4), 2, 3, H, D)  # v too narrow
    with pytest.raises(ValueError, match="needs"):
        na.attention(f(1, C), ok_kv, ok_kv, 2, 3, H, D)  # q one row short
    with pytest.raises(TypeError, match="CUDA"):
        na.attention(ok_q, ok_kv, ok_kv, 2, 3, H, D)  # the right shape, but not on the GPU
