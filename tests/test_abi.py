"""The C-ABI library loads on a machine without a GPU and exports every
function include/nanoinfer_kv.h declares; host-only handles work; the
device path refuses to run on them."""
import ctypes as C
import subprocess

import pytest

from nanoinfer_amd import _abi, build


def test_library_exports_every_declared_function():
    L = _abi.lib()
    declared = _abi.declared_functions()
    assert len(declared) >= 20
    missing = [f for f in declared if not hasattr(L, f)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", build.LIB], capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert set(declared) <= exported
    assert _abi.lib().ni_version().decode().startswith("nanoinfer-amd")


def test_library_is_built_for_gfx950():
    out = subprocess.run(["strings", "-n", "8", build.LIB], capture_output=True, text=True, check=True).stdout
    assert "gfx950" in out


def test_host_only_handle_refuses_device_work():
    import nanoinfer_amd as na

    kv = na.PagedKv(na.BatchOpts(kv_blocks=8, max_seqs=2, n_ctx=64, host_only=True))
    s = kv.add_seq()
    kv.reserve(s, 1)
    rows = (_abi.ni_row * 1)(_abi.ni_row(s, 0))
    rc = kv._L.ni_kv_append(kv.handle, -1, rows, 1, None, None, 0, 0, None)
    assert rc == _abi.NI_ERR_NO_DEVICE
    assert "host-only" in kv._L.ni_kv_last_error(kv.handle).decode()


def test_create_rejects_bad_options():
    import nanoinfer_amd as na

    with pytest.raises(na.KvError) as e:
        na.PagedKv(na.BatchOpts(head_dim=12, host_only=True))
    assert e.value.code == _abi.NI_ERR_BAD_ARG
    with pytest.raises(na.KvError) as e:
        na.PagedKv(na.BatchOpts(kv_blocks=4, page_order=[0, 1, 1, 2], host_only=True))
    assert "permutation" in str(e.value)


def test_attention_rejects_bad_arguments_before_any_launch():
    """ni_attention's checks come before anything touches the device."""
    L = _abi.lib()
    buf = (C.c_float * 64)()
    p = C.addressof(buf)
    rc = L.ni_attention(p, 768, p, 768, p, 768, p, 768, 1, 0, 12, 96, None)
    assert rc == _abi.NI_ERR_BAD_ARG and "head_dim 96" in L.ni_kv_last_error(None).decode()
    rc = L.ni_attention(p + 4, 768, p, 768, p, 768, p, 768, 1, 0, 12, 64, None)
    assert rc == _abi.NI_ERR_BAD_ARG and "out must be 16-byte aligned" in L.ni_kv_last_error(None).decode()
    rc = L.ni_attention(p, 768, p, 770, p, 768, p, 768, 1, 0, 12, 64, None)
    assert rc == _abi.NI_ERR_BAD_ARG and "q must be" in L.ni_kv_last_error(None).decode()
    rc = L.ni_attention(p, 768, p, 768, None, 768, p, 768, 1, 0, 12, 64, None)
    assert rc == _abi.NI_ERR_BAD_ARG and "k is NULL" in L.ni_kv_last_error(None).decode()
    assert L.ni_attention(None, 0, None, 0, None, 0, None, 0, 0, 0, 12, 64, None) == _abi.NI_OK  # nothing to do
