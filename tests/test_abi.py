"""The C-ABI library loads and exports every entry point include/vgx.h
declares, and the Python binding declares them all.  No device work: this runs
on hosts without a GPU."""
import ctypes
import os
import re

import numpy as np

from vgx import lib as vl

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header="vgx.h"):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vgx_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    L = vl.load()
    names = declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert sorted(vl.exported_symbols()) == names


def test_engine_symbols_exported():
    from vgx import engine as ve
    L = ve.load()
    names = declared("vgx_engine.h")
    assert not [n for n in names if not hasattr(L, n)]
    assert sorted(ve.exported_symbols()) == names
    assert os.access(ve.CLI_PATH, os.X_OK)


def test_host_only_calls():
    L = vl.load()
    assert L.vgx_abi_version() == 1
    assert L.vgx_strerror(vl.VGX_EINVAL) == b"invalid argument"
    # argument checks fail with a status and a message, no device needed
    assert L.vgx_ctx_create(0, None) == vl.VGX_EINVAL
    assert b"NULL" in L.vgx_last_error()
    assert L.vgx_mat_upload(None, None, None) == vl.VGX_EINVAL
    from vgx import gpu as vg
    import oracle as o
    v = np.random.default_rng(0).standard_normal(101).astype(np.float32) * 50
    assert np.array_equal(vg.quantize_act(v), o.quantize_act(v))
    assert np.array_equal(vg.x_pack_i16_2(v), o.x_pack(v, o.I16_2))
