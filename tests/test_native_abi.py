"""The C-ABI library loads on a host without a GPU and exports every entry point the header
declares; the ctypes binding covers the header exactly. No compute calls here (no GPU)."""

import ctypes
import os
import re

import pytest

from conftest import ROOT
from llmario_amd import _native as N

HEADER = os.path.join(ROOT, "include", "llmario_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lmh_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ["lmh_kv_create", "lmh_kv_reserve", "lmh_batch_prepare", "lmh_kv_store", "lmh_kv_gather",
                 "lmh_attend", "lmh_kv_destroy"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    if not os.path.exists(N.LIB_PATH):
        pytest.fail(f"{N.LIB_PATH} not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(N.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_matches_header():
    assert sorted(N.exported_symbols()) == declared()


def test_create_rejects_bad_options_without_touching_the_device():
    o = N.KvOptions(N.ABI_VERSION + 99, 0, 16, 0, None, 16, 1, 0, 0, 0)
    h = ctypes.c_void_p()
    assert N.lib().lmh_kv_create(ctypes.byref(o), ctypes.byref(h)) == N.INVALID_ARGUMENT
    assert b"ABI" in N.lib().lmh_create_error()
    layer = (N.LayerDesc * 1)(N.LayerDesc(8, 8, 64, 64, 0, 0))
    o = N.KvOptions(N.ABI_VERSION, 0, 24, 1, ctypes.cast(layer, ctypes.POINTER(N.LayerDesc)), 16, 1, 0, 0, 0)
    assert N.lib().lmh_kv_create(ctypes.byref(o), ctypes.byref(h)) == N.INVALID_ARGUMENT  # not a power of two
    o.block_tokens = 16
    layer[0] = N.LayerDesc(8, 8, 576, 512, 0, 0)
    assert N.lib().lmh_kv_create(ctypes.byref(o), ctypes.byref(h)) == N.UNSUPPORTED  # wider than 512 (Metal's bound)
    layer[0] = N.LayerDesc(8, 3, 64, 64, 0, 0)
    assert N.lib().lmh_kv_create(ctypes.byref(o), ctypes.byref(h)) == N.INVALID_ARGUMENT  # n_head % n_kv
    o.kv_type = N.KV_Q8_0
    layer[0] = N.LayerDesc(8, 8, 48, 48)
    assert N.lib().lmh_kv_create(ctypes.byref(o), ctypes.byref(h)) == N.INVALID_ARGUMENT  # kv.rs:103-109


def test_read_ceiling_hook_rejects_bad_arguments_without_touching_the_device():
    g = ctypes.c_double()
    lib = N.lib()
    assert lib.lmh_bench_read_ceiling(0, 0, 10, ctypes.byref(g)) == N.INVALID_ARGUMENT        # no bytes
    assert lib.lmh_bench_read_ceiling(0, 15, 10, ctypes.byref(g)) == N.INVALID_ARGUMENT       # under 16 bytes
    assert lib.lmh_bench_read_ceiling(0, 1 << 20, 0, ctypes.byref(g)) == N.INVALID_ARGUMENT   # no launches
    assert lib.lmh_bench_read_ceiling(0, 1 << 20, 10, None) == N.INVALID_ARGUMENT             # no result slot
