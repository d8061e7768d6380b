"""libtmq.so loads and exports every entry point include/tmq.h declares (CPU;
no compute calls without a GPU)."""
import ctypes
import os
import re

import pytest
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "tmq.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tmq_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = declared()
    for must in ("tmq_open", "tmq_tensor_upload", "tmq_matmul", "tmq_gemv_dev",
                 "tmq_vecmul_tile_q8", "tmq_phaseb_run", "tmq_chain_run"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import tmq
    if not os.path.exists(tmq.LIB_PATH):
        pytest.fail("libtmq.so not built: __graft_entry__.build() must run first")
    lib = ctypes.CDLL(tmq.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(tmq.EXPORTS) == declared()


def test_library_is_gfx950_code_object():
    """The fat binary carries a gfx950 code object (offload bundle id)."""
    import tmq
    blob = open(tmq.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob


def test_version_and_error_without_device():
    import tmq
    L = tmq.lib()
    assert b"gfx950" in L.tmq_version()
    assert isinstance(L.tmq_last_error(), bytes)


def test_arg_errors_need_no_device():
    import tmq
    L = tmq.lib()
    assert L.tmq_open(0, None) == -1           # TMQ_ERR_ARG
    assert L.tmq_tensor_info(None, None, None, None, None) == -1
    assert L.tmq_close(None) == 0 and L.tmq_tensor_free(None) == 0 and L.tmq_chain_free(None) == 0
