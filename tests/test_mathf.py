"""The engine's device expf and logf (tmac-zynq-fpga_amd/csrc/tmq_mathf.h),
built for the host from the same header, against the host libm expf and logf
that the reference engine calls (sim/tmac_gguf.cpp:460, :1650-1654).

Exhaustive runs over all 2^32 inputs (same checks, stride 1) found no
mismatch for either; the suite checks a strided sample plus the special
values.  The
same header's RoPE table is checked against the compiled reference's
apply_rope."""
import ctypes as C
import math
import os
import subprocess
import tempfile

import numpy as np
import pytest
from conftest import ROOT

HDR_DIR = os.path.join(ROOT, "tmac-zynq-fpga_amd", "csrc")
SRC = os.path.join(ROOT, "tests", "mathf_check.cpp")


@pytest.fixture(scope="module")
def mathf():
    out = os.path.join(tempfile.mkdtemp(prefix="tmq_mathf_"), "libmathf.so")
    # plain IEEE build: no fast-math, no -march (the reference's own flags)
    subprocess.run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-I", HDR_DIR, "-o", out, SRC],
                   check=True)
    L = C.CDLL(out)
    L.tmqm_expf_mismatches.restype = C.c_uint64
    L.tmqm_expf_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint32)]
    L.tmqm_expf.restype = C.c_float
    L.tmqm_expf.argtypes = [C.c_float]
    L.tmqm_logf_mismatches.restype = C.c_uint64
    L.tmqm_logf_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint32)]
    L.tmqm_logf.restype = C.c_float
    L.tmqm_logf.argtypes = [C.c_float]
    return L


def _libm(name):
    libm = C.CDLL("libm.so.6")
    f = getattr(libm, name)
    f.restype = C.c_float
    f.argtypes = [C.c_float]
    return f


def test_expf_sample_matches_libm(mathf):
    first = C.c_uint32(0)
    bad = mathf.tmqm_expf_mismatches(977, 13, C.byref(first))
    assert bad == 0, f"{bad} mismatches, first input bits {first.value:#010x}"


def test_expf_attention_range(mathf):
    """[-88, 0], the arguments of the softmax and of SiLU's exp(-g) for g > 0"""
    libm = C.CDLL("libm.so.6")
    libm.expf.restype = C.c_float
    libm.expf.argtypes = [C.c_float]
    for x in np.linspace(-88.0, 0.0, 30001, dtype=np.float32):
        a, e = mathf.tmqm_expf(float(x)), libm.expf(float(x))
        assert np.float32(a).view(np.uint32) == np.float32(e).view(np.uint32), x


@pytest.mark.parametrize("x", [0.0, -0.0, 1.0, -1.0, 88.0, 88.72283, 88.7229, -87.33655, -103.97208,
                               -103.9721, -150.0, float("inf"), float("-inf"), 1e-30, -1e-30, 0.5, -0.5])
def test_expf_special(mathf, x):
    libm = C.CDLL("libm.so.6")
    libm.expf.restype = C.c_float
    libm.expf.argtypes = [C.c_float]
    a, e = mathf.tmqm_expf(x), libm.expf(x)
    if math.isnan(e):
        assert math.isnan(a)
    else:
        assert np.float32(a).view(np.uint32) == np.float32(e).view(np.uint32)


def test_rope_table_matches_reference_apply_rope(mathf):
    """The engine's RoPE table (built on the host at load, tmq_math::rope_table)
    against the reference's apply_rope (sim/tmac_gguf.cpp:1528-1554): with q
    and k made of (1, 0) pairs, apply_rope writes exactly (cos, sin) of each
    pair (1*c - 0*s = c, 1*s + 0*c = s), so the whole table is compared bit
    for bit, positions 0..255 (the reference's context)."""
    from oracle import Reference
    if not Reference.available():
        pytest.skip("compiled reference (oracle/_ref) not built")
    ref = Reference()
    npos, H, KV = 256, 896, 128
    tab = np.zeros(npos * 32 * 2, dtype=np.float32)
    mathf.tmqm_rope_table.restype = None
    mathf.tmqm_rope_table.argtypes = [C.c_float, C.c_int, C.c_int, C.c_void_p]
    mathf.tmqm_rope_table(1000000.0, 64, npos, tab.ctypes.data)
    tab = tab.reshape(npos, 32, 2)
    for p in range(npos):
        q = np.zeros(H, dtype=np.float32)
        k = np.zeros(KV, dtype=np.float32)
        q[0::2] = 1.0
        k[0::2] = 1.0
        ref.lib.ref_apply_rope(q.ctypes.data, k.ctypes.data, p)
        for v in (q.reshape(-1, 32, 2), k.reshape(-1, 32, 2)):
            assert np.array_equal(v.view(np.uint32), np.broadcast_to(tab[p], v.shape).view(np.uint32)), p


def test_logf_sample_matches_libm(mathf):
    first = C.c_uint32(0)
    bad = mathf.tmqm_logf_mismatches(977, 29, C.byref(first))
    assert bad == 0, f"{bad} mismatches, first input bits {first.value:#010x}"


def test_logf_softmax_range(mathf):
    """[1, 4096]: the softmax denominators (the largest term is exp(0) = 1),
    every float of [1, 2) and a dense sample above"""
    libm_logf = _libm("logf")
    xs = np.concatenate([np.arange(0x3F800000, 0x40000000, 7, dtype=np.uint32).view(np.float32),
                         np.geomspace(2.0, 4096.0, 20001, dtype=np.float32)])
    for x in xs[::97]:
        a, e = mathf.tmqm_logf(float(x)), libm_logf(float(x))
        assert np.float32(a).view(np.uint32) == np.float32(e).view(np.uint32), x


@pytest.mark.parametrize("x", [0.0, -0.0, 1.0, -1.0, 2.0, 0.5, 1e-45, 1e-40, 1.1754942e-38, 3.4028235e38,
                               float("inf"), float("-inf"), float("nan"), 0.6999999, 1.4142135, 1.0000001])
def test_logf_special(mathf, x):
    a, e = mathf.tmqm_logf(x), _libm("logf")(x)
    if math.isnan(e):
        assert math.isnan(a)
    else:
        assert np.float32(a).view(np.uint32) == np.float32(e).view(np.uint32)
