"""GPU parity of the two other branches of `matmul` (sim/tmac_gguf.cpp:
473-493) on gfx950: matmul_fpga_int16 (:887-940) and the FP32 loop
(:488-492), through the C ABI, bit-exact against the compiled reference's
golden vectors and the CPU oracle (int64 tile results, row scales, fp32
outputs), and the routing of tmq_matmul_flags."""
import numpy as np
import pytest
from conftest import load_golden
from oracle import F16, F32, Q4_K, Q5_0, Q6_K, Q8_0
from tmq import synth

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def mism(got, exp):
    bad = np.flatnonzero(bits(got) != bits(exp))
    return f"{bad.size} mismatches, first rows {bad[:5]}"


@pytest.mark.parametrize("name", ["q8_0", "q5_0", "q4_k", "q6_k", "f32", "f16"])
def test_paths_golden(ctx, name):
    import tmq
    g = load_golden("matmul_paths.npz")
    qt, rows, cols = (int(v) for v in g[f"{name}_meta"])
    print(f"[paths] golden {name} {rows}x{cols}", flush=True)
    t = ctx.upload(qt, rows, cols, g[f"{name}_w"])
    try:
        y16 = ctx.matmul_path(t, g[f"{name}_x"], tmq.PATH_INT16)
        y32 = ctx.matmul_path(t, g[f"{name}_x"], tmq.PATH_FP32)
        edges = []
        if name == "q5_0":
            for tag in ("x0", "x1"):
                edges.append((tag, ctx.matmul_path(t, g[f"edge_{tag}"], tmq.PATH_INT16),
                              ctx.matmul_path(t, g[f"edge_{tag}"], tmq.PATH_FP32)))
    finally:
        t.free()
    assert np.array_equal(bits(y16), bits(g[f"{name}_y16"])), mism(y16, g[f"{name}_y16"])
    assert np.array_equal(bits(y32), bits(g[f"{name}_y32"])), mism(y32, g[f"{name}_y32"])
    for tag, a, b in edges:
        assert np.array_equal(bits(a), bits(g[f"edge_{tag}_y16"])), tag
        assert np.array_equal(bits(b), bits(g[f"edge_{tag}_y32"])), tag


SHAPES = [(Q5_0, 896, 896), (Q5_0, 4864, 896), (Q4_K, 896, 4864), (Q6_K, 896, 4864),
          (Q8_0, 128, 896), (Q8_0, 2000, 896), (Q8_0, 100, 96), (F32, 200, 4864), (F16, 64, 896)]


@pytest.mark.parametrize("qt,rows,cols", SHAPES)
def test_int16_vs_oracle(ctx, oracle, qt, rows, cols):
    """int64 tile results, x_scale and outputs of the INT16 path at the
    model's shapes"""
    import tmq
    print(f"[paths] int16 type={qt} {rows}x{cols}", flush=True)
    w = synth.gen_weights(qt, rows, cols, 700 + rows)
    x = synth.gen_x(cols, 800 + cols)
    t = ctx.upload(qt, rows, cols, w)
    try:
        acc, xs = ctx.partials_int16(t, x)
        y = ctx.matmul_path(t, x, tmq.PATH_INT16)
    finally:
        t.free()
    ye, te, _ = oracle.matmul_int16(qt, w, x, rows, cols)
    _, xse = oracle.quantize_act(x)
    assert xs == xse
    assert np.array_equal(acc, te), f"{np.sum(acc != te)} tile mismatches"
    assert np.array_equal(bits(y), bits(ye)), mism(y, ye)


@pytest.mark.parametrize("qt,rows,cols", [(Q5_0, 896, 896), (Q4_K, 896, 4864), (Q6_K, 128, 4864),
                                          (Q8_0, 1000, 896), (F32, 64, 896)])
def test_fp32_vs_oracle(ctx, oracle, qt, rows, cols):
    import tmq
    print(f"[paths] fp32 type={qt} {rows}x{cols}", flush=True)
    w = synth.gen_weights(qt, rows, cols, 900 + rows)
    x = synth.gen_x(cols, 950 + cols)
    t = ctx.upload(qt, rows, cols, w)
    try:
        y = ctx.matmul_path(t, x, tmq.PATH_FP32)
    finally:
        t.free()
    ye = oracle.matmul_fp32(qt, w, x, rows, cols)
    assert np.array_equal(bits(y), bits(ye)), mism(y, ye)


def test_matmul_flags_routes(ctx, oracle):
    """tmq_matmul_flags takes the branch the reference's matmul takes"""
    import tmq
    rows, cols = 256, 896
    w = synth.gen_weights(Q5_0, rows, cols, 31)
    x = synth.gen_x(cols, 32)
    t = ctx.upload(Q5_0, rows, cols, w)
    try:
        got = {f: ctx.matmul_flags(t, x, f) for f in (0, tmq.FLAG_FPGA, tmq.FLAG_FPGA | tmq.FLAG_Q5_0,
                                                       tmq.FLAGS_ALL & ~tmq.FLAG_Q5_0)}
    finally:
        t.free()
    assert np.array_equal(bits(got[0]), bits(oracle.matmul_fp32(Q5_0, w, x, rows, cols)))
    y16, _, _ = oracle.matmul_int16(Q5_0, w, x, rows, cols)
    assert np.array_equal(bits(got[tmq.FLAG_FPGA]), bits(y16))
    assert np.array_equal(bits(got[tmq.FLAGS_ALL & ~tmq.FLAG_Q5_0]), bits(y16))
    assert np.array_equal(bits(got[tmq.FLAG_FPGA | tmq.FLAG_Q5_0]), bits(oracle.matmul(Q5_0, w, x, rows, cols)))


def test_float_tensor_errors(ctx):
    import tmq
    w = synth.gen_weights(F32, 8, 64, 1)
    t = ctx.upload(F32, 8, 64, w)
    try:
        with pytest.raises(tmq.TmqError, match="matmul_fpga"):
            ctx.matmul(t, synth.gen_x(64, 2))
    finally:
        t.free()
    bad = w.copy().view(np.float32)
    bad[5] = np.inf
    with pytest.raises(tmq.TmqError) as e:
        ctx.upload(F32, 8, 64, bad.view(np.uint8))
    assert e.value.code == -3
