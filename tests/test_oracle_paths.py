"""Pins the oracle's restatement of the other two branches of `matmul`
(sim/tmac_gguf.cpp:473-493) -- matmul_fpga_int16 (:887-940) and the FP32
loop (:488-492) -- on the CPU: against the golden vectors written from the
compiled reference (tests/golden/matmul_paths.npz), the independent numpy
decode of the ggml layouts, and closed forms (one-hot activations, the
arg-max element's +-32767, zero rows, row-sharding independence), chosen so
that a dropped term, a transposed operand or a wrong rounding fails one of
them.  Also the routing table of `matmul` (tmq_route, host only)."""
import numpy as np
import pytest
from conftest import load_golden
from oracle import F16, F32, Q4_K, Q5_0, Q6_K, Q8_0
from tmq import synth
from test_oracle import np_decode


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def golden_cases():
    g = load_golden("matmul_paths.npz")
    return [str(n) for n in g["names"]]


@pytest.mark.parametrize("name", ["q8_0", "q5_0", "q4_k", "q6_k", "f32", "f16"])
def test_oracle_matches_reference_golden(oracle, name):
    g = load_golden("matmul_paths.npz")
    qt, rows, cols = (int(v) for v in g[f"{name}_meta"])
    w, x = g[f"{name}_w"], g[f"{name}_x"]
    y16, _, _ = oracle.matmul_int16(qt, w, x, rows, cols)
    assert np.array_equal(bits(y16), bits(g[f"{name}_y16"]))
    assert np.array_equal(bits(oracle.matmul_fp32(qt, w, x, rows, cols)), bits(g[f"{name}_y32"]))


def test_oracle_matches_reference_golden_edges(oracle):
    g = load_golden("matmul_paths.npz")
    w = g["q5_0_w"]
    for tag in ("x0", "x1"):
        y16, _, _ = oracle.matmul_int16(Q5_0, w, g[f"edge_{tag}"], 70, 896)
        assert np.array_equal(bits(y16), bits(g[f"edge_{tag}_y16"]))
        y32 = oracle.matmul_fp32(Q5_0, w, g[f"edge_{tag}"], 70, 896)
        assert np.array_equal(bits(y32), bits(g[f"edge_{tag}_y32"]))


def decode(qt, w, rows, cols):
    if qt == F32:
        return w.view(np.float32).reshape(rows, cols)
    if qt == F16:
        return w.view(np.float16).astype(np.float32).reshape(rows, cols)
    return np_decode(qt, w, rows, cols)


@pytest.mark.parametrize("qt,rows,cols", [(Q8_0, 70, 896), (Q5_0, 64, 896), (Q4_K, 16, 512),
                                          (Q6_K, 16, 512), (F32, 9, 96), (F16, 9, 96)])
def test_read_tensor_against_numpy_decode(oracle, qt, rows, cols):
    w = synth.gen_weights(qt, rows, cols, 8)
    E = decode(qt, w, rows, cols)
    got = np.array([[oracle.read_tensor(qt, w, cols, r, j) for j in range(cols)] for r in range(rows)],
                   dtype=np.float32)
    assert np.array_equal(bits(got), bits(E))


@pytest.mark.parametrize("qt,rows,cols", [(Q8_0, 70, 896), (Q5_0, 64, 896), (Q4_K, 16, 768),
                                          (Q6_K, 16, 768), (F32, 9, 160)])
def test_int16_one_hot_closed_form(oracle, qt, rows, cols):
    """x = c * e_j: x_scale = |c|/32767 and xq = +-32767 at j, 0 elsewhere, so
    every tile result is 0 except tile j//64, which is xq_j * w_rj with
    w_rj = roundf(E_rj / row_scale_r) (the arg-max element of a row -> +-32767)."""
    w = synth.gen_weights(qt, rows, cols, 9)
    E = decode(qt, w, rows, cols)
    m = np.max(np.abs(E), axis=1)
    rs = np.where(m < np.float32(1e-10), np.float32(1.0), m / np.float32(32767.0)).astype(np.float32)
    for j, c in ((0, 1.5), (cols - 1, -0.25), (cols // 2 + 3, 7.0)):
        x = np.zeros(cols, np.float32)
        x[j] = np.float32(c)
        y, tiles, rso = oracle.matmul_int16(qt, w, x, rows, cols)
        assert np.array_equal(bits(rso), bits(rs))
        q = (E[:, j] / rs).astype(np.float64)
        wq = (np.sign(q) * np.floor(np.abs(q) + 0.5)).astype(np.int64)
        exp = np.zeros_like(tiles)
        exp[:, j // 64] = np.int64(np.sign(c) * 32767) * wq
        assert np.array_equal(tiles, exp)
        a = np.argmax(np.abs(E), axis=1)
        assert np.all(np.abs(np.rint(E[np.arange(rows), a] / rs)) == 32767)
        # one non-zero tile: y = (float)((double)P * x_scale * row_scale)
        xs = np.float64(np.float32(abs(c)) / np.float32(32767.0))
        ye = ((exp[:, j // 64].astype(np.float64) * xs) * rs.astype(np.float64)).astype(np.float32)
        assert np.array_equal(bits(y), bits(ye))


@pytest.mark.parametrize("qt,rows,cols", [(Q8_0, 20, 896), (Q5_0, 20, 896), (Q4_K, 10, 768),
                                          (Q6_K, 10, 768), (F16, 9, 96)])
def test_fp32_closed_forms(oracle, qt, rows, cols):
    """one-hot x: y_r = 0 + E_rj * x_j exactly (the other terms add zeros);
    x = 1: y_r is the sequential fp32 sum of the row (np.add.accumulate
    adds in index order)."""
    w = synth.gen_weights(qt, rows, cols, 10)
    E = decode(qt, w, rows, cols)
    x = np.zeros(cols, np.float32)
    x[cols - 5] = np.float32(-3.25)
    # (0 + p: a -0 product comes out +0)
    exp = np.float32(0.0) + E[:, cols - 5] * x[cols - 5]
    assert np.array_equal(bits(oracle.matmul_fp32(qt, w, x, rows, cols)), bits(exp))
    ones = np.ones(cols, np.float32)
    seq = np.add.accumulate(E, axis=1, dtype=np.float32)[:, -1]
    assert np.array_equal(bits(oracle.matmul_fp32(qt, w, ones, rows, cols)), bits(seq))


def test_int16_rows_independent(oracle):
    """rows shard freely: a row slice gives the same outputs and tiles"""
    w = synth.gen_weights(Q5_0, 128, 896, 14)
    x = synth.gen_x(896, 15)
    y, t, _ = oracle.matmul_int16(Q5_0, w, x, 128, 896)
    per = 28 * 22
    y2, t2, _ = oracle.matmul_int16(Q5_0, w[40 * per:100 * per], x, 60, 896)
    assert np.array_equal(bits(y[40:100]), bits(y2)) and np.array_equal(t[40:100], t2)


def test_route_table():
    """sim/tmac_gguf.cpp:473-493: no --fpga flag -> FP32 loop; --fpga on ->
    the type's own matmul_fpga_* when its flag is set, else matmul_fpga_int16
    (F32/F16 have no flag of their own)."""
    import tmq
    for qt, own in ((Q8_0, tmq.FLAG_Q8_0), (Q5_0, tmq.FLAG_Q5_0), (Q4_K, tmq.FLAG_Q4_K), (Q6_K, tmq.FLAG_Q6_K)):
        assert tmq.route(qt, 0) == tmq.PATH_FP32
        assert tmq.route(qt, own) == tmq.PATH_FP32  # a type flag alone never happens without g_use_fpga
        assert tmq.route(qt, tmq.FLAG_FPGA) == tmq.PATH_INT16
        assert tmq.route(qt, tmq.FLAG_FPGA | own) == tmq.PATH_FPGA
        assert tmq.route(qt, tmq.FLAGS_ALL & ~own) == tmq.PATH_INT16
        assert tmq.route(qt, tmq.FLAGS_ALL) == tmq.PATH_FPGA
    for qt in (F32, F16):
        assert tmq.route(qt, tmq.FLAGS_ALL) == tmq.PATH_INT16
        assert tmq.route(qt, 0) == tmq.PATH_FP32
    with pytest.raises(tmq.TmqError):
        tmq.route(3, tmq.FLAGS_ALL)
