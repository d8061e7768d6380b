"""Pins the CPU oracle (oracle/tmq_oracle.c) -- runs on CPU.

Checks, per function, against what fixes it independently of the oracle's
own formulas: the golden vectors written from the compiled reference, the
reference's own known-answer tests (sim/test_integration.cpp,
verilog/tb_matmul_q8.v), an independent numpy decode of the ggml layouts,
and closed forms of the arithmetic.
"""
import numpy as np
import pytest
from conftest import load_golden
from oracle import Q4_K, Q5_0, Q6_K, Q8_0
from tmq import synth


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- f16
def test_f16_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib.tmqo_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    finite = np.isfinite(ref)
    # reference maps -0 -> +0 (sim/tmac_gguf.cpp:220) and NaN -> qNaN
    ref_f = np.where(ref == 0, np.float32(0.0), ref)
    assert np.array_equal(bits(got[finite]), bits(ref_f[finite]))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


# ------------------------------------------------------ activation quantiser
def test_quantize_act_closed_forms(oracle):
    x = synth.gen_x(4864, 5)
    xq, s = oracle.quantize_act(x)
    m = np.max(np.abs(x))
    assert s == np.float32(m / np.float32(32767.0))
    assert np.max(np.abs(xq.astype(np.int32))) == 32767
    assert xq[np.argmax(np.abs(x))] == np.sign(x[np.argmax(np.abs(x))]) * 32767
    # roundf = half away from zero on the quotient
    qf = x / s
    expect = np.where(qf >= 0, np.floor(qf + 0.5), -np.floor(-qf + 0.5)).astype(np.int16)
    assert np.array_equal(xq, expect)
    xq0, s0 = oracle.quantize_act(np.zeros(896, np.float32))
    assert s0 == 1.0 and not xq0.any()
    tiny = np.full(16, 1e-11, np.float32)
    xqt, st = oracle.quantize_act(tiny)
    assert st == 1.0 and not xqt.any()


# ----------------------------------------------- independent numpy decode
def np_decode(qt, w, rows, cols):
    """Dequantised E per element, from the ggml layout documentation
    (docs/architecture.md:62-114 with the corrected Q5_0 offsets of
    sim/tmac_gguf.cpp:310-319), vectorised and written independently."""
    f16 = lambda b: b.copy().view(np.float16).astype(np.float32)  # noqa: E731
    if qt == Q5_0:
        B = w.reshape(-1, 22)
        d = f16(B[:, 0:2]).reshape(-1, 1)
        qh = B[:, 2:6].copy().view(np.uint32).reshape(-1, 1)
        qs = B[:, 6:22]
        nib = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int32)
        hb = ((qh >> np.arange(32, dtype=np.uint32)) & 1).astype(np.int32)
        q = (nib | (hb << 4)) - 16
        return (d * q.astype(np.float32)).reshape(rows, cols)
    if qt == Q4_K:
        B = w.reshape(-1, 144)
        d = f16(B[:, 0:2]).reshape(-1, 1)
        dm = f16(B[:, 2:4]).reshape(-1, 1)
        s = B[:, 4:16].astype(np.int32)
        sc = np.zeros((B.shape[0], 8), np.int32)
        mn = np.zeros((B.shape[0], 8), np.int32)
        sc[:, :4], mn[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
        sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        qs = B[:, 16:].reshape(-1, 4, 32).astype(np.int32)
        q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32)
        A = (d * sc.astype(np.float32))[:, :, None] * q.astype(np.float32)
        Bm = (dm * mn.astype(np.float32))[:, :, None]
        return (A - Bm).reshape(rows, cols).astype(np.float32)
    if qt == Q6_K:
        B = w.reshape(-1, 210)
        ql, qh = B[:, 0:128].astype(np.int32), B[:, 128:192].astype(np.int32)
        sc = B[:, 192:208].view(np.int8).astype(np.float32)
        d = f16(B[:, 208:210]).reshape(-1, 1)
        out = np.zeros((B.shape[0], 256), np.float32)
        for half in range(2):
            for sub in range(4):
                for l in range(32):
                    qlb = ql[:, half * 64 + l + (sub & 1) * 32]
                    nib = (qlb & 15) if sub < 2 else (qlb >> 4)
                    hb = (qh[:, half * 32 + l] >> (2 * sub)) & 3
                    q = (nib | (hb << 4)) - 32
                    S = d[:, 0] * sc[:, half * 8 + l // 16 + sub * 2]
                    out[:, half * 128 + sub * 32 + l] = S * q.astype(np.float32)
        return out.reshape(rows, cols)
    if qt == Q8_0:
        B = w.reshape(-1, 34)
        d = f16(B[:, 0:2]).reshape(-1, 1)
        return (B[:, 2:].view(np.int8).astype(np.float32) * d).reshape(rows, cols)
    raise ValueError(qt)


@pytest.mark.parametrize("qt,rows,cols", [(Q5_0, 64, 896), (Q4_K, 32, 1024), (Q6_K, 32, 1024)])
def test_row_inv_against_numpy_decode(oracle, qt, rows, cols):
    w = synth.gen_weights(qt, rows, cols, 3)
    E = np_decode(qt, w, rows, cols)
    m = np.max(np.abs(E), axis=1)
    m = np.where(m < np.float32(1e-10), np.float32(1.0), m)
    expect = (np.float32(32767.0) / m).astype(np.float32)
    assert np.array_equal(bits(oracle.row_inv(qt, w, rows, cols)), bits(expect))


def test_q8_row_max_against_numpy_decode(oracle):
    w = synth.gen_weights(Q8_0, 64, 896, 4)
    E = np_decode(Q8_0, w, 64, 896)
    assert np.array_equal(bits(oracle.row_max_abs_q8(w, 64, 896)), bits(np.max(np.abs(E), axis=1)))


@pytest.mark.parametrize("qt,rows,cols", [(Q5_0, 32, 896), (Q4_K, 16, 512), (Q6_K, 16, 512)])
def test_acc_against_numpy_brute_force(oracle, qt, rows, cols):
    """int64 accumulators from an independent float32 numpy evaluation of
    w = clamp16(roundf(E*row_inv)) and an int64 dot product."""
    w = synth.gen_weights(qt, rows, cols, 9)
    x = synth.gen_x(cols, 10)
    xq, xs = oracle.quantize_act(x)
    ri = oracle.row_inv(qt, w, rows, cols)
    E = np_decode(qt, w, rows, cols)
    n = (E * ri[:, None]).astype(np.float32)
    r = np.where(n >= 0, np.floor(n + np.float32(0.5)), -np.floor(-n + np.float32(0.5)))
    # n is exactly representable and |n| < 2^23: floor(n+0.5) in float32 is exact
    wq = np.clip(r, -32768, 32767).astype(np.int64)
    expect = wq @ xq.astype(np.int64)
    assert np.array_equal(oracle.acc(qt, w, rows, cols, xq, ri), expect)
    # arg-max element of every row normalises to +-32767
    am = np.argmax(np.abs(E), axis=1)
    assert np.all(np.abs(wq[np.arange(rows), am]) == 32767)


# ----------------------------------------------------- reference KATs
def _f16_bytes(v):
    return np.array([v], np.float16).view(np.uint8)


def test_q4k_constant_block_kat(oracle):
    """sim/test_integration.cpp:98-155: d=1, dmin=0, sc=1, m=0, q4=8, act=1,
    row_inv=1, 16 blocks, 64-column tile -> every row sums to 8*64."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = _f16_bytes(1.0)
    blk[2:4] = _f16_bytes(0.0)
    blk[4:8] = 1
    blk[12:16] = 1
    blk[16:] = 8 | (8 << 4)
    blocks = np.tile(blk, 16)
    res = np.zeros(896, np.int64)
    oracle.tile_kquant(Q4_K, blocks, 16, np.ones(64, np.int16), 64, np.ones(896, np.float32), res, 0)
    assert np.all(res[:16] == 512) and not res[16:].any()


@pytest.mark.parametrize("wt,cs,act,expect", [(1, 256, 1, 64), (0, 256, 1, 0), (1, 512, 1, 128),
                                              (1, 256, 2, 128), (1, 256, 0, 0), (-1, 256, 1, -64)])
def test_q8_tile_kats(oracle, wt, cs, act, expect):
    """verilog/tb_matmul_q8.v:127-199 directed tests (same integer semantic
    as the C++ tile, deq = (q8*cs) >> 8)."""
    W = np.full(4096, wt, np.int8).view(np.uint8)
    r = oracle.tile_q8(W, np.full(128, cs, np.uint16), np.full(64, act, np.int16))
    assert np.all(r == expect)


def test_q8_combined_scale_special_cases(oracle):
    lib = oracle.lib
    one = int(np.array([1.0], np.float16).view(np.uint16)[0])
    # arg-max block always clamps (c = 32767/127 > 256) -> 65535
    rs = np.float32(127.0) / np.float32(32767.0)
    assert lib.tmqo_q8_combined_scale(one, float(rs)) == 65535
    # c*256+0.5 rounding up to 65536 wraps to 0 (x86 float->uint16)
    target = np.float32(255.999)
    rs2 = np.float32(1.0) / target
    ri2 = np.float32(1.0) / rs2
    if np.float32(ri2) * np.float32(256.0) + np.float32(0.5) >= np.float32(65536.0):
        assert lib.tmqo_q8_combined_scale(one, float(rs2)) == 0
    # negative scale -> clamped to 0
    neg = int(np.array([-1.0], np.float16).view(np.uint16)[0])
    assert lib.tmqo_q8_combined_scale(neg, float(rs)) == 0
    # zero row -> row_scale 1
    assert lib.tmqo_q8_row_scale(0.0) == 1.0


def test_zero_row_and_zero_activation(oracle):
    g = load_golden("edge_q5_0.npz")
    w = g["w"]
    y0 = oracle.matmul(Q5_0, w, g["x0"], 8, 896)
    assert not y0.any()
    ys = oracle.matmul(Q5_0, w, g["xs"], 8, 896)
    assert ys[5] == 0.0  # d = 0 row


def test_row_sharding_independence(oracle):
    """Rows are independent: a row slice of the weights gives the same
    outputs as the same rows of the full product (sharding by rows)."""
    for qt, cols in ((Q5_0, 896), (Q4_K, 512), (Q6_K, 512), (Q8_0, 896)):
        qk, bb = synth.BLOCK[qt]
        w = synth.gen_weights(qt, 64, cols, 12)
        x = synth.gen_x(cols, 13)
        full = oracle.matmul(qt, w, x, 64, cols)
        per = cols // qk * bb
        part = oracle.matmul(qt, w[16 * per:48 * per], x, 32, cols)
        assert np.array_equal(bits(full[16:48]), bits(part))


# ------------------------------------------------------------ golden
@pytest.mark.parametrize("name", ["q5_0", "q8_0", "q8_0_c64", "q4_k", "q6_k"])
def test_oracle_matches_golden_matmul(oracle, name):
    g = load_golden(f"matmul_{name}.npz")
    qt, rows, cols = int(g["qtype"]), int(g["rows"]), int(g["cols"])
    y = oracle.matmul(qt, g["w"], g["x"], rows, cols)
    assert np.array_equal(bits(y), bits(g["y"]))
    if qt == Q8_0:
        ya = oracle.matmul(qt, g["w"], g["x"], rows, cols, g["aux"])
        assert np.array_equal(bits(ya), bits(g["y_aux"]))
        assert np.array_equal(bits(ya), bits(y))  # aux tensor == inline scan


def test_oracle_matches_golden_edges(oracle):
    g = load_golden("edge_q5_0.npz")
    assert np.array_equal(bits(oracle.matmul(Q5_0, g["w"], g["x0"], 8, 896)), bits(g["y0"]))
    assert np.array_equal(bits(oracle.matmul(Q5_0, g["w"], g["xs"], 8, 896)), bits(g["ys"]))


def test_oracle_matches_golden_tiles(oracle):
    g = load_golden("tiles.npz")
    assert np.array_equal(oracle.tile_q8(g["W"], g["cs"], g["vec"]), g["tq8"])
    r5 = g["res5_in"].copy()
    oracle.tile_q5_0_8x896(g["b5"], g["act896"], g["ri8"], r5, 8)
    assert np.array_equal(r5, g["res5"])
    r6 = np.zeros(896, np.int64)
    oracle.tile_kquant(Q6_K, g["b6"], 32, g["act256"], 256, g["ri896"], r6, 864)
    assert np.array_equal(r6, g["res6"])
    r4 = np.zeros(896, np.int64)
    oracle.tile_kquant(Q4_K, g["b4"], 56, g["act256"], 200, g["ri896"], r4, 840)
    assert np.array_equal(r4, g["res4"])


def test_oracle_matches_golden_phaseb(oracle):
    g = load_golden("phaseb.npz")
    arena, base, head = g["arena"], int(g["base"]), int(g["head"])
    off, k, got_rows, got = head, 0, [], []
    while off:
        n, acc = oracle.phaseb_run(arena, base, off, 1024)
        got_rows.append(n)
        got.append(acc[:n])
        off = int(arena[off - base: off - base + 4].view(np.uint32)[0])
        k += 1
    assert got_rows == list(g["rows"])
    assert np.array_equal(np.concatenate(got), g["acc"])
