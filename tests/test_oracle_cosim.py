"""CPU checks of the PhaseB chain and cosimulation-dump goldens written from
the compiled reference (tests/golden/gen_phaseb_chain_golden.py,
gen_cosim_golden.py): the oracle's descriptor replay (tmqo_phaseb_run,
sim/tmac_gguf.cpp:761-831) run in chain order with every result written to
its slot reproduces the reference's replay of a chain holding matmul,
OP->OP, CPU_OP, Q8_0 and mixed-row_inv descriptors; the dump goldens have
the reference's byte layouts, their first tiles agree with the oracle's
tile primitives, and the later tiles show the reference's overflowed
(zero) results that the fixed values replace."""
import numpy as np
from conftest import load_golden
from oracle import Q6_K


def test_oracle_chain_replay_in_order(oracle):
    g = load_golden("phaseb_chain.npz")
    arena, base = g["arena"].copy(), int(g["base"])
    off, rows, accs = int(g["head"]), [], []
    while off:
        n, acc = oracle.phaseb_run(arena, base, off, 1024)
        d = arena[off - base: off - base + 32]
        ra = int(d[12:16].view(np.uint32)[0])
        if n:
            arena[ra - base: ra - base + 8 * n] = acc[:n].view(np.uint8)
        rows.append(n)
        accs.append(acc[:n])
        off = int(d[0:4].view(np.uint32)[0])
    assert rows == g["rows"].tolist()
    assert np.array_equal(np.concatenate(accs), g["acc"])
    assert np.array_equal(arena, g["arena_after"])
    # OP->OP: act_total_bytes derived from the previous tile_res_rows (56 * 8)
    assert g["atb"].tolist()[3] == 56 * 8


def test_cosim_dump_layouts(oracle):
    g = load_golden("cosim.npz")
    for k, rec, n in (("q8", 4992, 4), ("q5", 6816, 3), ("q6", 7616, 3)):
        d = g[k]
        assert d.size == 16 + n * rec
        assert d[:16].view(np.uint32).tolist() == [n, 0, 0, 0]
    # Q8 tile: the oracle's tile primitive reproduces every dumped result
    q8 = g["q8"]
    for t in range(4):
        r = q8[16 + t * 4992: 16 + (t + 1) * 4992]
        res = oracle.tile_q8(r[:4096].copy(), r[4096:4352].copy().view(np.uint16), r[4352:4480].copy().view(np.int16))
        assert np.array_equal(res, r[4480:].copy().view(np.int64))
    # Q5_0 / Q6_K: tile 0 as the oracle computes it, later tiles zero in the
    # reference's dump and non-zero in the fixed values
    q5 = g["q5"]
    for t in range(3):
        r = q5[16 + t * 6816: 16 + (t + 1) * 6816]
        res = np.zeros(8, np.int64)
        oracle.tile_q5_0_8x896(r[:4928].copy(), r[4928:6720].copy().view(np.int16),
                               r[6720:6752].copy().view(np.float32), res, 0)
        assert np.array_equal(res, g["q5_fixed"][t])
        dumped = r[6752:].copy().view(np.int64)
        assert np.array_equal(dumped, res) if t == 0 else (not dumped.any() and res.any())
    q6 = g["q6"]
    for t in range(3):
        r = q6[16 + t * 7616: 16 + (t + 1) * 7616]
        ri = np.zeros(896, np.float32)
        ri[32 * t: 32 * t + 32] = r[7232:7360].copy().view(np.float32)
        res = np.zeros(896, np.int64)
        oracle.tile_kquant(Q6_K, r[:6720].copy(), 32, r[6720:7232].copy().view(np.int16), 256, ri, res, 32 * t)
        assert np.array_equal(res[32 * t: 32 * t + 32], g["q6_fixed"][t])
        dumped = r[7360:].copy().view(np.int64)
        assert np.array_equal(dumped, g["q6_fixed"][t]) if t == 0 else not dumped.any()
