"""Golden PhaseB chain with every descriptor kind the reference's replay
knows (build container only, from the compiled reference):

  three matmul descriptors built by matmul_fpga_q5_0 / _q6_k / _q4_k with
  --fpga-phaseb semantics (sim/tmac_gguf.cpp:1140-1211, 1307-1355,
  1430-1516), then, added with phaseb_add_descriptor (:533-574):
  - an OP->OP descriptor: Q5_0 tiles whose activation address is the
    previous descriptor's result slot, so act_total_bytes is derived from
    the previous tile_res_rows (:551-561) and the replay reads the Q4_K
    results as its int16 activation;
  - a CPU_OP descriptor (type 15) and a Q8_0 descriptor, which the replay
    skips with 0 rows (:798-801, :823-829);
  - a Q6_K descriptor over copied tiles whose column group 1 carries other
    UQ24.8 row_inv values than group 0 (each tile's own value applies, :791-795).

The chain is replayed in order with every descriptor's results written to
its result slot before the next one runs, as phaseb_verify does (:846-852).
Stored in phaseb_chain.npz: arena (bytes from 0x18000000 as built, result
slots zero), arena_after (the same after the in-order replay), base, head,
rows per descriptor, results (concatenated), act_total_bytes per descriptor.

    make -C oracle && python tests/golden/gen_phaseb_chain_golden.py
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tmac-zynq-fpga_amd"))

from oracle import Q4_K, Q5_0, Q6_K, Reference  # noqa: E402
from tmq import synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
BASE = 0x18000000


def main():
    R = Reference()
    L = R.lib
    assert L.ref_phaseb_begin() == 0
    ddr = L.ref_ddr()

    def mem(addr, n):
        return np.frombuffer((C.c_uint8 * n).from_address(ddr + addr), dtype=np.uint8)

    w5 = synth.gen_weights(Q5_0, 16, 896, seed=131)
    w6 = synth.gen_weights(Q6_K, 64, 512, seed=132)
    w4 = synth.gen_weights(Q4_K, 112, 512, seed=133)
    xa, xb = synth.gen_x(896, 141), synth.gen_x(512, 142)
    for qt, w, x, rows, cols in ((Q5_0, w5, xa, 16, 896), (Q6_K, w6, xb, 64, 512), (Q4_K, w4, xb, 112, 512)):
        R.matmul(qt, w, x, rows, cols)
    offs = []
    off = L.ref_phaseb_head()
    while off:
        offs.append(off)
        off = int(mem(off, 4).view(np.uint32)[0])
    d5, d6, d4 = (mem(o, 32).copy() for o in offs)
    u32 = lambda d, o: int(d[o:o + 4].view(np.uint32)[0])  # noqa: E731
    # OP->OP: the Q5_0 tiles again, activation = the Q4_K result slot
    res_c = L.ref_phaseb_alloc(16 * 8)
    L.ref_phaseb_add_descriptor(u32(d5, 4), u32(d4, 12), res_c, 2, 4944, 6, 8, 0, 1792, 1)
    # CPU_OP and Q8_0: no matmul rows in the replay
    L.ref_phaseb_add_descriptor(0, 0, 0, 0, 0, 15, 0, 1, 0, 0)
    res_q8 = L.ref_phaseb_alloc(64 * 8)
    L.ref_phaseb_add_descriptor(u32(d5, 4), u32(d5, 8), res_q8, 2, 4352, 8, 64, 0, 128, 1)
    # Q6_K tiles copied, column group 1 with row_inv x 0.75 (UQ24.8)
    nt, tb = 4, 6848
    wt = L.ref_phaseb_alloc(nt * tb)
    tiles = mem(u32(d6, 4), nt * tb).copy()
    for ti in range(nt):
        if ti % 2 == 1:
            sc = tiles[ti * tb + 6720: ti * tb + 6848].view(np.uint32)
            sc[:] = (sc.astype(np.float64) * 0.75).astype(np.uint32)
    mem(wt, nt * tb)[:] = tiles
    res_k = L.ref_phaseb_alloc(64 * 8)
    L.ref_phaseb_add_descriptor(wt, u32(d6, 8), res_k, nt, tb, 14, 32, 0, 1024, 2)
    L.ref_phaseb_end()
    # replay in order, every result slot written before the next descriptor
    rows, results, atb, slots = [], [], [], []
    off = L.ref_phaseb_head()
    while off:
        d = mem(off, 32).copy()
        n, acc = R.phaseb_run(off, 1024)
        ra = u32(d, 12)
        if n:
            mem(ra, 8 * n)[:] = acc[:n].view(np.uint8)
            slots.append((ra, n))
        rows.append(n)
        results.append(acc[:n].copy())
        atb.append(int(d[0x17:0x19].view(np.uint16)[0]))
        off = u32(d, 0)
    end = L.ref_phaseb_next_off()
    after = mem(BASE, end - BASE).copy()
    # the arena before the replay: result slots as the build left them (zero)
    before = after.copy()
    for ra, n in slots:
        before[ra - BASE: ra - BASE + 8 * n] = 0
    np.savez_compressed(os.path.join(OUT, "phaseb_chain.npz"), base=BASE, head=L.ref_phaseb_head(),
                        arena=before, arena_after=after, rows=np.array(rows, np.int64),
                        acc=np.concatenate(results), atb=np.array(atb, np.int64))
    print("rows", rows, "act_total_bytes", atb, "arena", after.size)


if __name__ == "__main__":
    main()
