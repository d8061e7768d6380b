"""Write the golden vectors under tests/golden/ from the compiled reference.

Runs in the build container only: it loads oracle/_ref/libtmacref.so, the
reference's own sim/ sources (sim/tmac_gguf.cpp + sim/fpga_sim.hpp +
sim/matmul_q8.cpp) compiled in place by oracle/Makefile, feeds it seeded
synthetic inputs and stores inputs + reference outputs as .npz (no pickle).
The reference holds no golden vectors of its own for this path (no
*.bin/*.npz/*.hdr anywhere in it), so these are the pinned vectors.

    make -C oracle && python tests/golden/gen_golden.py
"""
from __future__ import annotations

import os
import zlib
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tmac-zynq-fpga_amd"))

from oracle import Q4_K, Q5_0, Q6_K, Q8_0, Reference  # noqa: E402
from tmq import synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def f16(v):
    return np.array([v], dtype=np.float16).view(np.uint16)[0]


def main():
    R = Reference()
    rng = np.random.Generator(np.random.PCG64(20261201))

    # 1. whole matmul_fpga_* calls (dispatch path), small shapes
    cases = [("q5_0", Q5_0, 24, 896), ("q8_0", Q8_0, 24, 896), ("q8_0_c64", Q8_0, 8, 96),
             ("q4_k", Q4_K, 24, 768), ("q6_k", Q6_K, 24, 768)]
    for name, qt, rows, cols in cases:
        w = synth.gen_weights(qt, rows, cols, seed=zlib.crc32(name.encode()) % 1000 + 7)
        x = synth.gen_x(cols, seed=len(name) * 31 + rows)
        y = R.matmul(qt, w, x, rows, cols)
        extra = {}
        if qt == Q8_0:
            # the logits path with the _row_max_abs aux tensor (sim/matmul_q8.cpp)
            d = w.reshape(-1, 34)[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(rows, -1)
            q = w.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.float32).reshape(rows, -1, 32)
            aux = np.max(np.abs(q * d[:, :, None]), axis=(1, 2)).astype(np.float32)
            extra["aux"] = aux
            extra["y_aux"] = R.matmul(qt, w, x, rows, cols, aux)
        # the reference's no-flag FP32 path, for context (not a parity target)
        extra["y_fp32"] = R.matmul_fp32(qt, w, x, rows, cols)
        np.savez(os.path.join(OUT, f"matmul_{name}.npz"), qtype=qt, rows=rows, cols=cols, w=w, x=x, y=y, **extra)

    # 2. edge cases of the dispatch path
    #    zero activation, zero weight row, one-element activation spike
    w = synth.gen_weights(Q5_0, 8, 896, seed=11)
    wz = w.reshape(8, 28, 22).copy()
    wz[3, :, 2:] = 0                        # row 3: all q = -16 ... but keep d
    wz[5, :, 0:2] = 0                       # row 5: d = 0 -> zero row
    x0 = np.zeros(896, dtype=np.float32)
    xs = np.zeros(896, dtype=np.float32)
    xs[17] = -3.5
    np.savez(os.path.join(OUT, "edge_q5_0.npz"), w=wz.reshape(-1), x0=x0, xs=xs,
             y0=R.matmul(Q5_0, wz.reshape(-1), x0, 8, 896), ys=R.matmul(Q5_0, wz.reshape(-1), xs, 8, 896))

    # 3. tile primitives
    W = rng.integers(-128, 128, size=4096, dtype=np.int8).view(np.uint8)
    cs = rng.integers(0, 65536, size=128, dtype=np.uint16)
    vec = rng.integers(-32767, 32768, size=64, dtype=np.int16)
    tq8 = R.tile_q8(W, cs, vec)
    b5 = synth.gen_weights(Q5_0, 8, 896, seed=21)
    act896 = rng.integers(-32767, 32768, size=896, dtype=np.int16)
    ri8 = (rng.random(8, dtype=np.float32) * np.float32(60000.0)).astype(np.float32)
    res5 = np.zeros(24, dtype=np.int64)
    res5[:] = rng.integers(-1000, 1000, size=24)
    res5_in = res5.copy()
    R.tile_q5_0_8x896(b5, act896, ri8, res5, 8)
    b6 = synth.gen_weights(Q6_K, 32, 256, seed=22)
    b4 = synth.gen_weights(Q4_K, 56, 256, seed=23)
    act256 = rng.integers(-32767, 32768, size=256, dtype=np.int16)
    ri896 = (rng.random(896, dtype=np.float32) * np.float32(3000.0) + np.float32(1.0)).astype(np.float32)
    res6 = np.zeros(896, dtype=np.int64)
    R.tile_kquant(Q6_K, b6, 32, act256, 256, ri896, res6, 864)   # rows 864..895
    res4 = np.zeros(896, dtype=np.int64)
    R.tile_kquant(Q4_K, b4, 56, act256, 200, ri896, res4, 840)   # ncols < 256
    np.savez(os.path.join(OUT, "tiles.npz"), W=W, cs=cs, vec=vec, tq8=tq8, b5=b5, act896=act896,
             ri8=ri8, res5_in=res5_in, res5=res5, b6=b6, b4=b4, act256=act256, ri896=ri896,
             res6=res6, res4=res4)

    # 4. a PhaseB descriptor chain (Q5_0 + Q6_K + Q4_K), built by the
    #    reference's matmul_fpga_* with --fpga-phaseb semantics, and its
    #    replay results (phaseb_run_descriptor)
    w5 = synth.gen_weights(Q5_0, 16, 896, seed=31)
    w6 = synth.gen_weights(Q6_K, 64, 512, seed=32)
    w4 = synth.gen_weights(Q4_K, 112, 512, seed=33)
    xa, xb = synth.gen_x(896, 41), synth.gen_x(512, 42)
    arena, base, head, nd = R.phaseb_build([(Q5_0, w5, xa, 16, 896), (Q6_K, w6, xb, 64, 512),
                                            (Q4_K, w4, xb, 112, 512)])
    rows = []
    accs = []
    off = head
    while off:
        d = arena[off - base: off - base + 32]
        n, acc = R.phaseb_run(off, 1024)
        rows.append(n)
        accs.append(acc[:n])
        off = int(d[0:4].view(np.uint32)[0])
    np.savez(os.path.join(OUT, "phaseb.npz"), arena=arena, base=base, head=head,
             rows=np.array(rows, dtype=np.int64), acc=np.concatenate(accs))
    print("golden vectors written to", OUT)


if __name__ == "__main__":
    main()
