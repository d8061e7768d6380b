"""Write tests/golden/matmul_paths.npz from the compiled reference: the two
branches of `matmul` besides matmul_fpga_* (sim/tmac_gguf.cpp:473-493) --
matmul_fpga_int16 (:887-940, taken when --fpga is on and the tensor type's
own flag is off) and the FP32 loop (:488-492, no --fpga flag) -- on every
tensor type they read (F32, F16, Q8_0, Q5_0, Q4_K, Q6_K), with seeded
synthetic inputs, plus edge cases (a zero row, a zero activation, a one-hot
activation, row counts that are not a multiple of 64).

Runs in the build container only (it loads oracle/_ref/libtmacref.so, the
reference's sim/ sources compiled in place by oracle/Makefile):

    make -C oracle && python tests/golden/gen_paths_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tmac-zynq-fpga_amd"))

from oracle import Reference  # noqa: E402
from tmq import synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# (name, type, rows, cols, weight seed)
CASES = [
    ("q8_0", synth.Q8_0, 24, 896, 71), ("q5_0", synth.Q5_0, 70, 896, 72),
    ("q4_k", synth.Q4_K, 24, 768, 73), ("q6_k", synth.Q6_K, 24, 768, 74),
    ("f32", synth.F32, 20, 160, 75), ("f16", synth.F16, 9, 96, 76),
]


def main():
    R = Reference()
    out = {}
    for name, qt, rows, cols, seed in CASES:
        w = synth.gen_weights(qt, rows, cols, seed)
        if qt == synth.Q5_0:
            # row 5: every block scale 0 -> a zero row (row_scale guard)
            per = (cols // 32) * 22
            w = w.copy()
            blk = w[5 * per:6 * per].reshape(-1, 22)
            blk[:, 0:2] = 0
        x = synth.gen_x(cols, seed + 1000)
        out[f"{name}_meta"] = np.array([qt, rows, cols], dtype=np.int64)
        out[f"{name}_w"] = w
        out[f"{name}_x"] = x
        out[f"{name}_y16"] = R.matmul_int16(qt, w, x, rows, cols)
        out[f"{name}_y32"] = R.matmul_fp32(qt, w, x, rows, cols)
    # activation edge cases on the Q5_0 case: all zero, one hot
    w, cols, rows = out["q5_0_w"], 896, 70
    x0 = np.zeros(cols, np.float32)
    x1 = np.zeros(cols, np.float32)
    x1[300] = np.float32(-2.75)
    for tag, xx in (("x0", x0), ("x1", x1)):
        out[f"edge_{tag}"] = xx
        out[f"edge_{tag}_y16"] = R.matmul_int16(synth.Q5_0, w, xx, rows, cols)
        out[f"edge_{tag}_y32"] = R.matmul_fp32(synth.Q5_0, w, xx, rows, cols)
    np.savez(os.path.join(OUT, "matmul_paths.npz"), names=np.array([c[0] for c in CASES]), **out)
    print("wrote", os.path.join(OUT, "matmul_paths.npz"))


if __name__ == "__main__":
    main()
