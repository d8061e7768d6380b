"""Golden tile and MAC counts of the reference's [FPGA TIMING SUMMARY], from the
compiled reference engine (build container only).

Every matmul_fpga_* adds rows*cols to g_timing.total_mac_ops and one to
total_tiles per tile it runs (sim/tmac_gguf.cpp:899-934, :963-1078,
:1109-1188, :1233-1300, :1379-1497); the FP32 loop adds nothing.  The summary
prints them with the time spent (sim/fpga_sim.hpp:156-172).  For the synthetic
C4 model and each flag set, timing.npz holds the counts of one decode step
(process_embedding + forward_all_layers) and of one logits call as generate /
main pick it (get_logits_q8 under --fpga-q8, else get_logits):

  <set>_flags, <set>_step (tiles, macs), <set>_logits (tiles, macs)

    make -C oracle && python tests/golden/gen_timing_golden.py
"""
from __future__ import annotations

import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tmac-zynq-fpga_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from oracle import Reference  # noqa: E402
from tmq import model_synth, tmacfile  # noqa: E402
from gen_model_golden import MODEL_SEED, prompt_token  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
# bit 0 g_use_fpga, 1 g_fpga_q8, 2 g_fpga_q5_0, 3 g_fpga_q4k, 4 g_fpga_q6_k
SETS = [("all", 31), ("q8q5", 1 | 2 | 4), ("int16", 1), ("q4k", 1 | 8), ("q6k", 1 | 16), ("fp32", 0)]


def main():
    R = Reference()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "c4.tmac")
        tmacfile.write(path, model_synth.gen_model(MODEL_SEED))
        R.model_load(path)
    tok = prompt_token()
    out = {"model_seed": MODEL_SEED}
    for name, flags in SETS:
        R.model_set_flags(flags)
        R.model_reset()
        hidden = np.zeros(R.HIDDEN, dtype=np.float32)
        R.timing_reset()
        R.model_step(hidden, tok, 0)
        step = R.timing_counts()
        R.timing_reset()
        R.model_logits_auto(hidden)
        lg = R.timing_counts()
        out[f"{name}_flags"] = np.int64(flags)
        out[f"{name}_step"] = np.array(step, dtype=np.int64)
        out[f"{name}_logits"] = np.array(lg, dtype=np.int64)
        print(f"{name}: step {step}, logits {lg}", flush=True)
    np.savez(os.path.join(OUT, "timing.npz"), **out)


if __name__ == "__main__":
    main()
