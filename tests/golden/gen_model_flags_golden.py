"""Golden greedy decode of the synthetic C4 model under the reference's other
flag sets, from the compiled reference engine (build container only).

The reference's `matmul` (sim/tmac_gguf.cpp:473-493) routes every projection
by its tensor type and the command-line flags (:2085-2091), and generate /
main pick get_logits_q8 only under --fpga-q8 (:2033-2037, :2151-2155):

  q8q5   --fpga-q8 --fpga-q5-0   Q5_0/Q8_0 by their own paths, the Q4_K/Q6_K
                                 ffn_down through matmul_fpga_int16
  int16  --fpga (= --fpga-int16)  every projection and the logits through
                                 matmul_fpga_int16 (get_logits)
  fp32   no flag                 the FP32 read_tensor loop everywhere

Stored per set in model_flags.npz (no pickle): <set>_flags, <set>_tokens[N]
(greedy: first index of the largest logit), <set>_top_ids / _top_vals
[N, 10], <set>_logits_sub (every 64th logit of step 0), <set>_layers0
[25, 896] (hidden after the embedding and each layer at position 0),
<set>_hidden_final.

    make -C oracle && python tests/golden/gen_model_flags_golden.py [--steps 8]
"""
from __future__ import annotations

import argparse
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tmac-zynq-fpga_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from oracle import Reference  # noqa: E402
from tmq import model_synth, tmacfile  # noqa: E402
from gen_model_golden import MODEL_SEED, prompt_token, top10  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
# bit 0 g_use_fpga, 1 g_fpga_q8, 2 g_fpga_q5_0, 3 g_fpga_q4k, 4 g_fpga_q6_k
SETS = [("q8q5", 1 | 2 | 4), ("int16", 1), ("fp32", 0)]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=8)
    args = ap.parse_args()
    R = Reference()
    t0 = time.time()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "c4.tmac")
        tmacfile.write(path, model_synth.gen_model(MODEL_SEED))
        R.model_load(path)
    tok = prompt_token()
    out = {"model_seed": MODEL_SEED, "prompt": np.array([tok], dtype=np.int32)}
    for name, flags in SETS:
        R.model_set_flags(flags)
        R.model_reset()
        hidden = np.zeros(R.HIDDEN, dtype=np.float32)
        layers0 = R.model_step(hidden, tok, 0, dump=True)
        toks, tids, tvals = [], [], []
        for gen in range(args.steps):
            t1 = time.time()
            logits = R.model_logits_auto(hidden)
            ids, vals = top10(logits)
            toks.append(int(ids[0]))
            tids.append(ids)
            tvals.append(vals)
            if gen == 0:
                out[f"{name}_logits_sub"] = logits[::64].copy()
            R.model_step(hidden, int(ids[0]), 1 + gen)
            print(f"{name} step {gen}: token {ids[0]} logit {vals[0]:.4f} gap {vals[0] - vals[1]:.4f} "
                  f"({time.time() - t1:.1f} s)", flush=True)
        out[f"{name}_flags"] = np.int64(flags)
        out[f"{name}_tokens"] = np.array(toks, dtype=np.int32)
        out[f"{name}_top_ids"] = np.array(tids, dtype=np.int32)
        out[f"{name}_top_vals"] = np.array(tvals, dtype=np.float32)
        out[f"{name}_layers0"] = layers0
        out[f"{name}_hidden_final"] = hidden.copy()
    np.savez_compressed(os.path.join(OUT, "model_flags.npz"), **out)
    print(f"done in {time.time() - t0:.1f} s", flush=True)


if __name__ == "__main__":
    main()
