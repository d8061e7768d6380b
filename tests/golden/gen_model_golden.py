"""Golden greedy decode of the full synthetic model from the compiled reference.

Runs in the build container only.  The model is tmq.model_synth.gen_model
(seed MODEL_SEED): Qwen2-0.5B-shaped, 24 layers, the reference's mixed
Q8_0/Q6_K vs Q5_0/Q4_K layer map.  It is written to a temporary .tmac and
loaded by the reference engine itself (oracle/_ref: sim/tmac_gguf.cpp's
load_tmac, process_prompt, get_logits_q8, forward_all_layers with the
--fpga-q8/-q5-0/-q4k/-q6-k paths), which then decodes greedily (the first
index of the largest logit; the reference's own generate samples with rand()).

Stored (model_c4.npz, no pickle):
  prompt            the one seeded prompt token
  tokens[N]         greedy tokens
  top_ids/top_vals  the 10 largest logits of every step (value desc, index asc)
  gap[N]            logit gap between the best and second-best token per step
  sub_steps, logits_sub[k, V/64]  every 64th logit at a few steps
  layers0[25, 896]  hidden state after the embedding and after each layer,
                    first position

    make -C oracle && python tests/golden/gen_model_golden.py [--steps 128]
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

from oracle import Reference  # noqa: E402
from tmq import model_synth, tmacfile  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
MODEL_SEED = 2024
PROMPT_SEED = 7
SUB_STEPS = (0, 1, 2, 63, 127)


def prompt_token(vocab: int = 151936) -> int:
    return int(np.random.Generator(np.random.PCG64(PROMPT_SEED)).integers(0, vocab))


def top10(logits: np.ndarray):
    order = np.lexsort((np.arange(logits.size), -logits))[:10]
    return order.astype(np.int32), logits[order]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=128)
    args = ap.parse_args()
    R = Reference()
    t0 = time.time()
    tensors = model_synth.gen_model(MODEL_SEED)
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "c4.tmac")
        tmacfile.write(path, tensors)
        R.model_load(path)
    print(f"model written and loaded in {time.time() - t0:.1f} s", flush=True)
    tok = prompt_token()
    R.model_reset()
    hidden = np.zeros(R.HIDDEN, dtype=np.float32)
    layers0 = R.model_step(hidden, tok, 0, dump=True)  # == process_prompt([tok])
    toks, tids, tvals, gaps, subs = [], [], [], [], []
    for gen in range(args.steps):
        t1 = time.time()
        logits = R.model_logits(hidden)
        ids, vals = top10(logits)
        nxt = int(ids[0])
        assert nxt == int(np.argmax(logits))
        toks.append(nxt)
        tids.append(ids)
        tvals.append(vals)
        gaps.append(float(vals[0] - vals[1]))
        if gen in SUB_STEPS:
            subs.append(logits[::64].copy())
        R.model_step(hidden, nxt, 1 + gen)
        print(f"step {gen}: token {nxt} logit {vals[0]:.4f} gap {gaps[-1]:.4f} ({time.time() - t1:.1f} s)",
              flush=True)
    steps = [s for s in SUB_STEPS if s < args.steps]
    np.savez_compressed(
        os.path.join(OUT, "model_c4.npz"),
        model_seed=MODEL_SEED, prompt=np.array([tok], dtype=np.int32), tokens=np.array(toks, dtype=np.int32),
        top_ids=np.array(tids, dtype=np.int32), top_vals=np.array(tvals, dtype=np.float32),
        gap=np.array(gaps, dtype=np.float32), sub_steps=np.array(steps, dtype=np.int32),
        logits_sub=np.array(subs, dtype=np.float32), layers0=layers0, hidden_final=hidden)
    print(f"done in {time.time() - t0:.1f} s; min gap {min(gaps):.5f}", flush=True)


if __name__ == "__main__":
    main()
