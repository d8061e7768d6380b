"""Golden multi-token prompt of the full synthetic model from the compiled
reference: the reference's own process_prompt over a seeded prompt, then
greedy decode steps.

Runs in the build container only.  The model is tmq.model_synth.gen_model
(seed MODEL_SEED); the reference engine (oracle/_ref: sim/tmac_gguf.cpp's
load_tmac, process_prompt, get_logits_q8, forward_all_layers with the
--fpga-q8/-q5-0/-q4k/-q6-k paths) loads it from a temporary .tmac file.

Stored (model_prompt.npz, no pickle):
  prompt[N]          seeded prompt token ids
  hidden             hidden state after the last prompt token
  top_ids/top_vals   the 10 largest logits after the prompt and after each
                     greedy step (value desc, index asc)
  logits_sub         every 64th logit of the position after the prompt
  tokens[S]          greedy tokens (first index of the largest logit)

    make -C oracle && python tests/golden/gen_prompt_golden.py
    # the reference's longest context (MAX_SEQ_LEN 256, sim/tmac_gguf.cpp:148):
    python tests/golden/gen_prompt_golden.py --len 250 --steps 5 --seed 13 --out model_prompt_long.npz
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
PROMPT_SEED = 11
PROMPT_LEN = 24
STEPS = 8


def top10(logits: np.ndarray):
    order = np.lexsort((np.arange(logits.size), -logits))[:10]
    return order.astype(np.int32), logits[order]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--len", type=int, default=PROMPT_LEN)
    ap.add_argument("--steps", type=int, default=STEPS)
    ap.add_argument("--seed", type=int, default=PROMPT_SEED)
    ap.add_argument("--out", default="model_prompt.npz")
    args = ap.parse_args()
    assert args.len + args.steps <= 256, "the reference's KV cache holds 256 positions"
    R = Reference()
    t0 = time.time()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "model.tmac")
        tmacfile.write(path, model_synth.gen_model(MODEL_SEED))
        R.model_load(path)
    prompt = np.random.Generator(np.random.PCG64(args.seed)).integers(0, 151936, size=args.len).astype(np.int32)
    R.model_reset()
    hidden = R.model_prompt(prompt)
    prompt_hidden = hidden.copy()
    logits = R.model_logits(hidden)
    logits_sub = logits[::64].copy()
    ids, vals = [], []
    tokens = []
    for s in range(args.steps + 1):
        i, v = top10(logits)
        ids.append(i)
        vals.append(v)
        if s == args.steps:
            break
        tok = int(np.argmax(logits))
        tokens.append(tok)
        R.model_step(hidden, tok, args.len + s)
        logits = R.model_logits(hidden)
        print(f"step {s}: token {tok} ({time.time() - t0:.0f} s)", flush=True)
    np.savez(os.path.join(OUT, args.out), model_seed=np.int64(MODEL_SEED), prompt=prompt,
             hidden=prompt_hidden, top_ids=np.array(ids), top_vals=np.array(vals), logits_sub=logits_sub,
             tokens=np.array(tokens, dtype=np.int32))
    print(f"wrote {args.out} in {time.time() - t0:.0f} s")


if __name__ == "__main__":
    main()
