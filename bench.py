#!/usr/bin/env python
"""bench.py -- quantized-GEMV weight-stream throughput on one MI355X.

Workload: the Q5_0 batch-1 projections of
Qwen2-0.5B -- attn_q 896x896 run as one descriptor with num_tiles=224 and
tile_res_rows=4, ffn_gate and ffn_up 4864x896 -- on a seeded N(0,1) fp32
activation.  The three tensors are replicated over enough distinct weight
sets that one step streams twice the 256 MiB Infinity Cache (84 sets,
550 MB); a step is one pass of the descriptor chain over all of them: one
activation-quantisation launch plus one launch of every GEMV.

value  = ggml weight bytes streamed per step / step time  (GB/s).  A step is
         one tmq_chain_run: the activation-quantisation launch plus the GEMV
         launch; K steps back to back between two HIP events on the
         library's stream.
roofline.achieved = the same bytes / average duration of the GEMV launch:
         200 launches on the prepared activation in 4 blocks that alternate
         with blocks of whole steps (same clock and cache state), against
         8 TB/s.  When the launch alone comes out longer than the step blocks
         beside it, achieved and frac are null.
warm-up: after a burst of launches the GPU's clock dips for a few hundred
         launches before it settles, so GEMV chain workloads run at least
         MIN_WARMUP untimed steps whatever --warmup asks; the line reports
         the count run ("warmup") and the count asked ("warmup_requested").
cpu_baseline = the reference's own matmul_fpga_q5_0 (sim/tmac_gguf.cpp:1221,
         compiled in place into oracle/_ref) or, where that was not built, its
         C restatement, on one host core over the same shapes; beside it the
         reference's no-flag FP32 loop (:488-492) on the same shapes, the
         host's core count and CPU model.
Weight sets are cycled to twice the 256 MiB Infinity Cache by default
(--sets-sweep measures 1x, 2x and 4x).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "tmac-zynq-fpga_amd")
sys.path.insert(0, PKG)

PEAK_GBPS = 8000.0  # MI355X HBM3E, datasheet
METRIC = "quant GEMV weight GB/s (% HBM peak); Qwen2-0.5B batch-1 decode tok/s"
MALL_BYTES = 256 << 20  # MI355X Infinity Cache
MALL_FACTOR = 2.0       # default working set: twice the Infinity Cache
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "chain_q5_0_c2_traffic.txt")
MIN_WARMUP = 300  # untimed chain steps before any GEMV measurement (clock settle)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# name -> (description, [(qtype, rows, cols, num_tiles, tile_res_rows, num_col_groups)], x len)
WORKLOADS = {
    "c2": ("BASELINE configs[1]: Q5_0 attn_q 896x896 (1 descriptor, num_tiles=224, tile_res_rows=4) "
           "+ ffn_gate/ffn_up 4864x896, batch 1",
           [(6, 896, 896, 224, 4, 1), (6, 4864, 896, 1216, 4, 1), (6, 4864, 896, 1216, 4, 1)], 896),
    "c1": ("BASELINE configs[0]: Q8_0 logits 151936x896 (num_tiles=2374 64-row tiles), batch 1",
           [(8, 151936, 896, 2374, 64, 14)], 896),
    "c3q4k": ("BASELINE configs[2]: Q4_K ffn_down 896x4864 (56-row tiles, 19 column groups), batch 1",
              [(12, 896, 4864, 304, 56, 19)], 4864),
    "c3q6k": ("BASELINE configs[2]: Q6_K ffn_down 896x4864 (32-row tiles, 19 column groups), batch 1",
              [(14, 896, 4864, 532, 32, 19)], 4864),
}
BLOCK = {6: (32, 22), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def set_bytes(name):
    return sum(r * (c // BLOCK[qt][0]) * BLOCK[qt][1] for qt, r, c, *_ in WORKLOADS[name][1])


def copies_for(name, factor=MALL_FACTOR):
    """distinct weight sets whose total exceeds factor x the Infinity Cache"""
    return int(factor * MALL_BYTES // set_bytes(name)) + 1


def build_workload(ctx, torch, dev, name, copies=None):
    from tmq import synth
    desc_txt, shapes, n = WORKLOADS[name]
    copies = copies or copies_for(name)
    x = synth.gen_x(n, 12345)
    x_d = torch.from_numpy(x).to(dev)
    tensors, descs, ys = [], [], []
    for s in range(copies):
        for k, (qt, rows, cols, nt, tr, ncg) in enumerate(shapes):
            w = synth.gen_weights(qt, rows, cols, seed=1000 * s + k)
            t = ctx.upload(qt, rows, cols, w)
            y = torch.empty(rows, dtype=torch.float32, device=dev)
            tensors.append(t)
            ys.append(y)
            descs.append((t, x_d.data_ptr(), y.data_ptr(), None, nt, tr, ncg))
        if s % 20 == 0:
            log(f"{name}: uploaded weight set {s + 1}/{copies}")
    return desc_txt, x_d, tensors, descs, ys


def time_events(torch, stream, fn, iters):
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(iters):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters  # ms


def read_traffic():
    """HBM bytes per chain launch measured with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE (scaled by a copy-kernel calibration), if committed."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def host_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


def _stdout_to_stderr(fn):
    """Runs fn with file descriptor 1 pointed at stderr: the compiled
    reference prints its progress (model loading) on stdout, which carries
    only the bench's JSON line.  The C library's buffer is flushed before the
    descriptor is restored."""
    import ctypes
    import functools

    @functools.wraps(fn)
    def run(*a, **k):
        sys.stdout.flush()
        saved = os.dup(1)
        os.dup2(2, 1)
        try:
            return fn(*a, **k)
        finally:
            ctypes.CDLL(None).fflush(None)
            os.dup2(saved, 1)
            os.close(saved)
    return run


@_stdout_to_stderr
def cpu_baseline(seconds):
    """Reference CPU path on one core, bounded sample of the same workload:
    (i) the --fpga-q5-0 integer path (matmul_fpga_q5_0) and (ii) the no-flag
    FP32 loop of matmul (sim/tmac_gguf.cpp:488-492), each ~seconds."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle, Reference
    from tmq import synth
    kind = "reference" if Reference.available() else "port"
    impl = Reference() if kind == "reference" else Oracle()
    x = synth.gen_x(896, 12345)
    ws = [(synth.gen_weights(qt, r, c, seed=k), r, c) for k, (qt, r, c, *_) in enumerate(WORKLOADS["c2"][1])]
    nbytes = sum(w.size for w, _, _ in ws)

    def run(fn):
        done, t0 = 0, time.perf_counter()
        while True:
            for w, r, c in ws:
                fn(6, w, x, r, c)
            done += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                return done, el

    done, el = run(impl.matmul)
    done32, el32 = run(impl.matmul_fp32)
    gbps = done * nbytes / el / 1e9
    name = "sim matmul_fpga_q5_0 (compiled reference)" if kind == "reference" else "C restatement of matmul_fpga_q5_0"
    out = {"value": round(gbps, 5), "unit": "GB/s", "cores": 1, "kind": kind,
           "sample": f"{name} over attn_q 896x896 + ffn_gate/ffn_up 4864x896 "
                     f"({nbytes} weight bytes) x {done} passes = {el:.1f} s on one host thread, "
                     f"per-call row scan included as in the reference",
           "fp32_path": {"value": round(done32 * nbytes / el32 / 1e9, 5), "unit": "GB/s", "cores": 1,
                         "sample": f"the no-flag FP32 loop of matmul (sim/tmac_gguf.cpp:488-492) on the same "
                                   f"shapes x {done32} passes = {el32:.1f} s on one host thread"}}
    out.update(host_info())
    return out


ROOF_BLOCKS = 4      # interleaved (step block, launch block) pairs of the roofline legs
ROOF_LAUNCHES = 200  # GEMV launches timed for the roofline, whatever --steps is


def time_primed(torch, stream, fn, iters, prime=2):
    """Average ms of fn over `iters` calls queued behind `prime` untimed
    ones: the start event is recorded while the GPU is still busy, so the
    host's time to issue the first timed launch is not counted."""
    for _ in range(prime):
        fn()
    return time_events(torch, stream, fn, iters)


def measure(ctx, torch, dev, stream, name, steps, warmup, copies=None):
    """Returns a dict: desc, weight bytes, step ms (the contract's K steps),
    kernel ms, the paired step ms, n descriptors, copies.

    A step = the activation-quantisation launch + the chain's GEMV launch.
    After the warm-up the roofline legs run as ROOF_BLOCKS alternating
    pairs: a block of steps, then a block of GEMV launches alone (on the
    activation the steps prepared), each block timed between two HIP events
    on a primed queue, ROOF_LAUNCHES launches in all; so both legs see the
    same clock and cache state.  Then the K steps of the contract are timed
    between two synchronisations (events only at the ends: an event between
    launches costs the step a few microseconds)."""
    copies = copies or copies_for(name)
    desc_txt, x_d, tensors, descs, ys = build_workload(ctx, torch, dev, name, copies)
    chain = ctx.chain(descs)
    wbytes = chain.weight_bytes
    log(f"{name}: {len(descs)} descriptors ({copies} weight sets), {wbytes} weight bytes per step")
    for _ in range(max(warmup, MIN_WARMUP)):
        chain.run()
    ctx.sync()
    torch.cuda.synchronize()
    blk = ROOF_LAUNCHES // ROOF_BLOCKS
    pair_step, pair_kern = [], []
    for _ in range(ROOF_BLOCKS):
        pair_step.append(time_primed(torch, stream, chain.run, blk))
        pair_kern.append(time_primed(torch, stream, chain.launch, blk))
    ctx.sync()
    torch.cuda.synchronize()
    step_ms = time_events(torch, stream, chain.run, steps)
    ctx.sync()
    torch.cuda.synchronize()
    chain.free()
    for t in tensors:
        t.free()
    return {"desc": desc_txt, "wbytes": wbytes, "step_ms": step_ms,
            "kern_ms": float(np.mean(pair_kern)), "pair_step_ms": float(np.mean(pair_step)),
            "kern_blocks_ms": [round(v, 5) for v in pair_kern],
            "ndesc": len(descs), "copies": copies}


def sets_scan(ctx, torch, dev, stream, name, lo, hi, step):
    """Chain kernel time over lo, lo+step, ..., hi weight sets of `name`,
    each chain over the first sets of one upload of hi sets; one JSON line
    per point.  Shows how the time steps with the number of workgroups
    per CU (the launch's last, partly filled round)."""
    per = len(WORKLOADS[name][1])
    desc_txt, x_d, tensors, descs, ys = build_workload(ctx, torch, dev, name, hi)
    for k in range(lo, hi + 1, step):
        chain = ctx.chain(descs[:k * per])
        for _ in range(MIN_WARMUP):
            chain.run()
        ctx.sync()
        kern = []
        for _ in range(ROOF_BLOCKS):
            time_primed(torch, stream, chain.run, ROOF_LAUNCHES // ROOF_BLOCKS)
            kern.append(time_primed(torch, stream, chain.launch, ROOF_LAUNCHES // ROOF_BLOCKS))
        ctx.sync()
        km = float(np.mean(kern))
        wb = chain.weight_bytes
        print(json.dumps({"scan": name, "sets": k, "weight_bytes": wb, "kernel_ms": round(km, 5),
                          "kernel_gbps": round(wb / (km * 1e-3) / 1e9, 1)}), flush=True)
        chain.free()
    for t in tensors:
        t.free()


def single_launch_us(ctx, torch, dev, stream, steps):
    """Latency of one attn_q GEMV launch (896x896 Q5_0), kernel only."""
    desc_txt, x_d, tensors, descs, ys = build_workload(ctx, torch, dev, "c2", copies=1)
    chain = ctx.chain(descs[:1])
    chain.run()
    chain.prepare()
    ctx.sync()
    ms = time_events(torch, stream, chain.launch, steps)
    ctx.sync()
    chain.free()
    for t in tensors:
        t.free()
    return ms * 1e3


def decode_bench(ctx, torch, stream, tokens=128, warmup=8, long_ctx=True):
    """greedy batch-1 decode of the synthetic Qwen2-0.5B
    model (tmq.model_synth, seed 2024) from one seeded prompt token; one
    step = logits GEMV + argmax + embedding + 24 layers, graph-replayed."""
    import tmq
    from tmq import model_synth, tmacfile
    log("decode: generating the synthetic C4 model")
    blob = tmacfile.to_bytes(model_synth.gen_model(2024))
    m = tmq.Model(ctx, blob, max_seq=512)
    del blob
    prompt = [int(np.random.Generator(np.random.PCG64(7)).integers(0, 151936))]
    m.prompt(prompt)
    m.generate(warmup)
    m.prompt(prompt)
    ctx.sync()
    ms = time_events(torch, stream, lambda: m.generate_async(tokens), 1) / tokens
    got = m.tokens(1, tokens)
    wb = m.weight_bytes
    out = {"tokens": tokens, "ms_per_token": round(ms, 4), "tok_s": round(1e3 / ms, 1),
           "weight_gbps": round(wb / (ms * 1e-3) / 1e9, 1), "weight_bytes_per_token": wb,
           "first_tokens": got[:8].tolist()}
    if long_ctx:
        # beside it (not the line's figure): the same decode with the cache
        # already at 384 positions (a seeded 384-token prompt through the
        # batched prefill), 64 steps up to position 447
        long_toks = np.random.Generator(np.random.PCG64(384)).integers(0, 151936, size=384).astype(np.int32)
        m.prompt(long_toks)
        m.generate(4)
        m.prompt(long_toks)
        ctx.sync()
        ms_long = time_events(torch, stream, lambda: m.generate_async(64), 1) / 64
        out["after_384_token_prompt"] = {"positions": "384-447", "ms_per_token": round(ms_long, 4),
                                         "tok_s": round(1e3 / ms_long, 1)}
    m.free()
    return out


# int8 MACs per token of the batched prefill: four digit products per
# weight of every layer projection (q,k,v,o,gate,up,down) of the C4 model
PF_LAYER_WEIGHTS = 24 * (1152 * 896 + 896 * 896 + 2 * 4864 * 896 + 896 * 4864)
PF_LAYER_BYTES = 246930432  # ggml bytes of those weights
MFMA_I8_PEAK_TOPS = 5000.0  # MI355X dense int8, datasheet


def prefill_bench(ctx, n=512, reps=5):
    """a seeded n-token prompt through the 24-layer model
    with the batched prefill (one chunk, every projection an int8-digit MFMA
    GEMM).  Timed per tmq_model_prompt call, wall clock (host launches and the
    final synchronisation included); the weight digit planes are built by the
    first, untimed call."""
    import tmq
    from tmq import model_synth, tmacfile
    log("prefill: generating the synthetic C4 model")
    blob = tmacfile.to_bytes(model_synth.gen_model(2024))
    m = tmq.Model(ctx, blob, max_seq=max(512, n + 16))
    del blob
    toks = np.random.Generator(np.random.PCG64(12345)).integers(0, 151936, size=n).astype(np.int32)
    m.set_prefill(512)
    m.prompt(toks)
    ctx.sync()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        m.prompt(toks)
        times.append(time.perf_counter() - t0)
    first = m.generate(4).tolist()
    m.free()
    ms = float(np.median(times)) * 1e3
    tops = 4 * PF_LAYER_WEIGHTS * n * 2 / (ms * 1e-3) / 1e12
    return {"prompt_tokens": n, "ms": round(ms, 4), "ms_min": round(min(times) * 1e3, 4),
            "tok_s": round(n / (ms * 1e-3), 1), "layer_weight_gbps": round(PF_LAYER_BYTES / (ms * 1e-3) / 1e9, 1),
            "int8_tops": round(tops, 2), "mfma_frac": round(tops / MFMA_I8_PEAK_TOPS, 4),
            "next_tokens": first}


@_stdout_to_stderr
def cpu_decode_baseline(seconds):
    """The reference engine (oracle/_ref: load_tmac + forward_all_layers +
    get_logits_q8 with the --fpga-* paths) on one host thread, greedy steps
    until `seconds` have passed."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Reference
    if not Reference.available():
        return None
    import tempfile
    from tmq import model_synth, tmacfile
    R = Reference()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "c4.tmac")
        tmacfile.write(path, model_synth.gen_model(2024))
        R.model_load(path)
    tok = int(np.random.Generator(np.random.PCG64(7)).integers(0, 151936))
    R.model_reset()
    hidden = np.zeros(R.HIDDEN, dtype=np.float32)
    R.model_step(hidden, tok, 0)
    done, t0 = 0, time.perf_counter()
    while True:
        lg = R.model_logits(hidden)
        R.model_step(hidden, int(np.argmax(lg)), 1 + done)
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(done / el, 4), "unit": "tok/s", "cores": 1, "kind": "reference",
            "sample": f"{done} greedy decode steps (positions 1..{done}) of the same model, {el:.1f} s"}


def copy_calibration(torch, dev, nbytes=1 << 30):
    """A plain device copy of known size, for scaling FETCH_SIZE/WRITE_SIZE."""
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "launches": 3}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # GEMV chains: the GPU's clock dips for a few hundred launches after a burst
    # and then settles, so the default warm-up runs into the settled state
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 200 GEMV chain launches, 128 decode tokens, 20 prefills)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default: 400 chain launches, 8 tokens, 1 prefill)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--sets", type=int, default=None, help="weight sets of the c2 chain (default: 2x the MALL)")
    ap.add_argument("--sets-sweep", action="store_true",
                    help="GEMV GB/s at working sets of 1x, 2x and 4x the Infinity Cache (c2, c3q4k, c3q6k, c1)")
    ap.add_argument("--sets-scan", nargs=4, metavar=("WORKLOAD", "LO", "HI", "STEP"), default=None,
                    help="kernel time of one GEMV chain over LO..HI weight sets (prefixes of one upload)")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS) + ["c4", "c5"],
                    help="c4: only the full-model greedy decode (BASELINE configs[3]); "
                         "c5: only the 512-token batched prefill (BASELINE configs[4])")
    ap.add_argument("--no-extra", action="store_true", help="skip the other BASELINE GEMV configs")
    ap.add_argument("--no-long-ctx", action="store_true",
                    help="decode legs: skip the steps with the cache at 384 positions")
    ap.add_argument("--prompt-tokens", type=int, default=512,
                    help="c5: prompt length (BASELINE configs[4] is 512; shorter ones show the fixed costs)")
    args = ap.parse_args()
    dflt = {"c4": (128, 8), "c5": (20, 1)}.get(args.workload, (200, 400))
    if args.steps is None:
        args.steps = dflt[0]
    if args.warmup is None:
        args.warmup = dflt[1]

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only; the GEMV shards by output rows with "
              "no exchange, and multi-GPU runs are not part of it", file=sys.stderr)
        sys.exit(2)

    import torch
    import tmq
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration(torch, dev)
        return

    ctx = tmq.Context(0)
    stream = torch.cuda.ExternalStream(ctx.stream)
    wl = args.workload
    if wl == "c4":
        dec = decode_bench(ctx, torch, stream, tokens=min(args.steps, 500), warmup=args.warmup,
                           long_ctx=not args.no_long_ctx)
        ctx.close()
        out = {"metric": "Qwen2-0.5B batch-1 greedy decode tok/s", "value": dec["tok_s"], "unit": "tok/s",
               "n_gpus": 1, "steps": dec["tokens"], "warmup": args.warmup, "ms_per_step": dec["ms_per_token"],
               "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int16",
               "data": "synthetic Qwen2-0.5B-shaped model (tmq.model_synth seed 2024), one seeded prompt token",
               "config": {"workload": "BASELINE configs[3]: 24-layer decode, mixed Q8_0/Q6_K and Q5_0/Q4_K "
                          "layers, Q8_0 tied logits, greedy", "weight_bytes_per_token": dec["weight_bytes_per_token"]},
               "extra": {"c4_decode": dec},
               "cpu_baseline": None if args.no_cpu else cpu_decode_baseline(args.cpu_seconds)}
        print(json.dumps(out), flush=True)
        return
    if wl == "c5":
        n_pf = args.prompt_tokens
        if not 1 <= n_pf <= 4096:
            sys.exit("bench.py: --prompt-tokens must be 1..4096")
        pf = prefill_bench(ctx, n_pf, max(3, min(args.steps, 20)))
        ctx.close()
        cpu = None
        if not args.no_cpu:
            dec = cpu_decode_baseline(args.cpu_seconds)
            if dec is not None:
                # the reference's process_prompt is the same per-token step
                cpu = dict(dec, sample=dec["sample"] + "; process_prompt runs the same step per prompt token")
        out = {"metric": f"Qwen2-0.5B batched prefill tok/s ({n_pf}-token prompt)", "value": pf["tok_s"],
               "unit": "tok/s", "n_gpus": 1, "steps": max(3, min(args.steps, 20)), "warmup": 1,
               "ms_per_step": pf["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
               "dtype": "int8 (exact int16 x int16 as digit products)",
               "data": f"synthetic Qwen2-0.5B-shaped model (tmq.model_synth seed 2024), {n_pf} seeded token ids",
               "config": {"workload": ("BASELINE configs[4]: 512-token prompt" if n_pf == 512 else
                                       f"{n_pf}-token prompt (BASELINE configs[4] is 512)") +
                          ", 24 layers, batched prefill (bit-exact with the one-token-at-a-time prompt)",
                          "prompt_tokens": n_pf},
               "roofline": {"bound": "mfma", "achieved": pf["int8_tops"], "peak": MFMA_I8_PEAK_TOPS,
                            "unit": "TFLOP/s", "frac": pf["mfma_frac"], "traffic": None,
                            "kernel": "whole prefill (int8 digit MACs / prompt time)"},
               "extra": {"c5_prefill": pf}, "cpu_baseline": cpu}
        print(json.dumps(out), flush=True)
        return
    if args.sets_scan:
        sets_scan(ctx, torch, dev, stream, args.sets_scan[0], *(int(v) for v in args.sets_scan[1:]))
        ctx.close()
        return
    if args.sets_sweep:
        for name in ("c2", "c3q4k", "c3q6k", "c1"):
            for f in (1.0, 2.0, 4.0):
                n = copies_for(name, f)
                m = measure(ctx, torch, dev, stream, name, args.steps, args.warmup, n)
                wb = m["wbytes"]
                print(json.dumps({"sweep": name, "mall_factor": f, "sets": n, "weight_bytes": wb,
                                  "ms_per_step": round(m["pair_step_ms"], 5), "kernel_ms": round(m["kern_ms"], 5),
                                  "step_gbps": round(wb / (m["pair_step_ms"] * 1e-3) / 1e9, 2),
                                  "kernel_gbps": round(wb / (m["kern_ms"] * 1e-3) / 1e9, 2)}), flush=True)
        ctx.close()
        return
    copies = args.sets if wl == "c2" else None
    m = measure(ctx, torch, dev, stream, wl, args.steps, args.warmup, copies)
    wbytes, step_ms, kern_ms, pair_ms = m["wbytes"], m["step_ms"], m["kern_ms"], m["pair_step_ms"]
    value = wbytes / (step_ms * 1e-3) / 1e9
    achieved = wbytes / (kern_ms * 1e-3) / 1e9
    # a step is the activation preparation plus the chain launch, so the
    # launch alone cannot take longer than the step blocks it alternates
    # with; if it did, the legs ran in different clock or cache states and
    # no fraction is reported
    within = bool(kern_ms <= pair_ms and kern_ms <= step_ms)
    traffic = read_traffic() if wl == "c2" else None
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": max(args.warmup, MIN_WARMUP),
        "warmup_requested": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16",
        "data": "synthetic (seeded ggml blocks as BASELINE.json specifies per format; x ~ N(0,1))",
        "config": {
            "workload": f"{m['desc']}; {m['copies']} weight sets cycled ({wbytes} B, "
                        f"{wbytes / MALL_BYTES:.2f}x the 256 MiB Infinity Cache), one chain launch per step",
            "descriptors_per_step": m["ndesc"],
            "weight_bytes_per_step": wbytes,
            "pct_hbm_peak": round(100.0 * value / PEAK_GBPS, 2),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2) if within else None,
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBPS, 4) if within else None,
            "traffic": traffic,
            "kernel": "chain_kernel",
            "kernel_ms": round(kern_ms, 5),
            "kernel_launches_timed": ROOF_LAUNCHES,
            "kernel_blocks_ms": m["kern_blocks_ms"],
            "paired_step_ms": round(pair_ms, 5),
            "kernel_within_step": within,
        },
    }
    if not args.no_extra and wl == "c2":
        extra = {}
        for name in ("c1", "c3q4k", "c3q6k"):
            e = measure(ctx, torch, dev, stream, name, ROOF_LAUNCHES, args.warmup)
            wb, km = e["wbytes"], e["kern_ms"]
            extra[name] = {"weight_bytes": wb, "descriptors": e["ndesc"], "weight_sets": e["copies"],
                           "ms_per_launch": round(km, 5), "launches_timed": ROOF_LAUNCHES,
                           "ms_per_step": round(e["pair_step_ms"], 5),
                           "kernel_within_step": bool(km <= e["pair_step_ms"]),
                           "gbps": round(wb / (km * 1e-3) / 1e9, 2),
                           "pct_hbm_peak": round(100.0 * wb / (km * 1e-3) / 1e9 / PEAK_GBPS, 2)}
        extra["c2_attn_q_single_launch_us"] = round(single_launch_us(ctx, torch, dev, stream, 50), 2)
        extra["c4_decode"] = decode_bench(ctx, torch, stream, long_ctx=not args.no_long_ctx)
        extra["c5_prefill"] = prefill_bench(ctx, 512, 20)
        out["extra"] = extra
    ctx.close()
    if not args.no_cpu:
        log(f"CPU baseline ({args.cpu_seconds:.0f} s sample)")
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        if not args.no_extra and wl == "c2":
            dec = cpu_decode_baseline(args.cpu_seconds)
            if dec is not None:
                out["cpu_baseline"]["c4_decode"] = dec
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
