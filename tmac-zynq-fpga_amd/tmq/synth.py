"""Deterministic synthetic ggml weights and activations.

The reference ships no model file (models/README.md:9-18), so every workload
here is synthetic, drawn from numpy's PCG64 with a recorded seed.  The value
distributions are the ones BASELINE.json fixes per format:

  Q8_0  q ~ U{-127..127}, d = fp16(|N(0,1)| * 0.01)           34 B / 32 weights
  Q5_0  qs, qh uniform random bits, d = fp16(|N(0,1)| * 0.02)  22 B / 32 weights
  Q4_K  d, dmin = fp16(|N| * 0.01), random 12-byte scales,
        random nibbles                                         144 B / 256 weights
  Q6_K  random ql/qh, sc ~ U{-32..31} int8, d = fp16(|N|*0.01)  210 B / 256 weights
  F32   N(0,1) * 0.05 (row-major fp32)                          4 B / weight
  F16   the same rounded to fp16                                2 B / weight
  x     fp32 N(0,1)

Block layouts follow ggml as read by the reference decoders
(sim/tmac_gguf.cpp:236-393, sim/fpga_sim.hpp:1004-1142): a row of `cols`
weights is cols/QK consecutive blocks, rows are consecutive.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q8_0, Q5_0, Q4_K, Q6_K = 0, 1, 8, 6, 12, 14
# type -> (weights per block, bytes per block)
BLOCK = {Q8_0: (32, 34), Q5_0: (32, 22), Q4_K: (256, 144), Q6_K: (256, 210), F32: (32, 128), F16: (32, 64)}
NAMES = {Q8_0: "q8_0", Q5_0: "q5_0", Q4_K: "q4_k", Q6_K: "q6_k", F32: "f32", F16: "f16"}


def nbytes(qtype: int, rows: int, cols: int) -> int:
    qk, bb = BLOCK[qtype]
    assert cols % qk == 0, f"cols={cols} not a multiple of {qk}"
    return rows * (cols // qk) * bb


def _f16_bits(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint16)


def gen_weights(qtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Return the ggml byte image (uint8, 1-D) of a rows x cols tensor."""
    rng = np.random.Generator(np.random.PCG64(seed))
    qk, bb = BLOCK[qtype]
    nblk = rows * (cols // qk)
    out = np.empty((nblk, bb), dtype=np.uint8)
    if qtype == Q8_0:
        d = _f16_bits(np.abs(rng.standard_normal(nblk, dtype=np.float32)) * np.float32(0.01))
        out[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
        out[:, 2:34] = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int8).view(np.uint8)
    elif qtype == Q5_0:
        d = _f16_bits(np.abs(rng.standard_normal(nblk, dtype=np.float32)) * np.float32(0.02))
        out[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
        out[:, 2:22] = rng.integers(0, 256, size=(nblk, 20), dtype=np.uint8)
    elif qtype == Q4_K:
        d = _f16_bits(np.abs(rng.standard_normal(nblk, dtype=np.float32)) * np.float32(0.01))
        dm = _f16_bits(np.abs(rng.standard_normal(nblk, dtype=np.float32)) * np.float32(0.01))
        out[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
        out[:, 2:4] = dm.view(np.uint8).reshape(nblk, 2)
        out[:, 4:144] = rng.integers(0, 256, size=(nblk, 140), dtype=np.uint8)
    elif qtype == Q6_K:
        out[:, 0:192] = rng.integers(0, 256, size=(nblk, 192), dtype=np.uint8)
        out[:, 192:208] = rng.integers(-32, 32, size=(nblk, 16), dtype=np.int8).view(np.uint8)
        d = _f16_bits(np.abs(rng.standard_normal(nblk, dtype=np.float32)) * np.float32(0.01))
        out[:, 208:210] = d.view(np.uint8).reshape(nblk, 2)
    elif qtype in (F32, F16):
        v = rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.05)
        return (v if qtype == F32 else v.astype(np.float16)).view(np.uint8).copy()
    else:
        raise ValueError(f"unsupported type {qtype}")
    return out.reshape(-1)


def gen_x(n: int, seed: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal(n, dtype=np.float32)
