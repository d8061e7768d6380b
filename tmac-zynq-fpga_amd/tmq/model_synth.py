"""Deterministic synthetic Qwen2-0.5B-shaped models as .tmac tensor lists.

The reference ships no model (models/README.md:9-18) and none can be fetched,
so the full-model workload is random-init weights of the reference's
architecture (sim/tmac_gguf.cpp:136-148): 24 layers, hidden 896, 14 query /
2 KV heads of 64, SwiGLU FFN 4864, vocab 151936, tied Q8_0
token_embd/logits.  The quantisation map is the one the reference documents
for its model (AGENTS.md:16): layers {0,1,3,6,7,8,9,10,13,16,19,21} carry a
Q8_0 attn_v and a Q6_K ffn_down, the others Q5_0 + Q4_K; attn_q/k/output and
ffn_gate/up are Q5_0.

Quantised blocks use the per-format distributions of tmq.synth.  The fp32
tensors are this generator's choice (the reference fixes none): RMSNorm
weights N(1, 0.1), attn_q/k/v biases N(0, 0.5).  Every tensor has its own
PCG64 stream, seeded from (seed, tensor index), so any subset can be
regenerated independently.
"""
from __future__ import annotations

import numpy as np

from . import synth
from .tmacfile import F32, Q4_K, Q5_0, Q6_K, Q8_0, TmacTensor

QWEN_Q8_V_LAYERS = (0, 1, 3, 6, 7, 8, 9, 10, 13, 16, 19, 21)

QWEN2_05B = dict(n_layers=24, hidden=896, inter=4864, vocab=151936, n_heads=14, n_kv_heads=2)


def _f32(rows: int, cols: int, data: np.ndarray, name: str) -> TmacTensor:
    return TmacTensor(name, rows, cols, F32, np.ascontiguousarray(data, dtype=np.float32).view(np.uint8).reshape(-1))


def gen_model(seed: int = 2024, n_layers: int = 24, hidden: int = 896, inter: int = 4864,
              vocab: int = 151936, n_heads: int = 14, n_kv_heads: int = 2,
              q8_v_layers=QWEN_Q8_V_LAYERS) -> list[TmacTensor]:
    """Tensors in the order a GGUF of the model lists them (token_embd,
    per-layer tensors, output_norm)."""
    if hidden != n_heads * 64 or hidden % 32 or inter % 256 or n_heads % n_kv_heads:
        raise ValueError("shape needs hidden = 64*n_heads (multiple of 32), inter % 256 == 0, "
                         "n_heads % n_kv_heads == 0")
    kv = n_kv_heads * 64
    out: list[TmacTensor] = []
    idx = [0]

    def sub_seed() -> int:
        idx[0] += 1
        return (seed * 1_000_003 + idx[0]) & 0x7FFFFFFF

    def quant(name: str, qtype: int, rows: int, cols: int):
        w = synth.gen_weights(qtype, rows, cols, seed=sub_seed())
        out.append(TmacTensor(name, rows, cols, qtype, w))

    def vec(name: str, n: int, mean: float, std: float):
        rng = np.random.Generator(np.random.PCG64(sub_seed()))
        v = (mean + std * rng.standard_normal(n)).astype(np.float32)
        out.append(_f32(1, n, v, name))

    quant("token_embd.weight", Q8_0, vocab, hidden)
    for layer in range(n_layers):
        p = f"blk.{layer}."
        big = layer in q8_v_layers
        vec(p + "attn_norm.weight", hidden, 1.0, 0.1)
        quant(p + "attn_q.weight", Q5_0, hidden, hidden)
        vec(p + "attn_q.bias", hidden, 0.0, 0.5)
        quant(p + "attn_k.weight", Q5_0, kv, hidden)
        vec(p + "attn_k.bias", kv, 0.0, 0.5)
        quant(p + "attn_v.weight", Q8_0 if big else Q5_0, kv, hidden)
        vec(p + "attn_v.bias", kv, 0.0, 0.5)
        quant(p + "attn_output.weight", Q5_0, hidden, hidden)
        vec(p + "ffn_norm.weight", hidden, 1.0, 0.1)
        quant(p + "ffn_gate.weight", Q5_0, inter, hidden)
        quant(p + "ffn_up.weight", Q5_0, inter, hidden)
        quant(p + "ffn_down.weight", Q6_K if big else Q4_K, hidden, inter)
    vec("output_norm.weight", hidden, 1.0, 0.1)
    return out


def matmul_shapes(n_layers: int = 24, hidden: int = 896, inter: int = 4864, vocab: int = 151936,
                  n_kv_heads: int = 2, q8_v_layers=QWEN_Q8_V_LAYERS) -> dict:
    """(type, rows, cols) of every matmul of one decode step in gen_model's
    map: "layers" lists each layer's q, k, v, output, gate, up, down;
    "logits" is the tied Q8_0 token_embd."""
    kv = n_kv_heads * 64
    layers = []
    for layer in range(n_layers):
        big = layer in q8_v_layers
        layers += [(Q5_0, hidden, hidden), (Q5_0, kv, hidden), (Q8_0 if big else Q5_0, kv, hidden),
                   (Q5_0, hidden, hidden), (Q5_0, inter, hidden), (Q5_0, inter, hidden),
                   (Q6_K if big else Q4_K, hidden, inter)]
    return {"layers": layers, "logits": (Q8_0, vocab, hidden)}


def weight_bytes(tensors: list[TmacTensor]) -> int:
    """ggml bytes streamed per decoded token: every quantised matrix once
    (token_embd as the logits matrix)."""
    return sum(t.n_bytes for t in tensors if t.type in (Q8_0, Q5_0, Q4_K, Q6_K))
