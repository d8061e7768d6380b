// tmq_engine.h -- device-side arguments of the decode-step kernels
// (tmq_engine.hip) shared with the host model runtime (tmq_model.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tmq_internal.h"

#define TMQ_HEAD_DIM 64
#define TMQ_MAX_POS 3072  // scores + weights (8 B each) beside 32 KB of staged V rows in 64 KB of LDS


struct TmqAttnArgs {
    TmqDeferred q, k, v;     // the QKV projections (K-split, with bias)
    float* kc;               // this layer's caches [max_pos][n_kv*64]
    float* vc;
    const float2* rope_cur;  // [32] (cos, sin) of the current position (the qkv launch's copy)
    TmqEngState* state;
    float* ctx;              // out [n_heads*64]
    int32_t n_heads, n_kv, max_pos, pad_;
};

int tmq_launch_attn(const TmqAttnArgs& a, hipStream_t s);
// greedy token from the logits GEMV's candidate keys; advances the position
int tmq_launch_argmax(const uint64_t* cand, int n, TmqEngState* state, int32_t* tokens, int max_pos,
                      hipStream_t s);
int tmq_launch_advance(TmqEngState* state, int max_pos, hipStream_t s);
