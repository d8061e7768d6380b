// tmq_engine.h -- device-side arguments of the decode-step kernels
// (tmq_engine.hip) shared with the host model runtime (tmq_model.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tmq_internal.h"

#define TMQ_HEAD_DIM 64
#define TMQ_MAX_POS 3072  // scores + weights, 8 B a position, beside the staged V rows in LDS
// dynamic LDS of the attention: scores, weights and up to vcap staged V rows
// (256 B each; all of them up to ~500 positions)
#define TMQ_ATTN_LDS_MAX (152 * 1024)


struct TmqAttnArgs {
    TmqDeferred q, k, v;     // the QKV projections (K-split, with bias)
    float* kc;               // this layer's caches [max_pos][n_kv*64]
    float* vc;
    const float2* rope_cur;  // [32] (cos, sin) of the current position (the qkv launch's copy)
    TmqEngState* state;
    float* ctx;              // out [n_heads*64]
    int32_t n_heads, n_kv, max_pos;
    int32_t vcap;            // V rows staged in LDS at a time (set by the launch)
};

int tmq_launch_attn(const TmqAttnArgs& a, hipStream_t s);
// one-time set-up (the dynamic LDS limit), so that a stream capture of the
// launches makes no such call; and the staged V rows / LDS bytes per max_pos
int tmq_attn_prepare();
int tmq_attn_vcap(int max_pos);
size_t tmq_attn_lds(int max_pos);
// greedy token from the logits GEMV's candidate keys; advances the position
int tmq_launch_argmax(const uint64_t* cand, int n, TmqEngState* state, int32_t* tokens, int max_pos,
                      hipStream_t s);
int tmq_launch_advance(TmqEngState* state, int max_pos, hipStream_t s);
