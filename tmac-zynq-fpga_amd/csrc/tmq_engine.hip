// tmq_engine.hip -- gfx950 kernels of the batch-1 decode step other than the
// GEMVs (whose activation prologues hold RMSNorm, SiLU*up and the embedding,
// tmq_kernels.hip): RoPE + KV cache + attention, greedy argmax, and the
// position advance.
//
// Every fp32 operation follows sim/tmac_gguf.cpp's order: sums the reference
// forms sequentially (attention scores, the softmax denominator, the context
// accumulation) are formed sequentially here too, by one lane per sum, from
// values staged in LDS.  Maxima are order free.  expf and logf are tmq_expf
// and tmq_logf (identical to the host libm's expf and logf).
//
// The current position lives in device memory (TmqEngState.pos); the first
// kernel of a step advances it, so a captured step replays without host
// involvement.
#include <hip/hip_runtime.h>

#include "tmq_device.h"
#include "tmq_engine.h"
#include "tmq_mathf.h"

namespace {

// RoPE (sim/tmac_gguf.cpp:1527-1554, adjacent pairs, cos/sin table from the
// host) + KV cache append (:1616-1617) + attention of one query head
// (:1619-1655).  One workgroup per query head; head_dim is 64.  The q/k/v
// terms and the RoPE row of this step (copied by the qkv launch) are read at
// entry, before the position arrives, so the q/k/v finalisation waits for one
// memory round trip; then the cached K row of each thread's first position
// and the first 64 V rows (rows below the position: reading the rows not yet
// written, as a position-free read would, measured 3 % slower per step).
template <bool Q8, bool K8, bool V8>
__global__ __launch_bounds__(256) void attn_kernel(TmqAttnArgs a) {
    tmq_warm_kernargs<sizeof(TmqAttnArgs)>();
    extern __shared__ float lds[];
    float* sc = lds;                  // scores, max_pos
    float* ex = lds + a.max_pos;      // exp terms / weights, max_pos
    __shared__ float qr[64], kr[64], vn[64];
    __shared__ float vbuf[2][64][64];
    __shared__ float red[8];
    __shared__ float s_stat[2];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int qpk = a.n_heads / a.n_kv;
    const int kv = h / qpk;
    const int KV = a.n_kv * 64;
    // the q/k/v terms do not depend on the position: their loads are issued
    // before the position arrives (valid addresses whatever it is)
    const int j = tid & 31, jv = tid & 63;
    const double qxs = (double)*a.q.xs, kxs = (double)*a.k.xs, vxs = (double)*a.v.xs;
    const TmqFinRaw<Q8> fq0 = fin_load<Q8>(a.q, h * 64 + 2 * j), fq1 = fin_load<Q8>(a.q, h * 64 + 2 * j + 1);
    const TmqFinRaw<K8> fk0 = fin_load<K8>(a.k, kv * 64 + 2 * j), fk1 = fin_load<K8>(a.k, kv * 64 + 2 * j + 1);
    const TmqFinRaw<V8> fv = fin_load<V8>(a.v, kv * 64 + jv);
    const float2 cs = a.rope_cur[j];
    const float* kb = a.kc + kv * 64;
    const float* vb = a.vc + kv * 64;
    const int pos = a.state->pos;
    if (a.state->err || pos < 0 || pos >= a.max_pos) return;
    float4 kk[16];
    {
        const float4* kp = (const float4*)(kb + (size_t)min(tid, max(pos - 1, 0)) * KV);
#pragma unroll
        for (int i = 0; i < 16; i++) kk[i] = kp[i];
    }
    // V rows 0..63 below pos (thread: rows tid/16 + 16 u, 16-byte column tid % 16)
    float4 v0[4];
    const int nv0 = max(min(64, pos), 1);
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int pr = (tid >> 4) + 16 * u;
        v0[u] = *(const float4*)(vb + (size_t)min(pr, nv0 - 1) * KV + 4 * (tid & 15));
    }
    // V rows [c0, c0+64) of cached positions (< pos) into vbuf[buf], by the
    // threads from `first` on
    auto stage = [&](int c0, int buf, int first) {
        const int nrow = min(64, pos - c0);
        for (int i = tid - first; i < nrow * 16; i += blockDim.x - first) {
            const int pr = i >> 4, q4 = i & 15;
            *(float4*)&vbuf[buf][pr][4 * q4] = *(const float4*)(vb + (size_t)(c0 + pr) * KV + 4 * q4);
        }
    };
    if (tid < 32) {
        const float q0 = fin_finish<Q8>(a.q, fq0, qxs), q1 = fin_finish<Q8>(a.q, fq1, qxs);
        qr[2 * tid] = q0 * cs.x - q1 * cs.y;
        qr[2 * tid + 1] = q0 * cs.y + q1 * cs.x;
        const float k0 = fin_finish<K8>(a.k, fk0, kxs), k1 = fin_finish<K8>(a.k, fk1, kxs);
        kr[2 * tid] = k0 * cs.x - k1 * cs.y;
        kr[2 * tid + 1] = k0 * cs.y + k1 * cs.x;
    } else if (tid >= 64 && tid < 128) {
        vn[tid - 64] = fin_finish<V8>(a.v, fv, vxs);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) *(float4*)&vbuf[0][(tid >> 4) + 16 * u][4 * (tid & 15)] = v0[u];
    __syncthreads();
    if (tid < 64) {
        if (h % qpk == 0) {
            a.kc[(size_t)pos * KV + kv * 64 + tid] = kr[tid];
            a.vc[(size_t)pos * KV + kv * 64 + tid] = vn[tid];
        }
        if (pos < 64) vbuf[0][pos][tid] = vn[tid];
    }
    // scores[p] = sum_d q[d]*k[p][d] (d ascending), / sqrt(64)
    for (int p = tid; p <= pos; p += blockDim.x) {
        float s = 0.0f;
        if (p == pos) {
            for (int d = 0; d < 64; d++) s += qr[d] * kr[d];
        } else {
            if (p != tid) {
                const float4* kp = (const float4*)(kb + (size_t)p * KV);
#pragma unroll
                for (int i = 0; i < 16; i++) kk[i] = kp[i];
            }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                s += qr[4 * i + 0] * kk[i].x;
                s += qr[4 * i + 1] * kk[i].y;
                s += qr[4 * i + 2] * kk[i].z;
                s += qr[4 * i + 3] * kk[i].w;
            }
        }
        sc[p] = s / 8.0f;
    }
    __syncthreads();
    float m = -__builtin_inff();
    for (int p = tid; p <= pos; p += blockDim.x) m = fmaxf(m, sc[p]);
    m = tmq_wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int p = tid; p <= pos; p += blockDim.x) ex[p] = tmq_math::tmq_expf(sc[p] - mx);
    __syncthreads();
    if (tid == 0) {
        // exp_sum in position order (:1648-1649), 16 terms per batch of LDS reads
        float es = 0.0f;
        int p = 0;
        for (; p + 16 <= pos + 1; p += 16) {
            float4 v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = *(const float4*)(ex + p + 4 * j);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                es += v[j].x;
                es += v[j].y;
                es += v[j].z;
                es += v[j].w;
            }
        }
        for (; p <= pos; p++) es += ex[p];
        s_stat[0] = tmq_math::tmq_logf(es) + mx;
    }
    __syncthreads();
    const float ls = s_stat[0];
    for (int p = tid; p <= pos; p += blockDim.x) ex[p] = tmq_math::tmq_expf(sc[p] - ls);
    __syncthreads();
    // context[d] = sum_p w[p]*v[p][d] (p ascending): wave 0 adds chunk c0
    // while waves 1-3 stage the next 64 rows
    float acc = 0.0f;
    int buf = 0;
    for (int c0 = 0; c0 <= pos; c0 += 64) {
        const int c1 = c0 + 64;
        if (c1 <= pos && tid >= 64) {
            stage(c1, buf ^ 1, 64);
            if (c1 + 64 > pos && tid < 128) vbuf[buf ^ 1][pos - c1][tid - 64] = vn[tid - 64];
        }
        if (tid < 64) {
            const int nrow = min(64, pos + 1 - c0);
            int pr = 0;
            for (; pr + 4 <= nrow; pr += 4) {
                const float4 e4 = *(const float4*)(ex + c0 + pr);
                const float v0 = vbuf[buf][pr][tid], v1 = vbuf[buf][pr + 1][tid];
                const float v2 = vbuf[buf][pr + 2][tid], v3 = vbuf[buf][pr + 3][tid];
                acc += e4.x * v0;
                acc += e4.y * v1;
                acc += e4.z * v2;
                acc += e4.w * v3;
            }
            for (; pr < nrow; pr++) acc += ex[c0 + pr] * vbuf[buf][pr][tid];
        }
        __syncthreads();
        buf ^= 1;
    }
    if (tid < 64) a.ctx[h * 64 + tid] = acc;
}

// Greedy pick from the logits GEMV's per-wave candidates (largest logit,
// then smallest index) -> tokens[pos + 1]; advances the position.
__global__ __launch_bounds__(256) void argmax_kernel(const uint64_t* __restrict__ cand, int n,
                                                     TmqEngState* state, int32_t* tokens, int max_pos) {
    __shared__ uint64_t best[4];
    if (state->err) return;
    uint64_t k = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) k = cand[i] > k ? cand[i] : k;
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t ok = __shfl_xor(k, o);
        k = ok > k ? ok : k;
    }
    if ((threadIdx.x & 63) == 0) best[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) k = best[w] > k ? best[w] : k;
        const int tok = k ? (int)(0xffffffffu - (uint32_t)(k & 0xffffffffu)) : 0;
        const int p = state->pos + 1;
        if (p >= 0 && p < max_pos) {
            tokens[p] = tok;
            state->pos = p;
        } else {
            state->err = 1;
        }
    }
}

// Start of a step whose token the host has stored: pos += 1.
__global__ void advance_kernel(TmqEngState* state, int max_pos) {
    if (state->err) return;
    const int p = state->pos + 1;
    if (p >= 0 && p < max_pos) state->pos = p;
    else state->err = 1;
}

}  // namespace

int tmq_launch_attn(const TmqAttnArgs& a, hipStream_t s) {
    // q, k, v: K-split sums (ntiles 0) or Q8_0 tile sums (at most TMQ_FIN_MAXT tiles)
    if (a.q.ntiles > TMQ_FIN_MAXT || a.k.ntiles > TMQ_FIN_MAXT || a.v.ntiles > TMQ_FIN_MAXT)
        return (int)hipErrorInvalidValue;
    const dim3 grid(a.n_heads), blk(256);
    const size_t lds = sizeof(float) * 2 * a.max_pos;
    const int code = (a.q.ntiles > 0 ? 4 : 0) | (a.k.ntiles > 0 ? 2 : 0) | (a.v.ntiles > 0 ? 1 : 0);
    switch (code) {
    case 0: hipLaunchKernelGGL((attn_kernel<false, false, false>), grid, blk, lds, s, a); break;
    case 1: hipLaunchKernelGGL((attn_kernel<false, false, true>), grid, blk, lds, s, a); break;
    case 2: hipLaunchKernelGGL((attn_kernel<false, true, false>), grid, blk, lds, s, a); break;
    case 3: hipLaunchKernelGGL((attn_kernel<false, true, true>), grid, blk, lds, s, a); break;
    case 4: hipLaunchKernelGGL((attn_kernel<true, false, false>), grid, blk, lds, s, a); break;
    case 5: hipLaunchKernelGGL((attn_kernel<true, false, true>), grid, blk, lds, s, a); break;
    case 6: hipLaunchKernelGGL((attn_kernel<true, true, false>), grid, blk, lds, s, a); break;
    default: hipLaunchKernelGGL((attn_kernel<true, true, true>), grid, blk, lds, s, a); break;
    }
    return (int)hipGetLastError();
}
int tmq_launch_argmax(const uint64_t* cand, int n, TmqEngState* state, int32_t* tokens, int max_pos,
                      hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(256), 0, s, cand, n, state, tokens, max_pos);
    return (int)hipGetLastError();
}
int tmq_launch_advance(TmqEngState* state, int max_pos, hipStream_t s) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, state, max_pos);
    return (int)hipGetLastError();
}
