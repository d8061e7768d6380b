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

#include <algorithm>

#include "tmq_device.h"
#include "tmq_engine.h"
#include "tmq_mathf.h"

namespace {

typedef __attribute__((address_space(3))) float lds_f32;

// RoPE (sim/tmac_gguf.cpp:1527-1554, adjacent pairs, cos/sin table from the
// host) + KV cache append (:1616-1617) + attention of one query head
// (:1619-1655).  One workgroup of 8 waves per query head; head_dim is 64.
// The q/k/v terms and the RoPE row of this step (copied by the qkv launch)
// are read at entry, before the position arrives.  Once it has, every
// thread loads the cached key row of its position (positions tid + 512 i,
// the first pass at once) and the workgroup's waves put the cached V rows
// into LDS by DMA (`vcap` rows at a time, all of them up to that count), so
// that no phase after the scores waits on memory.  The sums are formed in
// the reference's order: each score over d ascending, the exp sum and each
// context dimension over positions ascending, one lane per sum.
template <bool Q8, bool K8, bool V8>
__global__ __launch_bounds__(512) void attn_kernel(TmqAttnArgs a) {
    tmq_warm_kernargs<sizeof(TmqAttnArgs)>();
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int mp4 = (a.max_pos + 3) & ~3;  // (16-byte aligned regions)
    float* sc = lds;                       // scores, max_pos
    float* ex = lds + mp4;                 // exp terms / weights, max_pos
    float* vb = lds + 2 * mp4;             // V rows [vcap][64]
    __shared__ float qr[64], kr[64], vn[64];
    __shared__ float red[8];
    __shared__ float s_stat[1];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qpk = a.n_heads / a.n_kv;
    const int kv = h / qpk;
    const int KV = a.n_kv * 64;
    // the q/k/v terms do not depend on the position: their loads are issued
    // before the position arrives (valid addresses whatever it is)
    const int j = tid & 31, jv = tid & 63;
    const double qxs = (double)*a.q.xs, kxs = (double)*a.k.xs, vxs = (double)*a.v.xs;
    TmqFinRaw<Q8> fq0{}, fq1{};
    TmqFinRaw<K8> fk0{}, fk1{};
    TmqFinRaw<V8> fv{};
    if (tid < 32) {
        fq0 = fin_load<Q8>(a.q, h * 64 + 2 * j);
        fq1 = fin_load<Q8>(a.q, h * 64 + 2 * j + 1);
        fk0 = fin_load<K8>(a.k, kv * 64 + 2 * j);
        fk1 = fin_load<K8>(a.k, kv * 64 + 2 * j + 1);
    } else if (tid >= 64 && tid < 128) {
        fv = fin_load<V8>(a.v, kv * 64 + jv);
    }
    const float2 cs = a.rope_cur[j];
    const float* kb = a.kc + kv * 64;
    const float* vbase = a.vc + kv * 64;
    const int pos = a.state->pos;
    if (a.state->err || pos < 0 || pos >= a.max_pos) return;
    const int vcap = a.vcap;
    // (the q/k/v loads went out with the position's: finished first, so that
    // their registers are free before the key row's)
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
    // the cached key row of position tid (< pos; position pos is kr)
    float4 kk[16];
    {
        const float4* kp = (const float4*)(kb + (size_t)min(tid, max(pos - 1, 0)) * KV);
#pragma unroll
        for (int i = 0; i < 16; i++) kk[i] = kp[i];
    }
    // V rows [base, base + n) of the cache into vb[0, n) by DMA: wave w
    // takes rows 4w + 32i .. +3, lane l row + l / 16, 16 bytes at 4 (l % 16)
    // (rows past n re-read row n - 1 into vb rows below vcap: never used)
    auto stage_v = [&](int base, int n) {
        for (int r0 = 4 * wave; r0 < n; r0 += 32) {
            const int rr = min(r0 + (lane >> 4), n - 1);
            __builtin_amdgcn_global_load_lds((const void*)(vbase + (size_t)(base + rr) * KV + 4 * (lane & 15)),
                                             (lds_f32*)(vb + r0 * 64), 16, 0, 0);
        }
    };
    stage_v(0, min(pos, vcap));
    __syncthreads();
    if (tid < 64 && h % qpk == 0) {
        a.kc[(size_t)pos * KV + kv * 64 + tid] = kr[tid];
        a.vc[(size_t)pos * KV + kv * 64 + tid] = vn[tid];
    }
    // scores[p] = sum_d q[d]*k[p][d] (d ascending), / sqrt(64)
    for (int p = tid; p <= pos; p += 512) {
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
    for (int p = tid; p <= pos; p += 512) m = fmaxf(m, sc[p]);
    m = tmq_wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < 8; w++) mx = fmaxf(mx, red[w]);
    for (int p = tid; p <= pos; p += 512) ex[p] = tmq_math::tmq_expf(sc[p] - mx);
    __syncthreads();
    if (tid == 0) {
        // exp_sum in position order (:1648-1649), 16 terms per batch of LDS reads
        float es = 0.0f;
        int p = 0;
        for (; p + 16 <= pos + 1; p += 16) {
            float4 v[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) v[jj] = *(const float4*)(ex + p + 4 * jj);
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                es += v[jj].x;
                es += v[jj].y;
                es += v[jj].z;
                es += v[jj].w;
            }
        }
        for (; p <= pos; p++) es += ex[p];
        s_stat[0] = tmq_math::tmq_logf(es) + mx;
    }
    __syncthreads();
    const float ls = s_stat[0];
    for (int p = tid; p <= pos; p += 512) ex[p] = tmq_math::tmq_expf(sc[p] - ls);
    // this wave's V copies have landed; the barrier makes every wave's visible
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // context[d] = sum_p w[p]*v[p][d] (p ascending) in wave 0, vcap staged
    // rows at a time (the row of position pos is vn)
    float acc = 0.0f;
    for (int base = 0; base <= pos; base += vcap) {
        const int nb = min(vcap, pos + 1 - base);  // positions of this pass
        if (base > 0) {
            __syncthreads();  // wave 0 is done with the previous rows
            stage_v(base, min(vcap, pos - base));
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
        if (wave == 0) {
            if (pos - base < nb) vb[(pos - base) * 64 + lane] = vn[lane];
            const float* e = ex + base;
            int pr = 0;
            for (; pr + 4 <= nb; pr += 4) {
                const float4 e4 = *(const float4*)(e + pr);
                const float v0 = vb[pr * 64 + lane], v1 = vb[(pr + 1) * 64 + lane];
                const float v2 = vb[(pr + 2) * 64 + lane], v3 = vb[(pr + 3) * 64 + lane];
                acc += e4.x * v0;
                acc += e4.y * v1;
                acc += e4.z * v2;
                acc += e4.w * v3;
            }
            for (; pr < nb; pr++) acc += e[pr] * vb[pr * 64 + lane];
        }
    }
    if (wave == 0) a.ctx[h * 64 + lane] = acc;
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

namespace {
const void* attn_fns[8] = {
    (const void*)attn_kernel<false, false, false>, (const void*)attn_kernel<false, false, true>,
    (const void*)attn_kernel<false, true, false>,  (const void*)attn_kernel<false, true, true>,
    (const void*)attn_kernel<true, false, false>,  (const void*)attn_kernel<true, false, true>,
    (const void*)attn_kernel<true, true, false>,   (const void*)attn_kernel<true, true, true>};
bool attn_prepared = false;
}  // namespace

int tmq_attn_vcap(int max_pos) {
    const int mp4 = (max_pos + 3) & ~3;
    const int lim = (TMQ_ATTN_LDS_MAX / 4 - 2 * mp4) / 64;
    const int all = (max_pos + 63) & ~63;
    return std::min(all, lim & ~63);
}
size_t tmq_attn_lds(int max_pos) {
    return sizeof(float) * ((size_t)2 * ((max_pos + 3) & ~3) + (size_t)64 * tmq_attn_vcap(max_pos));
}

int tmq_attn_prepare() {
    if (attn_prepared) return 0;
    for (const void* f : attn_fns) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, TMQ_ATTN_LDS_MAX);
        if (e != hipSuccess) return (int)e;
    }
    attn_prepared = true;
    return 0;
}

int tmq_launch_attn(const TmqAttnArgs& a0, hipStream_t s) {
    // q, k, v: K-split sums (ntiles 0) or Q8_0 tile sums (at most TMQ_FIN_MAXT tiles)
    if (a0.q.ntiles > TMQ_FIN_MAXT || a0.k.ntiles > TMQ_FIN_MAXT || a0.v.ntiles > TMQ_FIN_MAXT)
        return (int)hipErrorInvalidValue;
    if (a0.max_pos < 1 || a0.max_pos > TMQ_MAX_POS || a0.n_kv < 1 || a0.n_heads % a0.n_kv)
        return (int)hipErrorInvalidValue;
    TmqAttnArgs a = a0;
    a.vcap = tmq_attn_vcap(a.max_pos);
    if (a.vcap < 64) return (int)hipErrorInvalidValue;
    if (!attn_prepared) {
        const int e = tmq_attn_prepare();
        if (e) return e;
    }
    const dim3 grid(a.n_heads), blk(512);
    const size_t lds = tmq_attn_lds(a.max_pos);
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
