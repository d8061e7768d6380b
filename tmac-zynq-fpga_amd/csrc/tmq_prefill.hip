// tmq_prefill.hip -- gfx950 kernels of the batched prefill (tmq_prefill.h):
// the digit GEMM on int8 MFMA with its fused epilogues, the attention of a
// block of positions, and the hand-over to the decode engine.
//
// GEMM mapping (v_mfma_i32_32x32x32_i8, 32 rows x 32 tokens x 32 columns):
// a wave owns two 32-row blocks and one 32-token block; the waves of a
// workgroup take consecutive token blocks of the same rows.  Lane l holds,
// for a 32x32x32 step, 16 bytes of row (l & 31) at columns 16*(l >> 5)..+15
// of both operands (rows of the weight planes, tokens of the activation
// planes, each K-contiguous); accumulator element v of lane l is row
// 8*(v/4) + 4*(l/32) + v%4 of the block, token l & 31.  Per block three
// int32 accumulators hold S(a,c), S(a,e)+S(b,c) and S(b,e).
#include <hip/hip_runtime.h>

#include "tmq_device.h"
#include "tmq_mathf.h"
#include "tmq_prefill.h"

namespace {

typedef int tmq_v4i __attribute__((ext_vector_type(4)));
typedef int tmq_v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(1))) const tmq_v4i gv4i;

__device__ __forceinline__ tmq_v4i ldq(const int8_t* p) { return *(const gv4i*)p; }
__device__ __forceinline__ tmq_v16i mfma(tmq_v4i a, tmq_v4i b, tmq_v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
// row (within a 32x32 block) of accumulator element v of lane l
__device__ __forceinline__ int blk_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

struct Frags {
    tmq_v4i a0, b0, a1, b1, c, e;
};
__device__ __forceinline__ Frags load_frags(const int8_t* pa0, const int8_t* pb0, const int8_t* pa1,
                                            const int8_t* pb1, const int8_t* pc, const int8_t* pe, int ko) {
    Frags f;
    f.a0 = ldq(pa0 + ko);
    f.b0 = ldq(pb0 + ko);
    f.a1 = ldq(pa1 + ko);
    f.b1 = ldq(pb1 + ko);
    f.c = ldq(pc + ko);
    f.e = ldq(pe + ko);
    return f;
}
// one 32-column step of both row blocks: 8 MFMAs, the two that add into
// the middle accumulators a second time issued last
__device__ __forceinline__ void step(tmq_v16i (&acc)[2][3], const Frags& f) {
    acc[0][0] = mfma(f.a0, f.c, acc[0][0]);
    acc[1][0] = mfma(f.a1, f.c, acc[1][0]);
    acc[0][1] = mfma(f.a0, f.e, acc[0][1]);
    acc[1][1] = mfma(f.a1, f.e, acc[1][1]);
    acc[0][2] = mfma(f.b0, f.e, acc[0][2]);
    acc[1][2] = mfma(f.b1, f.e, acc[1][2]);
    acc[0][1] = mfma(f.b0, f.c, acc[0][1]);
    acc[1][1] = mfma(f.b1, f.c, acc[1][1]);
}
__device__ __forceinline__ int64_t digit_sum(const tmq_v16i (&acc)[2][3], int bi, int v) {
    return 65536 * (int64_t)acc[bi][0][v] + 256 * (int64_t)acc[bi][1][v] + (int64_t)acc[bi][2][v];
}

template <int MODE, int NWV>
__global__ __launch_bounds__(64 * NWV) void pf_gemm_kernel(TmqPfGemm g) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    int rb[2];
    if (MODE == TMQ_PF_GU) {
        rb[0] = 32 * blockIdx.x;
        rb[1] = g.gu_rows + 32 * blockIdx.x;
    } else {
        rb[0] = 64 * blockIdx.x;
        rb[1] = rb[0] + 32;
    }
    const int tb = ((int)blockIdx.y * NWV + wave) * 32;
    if (tb >= g.T_pad) return;  // wave-uniform; the kernel has no barrier
    const int li = lane & 31, lk = (lane >> 5) * 16;
    const int8_t* pa0 = g.wa + (size_t)(rb[0] + li) * g.K + lk;
    const int8_t* pb0 = g.wb + (size_t)(rb[0] + li) * g.K + lk;
    const int8_t* pa1 = g.wa + (size_t)(rb[1] + li) * g.K + lk;
    const int8_t* pb1 = g.wb + (size_t)(rb[1] + li) * g.K + lk;
    const int8_t* pc = g.xc + (size_t)(tb + li) * g.K + lk;
    const int8_t* pe = g.xe + (size_t)(tb + li) * g.K + lk;
    const int nks = g.K >> 5;
    const int ks0 = (int)((int64_t)blockIdx.z * nks / g.split), ks1 = (int)((int64_t)(blockIdx.z + 1) * nks / g.split);
    const int t = tb + li;

    // the tensor of this row tile (QKV: q, k or v; GU: gate for block 0)
    int si = 0;
    if (MODE == TMQ_PF_QKV) {
        if (g.nseg > 1 && rb[0] >= g.seg[1].row0) si = 1;
        if (g.nseg > 2 && rb[0] >= g.seg[2].row0) si = 2;
    }
    const TmqPfSeg S = si == 0 ? g.seg[0] : si == 1 ? g.seg[1] : g.seg[2];

    tmq_v16i acc[2][3];
    for (int bi = 0; bi < 2; bi++)
        for (int j = 0; j < 3; j++) acc[bi][j] = tmq_v16i{};
    float y[2][16];

    if (MODE == TMQ_PF_QKV && S.q8) {
        // Q8_0: fold every 64-column tile into y in order, in double
        // (sim/tmac_gguf.cpp:1075-1076); split is 1
        const int nt = g.K / TMQ_PF_CHUNK;
        for (int bi = 0; bi < 2; bi++)
            for (int v = 0; v < 16; v++) y[bi][v] = 0.0f;
        const double xs = (double)g.xs[t];
        for (int tile = 0; tile < nt; tile++) {
            step(acc, load_frags(pa0, pb0, pa1, pb1, pc, pe, tile * 64));
            step(acc, load_frags(pa0, pb0, pa1, pb1, pc, pe, tile * 64 + 32));
            const int32_t tx = g.tx_c[(size_t)t * nt + tile];
            for (int bi = 0; bi < 2; bi++) {
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int r = rb[bi] + blk_row(v, lane);
                    const int64_t P = digit_sum(acc, bi, v) +
                                      128 * ((int64_t)g.rw_c[(size_t)r * nt + tile] + tx) + 16384 * 64;
                    y[bi][v] = (float)((double)y[bi][v] + ((double)P * xs) * (double)S.row_scale[r - S.row0]);
                }
                for (int j = 0; j < 3; j++) acc[bi][j] = tmq_v16i{};
            }
        }
        for (int bi = 0; bi < 2; bi++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int rr = rb[bi] + blk_row(v, lane) - S.row0;
                if (S.bias) y[bi][v] = y[bi][v] + S.bias[rr];
            }
    } else {
        Frags cur = load_frags(pa0, pb0, pa1, pb1, pc, pe, ks0 * 32);
        for (int ks = ks0; ks < ks1; ks++) {
            const Frags nxt = load_frags(pa0, pb0, pa1, pb1, pc, pe, (ks + 1 < ks1 ? ks + 1 : ks) * 32);
            step(acc, cur);
            cur = nxt;
        }
        if (MODE == TMQ_PF_PART) {
            int64_t* out = g.part + ((size_t)blockIdx.z * g.T_pad + t) * g.rows;
            for (int bi = 0; bi < 2; bi++)
#pragma unroll
                for (int v = 0; v < 16; v++) out[rb[bi] + blk_row(v, lane)] = digit_sum(acc, bi, v);
            return;
        }
        // finalise (sim/tmac_gguf.cpp:1303-1305) + bias (:1595-1597)
        const double xs = (double)g.xs[t];
        const int64_t tc = 128 * (int64_t)g.tx_t[t] + 16384 * (int64_t)g.K;
        for (int bi = 0; bi < 2; bi++) {
            const TmqPfSeg Sb = (MODE == TMQ_PF_GU && bi == 1) ? g.seg[1] : S;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int r = rb[bi] + blk_row(v, lane), rr = r - Sb.row0;
                const int64_t a = digit_sum(acc, bi, v) + 128 * (int64_t)g.rw_t[r] + tc;
                float f = (float)(((double)a * xs) / (double)Sb.row_inv[rr]);
                if (Sb.bias) f = f + Sb.bias[rr];
                y[bi][v] = f;
            }
        }
    }
    const bool live = t < g.T;

    if (MODE == TMQ_PF_QKV) {
        if (!live) return;
        const int pos = g.p0 + t;
        for (int bi = 0; bi < 2; bi++) {
#pragma unroll
            for (int v = 0; v < 16; v += 2) {
                const int rr = rb[bi] + blk_row(v, lane) - S.row0;  // even: (rr, rr+1) is a RoPE pair
                const float y0 = y[bi][v], y1 = y[bi][v + 1];
                if (si == 2) {
                    g.vc[(size_t)pos * g.KV + rr] = y0;
                    g.vc[(size_t)pos * g.KV + rr + 1] = y1;
                } else {
                    // apply_rope (sim/tmac_gguf.cpp:1537-1539)
                    const float2 cs = g.rope[(size_t)pos * 32 + ((rr & 63) >> 1)];
                    const float o0 = y0 * cs.x - y1 * cs.y;
                    const float o1 = y0 * cs.y + y1 * cs.x;
                    float* dst = si == 0 ? g.q_out + (size_t)t * g.H + rr : g.kc + (size_t)pos * g.KV + rr;
                    dst[0] = o0;
                    dst[1] = o1;
                }
            }
        }
    } else if (MODE == TMQ_PF_O) {
        if (!live) return;
        // residual add (sim/tmac_gguf.cpp:1663)
        for (int bi = 0; bi < 2; bi++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const size_t i = (size_t)t * g.rows + rb[bi] + blk_row(v, lane);
                g.x_out[i] = g.x_res[i] + y[bi][v];
            }
    } else if (MODE == TMQ_PF_GU) {
        // SwiGLU (sim/tmac_gguf.cpp:434-439): gate rows in block 0, the same
        // up rows in block 1
        float m = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float gv = y[0][v];
            const float sv = (gv / (1.0f + tmq_math::tmq_expf(-gv))) * y[1][v];
            if (live) g.s_out[(size_t)t * g.gu_rows + rb[0] + blk_row(v, lane)] = sv;
            m = fmaxf(m, fabsf(sv));
        }
        m = fmaxf(m, __shfl_xor(m, 32));
        if (live && lane < 32)
            __hip_atomic_fetch_max(g.max_bits + t, __builtin_bit_cast(uint32_t, m), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Attention of token t (position P = p0 + t) for the query heads of KV
// head g: the decode engine's chains (attn_kernel) per query -- scores
// summed over d in order and /8, max, exp terms summed over positions in
// order, log via fp64, weights, the context summed over positions in order.
__global__ __launch_bounds__(512) void pf_attn_kernel(TmqPfAttn a) {
    extern __shared__ float lds[];
    __shared__ float stat[2][8];
    const int t = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, nt = blockDim.x;
    const int qpk = a.n_heads / a.n_kv, KV = a.n_kv * 64, H = a.n_heads * 64;
    const int np = a.p0 + t + 1, npad = (np + 3) & ~3;
    const int wv = tid >> 6, ln = tid & 63;
    float* q = lds;                  // [qpk][64]
    float* sc = q + qpk * 64;        // [qpk][npad]
    float* ex = sc + qpk * npad;     // [qpk][npad]
    float* vb = ex + qpk * npad;     // [64][64]
    const float* kb = a.kc + g * 64;
    const float* vbase = a.vc + g * 64;
    for (int i = tid; i < qpk * 64; i += nt) q[i] = a.q[(size_t)t * H + g * qpk * 64 + i];
    __syncthreads();
    for (int p = tid; p < np; p += nt) {
        float4 kk[16];
        const float4* kp = (const float4*)(kb + (size_t)p * KV);
#pragma unroll
        for (int i = 0; i < 16; i++) kk[i] = kp[i];
        for (int h = 0; h < qpk; h++) {
            const float* qh = q + h * 64;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                s += qh[4 * i + 0] * kk[i].x;
                s += qh[4 * i + 1] * kk[i].y;
                s += qh[4 * i + 2] * kk[i].z;
                s += qh[4 * i + 3] * kk[i].w;
            }
            sc[h * npad + p] = s / 8.0f;
        }
    }
    __syncthreads();
    if (wv < qpk) {
        float m = -__builtin_inff();
        for (int p = ln; p < np; p += 64) m = fmaxf(m, sc[wv * npad + p]);
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        if (ln == 0) stat[0][wv] = m;
    }
    __syncthreads();
    for (int i = tid; i < qpk * np; i += nt) {
        const int h = i / np, p = i - h * np;
        ex[h * npad + p] = tmq_math::tmq_expf(sc[h * npad + p] - stat[0][h]);
    }
    __syncthreads();
    if (wv < qpk && ln == 0) {
        const float* e = ex + wv * npad;
        float es = 0.0f;
        int p = 0;
        for (; p + 16 <= np; p += 16) {
            float4 v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = *(const float4*)(e + p + 4 * j);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                es += v[j].x;
                es += v[j].y;
                es += v[j].z;
                es += v[j].w;
            }
        }
        for (; p < np; p++) es += e[p];
        stat[1][wv] = (float)log((double)es) + stat[0][wv];
    }
    __syncthreads();
    for (int i = tid; i < qpk * np; i += nt) {
        const int h = i / np, p = i - h * np;
        ex[h * npad + p] = tmq_math::tmq_expf(sc[h * npad + p] - stat[1][h]);
    }
    __syncthreads();
    float acc = 0.0f;
    for (int c0 = 0; c0 < np; c0 += 64) {
        const int nr = min(64, np - c0);
        for (int i = tid; i < nr * 16; i += nt) {
            const int pr = i >> 4, q4 = i & 15;
            *(float4*)&vb[pr * 64 + 4 * q4] = *(const float4*)(vbase + (size_t)(c0 + pr) * KV + 4 * q4);
        }
        __syncthreads();
        if (wv < qpk) {
            const float* e = ex + wv * npad + c0;
            for (int pr = 0; pr < nr; pr++) acc += e[pr] * vb[pr * 64 + ln];
        }
        __syncthreads();
    }
    if (wv < qpk) a.ctx[(size_t)t * H + (g * qpk + wv) * 64 + ln] = acc;
}

// The decode engine's residual state after the prefill's last token.
__global__ __launch_bounds__(256) void pf_handoff_kernel(TmqPfHandoff h) {
    for (int r = threadIdx.x; r < h.H; r += blockDim.x) {
        __hip_atomic_store(h.kacc + r, tmq_pf_acc(h.dn, h.t, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        h.hid[r] = h.x1[(size_t)h.t * h.H + r];
    }
    if (threadIdx.x == 0) *h.xs_slot = h.dn.xs[h.t];
}

template <int MODE>
int launch_gemm(const TmqPfGemm& g, int waves, hipStream_t s) {
    const int rt = MODE == TMQ_PF_GU ? g.gu_rows / 32 : g.rows / 64;
    const dim3 grid(rt, (g.T_pad + 32 * waves - 1) / (32 * waves), g.split);
    if (waves == 4) hipLaunchKernelGGL((pf_gemm_kernel<MODE, 4>), grid, dim3(256), 0, s, g);
    else if (waves == 8) hipLaunchKernelGGL((pf_gemm_kernel<MODE, 8>), grid, dim3(512), 0, s, g);
    else return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

}  // namespace

size_t tmq_pf_attn_lds(int qpk, int npos) {
    const size_t npad = ((size_t)npos + 3) & ~(size_t)3;
    return sizeof(float) * ((size_t)qpk * 64 + 2 * (size_t)qpk * npad + 64 * 64);
}

int tmq_launch_pf_gemm(const TmqPfGemm& g, int waves, hipStream_t s) {
    // shapes the kernel assumes: 64-column chunks, 32-token blocks, 64-row
    // tiles (GU: 32-row gate/up blocks), one split for fused epilogues
    if (g.K <= 0 || g.K % TMQ_PF_CHUNK || g.T_pad % 32 || g.T > g.T_pad || g.split < 1 || g.split > g.K / 32)
        return (int)hipErrorInvalidValue;
    if (g.mode != TMQ_PF_PART && g.split != 1) return (int)hipErrorInvalidValue;
    switch (g.mode) {
    case TMQ_PF_QKV:
        if (g.rows % 64) return (int)hipErrorInvalidValue;
        return launch_gemm<TMQ_PF_QKV>(g, waves, s);
    case TMQ_PF_O:
        if (g.rows % 64) return (int)hipErrorInvalidValue;
        return launch_gemm<TMQ_PF_O>(g, waves, s);
    case TMQ_PF_GU:
        if (g.gu_rows % 32 || g.rows != 2 * g.gu_rows) return (int)hipErrorInvalidValue;
        return launch_gemm<TMQ_PF_GU>(g, waves, s);
    case TMQ_PF_PART:
        if (g.rows % 64) return (int)hipErrorInvalidValue;
        return launch_gemm<TMQ_PF_PART>(g, waves, s);
    }
    return (int)hipErrorInvalidValue;
}

int tmq_launch_pf_attn(const TmqPfAttn& a, hipStream_t s) {
    const int qpk = a.n_heads / a.n_kv;
    if (qpk < 1 || qpk > 8 || a.n_heads % a.n_kv) return (int)hipErrorInvalidValue;
    const size_t lds = tmq_pf_attn_lds(qpk, a.p0 + a.T);
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)pf_attn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           160 * 1024 - 1024);
        if (e != hipSuccess) return (int)e;
        attr = true;
    }
    if (lds > 160 * 1024 - 1024) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(pf_attn_kernel, dim3(a.T, a.n_kv), dim3(512), lds, s, a);
    return (int)hipGetLastError();
}

int tmq_launch_pf_handoff(const TmqPfHandoff& h, hipStream_t s) {
    hipLaunchKernelGGL(pf_handoff_kernel, dim3(1), dim3(256), 0, s, h);
    return (int)hipGetLastError();
}
