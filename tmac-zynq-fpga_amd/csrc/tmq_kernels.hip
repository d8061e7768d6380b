// tmq_kernels.hip -- gfx950 kernels of the quantized-GEMV path.
//
// Mapping: one lane per output row, a wave covers 64 consecutive rows and
// streams their blocks from the row-interleaved planes (tmq_internal.h) with
// 16-byte loads that are contiguous across the wave.  The activation is
// wave-uniform and is read through the scalar cache.
//
// Exactness: every weight is normalised as the reference does
// (sim/fpga_sim.hpp:1034-1043, :1098-1104, :775-773):
//     w = clamp16(roundf(fl(E * row_inv)))
// with E the exact dequantised value.  roundf (ties away from zero) is done
// by one fp64 fma, see round_away().  Products w*xq are summed exactly:
// xq = 256*xh + xl with xh in [-128,127], xl in [0,255], and v_dot2_i32_i16
// accumulates w*xh and w*xl pairs in int32 (|sum| < 2^28 per 32-weight
// block), folded into int64 once per block.
#include <hip/hip_runtime.h>

#include "tmq_internal.h"

typedef short tmq_s16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 tmq_h2 __attribute__((ext_vector_type(2)));
// Activation words are wave-uniform: reading them through the constant
// address space makes the compiler use scalar (SMEM) loads.
typedef __attribute__((address_space(4))) const uint32_t cu32;

namespace {

constexpr int kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14;

__device__ __forceinline__ float h2f(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits & 0xffffu));
}

// roundf(n) for |n| < 2^31.  The fp64 fma forms n*(1+2^-30) + 1.5*2^52
// exactly and rounds it once to an integer.  n*2^-30 has n's sign and is
// below 1/64 of an fp32 ulp of n, so it cannot move n across a half-integer
// (any non-tie fp32 value is at least one ulp away from one) but it does
// push exact .5 ties away from zero -- which is roundf.  The low 32 bits of
// the fp64 result hold the integer in two's complement.
__device__ __forceinline__ int round_away(float n) {
    double t = __builtin_fma((double)n, 1.0 + 0x1p-30, 0x1.8p52);
    return (int)(uint32_t)__double_as_longlong(t);
}

// clamp16(roundf(n)) of the tile primitives.  With the row_inv computed at
// upload |n| <= 32767*(1+2^-24) and no clamp is needed; with an externally
// supplied row_inv (tile API, PhaseB replay) n is first clamped so that the
// saturating pack below reproduces the reference clamp exactly.
template <bool CLAMP>
__device__ __forceinline__ int wq(float n) {
    if (CLAMP) n = __builtin_amdgcn_fmed3f(n, -32769.0f, 32768.0f);
    return round_away(n);
}

// two int32 -> one dword of saturated int16 (lo = a, hi = b)
__device__ __forceinline__ uint32_t pk16(int a, int b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(a, b));
}

__device__ __forceinline__ int dot2(uint32_t w, uint32_t x, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(tmq_s16x2, w),
                                  __builtin_bit_cast(tmq_s16x2, x), c, false);
}

// weight planes live in global memory (address space 1): plain global loads
typedef uint32_t tmq_u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const tmq_u32x4 gu4;
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef __attribute__((address_space(1))) const uint16_t gu16;
__device__ __forceinline__ uint4 ld16(const uint8_t* p) {
    const tmq_u32x4 v = *(const gu4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) { return *(const gu32*)p; }
__device__ __forceinline__ uint32_t ld2(const uint8_t* p) { return *(const gu16*)p; }

// wave index, known to the compiler to be wave-uniform (an SGPR)
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ uint32_t byte_of(const uint4& v, int i) {
    uint32_t d = (i < 4) ? v.x : (i < 8) ? v.y : (i < 12) ? v.z : v.w;
    return (d >> (8 * (i & 3))) & 0xffu;
}
__device__ __forceinline__ uint32_t dw_of(const uint4& v, int i) {
    return (i == 0) ? v.x : (i == 1) ? v.y : (i == 2) ? v.z : v.w;
}
// byte k of a dword as float (v_cvt_f32_ubyteN)
__device__ __forceinline__ float ubf(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xffu); }

// bytes 0,1 (sel 0x0c010c00) or 2,3 (0x0c030c02) of w, each zero-extended
// into a 16-bit lane: as f16 those lanes are the subnormals b * 2^-24, exact
// inputs for v_fma_mix_f32 (fp16 denormals are not flushed)
__device__ __forceinline__ tmq_h2 lanes01(uint32_t w) {
    return __builtin_bit_cast(tmq_h2, __builtin_amdgcn_perm(0u, w, 0x0c010c00u));
}
__device__ __forceinline__ tmq_h2 lanes23(uint32_t w) {
    return __builtin_bit_cast(tmq_h2, __builtin_amdgcn_perm(0u, w, 0x0c030c02u));
}

struct Act {
    float xs;
    const cu32* xh;
    const cu32* xl;
};
__device__ __forceinline__ Act act_view(const uint8_t* a) {
    const cu32* p = (const cu32*)a;
    Act r;
    r.xs = __builtin_bit_cast(float, p[0]);
    const int n = (int)p[1];
    r.xh = p + 4;
    r.xl = r.xh + n / 2;
    return r;
}

__device__ __forceinline__ size_t p16(int b, int c, int C, size_t R, int r) {
    return (((size_t)b * C + c) * R + (size_t)r) * 16;
}

// 4 weights (quantised value u_k, normaliser E_k = f(u_k)) -> two int16
// pairs -> dot with the activation pairs kx, kx+1
template <bool CLAMP>
__device__ __forceinline__ void mac4(float e0, float e1, float e2, float e3, float inv,
                                     const Act& A, int kx, int& sh, int& sl) {
    const uint32_t P0 = pk16(wq<CLAMP>(e0 * inv), wq<CLAMP>(e1 * inv));
    const uint32_t P1 = pk16(wq<CLAMP>(e2 * inv), wq<CLAMP>(e3 * inv));
    sh = dot2(P0, A.xh[kx], sh);
    sl = dot2(P0, A.xl[kx], sl);
    sh = dot2(P1, A.xh[kx + 1], sh);
    sl = dot2(P1, A.xl[kx + 1], sl);
}

// ---------------------------------------------------------------- Q5_0
// Planes: qs[16] as in ggml; qh' = qh with its bits transposed so that bit
// (8k + g) holds the high bit of element 4g + k; d f16.  Group g of four
// weights (elements 4g..4g+3) is decoded SWAR-style into four bytes
// u = nibble | hb<<4, spread into f16 lanes 0x6400|u (= 1024+u) and turned
// into E = (u-16)*d exactly by one v_fma_mix: (1024+u)*d - 1040*d.
template <bool CLAMP>
__device__ __forceinline__ void q5_0_block(const TmqTensorDev& t, const Act& A, int b, int r,
                                           float inv, int& sh, int& sl) {
    const size_t o = (size_t)b * t.rows_pad + r;
    const uint4 qs = ld16(t.pa + o * 16);
    const uint32_t qhp = ld4(t.pb + o * 4);
    const float d = h2f(ld2(t.pd + o * 2));
    const float c = -1040.0f * d;  // exact: 7-bit x 11-bit
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t nib = (g < 4) ? (dw_of(qs, g) & 0x0f0f0f0fu) : ((dw_of(qs, g - 4) >> 4) & 0x0f0f0f0fu);
        const uint32_t hs = (g <= 4) ? (qhp << (4 - g)) : (qhp >> (g - 4));
        const uint32_t U = (hs & 0x10101010u) | nib;
        const tmq_h2 v0 = __builtin_bit_cast(tmq_h2, __builtin_amdgcn_perm(0x64646464u, U, 0x04010400u));
        const tmq_h2 v1 = __builtin_bit_cast(tmq_h2, __builtin_amdgcn_perm(0x64646464u, U, 0x04030402u));
        mac4<CLAMP>(__builtin_fmaf((float)v0.x, d, c), __builtin_fmaf((float)v0.y, d, c),
                    __builtin_fmaf((float)v1.x, d, c), __builtin_fmaf((float)v1.y, d, c), inv, A,
                    b * 16 + 2 * g, sh, sl);
    }
}

// ---------------------------------------------------------------- Q4_K
__device__ __forceinline__ void q4k_scale_min(const uint4& h, int s, int& sc, int& m) {
    // scales[12] are bytes 4..15 of the 16-byte header
    if (s < 4) {
        sc = (int)(byte_of(h, 4 + s) & 63u);
        m = (int)(byte_of(h, 8 + s) & 63u);
    } else {
        sc = (int)((byte_of(h, 8 + s) & 0xfu) | ((byte_of(h, s) >> 6) << 4));
        m = (int)((byte_of(h, 8 + s) >> 4) | ((byte_of(h, 4 + s) >> 6) << 4));
    }
}

// E = fl(d*sc*q4 - dmin*m): d*sc*q4 is exact, so one fma with -dmin*m rounds
// exactly where the reference's multiply-then-subtract does.  The nibbles go
// into f16 lanes as subnormals q*2^-24 (low nibbles) and 16q*2^-24 (high
// nibbles, masked in place), so E = fma_mix(lane, A*2^24 or A*2^20, -B):
// the scalings by powers of two are exact and the product is A*q exactly.
template <bool CLAMP>
__device__ __forceinline__ void q4_k_block(const TmqTensorDev& t, const Act& A, int b, int r,
                                           float inv, int& sh, int& sl) {
    const size_t R = t.rows_pad;
    const uint4 h = ld16(t.pb + p16(b, 0, 1, R, r));
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
#pragma unroll
    for (int sp = 0; sp < 4; sp++) {
        int sc0, m0, sc1, m1;
        q4k_scale_min(h, 2 * sp, sc0, m0);
        q4k_scale_min(h, 2 * sp + 1, sc1, m1);
        const float A0 = (d * (float)sc0) * 0x1p24f, B0 = -(dmin * (float)m0);
        const float A1 = (d * (float)sc1) * 0x1p20f, B1 = -(dmin * (float)m1);
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            const uint4 qs = ld16(t.pa + p16(b, 2 * sp + hf, 8, R, r));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t w = dw_of(qs, i);
                const uint32_t lo = w & 0x0f0f0f0fu, hi = w & 0xf0f0f0f0u;
                const tmq_h2 l0 = lanes01(lo), l1 = lanes23(lo), h0 = lanes01(hi), h1 = lanes23(hi);
                const int kx = (b * 256 + 64 * sp + 16 * hf + 4 * i) / 2;
                mac4<CLAMP>(__builtin_fmaf((float)l0.x, A0, B0), __builtin_fmaf((float)l0.y, A0, B0),
                            __builtin_fmaf((float)l1.x, A0, B0), __builtin_fmaf((float)l1.y, A0, B0),
                            inv, A, kx, sh, sl);
                mac4<CLAMP>(__builtin_fmaf((float)h0.x, A1, B1), __builtin_fmaf((float)h0.y, A1, B1),
                            __builtin_fmaf((float)h1.x, A1, B1), __builtin_fmaf((float)h1.y, A1, B1),
                            inv, A, kx + 16, sh, sl);
            }
        }
    }
}

// ---------------------------------------------------------------- Q6_K
// u6 = ql nibble | (qh 2 bits) << 4, built four at a time in byte lanes;
// E = S*(u-32) exactly (S = d*sc has <= 18 significant bits, u-32 <= 6).
template <bool CLAMP>
__device__ __forceinline__ void q6_k_block(const TmqTensorDev& t, const Act& A, int b, int r,
                                           float inv, int& sh, int& sl) {
    const size_t R = t.rows_pad;
    const uint4 sc = ld16(t.pc + p16(b, 0, 1, R, r));
    const float ss = h2f(ld2(t.pd + ((size_t)b * R + r) * 2));
#pragma unroll
    for (int half = 0; half < 2; half++) {
#pragma unroll
        for (int lc = 0; lc < 2; lc++) {
            const uint4 qla = ld16(t.pa + p16(b, half * 4 + lc, 8, R, r));
            const uint4 qlb = ld16(t.pa + p16(b, half * 4 + 2 + lc, 8, R, r));
            const uint4 qhc = ld16(t.pb + p16(b, half * 2 + lc, 4, R, r));
#pragma unroll
            for (int sub = 0; sub < 4; sub++) {
                const float S = ss * (float)(int8_t)byte_of(sc, half * 8 + lc + 2 * sub);
                const float nS = -32.0f * S, S24 = S * 0x1p24f;
                const uint4& src = (sub & 1) ? qlb : qla;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t ql = dw_of(src, i), qh = dw_of(qhc, i);
                    const uint32_t nib = (sub < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                    const uint32_t hs = (sub == 0) ? (qh << 4) : (sub == 1) ? (qh << 2) : (sub == 2) ? qh : (qh >> 2);
                    const uint32_t U = (hs & 0x30303030u) | nib;
                    const int kx = (b * 256 + half * 128 + sub * 32 + 16 * lc + 4 * i) / 2;
                    // E = S*(u-32) = fma_mix(u*2^-24, S*2^24, -32*S), exact
                    const tmq_h2 u0 = lanes01(U), u1 = lanes23(U);
                    mac4<CLAMP>(__builtin_fmaf((float)u0.x, S24, nS), __builtin_fmaf((float)u0.y, S24, nS),
                                __builtin_fmaf((float)u1.x, S24, nS), __builtin_fmaf((float)u1.y, S24, nS),
                                inv, A, kx, sh, sl);
                }
            }
        }
    }
}

// ---------------------------------------------------------------- Q8_0
// UQ8.8 combined scale of sim/tmac_gguf.cpp:1030-1037, including the x86
// float->uint16 conversion (truncate to int32, keep the low 16 bits).
__device__ __forceinline__ uint32_t q8_cs(float bs, float ri) {
    float c = bs * ri;
    if (c >= 256.0f) c = 255.996f;
    if (c < 0.0f) c = 0.0f;
    float tf = c * 256.0f + 0.5f;
    return (uint32_t)(int)tf & 0xffffu;
}

// deq = (q8*cs) >> 8: with |q8*cs| < 2^23, bytes 1..2 of the product are
// exactly that int16, so one v_perm packs two of them.
struct Q8Blk {
    uint4 v0, v1;
    uint32_t d;
};
__device__ __forceinline__ Q8Blk q8_load(const TmqTensorDev& t, int b, int r) {
    const size_t R = t.rows_pad;
    Q8Blk k;
    k.v0 = ld16(t.pa + p16(b, 0, 2, R, r));
    k.v1 = ld16(t.pa + p16(b, 1, 2, R, r));
    k.d = ld2(t.pd + ((size_t)b * R + r) * 2);
    return k;
}
__device__ __forceinline__ void q8_mac(const Q8Blk& k, const Act& A, int b, float ri, int& sh, int& sl) {
    const int cs = (int)q8_cs(h2f(k.d), ri);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint4& v = (j < 8) ? k.v0 : k.v1;
        const int p0 = (int)(int8_t)byte_of(v, (2 * j) & 15) * cs;
        const int p1 = (int)(int8_t)byte_of(v, (2 * j + 1) & 15) * cs;
        const uint32_t P = __builtin_amdgcn_perm((uint32_t)p1, (uint32_t)p0, 0x06050201u);
        sh = dot2(P, A.xh[b * 16 + j], sh);
        sl = dot2(P, A.xl[b * 16 + j], sl);
    }
}

// ------------------------------------------------------------ row groups
// K-split group (Q5_0 / K-quants): 4 waves share 64 rows, wave w takes
// blocks w, w+4, ...; the int32 pair sums are folded into int64 every
// 256 weights at most (|sum| < 2^31), then the waves meet in LDS.
template <int FMT, bool CLAMP>
__device__ __forceinline__ void group_ksplit(const TmqWork& w, int g) {
    __shared__ int64_t part[TMQ_WAVES][64];
    const TmqTensorDev& t = w.t;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    const float inv = t.row_inv[r];
    const Act A = act_view(w.act);
    int64_t acc = 0;
    if (FMT == kQ5_0) {
        int b = wave;
        for (; b + TMQ_WAVES < t.nb; b += 2 * TMQ_WAVES) {
            int sh = 0, sl = 0;
            q5_0_block<CLAMP>(t, A, b, r, inv, sh, sl);
            q5_0_block<CLAMP>(t, A, b + TMQ_WAVES, r, inv, sh, sl);
            acc += (int64_t)sh * 256 + sl;
        }
        if (b < t.nb) {
            int sh = 0, sl = 0;
            q5_0_block<CLAMP>(t, A, b, r, inv, sh, sl);
            acc += (int64_t)sh * 256 + sl;
        }
    } else {
        for (int b = wave; b < t.nb; b += TMQ_WAVES) {
            int sh = 0, sl = 0;
            if (FMT == kQ4_K) q4_k_block<CLAMP>(t, A, b, r, inv, sh, sl);
            if (FMT == kQ6_K) q6_k_block<CLAMP>(t, A, b, r, inv, sh, sl);
            acc += (int64_t)sh * 256 + sl;
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && r < t.rows) {
        int64_t tot = part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane];
        if (w.acc) w.acc[r] = tot;
        if (w.y) {
            // sim/tmac_gguf.cpp:1303-1305: y = 0.0f; y += (double)acc*x_scale/(double)row_inv
            w.y[r] = (float)(((double)tot * (double)A.xs) / (double)inv);
        }
    }
}

// Q8_0 group: 4 waves take 4 consecutive 64-row groups (256 rows) and each
// walks all 64-column tiles of its rows in order, folding the tile results
// into y in double exactly as sim/tmac_gguf.cpp:1075-1076 does.
__device__ __forceinline__ void group_q8(const TmqWork& w, int g) {
    const TmqTensorDev& t = w.t;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r0 = (g * TMQ_WAVES + wave) * 64;
    if (r0 >= t.rows_pad) return;
    const int r = r0 + lane;
    const float ri = t.row_inv[r], rs = t.row_scale[r];
    const Act A = act_view(w.act);
    const int nt = (t.cols + 63) / 64;
    float y = 0.0f;
    // software pipeline: the next block's loads are in flight while the
    // current block is multiplied
    Q8Blk cur = q8_load(t, 0, r);
    for (int tt = 0; tt < nt; tt++) {
        int sh = 0, sl = 0;
        const int b0 = 2 * tt, b1 = 2 * tt + 1;
        const bool has1 = b1 < t.nb;
        Q8Blk nxt = has1 ? q8_load(t, b1, r) : cur;
        q8_mac(cur, A, b0, ri, sh, sl);
        if (has1) {
            cur = (b1 + 1 < t.nb) ? q8_load(t, b1 + 1, r) : nxt;
            q8_mac(nxt, A, b1, ri, sh, sl);
        } else if (b0 + 1 < t.nb) {
            cur = q8_load(t, b0 + 1, r);
        }
        const int64_t P = (int64_t)sh * 256 + sl;
        if (w.acc && r < t.rows) w.acc[(size_t)r * nt + tt] = P;
        y = (float)((double)y + ((double)P * (double)A.xs) * (double)rs);
    }
    if (w.y && r < t.rows) w.y[r] = y;
}

template <int FMT, bool CLAMP>
__device__ __forceinline__ void run_group(const TmqWork& w, int g) {
    if (FMT == kQ8_0) group_q8(w, g);
    else group_ksplit<FMT, CLAMP>(w, g);
}

// one GEMV
template <int FMT, bool CLAMP>
__global__ __launch_bounds__(TMQ_WG) void gemv_kernel(TmqWork w) {
    run_group<FMT, CLAMP>(w, blockIdx.x);
}

// A chain segment: every descriptor of one format in one launch,
// workgroup -> (descriptor, group) through the group map.
template <int FMT, bool CLAMP>
__global__ __launch_bounds__(TMQ_WG) void chain_kernel(const TmqWork* __restrict__ works,
                                                       const int32_t* __restrict__ group_work) {
    const TmqWork& w = works[group_work[blockIdx.x]];
    run_group<FMT, CLAMP>(w, blockIdx.x - w.first_group);
}

// ------------------------------------------------------ activation prep
// sim/tmac_gguf.cpp:1225-1231: x_scale = max|x| (sequential fmaxf; the max
// is order independent), /32767 unless < 1e-10; xq = (int16)roundf(x/x_scale)
__global__ __launch_bounds__(1024) void act_prep_kernel(TmqActJobs jobs) {
    const TmqActJob& J = jobs.j[blockIdx.x];
    __shared__ float red[16];
    __shared__ float s_scale;
    const int n = J.n;
    float m = 0.0f;
    for (int j = threadIdx.x; j < n; j += blockDim.x) m = fmaxf(m, fabsf(J.x[j]));
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float mm = 0.0f;
        for (int i = 0; i < (int)(blockDim.x >> 6); i++) mm = fmaxf(mm, red[i]);
        s_scale = (mm < 1e-10f) ? 1.0f : mm / 32767.0f;
        *(float*)J.act = s_scale;
        *(int*)(J.act + 4) = n;
    }
    __syncthreads();
    const float s = s_scale;
    uint32_t* xh = (uint32_t*)(J.act + 16);
    uint32_t* xl = xh + n / 2;
    int16_t* xq = (int16_t*)(xl + n / 2);
    for (int k = threadIdx.x; k < n / 2; k += blockDim.x) {
        int a = (int)(int16_t)roundf(J.x[2 * k] / s);
        int c = (int)(int16_t)roundf(J.x[2 * k + 1] / s);
        xq[2 * k] = (int16_t)a;
        xq[2 * k + 1] = (int16_t)c;
        xh[k] = ((uint32_t)(a >> 8) & 0xffffu) | ((uint32_t)(c >> 8) << 16);
        xl[k] = ((uint32_t)a & 0xffu) | (((uint32_t)c & 0xffu) << 16);
    }
}

// ------------------------------------------------------------- repack
// ggml blocks (row-major) -> planes.  One thread per (row, block column).
__global__ void repack_kernel(int type, const uint8_t* __restrict__ src, TmqTensorDev t) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)t.rows * t.nb;
    if (idx >= total) return;
    const int r = (int)(idx / t.nb), b = (int)(idx % t.nb);
    const size_t R = t.rows_pad;
    uint8_t* pa = (uint8_t*)t.pa;
    uint8_t* pb = (uint8_t*)t.pb;
    uint8_t* pc = (uint8_t*)t.pc;
    uint8_t* pd = (uint8_t*)t.pd;
    if (type == kQ8_0) {
        const uint8_t* s = src + idx * 34;
        pd[((size_t)b * R + r) * 2 + 0] = s[0];
        pd[((size_t)b * R + r) * 2 + 1] = s[1];
        for (int i = 0; i < 32; i++) pa[p16(b, i >> 4, 2, R, r) + (i & 15)] = s[2 + i];
    } else if (type == kQ5_0) {
        const uint8_t* s = src + idx * 22;
        pd[((size_t)b * R + r) * 2 + 0] = s[0];
        pd[((size_t)b * R + r) * 2 + 1] = s[1];
        const uint32_t qh = (uint32_t)s[2] | ((uint32_t)s[3] << 8) | ((uint32_t)s[4] << 16) | ((uint32_t)s[5] << 24);
        uint32_t qhp = 0;  // bit 8k+g <- bit 4g+k
        for (int e = 0; e < 32; e++) qhp |= ((qh >> e) & 1u) << (8 * (e & 3) + (e >> 2));
        *(uint32_t*)(pb + ((size_t)b * R + r) * 4) = qhp;
        for (int i = 0; i < 16; i++) pa[p16(b, 0, 1, R, r) + i] = s[6 + i];
    } else if (type == kQ4_K) {
        const uint8_t* s = src + idx * 144;
        for (int i = 0; i < 16; i++) pb[p16(b, 0, 1, R, r) + i] = s[i];
        for (int i = 0; i < 128; i++) pa[p16(b, i >> 4, 8, R, r) + (i & 15)] = s[16 + i];
    } else if (type == kQ6_K) {
        const uint8_t* s = src + idx * 210;
        for (int i = 0; i < 128; i++) pa[p16(b, i >> 4, 8, R, r) + (i & 15)] = s[i];
        for (int i = 0; i < 64; i++) pb[p16(b, i >> 4, 4, R, r) + (i & 15)] = s[128 + i];
        for (int i = 0; i < 16; i++) pc[p16(b, 0, 1, R, r) + i] = s[192 + i];
        pd[((size_t)b * R + r) * 2 + 0] = s[208];
        pd[((size_t)b * R + r) * 2 + 1] = s[209];
    }
}

// ------------------------------------------------------------ row stats
// Per-row max|E| -> row_inv (sim/tmac_gguf.cpp:1242-1263, :1116-1136,
// :1381-1424) or, for Q8_0, row_scale and its guarded inverse
// (sim/tmac_gguf.cpp:979-1003, :1034-1035).  Flags Inf/NaN scales.
__device__ __forceinline__ bool finite_h(uint32_t bits) { return ((bits >> 10) & 0x1fu) != 0x1fu; }

__global__ void rowstat_kernel(TmqTensorDev t, const float* __restrict__ aux, float* row_inv,
                               float* row_scale, int* bad) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= t.rows_pad) return;
    const size_t R = t.rows_pad;
    float mx = 0.0f;
    bool ok = true;
    for (int b = 0; b < t.nb; b++) {
        if (t.type == kQ5_0) {
            uint32_t db = *(const uint16_t*)(t.pd + ((size_t)b * R + r) * 2);
            ok &= finite_h(db);
            const float d = h2f(db);
            const uint4 qs = ld16(t.pa + p16(b, 0, 1, R, r));
            const uint32_t qhp = *(const uint32_t*)(t.pb + ((size_t)b * R + r) * 4);
            for (int e = 0; e < 32; e++) {
                uint32_t by = byte_of(qs, e & 15);
                int nib = (e < 16) ? (int)(by & 15u) : (int)(by >> 4);
                int hb = (int)((qhp >> (8 * (e & 3) + (e >> 2))) & 1u);
                int q = (hb << 4) + nib - 16;
                float ab = fabsf(d * (float)q);
                if (ab > mx) mx = ab;
            }
        } else if (t.type == kQ4_K) {
            const uint4 h = ld16(t.pb + p16(b, 0, 1, R, r));
            ok &= finite_h(h.x) && finite_h(h.x >> 16);
            const float d = h2f(h.x), dmin = h2f(h.x >> 16);
            for (int s = 0; s < 8; s++) {
                int sc, m;
                q4k_scale_min(h, s, sc, m);
                const float A = d * (float)sc, B = dmin * (float)m;
                const uint4 qs = ld16(t.pa + p16(b, (s >> 1) * 2, 8, R, r));
                const uint4 qs2 = ld16(t.pa + p16(b, (s >> 1) * 2 + 1, 8, R, r));
                for (int j = 0; j < 32; j++) {
                    uint32_t by = byte_of(j < 16 ? qs : qs2, j & 15);
                    uint32_t q4 = (s & 1) ? (by >> 4) : (by & 15u);
                    float ab = fabsf(__builtin_fmaf((float)q4, A, -B));
                    if (ab > mx) mx = ab;
                }
            }
        } else if (t.type == kQ6_K) {
            uint32_t db = *(const uint16_t*)(t.pd + ((size_t)b * R + r) * 2);
            ok &= finite_h(db);
            const float ss = h2f(db);
            const uint4 sc = ld16(t.pc + p16(b, 0, 1, R, r));
            for (int wi = 0; wi < 256; wi++) {
                int half = wi >> 7, pos = wi & 127, l = pos & 31, sub = pos >> 5;
                int qlo = half * 64 + l + (sub & 1) * 32;
                uint32_t qlb = byte_of(ld16(t.pa + p16(b, qlo >> 4, 8, R, r)), qlo & 15);
                int qho = half * 32 + l;
                uint32_t qhb = byte_of(ld16(t.pb + p16(b, qho >> 4, 4, R, r)), qho & 15);
                uint32_t nib = (sub < 2) ? (qlb & 15u) : (qlb >> 4);
                int q6 = (int)(nib | (((qhb >> (2 * sub)) & 3u) << 4)) - 32;
                float S = ss * (float)(int8_t)byte_of(sc, half * 8 + (l >> 4) + sub * 2);
                float ab = fabsf(S * (float)q6);
                if (ab > mx) mx = ab;
            }
        } else if (t.type == kQ8_0) {
            uint32_t db = *(const uint16_t*)(t.pd + ((size_t)b * R + r) * 2);
            ok &= finite_h(db);
            const float d = h2f(db);
            const uint4 v0 = ld16(t.pa + p16(b, 0, 2, R, r));
            const uint4 v1 = ld16(t.pa + p16(b, 1, 2, R, r));
            for (int i = 0; i < 32; i++) {
                float a = fabsf((float)(int8_t)byte_of(i < 16 ? v0 : v1, i & 15) * d);
                if (a > mx) mx = a;
            }
        }
    }
    if (!ok && r < t.rows) atomicOr(bad, 1);
    if (t.type == kQ8_0) {
        if (aux && r < t.rows) mx = aux[r];
        float rs = (mx < 1e-10f) ? 1.0f : mx / 32767.0f;
        row_scale[r] = rs;
        row_inv[r] = (rs < 1e-10f) ? 1.0f : (1.0f / rs);
    } else {
        mx = (mx < 1e-10f) ? 1.0f : mx;
        row_inv[r] = 32767.0f / mx;
    }
}

// ----------------------------------------------------------- Q8 tile
// axi_vecmul_tile_q8: q8_W column-major [k][n], cs[n*2 + k/32] UQ8.8,
// deq = (q8*cs) >> 8, result[n] = sum_k vec[k]*deq (sim/fpga_sim.hpp:316-349)
__global__ void tile_q8_kernel(const uint8_t* __restrict__ W, const uint16_t* __restrict__ cs,
                               const int16_t* __restrict__ vec, int64_t* __restrict__ out) {
    const int n = threadIdx.x;
    int64_t a = 0;
    for (int k = 0; k < 64; k++) {
        int p = (int)(int8_t)W[k * 64 + n] * (int)cs[n * 2 + k / 32];
        a += (int64_t)vec[k] * (int64_t)(int16_t)(p >> 8);
    }
    out[n] = a;
}

}  // namespace

// ---------------------------------------------------------------- launchers
int tmq_launch_act_prep(const TmqActJobs& jobs, hipStream_t s) {
    if (jobs.count <= 0) return 0;
    hipLaunchKernelGGL(act_prep_kernel, dim3(jobs.count), dim3(1024), 0, s, jobs);
    return (int)hipGetLastError();
}

int tmq_launch_repack(int type, const uint8_t* src, const TmqTensorDev& t, hipStream_t s) {
    const size_t total = (size_t)t.rows * t.nb;
    const int bs = 256;
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((total + bs - 1) / bs)), dim3(bs), 0, s,
                       type, src, t);
    return (int)hipGetLastError();
}

int tmq_launch_rowstat(const TmqTensorDev& t, const float* aux, float* row_inv, float* row_scale,
                       int* bad, hipStream_t s) {
    const int bs = 64;
    hipLaunchKernelGGL(rowstat_kernel, dim3((t.rows_pad + bs - 1) / bs), dim3(bs), 0, s, t, aux,
                       row_inv, row_scale, bad);
    return (int)hipGetLastError();
}

template <template <int, bool> class K>
static void* kernel_for(int type, int clamp) {
    switch (type) {
    case kQ5_0: return clamp ? (void*)K<kQ5_0, true>::fn() : (void*)K<kQ5_0, false>::fn();
    case kQ4_K: return clamp ? (void*)K<kQ4_K, true>::fn() : (void*)K<kQ4_K, false>::fn();
    case kQ6_K: return clamp ? (void*)K<kQ6_K, true>::fn() : (void*)K<kQ6_K, false>::fn();
    case kQ8_0: return (void*)K<kQ8_0, false>::fn();
    default: return nullptr;
    }
}
template <int F, bool C> struct GemvK { static auto fn() { return gemv_kernel<F, C>; } };
template <int F, bool C> struct ChainK { static auto fn() { return chain_kernel<F, C>; } };

int tmq_launch_gemv(const TmqWork& w, hipStream_t s) {
    if (w.ngroups <= 0) return 0;
    void* k = kernel_for<GemvK>(w.t.type, w.t.clamp);
    if (!k) return (int)hipErrorInvalidValue;
    TmqWork arg = w;
    void* args[] = {&arg};
    return (int)hipLaunchKernel(k, dim3(w.ngroups), dim3(TMQ_WG), args, 0, s);
}

int tmq_launch_chain(int type, int clamp, const TmqWork* works_dev, const int32_t* group_work_dev,
                     int total_groups, hipStream_t s) {
    if (total_groups <= 0) return 0;
    void* k = kernel_for<ChainK>(type, clamp);
    if (!k) return (int)hipErrorInvalidValue;
    void* args[] = {&works_dev, &group_work_dev};
    return (int)hipLaunchKernel(k, dim3(total_groups), dim3(TMQ_WG), args, 0, s);
}

int tmq_launch_tile_q8(const uint8_t* W, const uint16_t* cs, const int16_t* vec, int64_t* out,
                       hipStream_t s) {
    hipLaunchKernelGGL(tile_q8_kernel, dim3(1), dim3(64), 0, s, W, cs, vec, out);
    return (int)hipGetLastError();
}
