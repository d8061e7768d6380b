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
#include <mutex>
#include <set>

#include <cstdlib>
#include <type_traits>

#include "tmq_internal.h"
#include "tmq_mathf.h"
#include "tmq_device.h"
#include "tmq_prefill.h"

typedef short tmq_s16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 tmq_h2 __attribute__((ext_vector_type(2)));
// Activation words are wave-uniform: reading them through the constant
// address space makes the compiler use scalar (SMEM) loads.
typedef __attribute__((address_space(4))) const uint32_t cu32;

namespace {

constexpr int kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kQ5_0M = TMQ_FMT_Q5_0_MFMA;
constexpr int kQ4_KM = TMQ_FMT_Q4_K_MFMA, kQ6_KM = TMQ_FMT_Q6_K_MFMA;
constexpr int kF32 = 0, kF16 = 1;  // element types of the INT16 / FP32 paths

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

// A fitted weight is the integer nearest (ties to even) to fl(u*A + B):
// adding 1.5*2^23 rounds that value to an integer in the low mantissa bits,
// the bit pattern being kFitM + w (|w| < 2^22).
constexpr uint32_t kFitM = 0x4B400000u;
__device__ __forceinline__ float fit_rne(float x) { return x + 0x1.8p23f; }
__device__ __forceinline__ int32_t fit_biased(float r) { return (int32_t)__float_as_uint(r); }
// two of them (fit_rne values) as one int16 pair: the low halves
__device__ __forceinline__ uint32_t pk_rne(float r0, float r1) {
    return __builtin_amdgcn_perm(__float_as_uint(r1), __float_as_uint(r0), 0x05040100u);
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
typedef __attribute__((address_space(1))) const uint8_t gu8;
__device__ __forceinline__ uint32_t ld1(const uint8_t* p) { return *(const gu8*)p; }

// Weight-stream loads: every weight byte is read once per GEMV, so they
// carry the nontemporal cache policy (gfx950 "nt": streamed through the
// caches without displacing reused lines), worth ~10 % of read bandwidth
// on a plain stream.  TMQ_CPOL_NT is the same bit for the LDS-DMA loads.
#ifndef TMQ_WEIGHT_NT
#define TMQ_WEIGHT_NT 1
#endif
#define TMQ_CPOL_NT (TMQ_WEIGHT_NT ? 2 : 0)
__device__ __forceinline__ uint4 ldw16(const uint8_t* p) {
#if TMQ_WEIGHT_NT
    const tmq_u32x4 v = __builtin_nontemporal_load((const gu4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return ld16(p);
#endif
}
__device__ __forceinline__ uint32_t ldw4(const uint8_t* p) {
#if TMQ_WEIGHT_NT
    return __builtin_nontemporal_load((const gu32*)p);
#else
    return ld4(p);
#endif
}
__device__ __forceinline__ uint32_t ldw2(const uint8_t* p) {
#if TMQ_WEIGHT_NT
    return __builtin_nontemporal_load((const gu16*)p);
#else
    return ld2(p);
#endif
}
__device__ __forceinline__ uint32_t ldw1(const uint8_t* p) {
#if TMQ_WEIGHT_NT
    return __builtin_nontemporal_load((const gu8*)p);
#else
    return ld1(p);
#endif
}

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

// Activation view: x_scale and the XH/XL pair arrays, read either through
// the scalar cache (standalone GEMVs: a prepared activation in HBM) or from
// LDS (engine GEMVs: each workgroup quantises its activation itself).
typedef __attribute__((address_space(3))) const uint32_t lu32;
template <class P>
struct ActT {
    static constexpr bool kSink = false;
    float xs;
    P xh;
    P xl;
    P x32;  // xq as int32 (scalar-cache view only)
};

// Weight sink: takes the place of an activation in the block decoders and
// stores each int16 weight pair as its prefill digits instead of multiplying
// it (hi = w >> 8, lo = (w & 255) - 128), at columns 2*kx, 2*kx+1 of `row`
// in fragment-major planes (tmq_prefill.h; the pair is two adjacent bytes
// of one fragment per digit).
struct WDigits {
    static constexpr bool kSink = true;
    int8_t* planes;
    int row, K;
    __device__ __forceinline__ void put(int kx, uint32_t P) const {
        const size_t o = tmq_pf_off(row, 2 * kx, K, 0);
        *(uint16_t*)(planes + o) = (uint16_t)__builtin_amdgcn_perm(0u, P, 0x0c0c0301u);
        *(uint16_t*)(planes + o + 1024) = (uint16_t)(__builtin_amdgcn_perm(0u, P, 0x0c0c0200u) ^ 0x8080u);
    }
};
typedef ActT<const cu32*> Act;
typedef ActT<const lu32*> ActL;

// N activation pairs in registers (element kx of the view is pair
// base + kx of the activation), read before a decoder branches.
template <int N>
struct ActN {
    static constexpr bool kSink = false;
    uint32_t xh[N], xl[N];
};
template <int N, class AT>
__device__ __forceinline__ ActN<N> act_n(const AT& A, int base) {
    ActN<N> r;
#pragma unroll
    for (int i = 0; i < N; i++) {
        r.xh[i] = A.xh[base + i];
        r.xl[i] = A.xl[base + i];
    }
    return r;
}

__device__ __forceinline__ Act act_view(const uint8_t* a) {
    const cu32* p = (const cu32*)a;
    Act r;
    r.xs = __builtin_bit_cast(float, p[0]);
    const int n = (int)p[1];
    r.xh = p + 4;
    r.xl = r.xh + n / 2;
    r.x32 = r.xh + 3 * (n / 2);
    return r;
}

__device__ __forceinline__ size_t p16(int b, int c, int C, size_t R, int r) {
    return (((size_t)b * C + c) * R + (size_t)r) * 16;
}

// 4 weights (quantised value u_k, normaliser E_k = f(u_k)) -> two int16
// pairs -> dot with the activation pairs kx, kx+1
template <bool CLAMP, class AT>
__device__ __forceinline__ void mac4(float e0, float e1, float e2, float e3, float inv,
                                     const AT& A, int kx, int& sh, int& sl) {
    const uint32_t P0 = pk16(wq<CLAMP>(e0 * inv), wq<CLAMP>(e1 * inv));
    const uint32_t P1 = pk16(wq<CLAMP>(e2 * inv), wq<CLAMP>(e3 * inv));
    if constexpr (AT::kSink) {
        A.put(kx, P0);
        A.put(kx + 1, P1);
    } else {
        sh = dot2(P0, A.xh[kx], sh);
        sl = dot2(P0, A.xl[kx], sl);
        sh = dot2(P1, A.xh[kx + 1], sh);
        sl = dot2(P1, A.xl[kx + 1], sl);
    }
}

// 4 fitted weights (fit_rne values) -> two int16 pairs -> dot with the
// activation pairs kx, kx+1
template <class AT>
__device__ __forceinline__ void mac4r(float r0, float r1, float r2, float r3, const AT& A, int kx, int& sh, int& sl) {
    const uint32_t P0 = pk_rne(r0, r1), P1 = pk_rne(r2, r3);
    if constexpr (AT::kSink) {
        A.put(kx, P0);
        A.put(kx + 1, P1);
    } else {
        sh = dot2(P0, A.xh[kx], sh);
        sl = dot2(P0, A.xl[kx], sl);
        sh = dot2(P1, A.xh[kx + 1], sh);
        sl = dot2(P1, A.xl[kx + 1], sl);
    }
}

// Each format: Blk = one block of one row in registers, blk_load() fetches
// it from the planes, blk_mac() multiplies it into the pair sums.

// ---------------------------------------------------------------- Q5_0
// Planes: the 32 5-bit codes in five dwords D0..D4 (A: D0-D3, B: D4), d f16.
// Byte k of D_g holds in bits 0-4 the code of element 4g + k (elements
// 0-19); bits 5-7 of the twenty bytes hold elements 20-31: element 20+k
// bits 0-2 in D0 byte k, bits 3-4 in D1 byte k bits 5-6; 24+k likewise in
// D2, D3; 28+k bits 0-2 in D4 byte k, bit 3 in D1 byte k bit 7, bit 4 in D3
// byte k bit 7.  Group g of four weights (elements 4g..4g+3) is then one
// mask (g < 5) or a few shifts and masks away as four code bytes u; the
// decoders spread them into f16 lanes 0x6400|u (= 1024+u) and turn them
// into E = (u-16)*d exactly by one v_fma_mix: (1024+u)*d - 1040*d.
//
// Fitted blocks (tensors normalised at upload): within one block of one row
// the int16 weight is a function g(u) of the 5-bit code u alone, and
// g(u) = rne(fl(u*A + B)) (nearest integer, ties to even) for a pair
// (A, B) found at upload (fit_kernel) and checked there against the exact
// g on every code the block holds.  A and B are d*row_inv and -16A (fp32,
// as computed here) moved by a few ulps, coded in one byte per block and
// row (plane pe, fit_a/fit_b).  The code goes into an f16 lane as the
// subnormal u*2^-24, so one v_fma_mix with A*2^24 forms u*A + B with a
// single rounding, and one add of 1.5*2^23 (fit_rne) leaves the weight in
// the low bits: 2 instructions per weight instead of 4.  The K-quants fit
// each 32-weight (Q4_K) or 16-weight (Q6_K) sub-block the same way.
struct Q5Blk {
    uint4 qs;           // D0..D3
    uint32_t qh, d, e;  // D4, d, fit code
};
__device__ __forceinline__ Q5Blk q5_load(const TmqTensorDev& t, int b, int r) {
    const size_t o = (size_t)b * t.rows_pad + r;
    Q5Blk k;
    k.qs = ldw16(t.pa + o * 16);
    k.qh = ldw4(t.pb + o * 4);
    k.d = ldw2(t.pd + o * 2);
    k.e = ldw1(t.pe + o);
    return k;
}
// the 5-bit codes of elements 4g..4g+3 as bytes
__device__ __forceinline__ uint32_t q5_codes(const Q5Blk& k, int g) {
    const uint32_t d0 = k.qs.x, d1 = k.qs.y, d2 = k.qs.z, d3 = k.qs.w, d4 = k.qh;
    switch (g) {
    case 0: return d0 & 0x1f1f1f1fu;
    case 1: return d1 & 0x1f1f1f1fu;
    case 2: return d2 & 0x1f1f1f1fu;
    case 3: return d3 & 0x1f1f1f1fu;
    case 4: return d4 & 0x1f1f1f1fu;
    case 5: return ((d0 >> 5) & 0x07070707u) | ((d1 >> 2) & 0x18181818u);
    case 6: return ((d2 >> 5) & 0x07070707u) | ((d3 >> 2) & 0x18181818u);
    default: return ((d4 >> 5) & 0x07070707u) | ((d1 >> 4) & 0x08080808u) | ((d3 >> 3) & 0x10101010u);
    }
}
// the code of element e (0..31) from the five dwords
__device__ __forceinline__ int q5_code(const uint4& qs, uint32_t d4, int e) {
    const int g = e >> 2, k = e & 3, sh = 8 * k + 5;
    if (e < 20) {
        const uint32_t v = g == 0 ? qs.x : g == 1 ? qs.y : g == 2 ? qs.z : g == 3 ? qs.w : d4;
        return (int)((v >> (8 * k)) & 31u);
    }
    if (e < 24) return (int)(((qs.x >> sh) & 7u) | (((qs.y >> sh) & 3u) << 3));
    if (e < 28) return (int)(((qs.z >> sh) & 7u) | (((qs.w >> sh) & 3u) << 3));
    return (int)(((d4 >> sh) & 7u) | (((qs.y >> (sh + 2)) & 1u) << 3) | (((qs.w >> (sh + 2)) & 1u) << 4));
}
// Fit code byte: bits 0-2 dA+4, bits 3-5 dB+4 (ulps), bit 7 set: no pair
// found, the (sub-)block takes the exact decode.  A = a0 moved by dA ulps;
// B = b0, computed from that A where it depends on it, moved by dB ulps.
__device__ __forceinline__ float fit_mv(float x, int k) { return __int_as_float(__float_as_int(x) + k); }
__device__ __forceinline__ float fit_a(float a0, uint32_t e) { return fit_mv(a0, (int)(e & 7u) - 4); }
__device__ __forceinline__ float fit_b(float b0, uint32_t e) { return fit_mv(b0, (int)((e >> 3) & 7u) - 4); }
template <class AT>
__device__ __forceinline__ void q5_mac_fit(const Q5Blk& k, const AT& A, int b, float inv, int& sh, int& sl) {
    const float a = fit_a(h2f(k.d) * inv, k.e);
    const float a24 = a * 0x1p24f, bb = fit_b(-16.0f * a, k.e);
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t U = q5_codes(k, g);
        const tmq_h2 l0 = lanes01(U), l1 = lanes23(U);
        mac4r(fit_rne(__builtin_fmaf((float)l0.x, a24, bb)), fit_rne(__builtin_fmaf((float)l0.y, a24, bb)),
              fit_rne(__builtin_fmaf((float)l1.x, a24, bb)), fit_rne(__builtin_fmaf((float)l1.y, a24, bb)), A,
              b * 16 + 2 * g, sh, sl);
    }
}
// a fitted block summed straight into int64 (v_mad_i64_i32 per weight, the
// activation as int32 through the scalar cache; x holds elements 32b..32b+31)
__device__ __forceinline__ void q5_fit64(const Q5Blk& k, const int32_t (&x)[32], float inv, int64_t& acc0,
                                         int64_t& acc1) {
    const float a = fit_a(h2f(k.d) * inv, k.e);
    const float a24 = a * 0x1p24f, bb = fit_b(-16.0f * a, k.e);
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t U = q5_codes(k, g);
        const tmq_h2 l0 = lanes01(U), l1 = lanes23(U);
        int64_t& c = (g & 1) ? acc1 : acc0;
        c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)l0.x, a24, bb))) * x[4 * g];
        c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)l0.y, a24, bb))) * x[4 * g + 1];
        c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)l1.x, a24, bb))) * x[4 * g + 2];
        c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)l1.y, a24, bb))) * x[4 * g + 3];
    }
    // every term carried kFitM: take kFitM * sum(x) off (a wave-uniform sum)
    int32_t xs = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) xs += x[i];
    acc1 -= (int64_t)kFitM * xs;
}
template <bool CLAMP, class AT>
__device__ __forceinline__ void q5_mac_exact(const Q5Blk& k, const AT& A, int b, float inv, int& sh, int& sl) {
    const float d = h2f(k.d);
    const float c = -1040.0f * d;  // exact: 7-bit x 11-bit
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t U = q5_codes(k, g);
        const tmq_h2 v0 = __builtin_bit_cast(tmq_h2, __builtin_amdgcn_perm(0x64646464u, U, 0x04010400u));
        const tmq_h2 v1 = __builtin_bit_cast(tmq_h2, __builtin_amdgcn_perm(0x64646464u, U, 0x04030402u));
        mac4<CLAMP>(__builtin_fmaf((float)v0.x, d, c), __builtin_fmaf((float)v0.y, d, c),
                    __builtin_fmaf((float)v1.x, d, c), __builtin_fmaf((float)v1.y, d, c), inv, A,
                    b * 16 + 2 * g, sh, sl);
    }
}
// Fitted blocks take the two-instruction decode, the others (and every
// block of a clamped tensor) the exact one.  The block's activation pairs
// are read before the branch.
template <bool CLAMP, class AT>
__device__ __forceinline__ void q5_mac(const Q5Blk& k, const AT& A, int b, float inv, int& sh, int& sl) {
    if constexpr (CLAMP) {
        q5_mac_exact<CLAMP>(k, A, b, inv, sh, sl);
    } else if constexpr (AT::kSink) {
        if (!(k.e & 0x80u)) q5_mac_fit(k, A, b, inv, sh, sl);
        else q5_mac_exact<CLAMP>(k, A, b, inv, sh, sl);
    } else {
        const ActN<16> X = act_n<16>(A, b * 16);
        if (!(k.e & 0x80u)) q5_mac_fit(k, X, 0, inv, sh, sl);
        else q5_mac_exact<CLAMP>(k, X, 0, inv, sh, sl);
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
struct Q4KBlk {
    uint4 h;
    uint4 qs[8];
    uint2 e;  // fit codes of the 8 sub-blocks
};
__device__ __forceinline__ Q4KBlk q4k_load(const TmqTensorDev& t, int b, int r) {
    const size_t R = t.rows_pad;
    Q4KBlk k;
    k.h = ld16(t.pb + p16(b, 0, 1, R, r));
#pragma unroll
    for (int i = 0; i < 8; i++) k.qs[i] = ld16(t.pa + p16(b, i, 8, R, r));
    k.e.x = ld4(t.pe + ((size_t)b * R + r) * 8);
    k.e.y = ld4(t.pe + ((size_t)b * R + r) * 8 + 4);
    return k;
}
// sub-block s = 2sp + hi of a quarter fitted: A = (d*sc)*row_inv and
// B = -(dmin*m)*row_inv, both moved by its code; the high
// nibbles sit in their lanes as 16u*2^-24, hence A*2^20.  Pair kx of
// dwords (hf, i) is kx0 + 8hf + 2i (+1).
template <class AT>
__device__ __forceinline__ void q4k_sub_fit(float Ad, float Bm, uint32_t e, const uint4& qsa, const uint4& qsb, int hi,
                                            const AT& A, int kx0, float inv, int& sh, int& sl) {
    const float a = fit_a(Ad * inv, e) * (hi ? 0x1p20f : 0x1p24f), bb = fit_b(-Bm * inv, e);
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        const uint4& qs = hf ? qsb : qsa;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = dw_of(qs, i) & (hi ? 0xf0f0f0f0u : 0x0f0f0f0fu);
            const tmq_h2 l0 = lanes01(w), l1 = lanes23(w);
            mac4r(fit_rne(__builtin_fmaf((float)l0.x, a, bb)), fit_rne(__builtin_fmaf((float)l0.y, a, bb)),
                  fit_rne(__builtin_fmaf((float)l1.x, a, bb)), fit_rne(__builtin_fmaf((float)l1.y, a, bb)), A,
                  kx0 + 8 * hf + 2 * i, sh, sl);
        }
    }
}
// the same sub-block fitted, summed into int64 against the int32
// activation x of its 32 elements (element 16hf + 4i + k: byte k of dword i
// of qs[hf])
__device__ __forceinline__ void q4k_sub_fit64(float Ad, float Bm, uint32_t e, const uint4& qsa, const uint4& qsb,
                                              int hi, const int32_t (&x)[32], float inv, int64_t& acc0,
                                              int64_t& acc1) {
    const float a = fit_a(Ad * inv, e) * (hi ? 0x1p20f : 0x1p24f), bb = fit_b(-Bm * inv, e);
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        const uint4& qs = hf ? qsb : qsa;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = dw_of(qs, i) & (hi ? 0xf0f0f0f0u : 0x0f0f0f0fu);
            const tmq_h2 l0 = lanes01(w), l1 = lanes23(w);
            const int o = 16 * hf + 4 * i;
            int64_t& c = (i & 1) ? acc1 : acc0;
            c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)l0.x, a, bb))) * x[o];
            c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)l0.y, a, bb))) * x[o + 1];
            c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)l1.x, a, bb))) * x[o + 2];
            c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)l1.y, a, bb))) * x[o + 3];
        }
    }
    int32_t xs = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) xs += x[i];
    acc1 -= (int64_t)kFitM * xs;
}
// the same sub-block, exact: E = fma_mix(lane, Ad*2^24 or Ad*2^20, -Bm)
template <bool CLAMP, class AT>
__device__ __forceinline__ void q4k_sub_exact(float Ad, float Bm, const uint4& qsa, const uint4& qsb, int hi,
                                              const AT& A, int kx0, float inv, int& sh, int& sl) {
    const float a = Ad * (hi ? 0x1p20f : 0x1p24f), nb = -Bm;
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        const uint4& qs = hf ? qsb : qsa;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = dw_of(qs, i) & (hi ? 0xf0f0f0f0u : 0x0f0f0f0fu);
            const tmq_h2 l0 = lanes01(w), l1 = lanes23(w);
            mac4<CLAMP>(__builtin_fmaf((float)l0.x, a, nb), __builtin_fmaf((float)l0.y, a, nb),
                        __builtin_fmaf((float)l1.x, a, nb), __builtin_fmaf((float)l1.y, a, nb), inv, A,
                        kx0 + 8 * hf + 2 * i, sh, sl);
        }
    }
}
// one quarter (sub-blocks 2sp, 2sp+1: 64 weights, pairs 128b + 32sp + 0..31;
// the low nibbles are sub-block 2sp, pairs 0..15 of the quarter)
template <bool CLAMP, class AT>
__device__ __forceinline__ void q4k_mac_q(const uint4& h, const uint4& qsa, const uint4& qsb, uint32_t e2, const AT& A,
                                          int b, int sp, float inv, int& sh, int& sl) {
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
#pragma unroll
    for (int hi = 0; hi < 2; hi++) {
        int sc, m;
        q4k_scale_min(h, 2 * sp + hi, sc, m);
        const float Ad = d * (float)sc, Bm = dmin * (float)m;
        const uint32_t e = (e2 >> (8 * hi)) & 0xffu;
        const int kx = 128 * b + 32 * sp + 16 * hi;
        if constexpr (CLAMP) {
            q4k_sub_exact<CLAMP>(Ad, Bm, qsa, qsb, hi, A, kx, inv, sh, sl);
        } else if constexpr (AT::kSink) {
            if (!(e & 0x80u)) q4k_sub_fit(Ad, Bm, e, qsa, qsb, hi, A, kx, inv, sh, sl);
            else q4k_sub_exact<CLAMP>(Ad, Bm, qsa, qsb, hi, A, kx, inv, sh, sl);
        } else {
            const ActN<16> X = act_n<16>(A, kx);
            if (!(e & 0x80u)) q4k_sub_fit(Ad, Bm, e, qsa, qsb, hi, X, 0, inv, sh, sl);
            else q4k_sub_exact<CLAMP>(Ad, Bm, qsa, qsb, hi, X, 0, inv, sh, sl);
        }
    }
}
template <bool CLAMP, class AT>
__device__ __forceinline__ void q4k_mac(const Q4KBlk& k, const AT& A, int b, float inv, int& sh, int& sl) {
#pragma unroll
    for (int sp = 0; sp < 4; sp++)
        q4k_mac_q<CLAMP>(k.h, k.qs[2 * sp], k.qs[2 * sp + 1], ((sp < 2 ? k.e.x : k.e.y) >> (16 * (sp & 1))) & 0xffffu,
                         A, b, sp, inv, sh, sl);
}

// ---------------------------------------------------------------- Q6_K
// u6 = ql nibble | (qh 2 bits) << 4, built four at a time in byte lanes;
// E = S*(u-32) exactly (S = d*sc has <= 18 significant bits, u-32 <= 6).
struct Q6KBlk {
    uint4 ql[8];
    uint4 qh[4];
    uint4 sc;
    uint4 e;  // fit codes of the 16 sub-blocks (byte j: scale j)
    uint32_t d;
};
__device__ __forceinline__ Q6KBlk q6k_load(const TmqTensorDev& t, int b, int r) {
    const size_t R = t.rows_pad;
    Q6KBlk k;
#pragma unroll
    for (int i = 0; i < 8; i++) k.ql[i] = ld16(t.pa + p16(b, i, 8, R, r));
#pragma unroll
    for (int i = 0; i < 4; i++) k.qh[i] = ld16(t.pb + p16(b, i, 4, R, r));
    k.sc = ld16(t.pc + p16(b, 0, 1, R, r));
    k.e = ld16(t.pe + ((size_t)b * R + r) * 16);
    k.d = ld2(t.pd + ((size_t)b * R + r) * 2);
    return k;
}
// the four 6-bit codes of quarter (half, lc), sub-block sub, dword i
__device__ __forceinline__ uint32_t q6_codes(const uint4& qla, const uint4& qlb, const uint4& qhc, int sub, int i) {
    const uint32_t ql = dw_of((sub & 1) ? qlb : qla, i), qh = dw_of(qhc, i);
    const uint32_t nib = (sub < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
    const uint32_t hs = (sub == 0) ? (qh << 4) : (sub == 1) ? (qh << 2) : (sub == 2) ? qh : (qh >> 2);
    return (hs & 0x30303030u) | nib;
}
// sub-block sub of quarter (half, lc) of a Q6_K block (16 weights, scale S);
// pair kx of dword i is kx0 + 2i (+1)
template <bool CLAMP, class AT>
__device__ __forceinline__ void q6k_sub_exact(float S, const uint4& qla, const uint4& qlb, const uint4& qhc, int sub,
                                              const AT& A, int kx0, float inv, int& sh, int& sl) {
    const float nS = -32.0f * S, S24 = S * 0x1p24f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // E = S*(u-32) = fma_mix(u*2^-24, S*2^24, -32*S), exact
        const tmq_h2 u0 = lanes01(q6_codes(qla, qlb, qhc, sub, i)), u1 = lanes23(q6_codes(qla, qlb, qhc, sub, i));
        mac4<CLAMP>(__builtin_fmaf((float)u0.x, S24, nS), __builtin_fmaf((float)u0.y, S24, nS),
                    __builtin_fmaf((float)u1.x, S24, nS), __builtin_fmaf((float)u1.y, S24, nS), inv, A, kx0 + 2 * i,
                    sh, sl);
    }
}
// the same sub-block fitted: A = S*row_inv and B = -32A, both moved by
// its code byte
template <class AT>
__device__ __forceinline__ void q6k_sub_fit(float S, uint32_t e, const uint4& qla, const uint4& qlb, const uint4& qhc,
                                            int sub, const AT& A, int kx0, float inv, int& sh, int& sl) {
    const float a = fit_a(S * inv, e);
    const float a24 = a * 0x1p24f, bb = fit_b(-32.0f * a, e);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t U = q6_codes(qla, qlb, qhc, sub, i);
        const tmq_h2 u0 = lanes01(U), u1 = lanes23(U);
        mac4r(fit_rne(__builtin_fmaf((float)u0.x, a24, bb)), fit_rne(__builtin_fmaf((float)u0.y, a24, bb)),
              fit_rne(__builtin_fmaf((float)u1.x, a24, bb)), fit_rne(__builtin_fmaf((float)u1.y, a24, bb)), A,
              kx0 + 2 * i, sh, sl);
    }
}
// the same sub-block fitted, summed into int64 against the int32 activation
// x of its 16 elements (element 4i + k: byte k of code dword i)
__device__ __forceinline__ void q6k_sub_fit64(float S, uint32_t e, const uint4& qla, const uint4& qlb,
                                              const uint4& qhc, int sub, const int32_t (&x)[16], float inv,
                                              int64_t& acc0, int64_t& acc1) {
    const float a = fit_a(S * inv, e);
    const float a24 = a * 0x1p24f, bb = fit_b(-32.0f * a, e);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t U = q6_codes(qla, qlb, qhc, sub, i);
        const tmq_h2 u0 = lanes01(U), u1 = lanes23(U);
        int64_t& c = (i & 1) ? acc1 : acc0;
        c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)u0.x, a24, bb))) * x[4 * i];
        c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)u0.y, a24, bb))) * x[4 * i + 1];
        c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)u1.x, a24, bb))) * x[4 * i + 2];
        c += (int64_t)fit_biased(fit_rne(__builtin_fmaf((float)u1.y, a24, bb))) * x[4 * i + 3];
    }
    int32_t xs = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) xs += x[i];
    acc1 -= (int64_t)kFitM * xs;
}
// one quarter (half, lc: 64 weights) of a Q6_K block: sub-blocks
// j = half*8 + lc + 2*sub, pairs 128b + 64half + 8lc + 16sub + 0..7
template <bool CLAMP, class AT>
__device__ __forceinline__ void q6k_mac_q(const uint4& sc, const uint4& e, float ss, const uint4& qla,
                                          const uint4& qlb, const uint4& qhc, const AT& A, int b, int half, int lc,
                                          float inv, int& sh, int& sl) {
#pragma unroll
    for (int sub = 0; sub < 4; sub++) {
        const int j = half * 8 + lc + 2 * sub, kx = 128 * b + 64 * half + 8 * lc + 16 * sub;
        const float S = ss * (float)(int8_t)byte_of(sc, j);
        const uint32_t ej = byte_of(e, j);
        if constexpr (CLAMP) {
            q6k_sub_exact<CLAMP>(S, qla, qlb, qhc, sub, A, kx, inv, sh, sl);
        } else if constexpr (AT::kSink) {
            if (!(ej & 0x80u)) q6k_sub_fit(S, ej, qla, qlb, qhc, sub, A, kx, inv, sh, sl);
            else q6k_sub_exact<CLAMP>(S, qla, qlb, qhc, sub, A, kx, inv, sh, sl);
        } else {
            const ActN<8> X = act_n<8>(A, kx);
            if (!(ej & 0x80u)) q6k_sub_fit(S, ej, qla, qlb, qhc, sub, X, 0, inv, sh, sl);
            else q6k_sub_exact<CLAMP>(S, qla, qlb, qhc, sub, X, 0, inv, sh, sl);
        }
    }
}
template <bool CLAMP, class AT>
__device__ __forceinline__ void q6k_mac(const Q6KBlk& k, const AT& A, int b, float inv, int& sh, int& sl) {
    const float ss = h2f(k.d);
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
        for (int lc = 0; lc < 2; lc++)
            q6k_mac_q<CLAMP>(k.sc, k.e, ss, k.ql[half * 4 + lc], k.ql[half * 4 + 2 + lc], k.qh[half * 2 + lc], A, b,
                             half, lc, inv, sh, sl);
}

// Quarter-block units (64 weights) of the K-quants, for the engine's K split.
struct Q4KQ {
    uint4 h, qa, qb;
    uint32_t e;  // fit codes of sub-blocks 2q, 2q+1
};
__device__ __forceinline__ Q4KQ q4kq_load(const TmqTensorDev& t, int b, int q, int r) {
    const size_t R = t.rows_pad;
    Q4KQ k;
    k.h = ldw16(t.pb + p16(b, 0, 1, R, r));
    k.qa = ldw16(t.pa + p16(b, 2 * q, 8, R, r));
    k.qb = ldw16(t.pa + p16(b, 2 * q + 1, 8, R, r));
    k.e = ldw2(t.pe + ((size_t)b * R + r) * 8 + 2 * q);
    return k;
}
struct Q6KQ {
    uint4 qla, qlb, qhc, sc, e;
    uint32_t d;
};
__device__ __forceinline__ Q6KQ q6kq_load(const TmqTensorDev& t, int b, int q, int r) {
    const size_t R = t.rows_pad;
    const int half = q >> 1, lc = q & 1;
    Q6KQ k;
    k.qla = ldw16(t.pa + p16(b, half * 4 + lc, 8, R, r));
    k.qlb = ldw16(t.pa + p16(b, half * 4 + 2 + lc, 8, R, r));
    k.qhc = ldw16(t.pb + p16(b, half * 2 + lc, 4, R, r));
    k.sc = ldw16(t.pc + p16(b, 0, 1, R, r));
    k.e = ldw16(t.pe + ((size_t)b * R + r) * 16);
    k.d = ldw2(t.pd + ((size_t)b * R + r) * 2);
    return k;
}

// format dispatch for the K-split group code
template <int FMT> struct BlkOf;
template <> struct BlkOf<kQ5_0> { typedef Q5Blk T; };
template <> struct BlkOf<kQ4_K> { typedef Q4KBlk T; };
template <> struct BlkOf<kQ6_K> { typedef Q6KBlk T; };
template <int FMT>
__device__ __forceinline__ typename BlkOf<FMT>::T blk_load(const TmqTensorDev& t, int b, int r) {
    if constexpr (FMT == kQ5_0) return q5_load(t, b, r);
    else if constexpr (FMT == kQ4_K) return q4k_load(t, b, r);
    else return q6k_load(t, b, r);
}
template <int FMT, bool CLAMP, class AT>
__device__ __forceinline__ void blk_mac(const typename BlkOf<FMT>::T& k, const AT& A, int b, float inv,
                                        int& sh, int& sl) {
    if constexpr (FMT == kQ5_0) q5_mac<CLAMP>(k, A, b, inv, sh, sl);
    else if constexpr (FMT == kQ4_K) q4k_mac<CLAMP>(k, A, b, inv, sh, sl);
    else q6k_mac<CLAMP>(k, A, b, inv, sh, sl);
}

// Work unit u of a row: Q5_0 block u, or K-quant quarter block (u >> 2, u & 3).
template <int FMT> struct UnitOf;
template <> struct UnitOf<kQ5_0> { typedef Q5Blk T; static constexpr int per_block = 1; };
template <> struct UnitOf<kQ4_K> { typedef Q4KQ T; static constexpr int per_block = 4; };
template <> struct UnitOf<kQ6_K> { typedef Q6KQ T; static constexpr int per_block = 4; };
template <int FMT>
__device__ __forceinline__ typename UnitOf<FMT>::T unit_load(const TmqTensorDev& t, int u, int r) {
    if constexpr (FMT == kQ5_0) return q5_load(t, u, r);
    else if constexpr (FMT == kQ4_K) return q4kq_load(t, u >> 2, u & 3, r);
    else return q6kq_load(t, u >> 2, u & 3, r);
}
template <int FMT, bool CLAMP = false, class AT>
__device__ __forceinline__ void unit_mac(const typename UnitOf<FMT>::T& k, const AT& A, int u, float inv,
                                         int& sh, int& sl) {
    if constexpr (FMT == kQ5_0) q5_mac<CLAMP>(k, A, u, inv, sh, sl);
    else if constexpr (FMT == kQ4_K) q4k_mac_q<CLAMP>(k.h, k.qa, k.qb, k.e, A, u >> 2, u & 3, inv, sh, sl);
    else q6k_mac_q<CLAMP>(k.sc, k.e, h2f(k.d), k.qla, k.qlb, k.qhc, A, u >> 2, (u & 3) >> 1, u & 1, inv, sh, sl);
}

// A quarter unit with fitted sub-blocks summed into int64 (against the
// int32 activation of the scalar-cache view) and the others exact.
template <int FMT>
__device__ __forceinline__ void unit_mac64(const typename UnitOf<FMT>::T& k, const Act& A, int u, float inv,
                                           int64_t& acc0, int64_t& acc1) {
    const int b = u >> 2, q = u & 3;
    if constexpr (FMT == kQ4_K) {
        const float d = h2f(k.h.x), dmin = h2f(k.h.x >> 16);
#pragma unroll
        for (int hi = 0; hi < 2; hi++) {
            int sc, m;
            q4k_scale_min(k.h, 2 * q + hi, sc, m);
            const float Ad = d * (float)sc, Bm = dmin * (float)m;
            const uint32_t e = (k.e >> (8 * hi)) & 0xffu;
            const int e0 = 256 * b + 64 * q + 32 * hi;
            int32_t x[32];
#pragma unroll
            for (int j = 0; j < 32; j++) x[j] = (int32_t)A.x32[e0 + j];
            if (!(e & 0x80u)) {
                q4k_sub_fit64(Ad, Bm, e, k.qa, k.qb, hi, x, inv, acc0, acc1);
            } else {
                int sh = 0, sl = 0;
                q4k_sub_exact<false>(Ad, Bm, k.qa, k.qb, hi, A, 128 * b + 32 * q + 16 * hi, inv, sh, sl);
                acc0 += (int64_t)sh * 256 + sl;
            }
        }
    } else {
        const int half = q >> 1, lc = q & 1;
        const float ss = h2f(k.d);
#pragma unroll
        for (int sub = 0; sub < 4; sub++) {
            const int j = half * 8 + lc + 2 * sub;
            const float S = ss * (float)(int8_t)byte_of(k.sc, j);
            const uint32_t ej = byte_of(k.e, j);
            const int e0 = 256 * b + 128 * half + 32 * sub + 16 * lc;
            int32_t x[16];
#pragma unroll
            for (int jj = 0; jj < 16; jj++) x[jj] = (int32_t)A.x32[e0 + jj];
            if (!(ej & 0x80u)) {
                q6k_sub_fit64(S, ej, k.qla, k.qlb, k.qhc, sub, x, inv, acc0, acc1);
            } else {
                int sh = 0, sl = 0;
                q6k_sub_exact<false>(S, k.qla, k.qlb, k.qhc, sub, A, 128 * b + 64 * half + 8 * lc + 16 * sub, inv,
                                     sh, sl);
                acc0 += (int64_t)sh * 256 + sl;
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
    k.v0 = ldw16(t.pa + p16(b, 0, 2, R, r));
    k.v1 = ldw16(t.pa + p16(b, 1, 2, R, r));
    k.d = ldw2(t.pd + ((size_t)b * R + r) * 2);
    return k;
}
template <class AT>
__device__ __forceinline__ void q8_mac(const Q8Blk& k, const AT& A, int b, float ri, int& sh, int& sl) {
    const int cs = (int)q8_cs(h2f(k.d), ri);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint4& v = (j < 8) ? k.v0 : k.v1;
        const int p0 = (int)(int8_t)byte_of(v, (2 * j) & 15) * cs;
        const int p1 = (int)(int8_t)byte_of(v, (2 * j + 1) & 15) * cs;
        const uint32_t P = __builtin_amdgcn_perm((uint32_t)p1, (uint32_t)p0, 0x06050201u);
        if constexpr (AT::kSink) {
            A.put(b * 16 + j, P);
        } else {
            sh = dot2(P, A.xh[b * 16 + j], sh);
            sl = dot2(P, A.xl[b * 16 + j], sl);
        }
    }
}

// ------------------------------------------------------------ row groups
// Output epilogue shared by all formats: bias, then residual (TmqWork).
__device__ __forceinline__ void store_y(const TmqWork& w, int r, float v) {
    if (w.bias) v = v + w.bias[r];
    if (w.resid) v = w.y[r] + v;
    w.y[r] = v;
}

// K-split group (Q5_0 / K-quants): NWV waves (gemv_waves) share 64 rows,
// wave w takes blocks w, w+NWV, ...; the int32 pair sums are folded into int64 every 256
// weights at most (|sum| < 2^31), then the waves meet in LDS.
template <int FMT, bool CLAMP>
__device__ __forceinline__ void group_ksplit(const TmqWork& w, int g) {
    constexpr int NWV = gemv_waves(FMT);
    __shared__ int64_t part[NWV][64];
    const TmqTensorDev& t = w.t;
    const int b0 = 0, b1 = t.nb;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    const float inv = t.row_inv[r];
    const Act A = act_view(w.act);
    int64_t acc = 0;
    if constexpr (FMT == kQ5_0) {
        // two blocks per step, the next step's two in flight (indices
        // clamped into the row, so every load is unconditional)
        constexpr int S = NWV;
        if (b1 - b0 == 7 * S) {
            // 896 columns (7 blocks per wave): every load of the wave is
            // issued at once, the blocks are multiplied as they arrive
            Q5Blk kk[7];
#pragma unroll
            for (int i = 0; i < 7; i++) kk[i] = q5_load(t, b0 + wave + S * i, r);
            if constexpr (CLAMP) {
                int sh = 0, sl = 0;
#pragma unroll
                for (int i = 0; i < 7; i++) {
                    q5_mac<CLAMP>(kk[i], A, b0 + wave + S * i, inv, sh, sl);
                    if (i & 1 || i == 6) {
                        acc += (int64_t)sh * 256 + sl;
                        sh = sl = 0;
                    }
                }
            } else {
                // fitted blocks into int64 directly, the others exact
                int64_t acc1 = 0;
#pragma unroll
                for (int i = 0; i < 7; i++) {
                    const int b = b0 + wave + S * i;
                    int32_t x[32];
#pragma unroll
                    for (int j = 0; j < 32; j++) x[j] = (int32_t)A.x32[32 * b + j];
                    if (!(kk[i].e & 0x80u)) {
                        q5_fit64(kk[i], x, inv, acc, acc1);
                    } else {
                        int sh = 0, sl = 0;
                        q5_mac_exact<CLAMP>(kk[i], A, b, inv, sh, sl);
                        acc += (int64_t)sh * 256 + sl;
                    }
                }
                acc += acc1;
            }
            goto reduce;
        }
        auto ld = [&](int bb) { return q5_load(t, min(bb, b1 - 1), r); };
        auto pair = [&](const Q5Blk& x0, const Q5Blk& x1, int bb) {
            int sh = 0, sl = 0;
            q5_mac<CLAMP>(x0, A, bb, inv, sh, sl);
            if (bb + S < b1) q5_mac<CLAMP>(x1, A, bb + S, inv, sh, sl);
            acc += (int64_t)sh * 256 + sl;
        };
        // two register sets in turn, so that no copy waits on a load
        Q5Blk k0 = ld(b0 + wave), k1 = ld(b0 + wave + S);
        for (int b = b0 + wave; b < b1; b += 4 * S) {
            const Q5Blk n0 = ld(b + 2 * S), n1 = ld(b + 3 * S);
            pair(k0, k1, b);
            if (b + 2 * S >= b1) break;
            k0 = ld(b + 4 * S);
            k1 = ld(b + 5 * S);
            pair(n0, n1, b + 2 * S);
        }
    } else {
        // K-quants in quarter blocks: each wave keeps its next quarter in
        // flight while it multiplies (the row sums are exact integers, so
        // the grouping does not change them)
        typedef typename UnitOf<FMT>::T Unit;
        constexpr int S = NWV;
        const int u1 = b1 * 4;
        int64_t acc1 = 0;
        auto ld = [&](int uu) { return unit_load<FMT>(t, min(uu, u1 - 1), r); };
        auto mac = [&](const Unit& k, int uu) {
            if constexpr (CLAMP) {
                int sh = 0, sl = 0;
                unit_mac<FMT, CLAMP>(k, A, uu, inv, sh, sl);
                acc += (int64_t)sh * 256 + sl;
            } else {
                unit_mac64<FMT>(k, A, uu, inv, acc, acc1);
            }
        };
        // two register sets in turn (clamped, unconditional loads), so that
        // no copy waits on a load
        Unit c0 = ld(b0 * 4 + wave);
        for (int u = b0 * 4 + wave; u < u1; u += 2 * S) {
            const Unit c1 = ld(u + S);
            mac(c0, u);
            if (u + S >= u1) break;
            c0 = ld(u + 2 * S);
            mac(c1, u + S);
        }
        acc += acc1;
    }
reduce:
    part[wave][lane] = acc;
    __syncthreads();
    int64_t tot = 0;
    if (wave == 0)
#pragma unroll
        for (int i = 0; i < NWV; i++) tot += part[i][lane];
    if (wave == 0 && r < t.rows) {
        if (w.acc) w.acc[r] = tot;
        // sim/tmac_gguf.cpp:1303-1305: y = 0.0f; y += (double)acc*x_scale/(double)row_inv
        if (w.y) store_y(w, r, (float)(((double)tot * (double)A.xs) / (double)inv));
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
    if (w.y && r < t.rows) store_y(w, r, y);
}

// 64-row quarter `sub` of row group g, a split group of a chain's last
// round: the four waves take the rows' 64-column tiles w, w + 4, ...; the
// tiles' int64 sums meet in LDS (dynamic, 512 B a tile) and wave 0 folds
// them in tile order as group_q8 does.
__device__ __forceinline__ void group_q8_quarter(const TmqWork& w, int g, int sub) {
    extern __shared__ __attribute__((aligned(16))) uint8_t mfma_lds[];
    int64_t* ps = (int64_t*)mfma_lds;
    const TmqTensorDev& t = w.t;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r0 = (g * TMQ_WAVES + sub) * 64;
    if (r0 >= t.rows_pad) return;  // the same for the whole workgroup
    const int r = r0 + lane;
    const float ri = t.row_inv[r], rs = t.row_scale[r];
    const Act A = act_view(w.act);
    const int nt = (t.cols + 63) / 64;
    for (int tt = wave; tt < nt; tt += TMQ_WAVES) {
        int sh = 0, sl = 0;
        const int b0 = 2 * tt, b1 = 2 * tt + 1;
        const bool has1 = b1 < t.nb;
        const Q8Blk k0 = q8_load(t, b0, r);
        const Q8Blk k1 = has1 ? q8_load(t, b1, r) : k0;
        q8_mac(k0, A, b0, ri, sh, sl);
        if (has1) q8_mac(k1, A, b1, ri, sh, sl);
        const int64_t P = (int64_t)sh * 256 + sl;
        if (w.acc && r < t.rows) w.acc[(size_t)r * nt + tt] = P;
        ps[tt * 64 + lane] = P;
    }
    __syncthreads();
    if (wave != 0) return;
    float y = 0.0f;
    for (int tt = 0; tt < nt; tt++)
        y = (float)((double)y + ((double)ps[tt * 64 + lane] * (double)A.xs) * (double)rs);
    if (w.y && r < t.rows) store_y(w, r, y);
}

// --------------------------------------------- MFMA decoders (Q5_0)
// Integer fit.  Within one block of one row the int16 weight of code u is
// g(u) = clamp16(roundf(fl(E(u) * row_inv))); ifit_kernel picks integers
// AN = 256*alpha + a, BN = 256*beta + bb (0 <= a, bb < 256) with
//     g(u) = floor((AN*u + BN) / 256) = alpha*u + beta + t(u),
//     t(u) = (a*u + bb) >> 8  (0 <= t < 32)
// for every code the block holds, AN and BN being the nominal slope
// trunc(d*row_inv*256) and intercept 128 - 16*AN moved by the fit code
// (plane pi: bits 0-2 dA + 4, bits 3-6 dB + 8).  Blocks it cannot fit keep
// the closest pair and list the differing codes as corrections (TmqCorr).
// t(u) is the high byte of the 16-bit a*u + bb, two codes per v_pk_mad_u16.
//
// The row sums go to v_mfma_i32_32x32x32_i8.  A wave owns 32 rows; lane
// (j, h) = (l & 31, l >> 5) decodes block 2p + h of row j into the code
// bytes U and the t bytes T: as B operands (32 columns = rows, K = the two
// blocks' 16-code halves) they meet an A operand whose rows 4h, 4h+1, 4h+2
// hold, over K half h only, xh, xl - 128 and ones of block 2p + h, so that
// accumulator elements 0, 1, 2 of lane (j, h) are
//     sum u*xh, sum u*(xl-128), sum u     over block 2p + h of row j
// (element v of lane l: A row 8*(v/4) + 4*(l/32) + v%4, B column l & 31).
// With xq = 256*xh + (xl - 128) + 128:
//     sum_k w_k xq_k = alpha * S(u) + S(t) + beta * sum_k xq_k,
//     S(v) = 256*sum v*xh + sum v*(xl-128) + 128*sum v.
// S(u) is read out per block (its alpha differs); S(t) has coefficient 1
// and stays in a second accumulator for the whole row.  Every partial is
// an exact integer: the MFMA sums stay below 2^31, the row sum is int64.
typedef int tmq_v4i __attribute__((ext_vector_type(4)));
typedef int tmq_v16i __attribute__((ext_vector_type(16)));
typedef unsigned short tmq_u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ tmq_v16i mfma_i8(tmq_v4i a, tmq_v4i b, tmq_v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
// two 16-bit lanes x*a + b (v_pk_mad_u16)
__device__ __forceinline__ uint32_t pk_mad_u16(uint32_t x, uint32_t a, uint32_t b) {
    const tmq_u16x2 r = __builtin_bit_cast(tmq_u16x2, x) * __builtin_bit_cast(tmq_u16x2, a) +
                        __builtin_bit_cast(tmq_u16x2, b);
    return __builtin_bit_cast(uint32_t, r);
}

struct IFit {
    int alpha, beta;
    uint32_t a2, b2;  // a and bb in both 16-bit lanes
};
// nominal slope: trunc(d * row_inv * 256), the float held inside +-(2^23 - 8)
// (no real block comes near: |g| <= 32767 bounds it for any code but 16)
__device__ __forceinline__ int ifit_an0(float d, float ri256) {
    return (int)__builtin_amdgcn_fmed3f(d * ri256, -8388600.0f, 8388600.0f);
}
__device__ __forceinline__ IFit ifit_q5(uint32_t dbits, float ri256, uint32_t e) {
    const int AN = ifit_an0(h2f(dbits), ri256) + (int)(e & 7u) - 4;
    const int BN = 120 - 16 * AN + (int)((e >> 3) & 15u);
    IFit f;
    f.alpha = AN >> 8;
    f.beta = BN >> 8;
    f.a2 = ((uint32_t)AN & 255u) * 0x10001u;
    f.b2 = ((uint32_t)BN & 255u) * 0x10001u;
    return f;
}
// the fitted weight of code u (what the MFMA sums amount to)
__device__ __forceinline__ int ifit_w(const IFit& f, int u) {
    return f.alpha * u + f.beta + (int)(((f.a2 & 0xffffu) * (uint32_t)u + (f.b2 & 0xffffu)) >> 8);
}
// t bytes of four code bytes
__device__ __forceinline__ uint32_t ifit_t4(uint32_t U, uint32_t a2, uint32_t b2) {
    const uint32_t PE = pk_mad_u16(U & 0x00ff00ffu, a2, b2);
    const uint32_t PO = pk_mad_u16(__builtin_amdgcn_perm(0u, U, 0x0c030c01u), a2, b2);
    return __builtin_amdgcn_perm(PO, PE, 0x07030501u);
}
// Integer fit of a K-quant sub-block (the same form as IFit): nominal
// slope AN = (int)an with an ~ A*row_inv*256 for the per-code step A (Q4_K
// d*sc, Q6_K d*sc), and the value at the pivot code p (Q4_K 8, Q6_K 32, the
// middle of the codes) BN(p) = (int)bn, bn ~ E(p)*row_inv*256 + 128 (kq_nom:
// any fixed rounding of these serves, the fit code absorbs it); the code
// moves AN by dA = (code & 7) - 4 and the pivot value by dB = (code >> 3) -
// 16, the intercept following from the pivot:
//     BN = BN(p) - p*AN,   g(u) = floor((AN*u + BN) / 256).
// an and bn are held inside +-(2^23 - 8) (|AN*u + BN| < 2^30 for u < 64).
__device__ __forceinline__ IFit kfit(float an, float bn, int p, uint32_t code) {
    const int AN = (int)__builtin_amdgcn_fmed3f(an, -8388600.0f, 8388600.0f) + (int)(code & 7u) - 4;
    const int BN = (int)__builtin_amdgcn_fmed3f(bn, -8388600.0f, 8388600.0f) - p * AN +
                   (int)((code >> 3) & 31u) - 16;
    IFit f;
    f.alpha = AN >> 8;
    f.beta = BN >> 8;
    f.a2 = ((uint32_t)AN & 255u) * 0x10001u;
    f.b2 = ((uint32_t)BN & 255u) * 0x10001u;
    return f;
}

// Nominal fit values of a Q4_K sub-block from dri = d*row_inv*256 and
// mri = dmin*row_inv*256 (per block): an = dri*sc, bn = 8*an - mri*m + 128
// (E(8)*row_inv*256 + 128 up to rounding).  The upload fit and the decoder
// both use this function.
__device__ __forceinline__ void q4k_nomf(float dri, float mri, float sc, float m, float& an, float& bn) {
    an = dri * sc;
    bn = __builtin_fmaf(an, 8.0f, __builtin_fmaf(-mri, m, 128.0f));
}
__device__ __forceinline__ void q4k_nom(float dri, float mri, int sc, int m, float& an, float& bn) {
    q4k_nomf(dri, mri, (float)sc, (float)m, an, bn);
}
template <bool B> struct BoolC {
    static constexpr bool value = B;
};

// block pairs in flight per lane
#ifndef TMQ_MFMA_DEPTH
#define TMQ_MFMA_DEPTH 2
#endif

typedef __attribute__((address_space(3))) const tmq_v4i lv4i;
typedef __attribute__((address_space(3))) const int32_t li32;
typedef __attribute__((address_space(3))) const uint32_t lu32c;
typedef __attribute__((address_space(3))) const uint16_t lu16;
typedef __attribute__((address_space(3))) const uint8_t lu8;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Dynamic LDS of the Q5_0 MFMA decoder (mfma_lds_bytes): per wave a ring of
// TMQ_MFMA_DEPTH stages, each one block of the wave's 64 rows as the LDS DMA
// lays it down (lane l at 16*l of the qs part, 4*l of the others): qs
// 1024 B, qh' 256 B, d 256 B, the fit-code dword (the block's code in byte
// wave) 256 B; then the activation's operand bytes (XA, then runs of zero
// and one bytes), the block sums, the waves' row sums and the 64 rows'
// corrections.
constexpr int kMfmaStage = 1792;
constexpr int kMfmaWaves = gemv_waves(kQ5_0M);
__host__ __device__ constexpr int mfma_xa_off() { return kMfmaWaves * TMQ_MFMA_DEPTH * kMfmaStage; }
// behind the operand bytes: 64 zero bytes, then 64 one bytes
constexpr int kMfmaConst = 128;
__host__ __device__ constexpr int mfma_xs_off(int nb) { return mfma_xa_off() + nb * 64 + kMfmaConst; }
__host__ __device__ constexpr int mfma_part_off(int nb) { return mfma_xs_off(nb) + ((nb * 4 + 15) & ~15); }
__host__ __device__ constexpr int mfma_lds_bytes(int nb) { return mfma_part_off(nb) + (kMfmaWaves + 1) * 64 * 8; }

// raw buffer resource over `bytes` bytes at p (gfx9 word 3: 32-bit data
// format, no stride / swizzle); out-of-range reads return 0
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt vmcnt(n) for the ring (n = loads issued after the awaited stage)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N <= 63, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// s_waitcnt vmcnt(STEP * k) for a wave-uniform k in 0..K
template <int STEP, int K>
__device__ __forceinline__ void wait_vm_k(int k) {
    if constexpr (K == 0) {
        wait_vm<0>();
    } else {
        if (k >= K)
            wait_vm<STEP * K>();
        else
            wait_vm_k<STEP, K - 1>(k);
    }
}

__device__ __forceinline__ tmq_v4i mfma16(tmq_v4i a, tmq_v4i b, tmq_v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// 64 rows (group g), one per lane, the row's blocks split over the waves
// (wave w: blocks w, w + 4, ...; any block count).  v_mfma_i32_16x16x64_i8 sees lane
// l = 16q + n as B column n, K group q (16 codes) and A row n, K group q,
// so lane l's codes of a block pair with A rows 4q .. 4q+2 only where those
// hold the block's xh, xl - 128 and ones for K group q and zero elsewhere;
// accumulator element v of lane l is then A row 4q + v, column n = lane l's
// row: elements 0, 1, 2 are that row's S(u) parts.  Two MFMAs per block
// take codes 0-15 and 16-31 (u), two more the t bytes.  The weights
// stream global -> LDS through each wave's ring (LDS DMA: no registers hold
// data in flight, and each wait is for the oldest stage alone); the
// activation's operand bytes are copied into LDS once per workgroup.
// The int64 sums of rows 64g .. 64g+63 over blocks [b0, b1): the NW waves
// take blocks b0 + wave, b0 + wave + NW, ...  The caller lays out LDS:
// xa / xsl the activation's operand bytes and block sums over the whole row
// (with the constant runs at xa + 64 nb), ring NW * D stages, part (NW + 1)
// * 64 int64.  ready(prime, nbw) must prime the ring (prime()), make xa and
// xsl visible to every wave and leave no vector-memory operation of its own
// outstanding behind the primed stages.  The corrections of the group whose
// elements lie in columns [clo, chi) are added, xq(col) giving their
// activation values.  STATIC_PRIME: the prime issues D stages whatever the
// wave's block count (the surplus ones reload a block the wave or its
// workgroup loads anyway), so that code around it sees a fixed number of
// memory operations.  Returns the row's sum in wave 0 (after a workgroup
// barrier; the other waves' values are meaningless).
template <int NW, bool STATIC_PRIME = false, class Ready, class XQ>
__device__ __forceinline__ int64_t mfma_q5_rows(const TmqTensorDev& t, int g, int b0, int b1, const uint8_t* xa,
                                                const int32_t* xsl, uint8_t* ring0, int64_t* part, int clo, int chi,
                                                Ready&& ready, XQ&& xq) {
    constexpr int D = TMQ_MFMA_DEPTH;
    const int nb = t.nb;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    const int nbw = max(0, (b1 - b0 - wave + NW - 1) / NW);  // this wave's blocks (wave-uniform)
    // corrections of the group (uniform), fetched first
    const bool corr = t.corr_off && chi > clo;
    const int c0 = corr ? t.corr_off[g] : 0, c1 = corr ? t.corr_off[g + 1] : 0;
    const float inv = t.row_inv[r], ri256 = inv * 256.0f;
    int64_t* fix = part + NW * 64;

    uint8_t* ring = ring0 + wave * D * kMfmaStage;
    const size_t R = t.rows_pad;
    // stage `slot` <- the wave's block i, i < nbw (nothing is loaded past
    // the wave's last block: every weight byte is read from memory once;
    // a wave with no block of its own loads nothing).
    // Buffer loads: the planes' base addresses and sizes in scalar resources,
    // the block's element offset (wave-uniform) in a scalar register and
    // the lane's in a constant vector register, so no vector instruction
    // forms an address (the host keeps every plane below 2^31 bytes).
    const uint32_t pl = (uint32_t)(R * (size_t)nb);  // elements per plane
    const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(t.pa, 16 * pl), rsb = buf_rsrc(t.pb, 4 * pl);
    const __amdgpu_buffer_rsrc_t rsd = buf_rsrc(t.pd, 2 * pl), rsi = buf_rsrc(t.pi, 4 * (uint32_t)R * ((nb + 3) / 4));
    const int la16 = lane * 16, la4 = lane * 4, la2 = lane * 2;
    auto issue = [&](int i, int slot) {
        // (i < nbw, but for a static prime's surplus stages: the wave's
        // last block, or the range's first when it has none)
        const int blk = __builtin_amdgcn_readfirstlane(
            i < nbw ? b0 + wave + NW * i : nbw > 0 ? b0 + wave + NW * (nbw - 1) : min(b0, nb - 1));
        const int ob = blk * (int)R + g * 64;
        uint8_t* st = ring + slot * kMfmaStage;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_u8*)st, 16, la16, 16 * ob, 0, TMQ_CPOL_NT);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_u8*)(st + 1024), 4, la4, 4 * ob, 0, TMQ_CPOL_NT);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsd, (lds_u8*)(st + 1280), 2, la2, 2 * ob, 0, TMQ_CPOL_NT);
        // the fit codes of blocks 4j .. 4j+3 of a row in one dword (plane
        // [b/4][r]): the four waves read the same 256 B, each its own byte
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsi, (lds_u8*)(st + 1536), 4, la4, 4 * ((blk >> 2) * (int)R + g * 64),
                                                 0, TMQ_CPOL_NT);
    };
    ready(
        [&] {
#pragma unroll
            for (int i = 0; i < D; i++)
                if (STATIC_PRIME || i < nbw) issue(i, i);
        },
        nbw);

    // this lane's A operand: rows 4q, 4q+1 the block's xh and xl - 128 over
    // K group q, row 4q+2 ones, the rest zero: block b's two halves at
    // abase + b*astride and 32 bytes on (the rows of zeros and ones,
    // astride 0, read both inside their 64-byte constant runs)
    const lds_u8* ap0;
    uint32_t astride;
    {
        const int q = lane >> 4, m = lane & 15, dg = m & 3;
        const bool own = (m >> 2) == q;
        const uint32_t zero = (uint32_t)nb * 64u;
        const uint32_t abase = own && dg < 2 ? (uint32_t)(dg * 16) : own && dg == 2 ? zero + kMfmaConst / 2 : zero;
        astride = own && dg < 2 ? 64u : 0u;
        ap0 = (const lds_u8*)(xa + abase);
    }

    int64_t acc = 0;
    tmq_v4i Ct = {}, Cu = {};
    int ap = 0, bp = 0, xp = 0;  // previous block: alpha, beta, block sum
    const tmq_v4i Z = {};
    // the wave's block i from stage `slot`: decode, read out the previous
    // block's u sums (their MFMAs have long finished), then this block's
    // MFMAs into the same accumulator; the stage is refilled D blocks ahead
    // while that block exists.  FULL: block i + D exists (the stages of
    // blocks i+1 .. i+D-1 are in flight behind this one); otherwise the
    // count of stages behind it is min(D - 1, nbw - 1 - i).
    auto step = [&](int i, int slot, auto fullc) {
        constexpr bool FULL = decltype(fullc)::value;
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (FULL)
            wait_vm<4 * (D - 1)>();
        else
            wait_vm_k<4, D - 1>(min(D - 1, nbw - 1 - i));
        const int b = b0 + wave + NW * i;
        const uint8_t* st = ring + slot * kMfmaStage;
        Q5Blk k;
        {
            const tmq_v4i v = *(lv4i*)(st + lane * 16);
            k.qs = make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
        }
        k.qh = *(lu32c*)(st + 1024 + lane * 4);
        k.d = *(lu16*)(st + 1280 + lane * 4);
        k.e = *(lu8*)(st + 1536 + lane * 4 + (b & 3));
        const lds_u8* xp0 = ap0 + (uint32_t)b * astride;
        const tmq_v4i A0 = *(lv4i*)xp0, A1 = *(lv4i*)(xp0 + 32);
        const int xsv = *(li32*)(xsl + b);
        // the stage's reads are in registers before its refill overwrites it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (FULL || i + D < nbw) issue(i + D, slot);
        const IFit f = ifit_q5(k.d, ri256, k.e);
        uint32_t U[8], T[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            U[e] = q5_codes(k, e);
            T[e] = ifit_t4(U[e], f.a2, f.b2);
        }
        const tmq_v4i U0 = {(int)U[0], (int)U[1], (int)U[2], (int)U[3]};
        const tmq_v4i U1 = {(int)U[4], (int)U[5], (int)U[6], (int)U[7]};
        const tmq_v4i T0 = {(int)T[0], (int)T[1], (int)T[2], (int)T[3]};
        const tmq_v4i T1 = {(int)T[4], (int)T[5], (int)T[6], (int)T[7]};
        acc += (int64_t)ap * (Cu[0] * 256 + Cu[1] + Cu[2] * 128) + (int64_t)bp * xp;
        __builtin_amdgcn_sched_barrier(0);  // the read-out before the overwrite: one accumulator
        Cu = mfma16(A0, U0, Z);
        Cu = mfma16(A1, U1, Cu);
        Ct = mfma16(A0, T0, Ct);
        Ct = mfma16(A1, T1, Ct);
        ap = f.alpha;
        bp = f.beta;
        xp = xsv;
    };
    int ib = 0;
    for (; ib + 2 * D <= nbw; ib += D) {
#pragma unroll
        for (int i = 0; i < D; i++) step(ib + i, i, BoolC<true>{});
    }
#pragma unroll
    for (int i = 0; i < 2 * D - 1; i++)
        if (ib + i < nbw) step(ib + i, i % D, BoolC<false>{});
    acc += (int64_t)ap * (Cu[0] * 256 + Cu[1] + Cu[2] * 128) + (int64_t)bp * xp;
    acc += (int64_t)Ct[0] * 256 + Ct[1] + (int64_t)Ct[2] * 128;
    // no DMA into the ring may still run past this point
    wait_vm<0>();
    part[wave * 64 + lane] = acc;
    if (threadIdx.x < 64) fix[threadIdx.x] = 0;
    __syncthreads();
    if (c1 > c0) {
        // corrections (uniform branch): delta * sum of xq over their elements
        for (int c = c0 + (int)threadIdx.x; c < c1; c += 64 * NW) {
            const uint4 e = t.corr[c];
            // (a correction's elements lie in one block or sub-block)
            if ((int)e.y < clo || (int)e.y >= chi) continue;
            int64_t s = 0;
            for (uint32_t m = e.z; m; m &= m - 1) s += xq((int)e.y + __builtin_ctz(m));
            atomicAdd((unsigned long long*)&fix[(int)e.x - g * 64], (unsigned long long)((int64_t)(int32_t)e.w * s));
        }
        __syncthreads();
    }
    int64_t tot = 0;
    if (wave == 0) {
        tot = fix[lane];
#pragma unroll
        for (int i = 0; i < NW; i++) tot += part[i * 64 + lane];
    }
    return tot;
}

// A standalone / chain row group: the activation's operand bytes copied
// from the prepared activation (global -> LDS), every block of the row.
__device__ __forceinline__ void group_mfma_q5(const TmqWork& w, int g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t mfma_lds[];
    constexpr int NW = kMfmaWaves, D = TMQ_MFMA_DEPTH;
    const TmqTensorDev& t = w.t;
    const int nb = t.nb, n = t.cols;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    uint8_t* xa = mfma_lds + mfma_xa_off();
    int32_t* xsl = (int32_t*)(mfma_lds + mfma_xs_off(nb));
    int64_t* part = (int64_t*)(mfma_lds + mfma_part_off(nb));
    // the finalisation's operands, loaded at the start (not behind the sums)
    const float inv = t.row_inv[r], xsc = *(const float*)w.act;
    auto ready = [&](auto&& prime, int nbw) {
        // the activation copy first (global -> LDS), so that waiting for it
        // does not wait for the ring's stages
        const uint8_t* src = w.act + tmq_act_xa(n);
        const int n16 = nb * 4;
        for (int i0 = wave * 64; i0 < n16; i0 += NW * 64)
            if (i0 + lane < n16)
                __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)(i0 + lane) * 16), (lds_u8*)(xa + i0 * 16),
                                                 16, 0, 0);
        if (wave == NW - 1 && lane < kMfmaConst / 16) {
            const uint32_t v = lane < kMfmaConst / 32 ? 0u : 0x01010101u;
            *(uint4*)(xa + nb * 64 + lane * 16) = make_uint4(v, v, v, v);
        }
        const uint8_t* xs = w.act + tmq_act_xs(n);
        for (int i0 = wave * 64; i0 < nb; i0 += NW * 64)
            if (i0 + lane < nb)
                __builtin_amdgcn_global_load_lds((const void*)(xs + (size_t)(i0 + lane) * 4),
                                                 (lds_u8*)((uint8_t*)xsl + i0 * 4), 4, 0, 0);
        prime();
        // this wave's part of the activation copy (issued before the ring)
        // has landed and the constant bytes are written; the barrier makes
        // every part visible (a plain s_barrier: the workgroup fence of
        // __syncthreads would also wait for the ring's stages)
        wait_vm_k<4, D>(min(nbw, D));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    const int32_t* x32 = (const int32_t*)(w.act + 16 + 6 * (size_t)n);
    const int64_t tot = mfma_q5_rows<NW>(t, g, 0, nb, xa, xsl, mfma_lds, part, 0, n, ready,
                                         [&](int col) { return x32[col]; });
    if (wave == 0 && r < t.rows) {
        if (w.acc) w.acc[r] = tot;
        // sim/tmac_gguf.cpp:1303-1305: y = 0.0f; y += (double)acc*x_scale/(double)row_inv
        if (w.y) store_y(w, r, (float)(((double)tot * (double)xsc) / (double)inv));
    }
}

// --------------------------------------- MFMA decoders (Q4_K, Q6_K)
// The K-quant blocks on the same int8 MFMA form as group_mfma_q5, per
// sub-block (Q4_K 32 weights, Q6_K 16 weights) with its own kfit pair:
//     sum_k w_k xq_k = alpha*S(u) + beta*sum_k xq_k + S(t),
// S(u) read out per sub-block, S(t) summed in one accumulator for the row.
// A workgroup owns 64 rows (one per lane) and splits their quarter blocks
// (64 weights: Q4_K sub-blocks 2q, 2q+1; Q6_K quarter (h, lc) = the four
// 16-weight sub-blocks 128h + 32sub + 16lc + (0..15)) over its 4 waves:
// wave w takes quarters w, w + 4, ..., i.e. quarter w of every super-block,
// so a 4864-column row gives each wave 19.  Each wave streams its quarters
// global -> LDS through a ring of TMQ_MFMA_DEPTH stages (buffer loads with
// scalar offsets; the per-block header / scales / d, which the four waves
// of the workgroup all read, keep the default cache policy).  The LDS DMA
// puts lane l's data at 16*l for 16-byte loads and at 4*l for the 1-, 2-
// and 4-byte ones:
//   Q4_K stage: qs chunks 2q, 2q+1 (1024 B each), header (1024 B), the two
//               fit codes (256 B);
//   Q6_K stage: the quarter's three chunks of the packed code plane
//               (q6_pack_kernel, 1024 B each), the quarter's four sub-block
//               scales (256 B), d (256 B), the four fit codes (256 B).
// The activation's operand bytes, 32- and 16-element sums are copied into
// LDS once per workgroup (the range's part of them for a split group).
constexpr int kKqWaves = 4;
template <int FMT> __host__ __device__ constexpr int kq_stage() { return FMT == kQ4_K ? 3328 : 3840; }
template <int FMT> __host__ __device__ constexpr int kq_ndma() { return FMT == kQ4_K ? 4 : 6; }
template <int FMT> __host__ __device__ constexpr int kq_xa_off() { return kKqWaves * TMQ_MFMA_DEPTH * kq_stage<FMT>(); }
// behind the operand bytes: 256 zero bytes, then 256 one bytes (the A rows
// that hold no activation read there, at the same offsets as the others)
constexpr int kKqConst = 512;
template <int FMT> __host__ __device__ constexpr int kq_xs_off(int nbx) {
    return kq_xa_off<FMT>() + nbx * 64 + kKqConst;
}
template <int FMT> __host__ __device__ constexpr int kq_xs16_off(int nbx) { return kq_xs_off<FMT>(nbx) + ((nbx * 4 + 15) & ~15); }
template <int FMT> __host__ __device__ constexpr int kq_part_off(int nbx) {
    return kq_xs16_off<FMT>(nbx) + (FMT == kQ6_K ? ((nbx * 8 + 15) & ~15) : 0);
}
template <int FMT> __host__ __device__ constexpr int kq_lds_bytes(int nbx) {
    return kq_part_off<FMT>(nbx) + (kKqWaves + 1) * 64 * 8;
}

// The int64 sums of rows 64g .. 64g+63 over super-blocks [b0, b1) (b1 > b0)
// on the K-quant MFMA decoder, with LDS laid out by the caller as for
// mfma_q5_rows (xs16l: Q6_K's 16-element sums; part (NW + 1) * 64 int64;
// ring NW * D stages; xa's constant runs kKqConst bytes at xa + 64 * 8nb)
// and the same ready / corr / xq contract.  Returns the rows' sums in wave 0.
template <int FMT, bool STATIC_PRIME = false, class Ready, class XQ>
__device__ __forceinline__ int64_t mfma_kq_rows(const TmqTensorDev& t, int g, int b0, int b1, const uint8_t* xa,
                                                const int32_t* xsl, const int32_t* xs16l, uint8_t* ring0,
                                                int64_t* part, int clo, int chi, Ready&& ready, XQ&& xq) {
    constexpr int NW = kKqWaves, D = TMQ_MFMA_DEPTH, ST = kq_stage<FMT>(), ND = kq_ndma<FMT>();
    constexpr int NS = FMT == kQ4_K ? 2 : 4;  // sub-blocks per quarter
    const int nb = t.nb, nbx = nb * 8;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    // quarter u = 4b + q of the row; wave w takes quarters u0 + w + NW*i:
    // quarter w of each super-block of the range (NW = 4 = quarters per
    // super-block), b1 - b0 >= 1 of them
    const int u0 = 4 * b0;
    const int nuw = b1 - b0;
    const bool corr = t.corr_off && chi > clo;
    const int c0 = corr ? t.corr_off[g] : 0, c1 = corr ? t.corr_off[g + 1] : 0;
    const float inv = t.row_inv[r], ri256 = inv * 256.0f;
    int64_t* fix = part + NW * 64;

    uint8_t* ring = ring0 + wave * D * ST;
    const int R = t.rows_pad, g64 = g * 64;
    // planes (the host keeps each below 2^31 bytes)
    const uint32_t pb = (uint32_t)R * (uint32_t)nb;  // (row, block) pairs
    const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(t.pa, 128 * pb), rsi = buf_rsrc(t.pi, (FMT == kQ4_K ? 8 : 16) * pb);
    const __amdgpu_buffer_rsrc_t rsb = buf_rsrc(t.pb, (FMT == kQ4_K ? 16 : 64) * pb);
    const __amdgpu_buffer_rsrc_t rsd = buf_rsrc(FMT == kQ6_K ? t.pd : t.pb, 2 * pb);
    const __amdgpu_buffer_rsrc_t rsq = buf_rsrc(FMT == kQ6_K ? t.pq : t.pb, 208 * pb);
    const int l16 = lane * 16;
    // stage `slot` <- the wave's quarter i, i < nuw (nothing is loaded past
    // the wave's last quarter: every weight byte is read from memory once)
    auto issue = [&](int i, int slot) {
        // (i < nuw, but for a static prime's surplus stages: the last
        // quarter, or the row's first super-block's when the range is empty)
        const int u = __builtin_amdgcn_readfirstlane(i < nuw ? u0 + wave + NW * i
                                                     : nuw > 0 ? u0 + wave + NW * (nuw - 1)
                                                               : 4 * min(b0, nb - 1) + wave);
        const int b = u >> 2, q = u & 3;
        uint8_t* st = ring + slot * ST;
        if constexpr (FMT == kQ4_K) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_u8*)st, 16, l16, ((b * 8 + 2 * q) * R + g64) * 16, 0,
                                                     TMQ_CPOL_NT);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_u8*)(st + 1024), 16, l16,
                                                     ((b * 8 + 2 * q + 1) * R + g64) * 16, 0, TMQ_CPOL_NT);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_u8*)(st + 2048), 16, l16, (b * R + g64) * 16, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsi, (lds_u8*)(st + 3072), 2, lane * 2, ((b * 4 + q) * R + g64) * 2,
                                                     0, TMQ_CPOL_NT);
        } else {
            // the quarter's three code chunks of the packed plane
#pragma unroll
            for (int k = 0; k < 3; k++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsq, (lds_u8*)(st + 1024 * k), 16, l16,
                                                         ((b * 12 + 3 * q + k) * R + g64) * 16, 0, TMQ_CPOL_NT);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsq, (lds_u8*)(st + 3072), 4, lane * 4,
                                                     (int)(192 * pb) + ((b * 4 + q) * R + g64) * 4, 0, TMQ_CPOL_NT);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsd, (lds_u8*)(st + 3328), 2, lane * 2, (b * R + g64) * 2, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsi, (lds_u8*)(st + 3584), 4, lane * 4, ((b * 4 + q) * R + g64) * 4,
                                                     0, TMQ_CPOL_NT);
        }
    };
    ready(
        [&] {
#pragma unroll
            for (int i = 0; i < D; i++)
                if (STATIC_PRIME || i < nuw) issue(i, i);
        },
        nuw);

    // this lane's A operand: rows 4q', 4q'+1 the sub-block's xh and
    // xl - 128 over K group q' (lane >> 4), row 4q'+2 ones, the rest zero;
    // the 16 elements of (32-element block xb, half hf) at
    // ((64*xb + 32*hf) & amask) | abase.  A step's blocks lie at
    // immediate offsets 0-192 from its first, which the rows of ones and
    // zeros (amask 0) read inside their 256-byte constant runs.
    // (the offset is a multiple of 32 and abase < 32 where amask is set, so
    // (offset & amask) | abase is one v_and_or)
    uint32_t abase, amask;
    {
        const int qg = lane >> 4, m = lane & 15, dg = m & 3;
        const bool own = (m >> 2) == qg;
        const uint32_t zero = (uint32_t)nbx * 64u;
        abase = own && dg < 2 ? (uint32_t)(dg * 16) : own && dg == 2 ? zero + kKqConst / 2 : zero;
        amask = own && dg < 2 ? 0xffffffffu : 0u;
    }
    auto abase_of = [&](uint32_t off) { return (off & amask) | abase; };

    int64_t acc = 0;
    tmq_v4i Ct = {};
    tmq_v4i Cu[NS];
    int ap[NS], bp[NS], xp[NS];  // the previous quarter's sub-blocks: alpha, beta, activation sum
#pragma unroll
    for (int k = 0; k < NS; k++) {
        Cu[k] = tmq_v4i{};
        ap[k] = bp[k] = xp[k] = 0;
    }
    const tmq_v4i Z = {};
    // Q4_K: a wave's quarter q is the same in every super-block (wave & 3,
    // as NW is 4); its sub-blocks s = 2q + k take their 6-bit scale and min
    // from the header's scale bytes (q4k_scale_min's cases):
    //   q < 2:  sc_k = scales[s] & 63, m_k = scales[4 + s] & 63
    //   q >= 2: s' = s - 4, sc_k = (scales[8 + s'] & 15) | (scales[s'] >> 6) << 4,
    //           m_k = (scales[8 + s'] >> 4) | (scales[4 + s'] >> 6) << 4
    // gathered by v_perm as the bytes (sc_0, sc_1, m_0, m_1) of one dword:
    // bytes s0, s0 + 1 of a header dword and of the next, s0 = 2 * (q & 1)
    static_assert(NW == 4, "the quarter of a wave is wave & 3");
    const int qw = wave & 3;
    const uint32_t hs0 = 2u * (uint32_t)(qw & 1);
    const uint32_t hsel = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(hs0 | (hs0 + 1) << 8 | (hs0 + 4) << 16 | (hs0 + 5) << 24));
    // the loop, compiled per header case (q < 2 or not; Q6_K: one case)
    auto run = [&](auto lo2c) {
        constexpr bool LO2 = decltype(lo2c)::value;
        // FULL: quarter i + D exists (see group_mfma_q5's step)
        auto step = [&](int i, int slot, auto fullc) {
            constexpr bool FULL = decltype(fullc)::value;
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (FULL)
                wait_vm<ND * (D - 1)>();
            else
                wait_vm_k<ND, D - 1>(min(D - 1, nuw - 1 - i));
            const int u = u0 + wave + NW * i, b = u >> 2, q = u & 3;
            const uint8_t* st = ring + slot * ST;
            IFit f[NS];
            tmq_v4i UA[NS][2], TA[NS][2], AA[NS][2];
            int xsv[NS];
            if constexpr (FMT == kQ4_K) {
                const tmq_v4i qa = *(lv4i*)(st + lane * 16), qb = *(lv4i*)(st + 1024 + lane * 16);
                const tmq_v4i hv = *(lv4i*)(st + 2048 + lane * 16);
                const uint32_t codes = *(lu16*)(st + 3072 + lane * 4);
                // sub-block k, half hf: block 8b + 2q + k
                const uint32_t ab = abase_of(64u * (uint32_t)(8 * b + 2 * q));
#pragma unroll
                for (int k = 0; k < NS; k++) {
                    AA[k][0] = *(lv4i*)(xa + ab + 64 * k);
                    AA[k][1] = *(lv4i*)(xa + ab + 64 * k + 32);
                    xsv[k] = xsl[8 * b + 2 * q + k];
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (FULL || i + D < nuw) issue(i + D, slot);
                const uint32_t hx = (uint32_t)hv.x, hy = (uint32_t)hv.y, hz = (uint32_t)hv.z, hw = (uint32_t)hv.w;
                const float dri = h2f(hx) * ri256, mri = h2f(hx >> 16) * ri256;
                uint32_t scm;
                if constexpr (LO2)
                    scm = __builtin_amdgcn_perm(hz, hy, hsel) & 0x3f3f3f3fu;
                else
                    scm = (__builtin_amdgcn_perm(hw >> 4, hw, hsel) & 0x0f0f0f0fu) |
                          ((__builtin_amdgcn_perm(hz, hy, hsel) >> 2) & 0x30303030u);
#pragma unroll
                for (int k = 0; k < NS; k++) {
                    float an, bn;
                    q4k_nomf(dri, mri, (float)((scm >> (8 * k)) & 255u), (float)((scm >> (16 + 8 * k)) & 255u), an,
                             bn);
                    f[k] = kfit(an, bn, 8, (codes >> (8 * k)) & 255u);
                    const tmq_v4i src[2] = {qa, qb};
#pragma unroll
                    for (int hf = 0; hf < 2; hf++) {
                        uint32_t U[4], T[4];
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const uint32_t v = (uint32_t)src[hf][e];
                            U[e] = (k ? (v >> 4) : v) & 0x0f0f0f0fu;
                            T[e] = ifit_t4(U[e], f[k].a2, f[k].b2);
                        }
                        UA[k][hf] = tmq_v4i{(int)U[0], (int)U[1], (int)U[2], (int)U[3]};
                        TA[k][hf] = tmq_v4i{(int)T[0], (int)T[1], (int)T[2], (int)T[3]};
                    }
                }
            } else {
                const int h = q >> 1, lc = q & 1;
                const tmq_v4i va = *(lv4i*)(st + lane * 16), vb = *(lv4i*)(st + 1024 + lane * 16);
                const tmq_v4i vh = *(lv4i*)(st + 2048 + lane * 16);
                const uint32_t scq = *(lu32c*)(st + 3072 + lane * 4);
                const uint32_t dbits = *(lu16*)(st + 3328 + lane * 4);
                const uint32_t codes = *(lu32c*)(st + 3584 + lane * 4);
                // sub-block k: half lc of block 8b + 4h + k
                const uint32_t ab = abase_of(64u * (uint32_t)(8 * b + 4 * h) + 32u * (uint32_t)lc);
#pragma unroll
                for (int k = 0; k < NS; k++) {
                    AA[k][0] = *(lv4i*)(xa + ab + 64 * k);
                    xsv[k] = xs16l[2 * (8 * b + 4 * h + k) + lc];
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (FULL || i + D < nuw) issue(i + D, slot);
                const float ssri = h2f(dbits) * ri256;
#pragma unroll
                for (int k = 0; k < NS; k++) {
                    // scale 8h + lc + 2k: byte k of the quarter's scale dword
                    const int sc = (int)(int8_t)(uint8_t)(scq >> (8 * k));
                    f[k] = kfit(ssri * (float)sc, 128.0f, 32, (codes >> (8 * k)) & 255u);
                    uint32_t U[4], T[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        // sub-blocks 0-2: the low 6 bits of chunk k; sub-block 3:
                        // the top 2 bits of chunks 0, 1, 2 as its bits 0-1, 2-3, 4-5
                        const uint32_t d0 = (uint32_t)va[e], d1 = (uint32_t)vb[e], d2 = (uint32_t)vh[e];
                        U[e] = k == 0   ? d0 & 0x3f3f3f3fu
                               : k == 1 ? d1 & 0x3f3f3f3fu
                               : k == 2 ? d2 & 0x3f3f3f3fu
                                        : ((d0 >> 6) & 0x03030303u) | ((d1 >> 4) & 0x0c0c0c0cu) |
                                              ((d2 >> 2) & 0x30303030u);
                        T[e] = ifit_t4(U[e], f[k].a2, f[k].b2);
                    }
                    UA[k][0] = tmq_v4i{(int)U[0], (int)U[1], (int)U[2], (int)U[3]};
                    TA[k][0] = tmq_v4i{(int)T[0], (int)T[1], (int)T[2], (int)T[3]};
                }
            }
            // the previous quarter's u sums (their MFMAs have long finished)
#pragma unroll
            for (int k = 0; k < NS; k++)
                acc += (int64_t)ap[k] * (Cu[k][0] * 256 + Cu[k][1] + Cu[k][2] * 128) + (int64_t)bp[k] * xp[k];
            __builtin_amdgcn_sched_barrier(0);  // the read-out before the overwrite
#pragma unroll
            for (int k = 0; k < NS; k++) {
                if constexpr (FMT == kQ4_K) {
                    Cu[k] = mfma16(AA[k][0], UA[k][0], Z);
                    Cu[k] = mfma16(AA[k][1], UA[k][1], Cu[k]);
                    Ct = mfma16(AA[k][0], TA[k][0], Ct);
                    Ct = mfma16(AA[k][1], TA[k][1], Ct);
                } else {
                    Cu[k] = mfma16(AA[k][0], UA[k][0], Z);
                    Ct = mfma16(AA[k][0], TA[k][0], Ct);
                }
                ap[k] = f[k].alpha;
                bp[k] = f[k].beta;
                xp[k] = xsv[k];
            }
        };
        int ib = 0;
        for (; ib + 2 * D <= nuw; ib += D) {
#pragma unroll
            for (int i = 0; i < D; i++) step(ib + i, i, BoolC<true>{});
        }
#pragma unroll
        for (int i = 0; i < 2 * D - 1; i++)
            if (ib + i < nuw) step(ib + i, i % D, BoolC<false>{});
    };
    if constexpr (FMT == kQ4_K) {
        if (qw < 2)
            run(BoolC<true>{});
        else
            run(BoolC<false>{});
    } else {
        run(BoolC<true>{});
    }
#pragma unroll
    for (int k = 0; k < NS; k++)
        acc += (int64_t)ap[k] * (Cu[k][0] * 256 + Cu[k][1] + Cu[k][2] * 128) + (int64_t)bp[k] * xp[k];
    acc += (int64_t)Ct[0] * 256 + Ct[1] + (int64_t)Ct[2] * 128;
    // no DMA into the ring may still run past this point
    wait_vm<0>();
    part[wave * 64 + lane] = acc;
    if (threadIdx.x < 64) fix[threadIdx.x] = 0;
    __syncthreads();
    if (c1 > c0) {
        // corrections (uniform branch): delta * sum of xq over their elements
        for (int c = c0 + (int)threadIdx.x; c < c1; c += 64 * NW) {
            const uint4 e = t.corr[c];
            // (a correction's elements lie in one block or sub-block)
            if ((int)e.y < clo || (int)e.y >= chi) continue;
            int64_t s = 0;
            for (uint32_t m = e.z; m; m &= m - 1) s += xq((int)e.y + __builtin_ctz(m));
            atomicAdd((unsigned long long*)&fix[(int)e.x - g * 64], (unsigned long long)((int64_t)(int32_t)e.w * s));
        }
        __syncthreads();
    }
    int64_t tot = 0;
    if (wave == 0) {
        tot = fix[lane];
#pragma unroll
        for (int i = 0; i < NW; i++) tot += part[i * 64 + lane];
    }
    return tot;
}

// A standalone / chain row group over super-blocks [b0, b1).  pieces > 1:
// one of the workgroups sharing the group, which meet in tail slot `slot`
// (a TmqGroupRef split; each piece adds the corrections of its columns).
template <int FMT>
__device__ __forceinline__ void group_mfma_kq(const TmqWork& w, int g, int b0, int b1, int slot, int pieces,
                                              uint64_t* tail) {
    extern __shared__ __attribute__((aligned(16))) uint8_t mfma_lds[];
    constexpr int NW = kKqWaves, D = TMQ_MFMA_DEPTH, ND = kq_ndma<FMT>();
    const TmqTensorDev& t = w.t;
    const int nb = t.nb, nbx = nb * 8, n = t.cols;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    uint8_t* xa = mfma_lds + kq_xa_off<FMT>();
    int32_t* xsl = (int32_t*)(mfma_lds + kq_xs_off<FMT>(nbx));
    int32_t* xs16l = (int32_t*)(mfma_lds + kq_xs16_off<FMT>(nbx));
    int64_t* part = (int64_t*)(mfma_lds + kq_part_off<FMT>(nbx));
    // the finalisation's operands, loaded at the start (not behind the sums)
    const float inv = t.row_inv[r], xsc = *(const float*)w.act;
    auto ready = [&](auto&& prime, int nuw) {
        // the activation copy first (global -> LDS), so that waiting for it
        // does not wait for the ring's stages: the range's 16-byte chunks
        // (32 a super-block) and block sums, at their offsets in the whole
        // row, and the runs of zeros and ones behind the row
        const uint8_t* src = w.act + tmq_act_xa(n);
        const int a0 = 32 * b0, a1 = 32 * b1;
        for (int i0 = a0 + wave * 64; i0 < a1; i0 += NW * 64)
            if (i0 + lane < a1)
                __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)(i0 + lane) * 16), (lds_u8*)(xa + i0 * 16),
                                                 16, 0, 0);
        if (wave == NW - 1 && lane < kKqConst / 16) {
            const uint32_t v = lane < kKqConst / 32 ? 0u : 0x01010101u;
            *(uint4*)(xa + nbx * 64 + lane * 16) = make_uint4(v, v, v, v);
        }
        const uint8_t* xs = w.act + tmq_act_xs(n);
        const int s0 = 8 * b0, s1 = 8 * b1;
        for (int i0 = s0 + wave * 64; i0 < s1; i0 += NW * 64)
            if (i0 + lane < s1)
                __builtin_amdgcn_global_load_lds((const void*)(xs + (size_t)(i0 + lane) * 4),
                                                 (lds_u8*)((uint8_t*)xsl + i0 * 4), 4, 0, 0);
        if constexpr (FMT == kQ6_K) {
            const uint8_t* x16 = w.act + tmq_act_xs16(n);
            for (int i0 = 2 * s0 + wave * 64; i0 < 2 * s1; i0 += NW * 64)
                if (i0 + lane < 2 * s1)
                    __builtin_amdgcn_global_load_lds((const void*)(x16 + (size_t)(i0 + lane) * 4),
                                                     (lds_u8*)((uint8_t*)xs16l + i0 * 4), 4, 0, 0);
        }
        prime();
        // this wave's part of the activation copy (issued before the ring)
        // has landed and the constant bytes are written; the barrier makes
        // every part visible (a plain s_barrier: the workgroup fence of
        // __syncthreads would also wait for the ring's stages)
        wait_vm_k<ND, D>(min(nuw, D));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    const int32_t* x32 = (const int32_t*)(w.act + 16 + 6 * (size_t)n);
    int64_t tot = mfma_kq_rows<FMT>(t, g, b0, b1, xa, xsl, xs16l, mfma_lds, part, 256 * b0, 256 * b1, ready,
                                    [&](int col) { return x32[col]; });
    if (wave != 0) return;
    if (pieces > 1) {
        // The pieces' row sums meet through device-scope atomics, which
        // every XCD performs at the same coherence point: each piece adds
        // its sums and waits for their return before it counts itself in;
        // the piece whose count completes the slot therefore reads the
        // whole sums, and leaves the slot zero for the next launch.
        // Integer addition: the sums do not depend on the order.
        uint64_t* sl = tail + (size_t)slot * TMQ_TAIL_SLOT_WORDS;
        const uint64_t prev = __hip_atomic_fetch_add(sl + lane, (uint64_t)tot, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(prev));
        wait_vm<0>();
        uint32_t cnt = 0;
        if (lane == 0)
            cnt = (uint32_t)__hip_atomic_fetch_add(sl + 64, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        cnt = __builtin_amdgcn_readfirstlane(cnt);
        if ((int)cnt != pieces - 1) return;
        tot = (int64_t)__hip_atomic_exchange(sl + lane, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) __hip_atomic_store(sl + 64, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (r < t.rows) {
        if (w.acc) w.acc[r] = tot;
        // sim/tmac_gguf.cpp:1192-1194 (Q4_K), :1501-1503 (Q6_K):
        // y = (float)((double)acc*x_scale/(double)row_inv)
        if (w.y) store_y(w, r, (float)(((double)tot * (double)xsc) / (double)inv));
    }
}

template <int FMT, bool CLAMP>
__device__ __forceinline__ void run_group(const TmqWork& w, int g, int b0, int b1, int slot, int pieces,
                                          uint64_t* tail) {
    if constexpr (FMT == kQ8_0) {
        if (pieces > 1)
            group_q8_quarter(w, g, b0);
        else
            group_q8(w, g);
    } else if constexpr (FMT == kQ5_0M) {
        group_mfma_q5(w, g);
    } else if constexpr (FMT == kQ4_KM) {
        group_mfma_kq<kQ4_K>(w, g, b0, b1 ? b1 : w.t.nb, slot, pieces, tail);
    } else if constexpr (FMT == kQ6_KM) {
        group_mfma_kq<kQ6_K>(w, g, b0, b1 ? b1 : w.t.nb, slot, pieces, tail);
    } else {
        group_ksplit<FMT, CLAMP>(w, g);
    }
}

// one GEMV
template <int FMT, bool CLAMP>
__global__ __launch_bounds__(64 * gemv_waves(FMT)) void gemv_kernel(TmqWork w) {
    run_group<FMT, CLAMP>(w, blockIdx.x, 0, 0, 0, 1, nullptr);
}

// A chain segment: every descriptor of one format in one launch,
// workgroup -> (descriptor, group, super-block range) through the group map.
// The Q5_0 decoder is held to 64 registers, eight waves a SIMD (1.5 % a C2
// launch over seven; the Q4_K decoder at five would spill).
template <int FMT, bool CLAMP>
__global__ __launch_bounds__(64 * gemv_waves(FMT), FMT == kQ5_0M ? 8 : 1) void chain_kernel(
    const TmqWork* __restrict__ works, const TmqGroupRef* __restrict__ groups, uint64_t* tail) {
    const TmqGroupRef ref = groups[blockIdx.x];
    run_group<FMT, CLAMP>(works[ref.work], ref.group, ref.b0, ref.b1, ref.slot, ref.pieces, tail);
}

// ------------------------------------------------- INT16 and FP32 paths
// The two other branches of the reference's `matmul` (sim/tmac_gguf.cpp:
// 473-493): matmul_fpga_int16 (:887-940), taken when --fpga is on but the
// tensor type's own flag is off, and the FP32 loop (:488-492) of a run
// without any --fpga flag.  Both start from the exact element values of
// read_tensor (:398-411, the decoders :236-393).

// 32 exact elements of row r, columns j0..j0+31 (j0 % 32 == 0), evaluated as
// read_tensor does: Q8_0 val*scale (:247), Q5_0 d*q (:322), Q6_K d*sc*q
// (:360), Q4_K d*sc*q4 - dmin*m (:392), F32 as stored, F16 half->float.
__device__ __forceinline__ void elems32(const TmqTensorDev& t, int r, int j0, float (&E)[32]) {
    const size_t R = t.rows_pad;
    if (t.type == kQ8_0) {
        const int b = j0 >> 5;
        const uint4 v0 = ld16(t.pa + p16(b, 0, 2, R, r)), v1 = ld16(t.pa + p16(b, 1, 2, R, r));
        const float d = h2f(ld2(t.pd + ((size_t)b * R + r) * 2));
#pragma unroll
        for (int i = 0; i < 16; i++) {
            E[i] = (float)(int8_t)byte_of(v0, i) * d;
            E[16 + i] = (float)(int8_t)byte_of(v1, i) * d;
        }
    } else if (t.type == kQ5_0) {
        const int b = j0 >> 5;
        const size_t o = (size_t)b * R + r;
        const uint4 qs = ld16(t.pa + o * 16);
        const uint32_t d4 = ld4(t.pb + o * 4);
        const float d = h2f(ld2(t.pd + o * 2));
#pragma unroll
        for (int e = 0; e < 32; e++) E[e] = d * (float)(q5_code(qs, d4, e) - 16);
    } else if (t.type == kQ4_K) {
        const int b = j0 >> 8, s = (j0 & 255) >> 5;
        const uint4 h = ld16(t.pb + p16(b, 0, 1, R, r));
        const uint4 qa = ld16(t.pa + p16(b, (s >> 1) * 2, 8, R, r)), qb = ld16(t.pa + p16(b, (s >> 1) * 2 + 1, 8, R, r));
        const float d = h2f(h.x), dmin = h2f(h.x >> 16);
        int sc, m;
        q4k_scale_min(h, s, sc, m);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t by = byte_of(i < 16 ? qa : qb, i & 15);
            const int q4 = (s & 1) ? (int)(by >> 4) : (int)(by & 15u);
            E[i] = d * (float)sc * (float)q4 - dmin * (float)m;
        }
    } else if (t.type == kQ6_K) {
        const int b = j0 >> 8, off = j0 & 255, half = off >> 7, sub = (off & 127) >> 5;
        const int cl = half * 4 + (sub & 1) * 2, ch = half * 2;
        const uint4 l0 = ld16(t.pa + p16(b, cl, 8, R, r)), l1 = ld16(t.pa + p16(b, cl + 1, 8, R, r));
        const uint4 h0 = ld16(t.pb + p16(b, ch, 4, R, r)), h1 = ld16(t.pb + p16(b, ch + 1, 4, R, r));
        const uint4 scv = ld16(t.pc + p16(b, 0, 1, R, r));
        const float d = h2f(ld2(t.pd + ((size_t)b * R + r) * 2));
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t qlb = byte_of(l < 16 ? l0 : l1, l & 15), qhb = byte_of(l < 16 ? h0 : h1, l & 15);
            const uint32_t nib = (sub < 2) ? (qlb & 15u) : (qlb >> 4);
            const int q = (int)(nib | (((qhb >> (2 * sub)) & 3u) << 4)) - 32;
            const int sc = (int)(int8_t)byte_of(scv, half * 8 + (l >> 4) + sub * 2);
            E[l] = d * (float)sc * (float)q;
        }
    } else if (t.type == kF32) {
        const int b = j0 >> 5;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const uint4 v = ld16(t.pa + p16(b, c, 8, R, r));
            E[4 * c] = __uint_as_float(v.x);
            E[4 * c + 1] = __uint_as_float(v.y);
            E[4 * c + 2] = __uint_as_float(v.z);
            E[4 * c + 3] = __uint_as_float(v.w);
        }
    } else {  // F16
        const int b = j0 >> 5;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint4 v = ld16(t.pa + p16(b, c, 4, R, r));
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t w = dw_of(v, k);
                E[8 * c + 2 * k] = h2f(w);
                E[8 * c + 2 * k + 1] = h2f(w >> 16);
            }
        }
    }
}

// matmul_fpga_int16's weight quantisation (sim/tmac_gguf.cpp:905-925), a
// function of the weights alone, done once per tensor: per row
// row_scale = max|E|/32767 (1 below 1e-10), w = (int16)roundf(E/row_scale)
// with the IEEE division; 8 weights per 16-byte chunk of plane pw.
// (|E/row_scale| <= 32767*(1+2^-24), so the cast never overflows.)
__global__ __launch_bounds__(64) void i16_prep_kernel(TmqTensorDev t) {
    const int r = blockIdx.x * 64 + threadIdx.x;
    if (r >= t.rows_pad) return;
    const size_t R = t.rows_pad;
    float m = 0.0f;
    for (int j0 = 0; j0 < t.cols; j0 += 32) {
        float E[32];
        elems32(t, r, j0, E);
#pragma unroll
        for (int i = 0; i < 32; i++) m = fmaxf(m, fabsf(E[i]));
    }
    const float rs = (m < 1e-10f) ? 1.0f : m / 32767.0f;
    ((float*)t.rs16)[r] = rs;
    uint8_t* pw = (uint8_t*)t.pw;
    for (int j0 = 0; j0 < t.cols; j0 += 32) {
        float E[32];
        elems32(t, r, j0, E);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            uint32_t d[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int a = (int)(int16_t)roundf(E[8 * c + 2 * k] / rs);
                const int b = (int)(int16_t)roundf(E[8 * c + 2 * k + 1] / rs);
                d[k] = ((uint32_t)a & 0xffffu) | ((uint32_t)b << 16);
            }
            *(uint4*)(pw + p16(j0 / 8 + c, 0, 1, R, r)) = make_uint4(d[0], d[1], d[2], d[3]);
        }
    }
}

// F32 / F16 tensors: every element finite (the quantized types check their
// fp16 scales in rowstat_kernel).
__global__ __launch_bounds__(64) void check_finite_kernel(TmqTensorDev t, int* bad) {
    const int r = blockIdx.x * 64 + threadIdx.x;
    if (r >= t.rows) return;
    bool ok = true;
    for (int j0 = 0; j0 < t.cols; j0 += 32) {
        float E[32];
        elems32(t, r, j0, E);
#pragma unroll
        for (int i = 0; i < 32; i++) ok = ok && __builtin_isfinite(E[i]);
    }
    if (!ok) atomicOr(bad, 1);
}

// INT16 64-column tile tt of row r: result = sum_k xq[c+k] * w[r][c+k]
// (axi_vecmul_tile_int16 -> vecmul_1x64_int16, sim/fpga_sim.hpp:437-446,
// :45-54) from the xh/xl pairs: |sum w*xh|, |sum w*xl| < 2^30 over 64
// columns, so both stay inside int32.
template <class AT>
__device__ __forceinline__ int64_t i16_tile(const TmqTensorDev& t, const AT& A, int r, int tt) {
    const size_t R = t.rows_pad;
    const int c0 = 8 * tt, c1 = min(c0 + 8, t.cols >> 3);
    uint4 v[8];
#pragma unroll
    for (int c = 0; c < 8; c++) v[c] = ld16(t.pw + p16(min(c0 + c, c1 - 1), 0, 1, R, r));
    int sh = 0, sl = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        if (c0 + c >= c1) break;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int kx = 4 * (c0 + c) + k;
            sh = dot2(dw_of(v[c], k), A.xh[kx], sh);
            sl = dot2(dw_of(v[c], k), A.xl[kx], sl);
        }
    }
    return (int64_t)sh * 256 + sl;
}

// matmul_fpga_int16 (sim/tmac_gguf.cpp:887-940): 4 waves, each owning 64
// rows, walk the 64-column tiles in order and fold every tile's result as
// y += (double)result * x_scale * row_scale (:930-931).
__global__ __launch_bounds__(64 * TMQ_WAVES) void i16_gemv_kernel(TmqWork w) {
    const TmqTensorDev& t = w.t;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r0 = (blockIdx.x * TMQ_WAVES + wave) * 64;
    if (r0 >= t.rows_pad) return;
    const int r = r0 + lane;
    const float rs = t.rs16[r];
    const Act A = act_view(w.act);
    const int nt = (t.cols + 63) / 64;
    float y = 0.0f;
    for (int tt = 0; tt < nt; tt++) {
        const int64_t P = i16_tile(t, A, r, tt);
        if (w.acc && r < t.rows) w.acc[(size_t)r * nt + tt] = P;
        y = (float)((double)y + ((double)P * (double)A.xs) * (double)rs);
    }
    if (w.y && r < t.rows) store_y(w, r, y);
}

// The FP32 loop of `matmul` (sim/tmac_gguf.cpp:488-492): y_r = sum over
// j in order of read_tensor(r, j) * x[j], every product and sum rounded to
// fp32 (no fma: the library is built with -ffp-contract=off).  One lane per
// row, 4 waves of 64 rows; x is read through the scalar cache.
__global__ __launch_bounds__(64 * TMQ_WAVES) void f32_gemv_kernel(TmqWork w) {
    const TmqTensorDev& t = w.t;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r0 = (blockIdx.x * TMQ_WAVES + wave) * 64;
    if (r0 >= t.rows_pad) return;
    const int r = r0 + lane;
    const cu32* xp = (const cu32*)w.xf;
    float sum = 0.0f;
    for (int j0 = 0; j0 < t.cols; j0 += 32) {
        float E[32];
        elems32(t, r, j0, E);
#pragma unroll
        for (int i = 0; i < 32; i++) sum = sum + E[i] * __uint_as_float(xp[j0 + i]);
    }
    if (w.y && r < t.rows) store_y(w, r, sum);
}

// ------------------------------------------------------------ engine GEMV
// One launch = one activation recipe (TmqEngAct) + row groups of works of
// any formats.  Every workgroup first issues the loads of its first weight
// block(s), then computes the launch's activation into LDS (the loads are in
// flight meanwhile), then multiplies.  K is split over the NW waves of the
// workgroup (Q5_0 / K-quants); a Q8_0 wave owns 64 rows and walks all tiles.

// Exact dequantised element (row r, column j) of an uploaded tensor, read
// from its planes (sim/tmac_gguf.cpp:236-393, read_embedding :400-411).
__device__ float tensor_elem(const TmqTensorDev& t, int r, int j) {
    const size_t R = t.rows_pad;
    if (t.type == kQ8_0) {
        const int b = j >> 5, i = j & 31;
        const float d = h2f(ld2(t.pd + ((size_t)b * R + r) * 2));
        const int q = (int)(int8_t)t.pa[p16(b, i >> 4, 2, R, r) + (i & 15)];
        return (float)q * d;  // :247 val * scale
    }
    if (t.type == kQ5_0) {
        const int b = j >> 5, e = j & 31;
        const size_t o = (size_t)b * R + r;
        const float d = h2f(ld2(t.pd + o * 2));
        return d * (float)(q5_code(ld16(t.pa + o * 16), ld4(t.pb + o * 4), e) - 16);  // :307-322
    }
    if (t.type == kQ4_K) {
        const int b = j >> 8, off = j & 255, s = off >> 5, qp = off & 31;
        const uint8_t* h = t.pb + p16(b, 0, 1, R, r);
        const float d = h2f(ld2(h)), dmin = h2f(ld2(h + 2));
        const uint8_t* sc = h + 4;
        int scv, m;
        if (s < 4) {
            scv = sc[s] & 63;
            m = sc[s + 4] & 63;
        } else {
            scv = (sc[s + 4] & 0xf) | ((sc[s - 4] >> 6) << 4);
            m = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4);
        }
        const int qi = (s >> 1) * 32 + qp;
        const uint32_t by = t.pa[p16(b, qi >> 4, 8, R, r) + (qi & 15)];
        const int q4 = (s & 1) ? (int)(by >> 4) : (int)(by & 15u);
        return d * (float)scv * (float)q4 - dmin * (float)m;  // :363-393
    }
    if (t.type == kQ6_K) {
        const int b = j >> 8, off = j & 255, half = off >> 7, pos = off & 127, l = pos & 31, sub = pos >> 5;
        const float d = h2f(ld2(t.pd + ((size_t)b * R + r) * 2));
        const int qlo = half * 64 + l + (sub & 1) * 32;
        const uint32_t qlb = t.pa[p16(b, qlo >> 4, 8, R, r) + (qlo & 15)];
        const int qho = half * 32 + l;
        const uint32_t qhb = t.pb[p16(b, qho >> 4, 4, R, r) + (qho & 15)];
        const uint32_t nib = (sub < 2) ? (qlb & 15u) : (qlb >> 4);
        const int q = (int)(nib | (((qhb >> (2 * sub)) & 3u) << 4)) - 32;
        const int sc = (int)(int8_t)t.pc[p16(b, 0, 1, R, r) + half * 8 + (l >> 4) + sub * 2];
        return d * (float)sc * (float)q;  // :324-361
    }
    return 0.0f;
}

// LDS carve-up of an engine workgroup: x[n] fp32 | xh[n/2] xl[n/2] (the
// squares of RMSNorm alias xh/xl before the quantisation) | part[(NW+1)*64]
// int64 | red[64] | spec[16*64] spec_c[16] (the norm's segmented sum) | the
// MFMA decoders' weight ring (ring bytes, 16-aligned).  An MFMA format's
// activation operand bytes (64 a 32-column block, then 512 bytes of
// constant runs), block sums (n/32 int32) and 16-column sums (n/16 int32)
// take the place of xh/xl where they fit (eng_mx_bytes <= 4n), else follow
// the ring.
struct EngLds {
    float* x;
    uint32_t* xh;
    uint32_t* xl;
    int64_t* part;
    float* red;
    float* spec;
    int* spec_c;
    uint8_t* ring;
    uint8_t* mxa;
    int32_t* mxs;
    int32_t* mxs16;
};
__host__ __device__ constexpr size_t eng_base_bytes(int n, int nw) {
    return (8 * (size_t)n + 8 * 64 * ((size_t)nw + 1) + 256 + 4 * (16 * 64 + 16) + 15) & ~(size_t)15;
}
__host__ __device__ constexpr size_t eng_mx_bytes(int n) {
    return 2 * (size_t)n + 512 + (size_t)n / 8 + (size_t)n / 4;
}
__device__ __forceinline__ EngLds eng_lds(unsigned char* base, int n, int nw, size_t ring_bytes) {
    EngLds L;
    L.x = (float*)base;
    L.xh = (uint32_t*)(base + 4 * (size_t)n);
    L.xl = L.xh + n / 2;
    L.part = (int64_t*)(base + 8 * (size_t)n);
    L.red = (float*)(L.part + (nw + 1) * 64);
    L.spec = L.red + 64;
    L.spec_c = (int*)(L.spec + 16 * 64);
    L.ring = base + eng_base_bytes(n, nw);
    L.mxa = eng_mx_bytes(n) <= 4 * (size_t)n ? (uint8_t*)L.xh : L.ring + ring_bytes;
    L.mxs = (int32_t*)(L.mxa + 2 * (size_t)n + 512);
    L.mxs16 = L.mxs + n / 32;
    return L;
}

// sum += the 64 values of a group, in order, in every lane: each lane of a
// 16-lane row holds four of them (lane i: values 4i .. 4i+3, the same in the
// four rows), and v_add_f32_dpp row_newbcast:i adds lane i's value of the
// lane's own row as src0 (src0 + src1 = v + sum, the same rounded value as
// sum + v).  No LDS traffic inside the chain; a dependent DPP add issues
// about every 7 cycles.  s_nop 1: the two wait states a DPP read of a VGPR
// needs after a VALU write of it.
__device__ __forceinline__ float add64_rowbcast(float4 x, float sum) {
#define TMQ_RB4(N)                                                                 \
    "v_add_f32_dpp %0, %1, %0 row_newbcast:" #N " row_mask:0xf bank_mask:0xf\n\t" \
    "v_add_f32_dpp %0, %2, %0 row_newbcast:" #N " row_mask:0xf bank_mask:0xf\n\t" \
    "v_add_f32_dpp %0, %3, %0 row_newbcast:" #N " row_mask:0xf bank_mask:0xf\n\t" \
    "v_add_f32_dpp %0, %4, %0 row_newbcast:" #N " row_mask:0xf bank_mask:0xf\n\t"
    asm volatile("s_nop 1\n\t" TMQ_RB4(0) TMQ_RB4(1) TMQ_RB4(2) TMQ_RB4(3) TMQ_RB4(4) TMQ_RB4(5) TMQ_RB4(6)
                     TMQ_RB4(7) TMQ_RB4(8) TMQ_RB4(9) TMQ_RB4(10) TMQ_RB4(11) TMQ_RB4(12) TMQ_RB4(13)
                         TMQ_RB4(14) TMQ_RB4(15)
                 : "+v"(sum)
                 : "v"(x.x), "v"(x.y), "v"(x.z), "v"(x.w));
#undef TMQ_RB4
    return sum;
}
// Lane i's four values of group g of [i0, i1) (v[i0 + 64g + 4i ..]), +0.0
// past i1.
__device__ __forceinline__ float4 seq_group(const float* v, int i0, int i1, int g, int i) {
    const int b = i0 + 64 * g + 4 * i;
    if (b + 4 <= i1) return *(const float4*)(v + b);
    float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (b + 0 < i1) r.x = v[b + 0];
    if (b + 1 < i1) r.y = v[b + 1];
    if (b + 2 < i1) r.z = v[b + 2];
    return r;
}
// Sequential fp32 sum of v[i0..i1) in index order from each lane's `sum`
// (the reference's loops), by a whole wave (the same i0, i1 in every lane;
// i0 a multiple of 4), from LDS, in groups of 64 (add64_rowbcast), the next
// group's values read during the current one's adds.  The values past i1 in
// the last group are +0.0: adding +0.0 leaves any sum whose sign bit is
// clear unchanged, which the callers guarantee (v >= 0, starts of
// non-negative bits).
__device__ __forceinline__ float seq_chain_lds(const float* v, int i0, int i1, float sum) {
    const int i = threadIdx.x & 15, ng = (i1 - i0 + 63) >> 6;
    float4 x = ng > 0 ? seq_group(v, i0, i1, 0, i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int g = 0; g < ng; g++) {
        const float4 cur = x;
        if (g + 1 < ng) x = seq_group(v, i0, i1, g + 1, i);
        sum = add64_rowbcast(cur, sum);
    }
    return sum;
}

// One DPP move of a double across lanes (lanes the control leaves without a
// source, or outside ROW_MASK, read 0.0).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, ROW_MASK, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, ROW_MASK, 0xf, false);
    return __hiloint2double(hi, lo);
}
// Sum of x over the wave's 64 lanes, complete in lane 63: pairs and quads
// (quad permutations), rows of 8 and 16 (half-row and row mirrors), then
// row 0 into row 1 and row 2 into row 3 (row_bcast15), rows 0-1 into row 3
// (row_bcast31).  VALU lane moves only, no LDS round trips.
__device__ __forceinline__ double wave_sum_f64(double x) {
    x += dpp_f64<0xb1>(x);       // quad_perm [1,0,3,2]
    x += dpp_f64<0x4e>(x);       // quad_perm [2,3,0,1]
    x += dpp_f64<0x141>(x);      // row_half_mirror
    x += dpp_f64<0x140>(x);      // row_mirror
    x += dpp_f64<0x142, 0xa>(x);  // row_bcast15
    x += dpp_f64<0x143, 0xc>(x);  // row_bcast31
    return x;
}

// The same sequential sum of v[0..n) (0 + v[0] + v[1] + ..., each add
// rounded; n a multiple of 4), by S waves of the workgroup at once (S at
// most the workgroup's waves); every thread calls it, and the result is
// returned to the lanes of wave 0.  The range is cut into S segments of L
// values (whole batches of 64); wave j runs segment j from 64 starting
// values, lane l from the float whose bits are those of c_j plus l - 32, c_j
// being the fp64 sum of v[0 .. jL) rounded to float (wave 0 from the exact
// start, 0).  Wave 0 then walks the segments in order: the exact start of
// segment j is the result of segment j-1, and the lane that started from
// those very bits performed exactly the sequential adds of that segment, so
// its result is taken.  When no lane did (the fp32 chain drifted more than
// 32 ulps from the fp64 sum, as over long runs of equal values), wave 0 runs
// the segment again from the exact start.  For v >= 0 the float bits order
// the values, so the 64 starts are 64 consecutive floats; lane l started
// from max(0, c_j + l - 32), which for the index l = b - c_j + 32 in
// [0, 64) of an exact start with bits b is b itself whenever b >= 0 as an
// integer (a float without its sign bit).  miss != 0 moves every window
// away (each segment then runs again: a test of that path).  scr: S*64
// words of LDS, scr_c: S words.
template <int S>
__device__ __forceinline__ float seq_sum_spec(const float* v, int n, float* scr, int* scr_c, int miss) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int L = ((n + S - 1) / S + 63) & ~63;
    if (wave < S) {
        const int j0 = min(n, wave * L), j1 = min(n, j0 + L);
        // centre: lane l adds the runs of 16 values at 16 l + 1024 i
        double p = 0.0;
        for (int base = 16 * lane; base < j0; base += 1024) {
            float4 q4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) q4[e] = *(const float4*)(v + min(base + 4 * e, n - 4));
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x[4] = {q4[e].x, q4[e].y, q4[e].z, q4[e].w};
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (base + 4 * e + u < j0) p += (double)x[u];
            }
        }
        const int cb = min(__builtin_amdgcn_readlane((int)__float_as_uint((float)wave_sum_f64(p)), 63), 0x7f800000) +
                       (miss ? (1 << 20) : 0);
        const float s0 = __uint_as_float((uint32_t)(wave == 0 ? 0 : max(0, cb + lane - 32)));
        scr[wave * 64 + lane] = seq_chain_lds(v, j0, j1, s0);
        if (lane == 0) scr_c[wave] = cb;
    }
    __syncthreads();
    float sum = 0.0f;
    if (wave == 0) {
        // the segments' results (lane l holds lane l's) and centres into
        // registers, all read at once (the empty asm keeps the compiler from
        // moving each read down to its step), then the walk reads them across
        // lanes with uniform indices
        float o[S];
        int c[S];
#pragma unroll
        for (int j = 0; j < S; j++) {
            o[j] = scr[j * 64 + lane];
            c[j] = scr_c[j];
        }
#pragma unroll
        for (int j = 0; j < S; j++) {
            c[j] = __builtin_amdgcn_readfirstlane(c[j]);
            asm volatile("" : "+v"(o[j]), "+s"(c[j]));
        }
        // the exact running sum as bits in a scalar register: a step is a
        // few scalar instructions and one lane read
        int sb = __builtin_amdgcn_readfirstlane(__float_as_int(o[0]));  // segment 0: exact in every lane
#pragma unroll
        for (int j = 1; j < S; j++) {
            const int j0 = min(n, j * L), j1 = min(n, j0 + L);
            if (j0 >= j1) break;
            // idx = sb - c_j + 32; a hit when idx is in [0, 64) and sb >= 0
            int nsb, miss, idx;
            asm volatile(
                "s_sub_i32 %[i], %[sb], %[c]\n\t"
                "s_add_i32 %[i], %[i], 32\n\t"
                "s_cmp_lt_u32 %[i], 64\n\t"
                "s_cselect_b32 %[m], 0, 1\n\t"
                "s_cmp_lt_i32 %[sb], 0\n\t"
                "s_cselect_b32 %[m], 1, %[m]\n\t"
                "s_and_b32 %[i], %[i], 63\n\t"
                "v_readlane_b32 %[r], %[o], %[i]"
                : [r] "=s"(nsb), [m] "=&s"(miss), [i] "=&s"(idx)
                : [sb] "s"(sb), [c] "s"(c[j]), [o] "v"(o[j])
                : "scc");
            sb = __builtin_expect(miss, 0)
                     ? __builtin_amdgcn_readfirstlane(__float_as_int(seq_chain_lds(v, j0, j1, __int_as_float(sb))))
                     : nsb;
        }
        sum = __int_as_float(sb);
    }
    return sum;
}

// The activation of the launch (TmqEngAct), quantised into L.xh / L.xl over
// the columns [c0, c1) the workgroup reads (all of them for the modes that
// need the whole vector); returns x_scale.
//   rms_norm (sim/tmac_gguf.cpp:447-453): o = fl(fl(x*w)*s), s from the
//   sequential sum of squares (seq_sum_spec over the squares in LDS).  The
//   max of |o| is taken as fl(max|fl(x*w)| * s), the wave maxima gathered
//   before the sum: rounding is monotone and s > 0, so it is the same value,
//   without waiting for s.
//   quantisation (:1225-1231): x_scale = max|o| / 32767 (1 below 1e-10),
//   xq = (int16)roundf(o / x_scale).
// `pre` issues the caller's weight prefetch.  It runs right after the
// activation loads are issued and before any of them is used: loads retire
// in order, so the activation arrives without waiting for the (cold) weights.
// The common modes take up to EP elements per thread with every load issued
// unconditionally (clamped indices), so no load waits for another.
// Segments of the norm's sum (seq_sum_spec), one a wave: 8 of a 16-wave
// workgroup (4 where the format's units, or several works in one launch,
// leave fewer of the 128 registers), or the four waves.  (16 segments of 64
// measured slower: the walk's 13 steps cost more than the shorter chains
// save.)
template <int NW, int FMT, bool MULTI = false>
constexpr int eng_norm_segs() { return NW < 16 || MULTI || FMT == kQ6_K ? 4 : 8; }
// MX: 0 quantises columns [c0, c1) into xh/xl; an MFMA format (kQ5_0M,
// kQ4_KM, kQ6_KM) into that decoder's operand bytes and sums (mxa, mxs,
// mxs16) with its constant runs ([c0, c1) whole 32-column blocks).
template <int NW, int SEGS, int MX = 0, class Pre>
__device__ __forceinline__ float eng_prologue(const TmqEngAct& a, const EngLds& L, int c0, int c1, Pre&& pre) {
    constexpr int EP = NW >= 16 ? 1 : 4;
    const int n = a.n, tid = threadIdx.x, nt = blockDim.x;
    const bool wr = a.hidden_out && blockIdx.x == 0;
    const bool norm = (a.mode == TMQ_ACT_RESID_NORM || a.mode == TMQ_ACT_EMBED_NORM) && a.w;
    float* sq = (float*)L.xh;  // squares, consumed before xh/xl are written
    float m = 0.0f;
    if (a.mode == TMQ_ACT_PRESCALED) {
        // max given as a_max_n slots (one per producing workgroup, bits of
        // non-negative floats); only the workgroup's columns are needed
        uint32_t mv = 0;
        if (c1 - c0 <= EP * nt) {
            float xin[EP];
#pragma unroll
            for (int e = 0; e < EP; e++) xin[e] = a.x[min(c0 + tid + e * nt, c1 - 1)];
            if (tid < a.max_n) mv = __hip_atomic_load(a.max_bits + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_sched_barrier(0);
            pre();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < EP; e++)
                if (c0 + tid + e * nt < c1) L.x[c0 + tid + e * nt] = xin[e];
        } else {
            pre();
            for (int i = c0 + tid; i < c1; i += nt) L.x[i] = a.x[i];
            if (tid < a.max_n) mv = __hip_atomic_load(a.max_bits + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        m = __builtin_bit_cast(float, mv);
        m = tmq_wave_max(m);
        if ((tid & 63) == 0) L.red[2 + (tid >> 6)] = m;
    } else if ((a.mode == TMQ_ACT_PLAIN || (a.mode == TMQ_ACT_RESID_NORM && a.d1.ntiles == 0 && !a.d1.val)) &&
               n <= EP * nt) {
        // every load first (indices clamped into [0, n), pointers always
        // valid), then the arithmetic; one straight-line path per mode
        auto fast = [&](auto resid_tag) {
            constexpr bool resid = decltype(resid_tag)::value;
            float xin[EP], wv[EP], ri[EP], bi[EP];
            int64_t ac[EP];
            float dxs = 1.0f;
            if constexpr (resid) dxs = *a.d1.xs;
            const float* bp = resid && a.d1.bias ? a.d1.bias : a.x;
            const float* wp = norm ? a.w : a.x;
#pragma unroll
            for (int e = 0; e < EP; e++) {
                const int i = min(tid + e * nt, n - 1);
                xin[e] = a.x[i];
                wv[e] = wp[i];
                if constexpr (resid) {
                    ac[e] = tmq_ld_acc(a.d1.acc + i);
                    ri[e] = a.d1.row_inv[i];
                    bi[e] = bp[i];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            pre();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < EP; e++) {
                const int i = tid + e * nt;
                if (i < n) {
                    float v = xin[e];
                    if constexpr (resid) {
                        float d = (float)(((double)ac[e] * (double)dxs) / (double)ri[e]);
                        if (a.d1.bias) d = d + bi[e];
                        v = v + d;
                    }
                    if (wr) a.hidden_out[i] = v;
                    if (norm) {
                        sq[i] = v * v;
                        v = v * wv[e];
                    }
                    L.x[i] = v;
                    m = fmaxf(m, fabsf(v));
                }
            }
        };
        if (a.mode == TMQ_ACT_RESID_NORM) fast(std::true_type{});
        else fast(std::false_type{});
        m = tmq_wave_max(m);
        if ((tid & 63) == 0) L.red[2 + (tid >> 6)] = m;
    } else {
        pre();
        int tok = 0;
        if (a.mode == TMQ_ACT_EMBED_NORM) tok = a.tokens[a.state->pos];
        for (int i = tid; i < n; i += nt) {
            float v;
            if (a.mode == TMQ_ACT_EMBED_NORM) v = tensor_elem(a.emb, tok, i);
            else if (a.mode == TMQ_ACT_RESID_NORM) v = a.x[i] + tmq_fin(a.d1, i);
            else v = a.x[i];
            if (wr) a.hidden_out[i] = v;
            if (norm) {
                sq[i] = v * v;
                v = v * a.w[i];
            }
            L.x[i] = v;
            m = fmaxf(m, fabsf(v));
        }
        m = tmq_wave_max(m);
        if ((tid & 63) == 0) L.red[2 + (tid >> 6)] = m;
    }
    __syncthreads();
    float s = 1.0f;  // the norm's scale
    if (norm) {
        static_assert(SEGS <= NW && SEGS <= 16, "a segment per wave");
        const float ss = seq_sum_spec<SEGS>(sq, n, L.spec, L.spec_c, a.spec_miss);
        if (tid == 0) L.red[0] = 1.0f / sqrtf(ss / (float)n + a.eps);
        __syncthreads();
        s = L.red[0];
    }
    // the FP32 path reads the activation itself: o = L.x * red[1]
    if (tid == 0) L.red[1] = s;
    // capture of the norm output (the matmuls' fp32 input, rms_norm's o)
    if (norm && a.act_out && blockIdx.x == 0)
        for (int i = tid; i < n; i += nt) a.act_out[i] = L.x[i] * s;
    float mm = 0.0f;
    for (int i = 0; i < (int)(nt >> 6); i++) mm = fmaxf(mm, L.red[2 + i]);
    if (norm) mm = mm * s;
    const float xs = (mm < 1e-10f) ? 1.0f : mm / 32767.0f;
    if constexpr (MX != 0) {
        // element i: xh byte at 64*(i/32) + 32*(i/16 % 2) + i%16, xl - 128
        // 16 bytes on; the sums of 16 and 32 consecutive elements from the
        // lanes of one 16-lane row and of two (c0, c1 and every 64-element
        // step being whole blocks, a row's lanes are all inside or all
        // outside [c0, c1))
        uint8_t* xa = L.mxa;
        for (int base = c0; base < c1; base += nt) {
            const int i = base + tid;
            int p = 0;
            if (i < c1) {
                float u = L.x[i];
                if (norm) u = u * s;
                p = (int)(int16_t)roundf(u / xs);
                const int o = 64 * (i >> 5) + 32 * ((i >> 4) & 1) + (i & 15);
                xa[o] = (uint8_t)(p >> 8);
                xa[o + 16] = (uint8_t)((p & 255) ^ 128);
            }
            const int s16 = tmq_row_sum(p);
            const int s32 = s16 + __shfl_xor(s16, 16);
            if (i < c1) {
                if (MX == kQ6_KM && (tid & 15) == 0) L.mxs16[i >> 4] = s16;
                if ((tid & 31) == 0) L.mxs[i >> 5] = s32;
            }
        }
        // the constant runs behind the row: zeros then ones, 64 bytes each
        // (Q5_0 decoder) or 256 (K-quants)
        constexpr int CR = MX == kQ5_0M ? 64 : 256;
        if (tid < CR / 8) {
            const uint32_t v = tid < CR / 16 ? 0u : 0x01010101u;
            *(uint4*)(xa + 64 * (n >> 5) + 16 * tid) = make_uint4(v, v, v, v);
        }
    } else {
        for (int k = (c0 >> 1) + tid; k < (c1 >> 1); k += nt) {
            float u = L.x[2 * k], v = L.x[2 * k + 1];
            if (norm) {
                u = u * s;
                v = v * s;
            }
            const int p = (int)(int16_t)roundf(u / xs);
            const int q = (int)(int16_t)roundf(v / xs);
            L.xh[k] = ((uint32_t)(p >> 8) & 0xffffu) | ((uint32_t)(q >> 8) << 16);
            L.xl[k] = ((uint32_t)p & 0xffu) | (((uint32_t)q & 0xffu) << 16);
        }
    }
    __syncthreads();
    return xs;
}

__device__ __forceinline__ ActL eng_act(const EngLds& L, float xs) {
    ActL A;
    A.xs = xs;
    A.xh = (const lu32*)L.xh;
    A.xl = (const lu32*)L.xl;
    return A;
}

// Q5_0 / K-quant row group g, K chunk c: the workgroup's units are split
// over its waves; each wave keeps its next unit in flight while it
// multiplies.  With kc > 1 (or a kacc) the int64 row sums go to w.kacc.
template <int FMT, int NW, bool MULTI>
__device__ __forceinline__ void eng_group_k(const TmqEngAct& a, const EngLds& L, const TmqWork& w, int gi) {
    typedef typename UnitOf<FMT>::T Unit;
    const TmqTensorDev& t = w.t;
    const int kc = w.kc, g = gi / kc, c = gi - g * kc;
    const int nu = t.nb * UnitOf<FMT>::per_block;
    const int u0 = c * nu / kc, u1 = (c + 1) * nu / kc;  // nu * kc < 2^31
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    Unit cur{};
    float inv = 0.0f;
    constexpr int QK = FMT == kQ5_0 ? 32 : 256, PB = UnitOf<FMT>::per_block;
    const float xs = eng_prologue<NW, eng_norm_segs<NW, FMT, MULTI>()>(a, L, (u0 / PB) * QK, ((u1 + PB - 1) / PB) * QK, [&] {
        // unconditional (a clamped, valid unit): the prologue's waits then
        // count these loads exactly and skip them
        cur = unit_load<FMT>(t, max(0, min(u0 + wave, nu - 1)), r);
        inv = t.row_inv[r];
    });
    if (w.xs_out && gi == 0 && threadIdx.x == 0) *w.xs_out = xs;
    const ActL A = eng_act(L, xs);
    int64_t acc = 0;
    for (int u = u0 + wave; u < u1; u += NW) {
        const bool more = u + NW < u1;
        Unit nxt{};
        if (more) nxt = unit_load<FMT>(t, u + NW, r);
        int sh = 0, sl = 0;
        unit_mac<FMT>(cur, A, u, inv, sh, sl);
        acc += (int64_t)sh * 256 + sl;
        if (more) cur = nxt;
    }
    L.part[wave * 64 + lane] = acc;
    __syncthreads();
    if (w.silu) {
        // fused SwiGLU (sim/tmac_gguf.cpp:459-461, :1696-1700): lane i < 32
        // holds gate row 32g+i, lane i+32 the same up row; both finalised
        // as the K-split consumers do (tmq_fin, no bias)
        if (wave == 0) {
            int64_t tot = 0;
#pragma unroll
            for (int i = 0; i < NW; i++) tot += L.part[i * 64 + lane];
            const float f = (float)(((double)tot * (double)xs) / (double)inv);
            const float up = __shfl_down(f, 32);
            float m = __int_as_float(0x7fc00000);  // lanes 32-63: fmaxf's identity
            if (lane < 32) {
                const float v = (f / (1.0f + tmq_math::tmq_expf(-f))) * up;
                w.silu[g * 32 + lane] = v;
                m = fabsf(v);
            }
            m = tmq_wave_max(m);
            // this group's max in its own slot (the consumer takes the largest)
            if (lane == 0)
                __hip_atomic_store(w.silu_max + g, __builtin_bit_cast(uint32_t, m), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    if (wave == 0 && r < t.rows) {
        int64_t tot = 0;
#pragma unroll
        for (int i = 0; i < NW; i++) tot += L.part[i * 64 + lane];
        if (w.kacc) {
            __hip_atomic_fetch_add(w.kacc + r, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            if (w.acc) w.acc[r] = tot;
            if (w.y) store_y(w, r, (float)(((double)tot * (double)xs) / (double)inv));
        }
    }
}

// Weight-ring bytes of an engine launch's MFMA format (0: not an MFMA format)
__host__ __device__ constexpr size_t eng_ring_bytes(int fmt, int nw) {
    return fmt == kQ5_0M   ? (size_t)nw * TMQ_MFMA_DEPTH * kMfmaStage
           : fmt == kQ4_KM ? (size_t)kKqWaves * TMQ_MFMA_DEPTH * kq_stage<kQ4_K>()
           : fmt == kQ6_KM ? (size_t)kKqWaves * TMQ_MFMA_DEPTH * kq_stage<kQ6_K>()
                           : 0;
}

// Q5_0 / K-quant row group g, K chunk c on the MFMA decoders: chunk c of kc
// takes blocks (Q5_0) or super-blocks (K-quants) [c*nb/kc, (c+1)*nb/kc),
// whose columns the prologue quantises into the decoder's operand bytes
// while the ring's first stages load; the chunk adds the corrections of its
// own columns.  The int64 row sums go where eng_group_k sends them.
template <int FMT, int NW, bool MULTI>
__device__ __forceinline__ void eng_group_mfma(const TmqEngAct& a, const EngLds& L, const TmqWork& w, int gi) {
    const TmqTensorDev& t = w.t;
    const int kc = w.kc, g = gi / kc, c = gi - g * kc;
    const int nb = t.nb, b0 = c * nb / kc, b1 = (c + 1) * nb / kc;
    constexpr int QK = FMT == kQ5_0M ? 32 : 256;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    const float inv = t.row_inv[r];
    float xs = 1.0f;
    // the prologue runs the prime between its loads and their use; after
    // it the stages have long landed (the wait also covers the prologue's
    // own stores), so the loop starts with no operation in flight
    auto ready = [&](auto&& prime, int) {
        xs = eng_prologue<NW, eng_norm_segs<NW, FMT, MULTI>(), FMT>(a, L, b0 * QK, b1 * QK, prime);
        wait_vm<0>();
    };
    // a correction's activation value from the operand bytes
    auto xq = [&](int col) {
        const int o = 64 * (col >> 5) + 32 * ((col >> 4) & 1) + (col & 15);
        return (int)(int8_t)L.mxa[o] * 256 + (int)(L.mxa[o + 16] ^ 128u);
    };
    int64_t tot;
    if constexpr (FMT == kQ5_0M)
        tot = mfma_q5_rows<NW, true>(t, g, b0, b1, L.mxa, L.mxs, L.ring, L.part, b0 * QK, b1 * QK, ready, xq);
    else
        tot = mfma_kq_rows<FMT == kQ4_KM ? kQ4_K : kQ6_K, true>(t, g, b0, b1, L.mxa, L.mxs, L.mxs16, L.ring, L.part,
                                                               b0 * QK, b1 * QK, ready, xq);
    if (w.xs_out && gi == 0 && threadIdx.x == 0) *w.xs_out = xs;
    if (wave != 0) return;
    if (w.silu) {
        // fused SwiGLU, as eng_group_k
        const float f = (float)(((double)tot * (double)xs) / (double)inv);
        const float up = __shfl_down(f, 32);
        float m = __int_as_float(0x7fc00000);  // lanes 32-63: fmaxf's identity
        if (lane < 32) {
            const float v = (f / (1.0f + tmq_math::tmq_expf(-f))) * up;
            w.silu[g * 32 + lane] = v;
            m = fabsf(v);
        }
        m = tmq_wave_max(m);
        if (lane == 0)
            __hip_atomic_store(w.silu_max + g, __builtin_bit_cast(uint32_t, m), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (r < t.rows) {
        if (w.kacc) {
            __hip_atomic_fetch_add(w.kacc + r, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            if (w.acc) w.acc[r] = tot;
            if (w.y) store_y(w, r, (float)(((double)tot * (double)xs) / (double)inv));
        }
    }
}

// Q8_0 K-split (attn_v): 64-row group g, tile chunk c; each wave takes
// tiles (two blocks) of the chunk and stores their int64 P into
// kacc[r][tile] (one writer per slot; the consumer folds the tiles in order).
template <int NW, bool MULTI>
__device__ __forceinline__ void eng_group_q8_split(const TmqEngAct& a, const EngLds& L, const TmqWork& w, int gi) {
    const TmqTensorDev& t = w.t;
    const int kc = w.kc, g = gi / kc, c = gi - g * kc;
    const int nt = (t.cols + 63) / 64;
    const int t0 = c * nt / kc, t1 = (c + 1) * nt / kc;  // nt * kc < 2^31
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    Q8Blk b0{}, b1{};
    float ri = 0.0f;
    const float xs = eng_prologue<NW, eng_norm_segs<NW, kQ8_0, MULTI>()>(a, L, 64 * t0, min(64 * t1, t.cols), [&] {
        const int tt = max(0, min(t0 + wave, nt - 1));
        b0 = q8_load(t, 2 * tt, r);
        b1 = q8_load(t, min(2 * tt + 1, t.nb - 1), r);
        ri = t.row_inv[r];
    });
    if (w.xs_out && gi == 0 && threadIdx.x == 0) *w.xs_out = xs;
    const ActL A = eng_act(L, xs);
    for (int tt = t0 + wave; tt < t1; tt += NW) {
        if (tt != t0 + wave) {
            b0 = q8_load(t, 2 * tt, r);
            if (2 * tt + 1 < t.nb) b1 = q8_load(t, 2 * tt + 1, r);
        }
        int sh = 0, sl = 0;
        q8_mac(b0, A, 2 * tt, ri, sh, sl);
        if (2 * tt + 1 < t.nb) q8_mac(b1, A, 2 * tt + 1, ri, sh, sl);
        if (r < t.rows)
            __hip_atomic_store(w.kacc + (size_t)r * nt + tt, (int64_t)sh * 256 + sl, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Orderable key of (logit, row): larger logit first, then smaller row.
__device__ __forceinline__ uint64_t argmax_key(float v, int r) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)r);
}

// Q8_0 direct (the logits): each wave owns 64 rows and walks all tiles,
// folding in double (sim/tmac_gguf.cpp:1075-1076), and leaves its argmax
// candidate.
template <int NW>
__device__ __forceinline__ void eng_group_q8(const TmqEngAct& a, const EngLds& L, const TmqWork& w, int g) {
    const TmqTensorDev& t = w.t;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int grp = g * NW + wave;
    const int r0 = grp * 64;
    const bool active = r0 < t.rows_pad;
    const int r = active ? r0 + lane : lane;
    Q8Blk cur{};
    float ri = 0.0f, rs = 0.0f;
    const ActL A = eng_act(L, eng_prologue<NW, eng_norm_segs<NW, kQ8_0>()>(a, L, 0, t.cols, [&] {
        cur = q8_load(t, 0, r);
        ri = t.row_inv[r];
        rs = t.row_scale[r];
    }));
    if (!active) return;
    const int nt = (t.cols + 63) / 64;
    float y = 0.0f;
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
    if (w.y && r < t.rows) store_y(w, r, y);
    if (w.cand) {
        uint64_t k = (r < t.rows) ? argmax_key(y, r) : 0ull;
        for (int o = 32; o > 0; o >>= 1) {
            const uint64_t ok = __shfl_xor(k, o);
            k = ok > k ? ok : k;
        }
        if (lane == 0) w.cand[grp] = k;
    }
}

// INT16 path in the engine (matmul_fpga_int16, sim/tmac_gguf.cpp:887-940),
// K split over 64-column tiles as the Q8_0 split is: each wave takes tiles of
// its chunk and stores their int64 results into kacc[r][tile] (one writer
// per slot); the consumer folds them in order with the INT16 row scales.
template <int NW, bool MULTI>
__device__ __forceinline__ void eng_group_i16_split(const TmqEngAct& a, const EngLds& L, const TmqWork& w, int gi) {
    const TmqTensorDev& t = w.t;
    const int kc = w.kc, g = gi / kc, c = gi - g * kc;
    const int nt = (t.cols + 63) / 64;
    const int t0 = c * nt / kc, t1 = (c + 1) * nt / kc;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = g * 64 + lane;
    const float xs = eng_prologue<NW, eng_norm_segs<NW, kQ8_0, MULTI>()>(a, L, 64 * t0, min(64 * t1, t.cols), [] {});
    if (w.xs_out && gi == 0 && threadIdx.x == 0) *w.xs_out = xs;
    const ActL A = eng_act(L, xs);
    for (int tt = t0 + wave; tt < t1; tt += NW) {
        const int64_t P = i16_tile(t, A, r, tt);
        if (r < t.rows)
            __hip_atomic_store(w.kacc + (size_t)r * nt + tt, P, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// argmax candidate of a wave's 64 rows (y of row r, rows past t.rows excluded)
__device__ __forceinline__ void wave_cand(const TmqWork& w, int r, float y, int grp) {
    uint64_t k = (r < w.t.rows) ? argmax_key(y, r) : 0ull;
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t ok = __shfl_xor(k, o);
        k = ok > k ? ok : k;
    }
    if ((threadIdx.x & 63) == 0) w.cand[grp] = k;
}

// INT16 path, direct (the logits through get_logits, :1852-1866): each
// wave owns 64 rows and folds all its tiles; argmax candidates as the
// Q8_0 logits leave them.
template <int NW>
__device__ __forceinline__ void eng_group_i16(const TmqEngAct& a, const EngLds& L, const TmqWork& w, int g) {
    const TmqTensorDev& t = w.t;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int grp = g * NW + wave, r0 = grp * 64;
    const bool active = r0 < t.rows_pad;
    const int r = active ? r0 + lane : lane;
    const ActL A = eng_act(L, eng_prologue<NW, eng_norm_segs<NW, kQ8_0>()>(a, L, 0, t.cols, [] {}));
    if (!active) return;
    const float rs = t.rs16[r];
    const int nt = (t.cols + 63) / 64;
    float y = 0.0f;
    for (int tt = 0; tt < nt; tt++)
        y = (float)((double)y + ((double)i16_tile(t, A, r, tt) * (double)A.xs) * (double)rs);
    if (w.y && r < t.rows) w.y[r] = y;
    if (w.cand) wave_cand(w, r, y, grp);
}

// FP32 path in the engine (the loop of :488-492): each wave owns 64 rows,
// one lane per row, and sums read_tensor(r, j) * o_j in column order from
// the launch's fp32 activation o = L.x * red[1] (the rms_norm output
// fl(fl(x*w)*scale), :447-453, or the input itself).  The rows are final
// values (TmqDeferred.val); the logits also leave argmax candidates.
template <int NW, bool MULTI>
__device__ __forceinline__ void eng_group_f32(const TmqEngAct& a, const EngLds& L, const TmqWork& w, int g) {
    const TmqTensorDev& t = w.t;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int grp = g * NW + wave, r0 = grp * 64;
    const bool active = r0 < t.rows_pad;
    const int r = active ? r0 + lane : lane;
    (void)eng_prologue<NW, eng_norm_segs<NW, kQ8_0, MULTI>()>(a, L, 0, t.cols, [] {});
    if (!active) return;
    const float sc = L.red[1];
    float sum = 0.0f;
    for (int j0 = 0; j0 < t.cols; j0 += 32) {
        float E[32];
        elems32(t, r, j0, E);
#pragma unroll
        for (int i = 0; i < 32; i++) sum = sum + E[i] * (L.x[j0 + i] * sc);
    }
    if (w.y && r < t.rows) __hip_atomic_store(w.y + r, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (w.cand) wave_cand(w, r, sum, grp);
}

// Format codes of the engine kernel variants: the ggml types, and
// kQ8_DIRECT for the logits (Q8_0, one wave per 64 rows, direct output).
constexpr int kQ8_DIRECT = 108;
// the other branches of matmul: INT16 K-split / direct, FP32
constexpr int kI16 = 116, kI16_DIRECT = 117, kF32P = 200;

template <int NW, int FMT, bool MULTI>
__device__ __forceinline__ void eng_dispatch(const TmqEngAct& a, const EngLds& L, const TmqWork& w) {
    const int g = blockIdx.x - w.first_group;
    if constexpr (FMT == kQ8_0) eng_group_q8_split<NW, MULTI>(a, L, w, g);
    else if constexpr (FMT == kQ8_DIRECT) eng_group_q8<NW>(a, L, w, g);
    else if constexpr (FMT == kI16) eng_group_i16_split<NW, MULTI>(a, L, w, g);
    else if constexpr (FMT == kI16_DIRECT) eng_group_i16<NW>(a, L, w, g);
    else if constexpr (FMT == kF32P) eng_group_f32<NW, MULTI>(a, L, w, g);
    else if constexpr (FMT == kQ5_0M || FMT == kQ4_KM || FMT == kQ6_KM) eng_group_mfma<FMT, NW, MULTI>(a, L, w, g);
    else eng_group_k<FMT, NW, MULTI>(a, L, w, g);
}

// The launch arrives by value (kernel arguments): no dependent loads
// before the weight prefetch and the activation prologue start.  One
// instantiation per format pair keeps the code small: every work uses FA
// except the last, which uses FB.
template <int NW, int FA, int FB, bool MULTI>
__global__ __launch_bounds__(NW * 64) void eng_gemv_kernel(TmqEngLaunch P) {
    tmq_warm_kernargs<sizeof(TmqEngLaunch)>();
    if ((int)blockIdx.x >= P.ngroups) {
        // the RoPE-row workgroup (launched only with rope_out set)
        const int pos = P.rope_state->pos;
        if (threadIdx.x < 32 && pos >= 0 && pos < P.rope_max_pos)
            P.rope_out[threadIdx.x] = P.rope_src[(size_t)pos * 32 + threadIdx.x];
        return;
    }
    extern __shared__ __attribute__((aligned(16))) unsigned char eng_smem[];
    constexpr size_t RB = eng_ring_bytes(FA, NW) > eng_ring_bytes(FB, NW) ? eng_ring_bytes(FA, NW)
                                                                          : eng_ring_bytes(FB, NW);
    const EngLds L = eng_lds(eng_smem, P.act.n, NW, RB);
    if constexpr (!MULTI) {
        // one work: every launch parameter sits at a fixed kernarg offset,
        // so all of them come in the first batch of scalar loads
        eng_dispatch<NW, FA, MULTI>(P.act, L, P.w[0]);
    } else {
        const int b = blockIdx.x;
        const int wi = (P.nworks > 2 && b >= P.w[2].first_group) ? 2 : (P.nworks > 1 && b >= P.w[1].first_group) ? 1 : 0;
        const TmqWork w = wi == 2 ? P.w[2] : wi == 1 ? P.w[1] : P.w[0];
        if (FA != FB && wi == P.nworks - 1) eng_dispatch<NW, FB, MULTI>(P.act, L, w);
        else eng_dispatch<NW, FA, MULTI>(P.act, L, w);
    }
}

// x = silu(g) * u (sim/tmac_gguf.cpp:459-461, :1696-1700) from two K-split
// GEMVs, once per layer; the workgroups' max |x| meet in max_bits.
__global__ __launch_bounds__(256) void silu_kernel(TmqDeferred g, TmqDeferred u, int n, float* x,
                                                   uint32_t* max_bits) {
    __shared__ float red[4];
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    float m = 0.0f;
    if (i < n) {
        const float gv = tmq_fin(g, i);
        const float v = (gv / (1.0f + tmq_math::tmq_expf(-gv))) * tmq_fin(u, i);
        x[i] = v;
        m = fabsf(v);
    }
    m = tmq_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __hip_atomic_fetch_max(max_bits, __builtin_bit_cast(uint32_t, m), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// hidden + the pending deferred rows (the residual stream as the host sees
// it), for reads from outside a step (dumps, tmq_model_hidden).
__global__ __launch_bounds__(256) void resid_view_kernel(const float* __restrict__ x, TmqDeferred d, int n,
                                                         float* out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = x[i] + tmq_fin(d, i);
}

// Zeroes n int64 K-split accumulators (at the device coherence point).
__global__ __launch_bounds__(256) void zero_acc_kernel(int64_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        __hip_atomic_store(p + i, (int64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------ activation prep
// sim/tmac_gguf.cpp:1225-1231: x_scale = max|x| (sequential fmaxf; the max
// is order independent), /32767 unless < 1e-10; xq = (int16)roundf(x/x_scale)
__global__ __launch_bounds__(1024) void act_prep_kernel(TmqActJobs jobs) {
    tmq_warm_kernargs<sizeof(TmqActJobs)>();
    const TmqActJob& J = jobs.j[blockIdx.x];
    __shared__ float red[16];
    __shared__ float s_scale;
    const int n = J.n;
    float m = 0.0f;
    for (int j = threadIdx.x; j < n; j += blockDim.x) m = fmaxf(m, fabsf(J.x[j]));
    m = tmq_wave_max(m);
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
    int32_t* x32 = (int32_t*)(xq + n);
    for (int k = threadIdx.x; k < n / 2; k += blockDim.x) {
        int a = (int)(int16_t)roundf(J.x[2 * k] / s);
        int c = (int)(int16_t)roundf(J.x[2 * k + 1] / s);
        xq[2 * k] = (int16_t)a;
        xq[2 * k + 1] = (int16_t)c;
        x32[2 * k] = a;
        x32[2 * k + 1] = c;
        xh[k] = ((uint32_t)(a >> 8) & 0xffffu) | ((uint32_t)(c >> 8) << 16);
        xl[k] = ((uint32_t)a & 0xffu) | (((uint32_t)c & 0xffu) << 16);
    }
    // the MFMA decoders' operand bytes and block sums: four lanes per
    // 32-element block, eight elements each (xq recomputed, as above)
    const int nbx = (n + 31) / 32;
    uint8_t* XA = J.act + tmq_act_xa(n);
    int32_t* XS = (int32_t*)(J.act + tmq_act_xs(n));
    int32_t* XS16 = (int32_t*)(J.act + tmq_act_xs16(n));
    for (int q = threadIdx.x; q < nbx * 4; q += blockDim.x) {
        const int b = q >> 2, e0 = 32 * b + 8 * (q & 3);
        uint32_t hi[2] = {0, 0}, lo[2] = {0x80808080u, 0x80808080u};
        int sum = 0;
        for (int i = 0; i < 8; i++) {
            const int a = e0 + i < n ? (int)(int16_t)roundf(J.x[e0 + i] / s) : 0;
            sum += a;
            hi[i >> 2] = (hi[i >> 2] & ~(0xffu << (8 * (i & 3)))) | (((uint32_t)(a >> 8) & 0xffu) << (8 * (i & 3)));
            lo[i >> 2] = (lo[i >> 2] & ~(0xffu << (8 * (i & 3)))) | ((((uint32_t)a & 0xffu) ^ 0x80u) << (8 * (i & 3)));
        }
        const int c = (q >> 1) & 1, pos = 8 * (q & 1);
        *(uint2*)(XA + 64 * b + 32 * c + pos) = make_uint2(hi[0], hi[1]);
        *(uint2*)(XA + 64 * b + 32 * c + 16 + pos) = make_uint2(lo[0], lo[1]);
        sum += __shfl_xor(sum, 1);
        if ((q & 1) == 0) XS16[2 * b + ((q >> 1) & 1)] = sum;
        sum += __shfl_xor(sum, 2);
        if ((q & 3) == 0) XS[b] = sum;
    }
    if (threadIdx.x < 8) ((uint32_t*)(XA + 64 * nbx))[threadIdx.x] = threadIdx.x < 4 ? 0u : 0x01010101u;
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
        // ggml: code(e) = nibble e of qs (low nibbles 0-15, high 16-31) | bit e of qh << 4
        const uint32_t qh = (uint32_t)s[2] | ((uint32_t)s[3] << 8) | ((uint32_t)s[4] << 16) | ((uint32_t)s[5] << 24);
        uint32_t D[5] = {0, 0, 0, 0, 0};
        for (int e = 0; e < 32; e++) {
            const uint32_t c = (uint32_t)((e < 16 ? s[6 + e] & 15 : s[6 + e - 16] >> 4) | (((qh >> e) & 1u) << 4));
            const int k = e & 3, sh = 8 * k + 5;
            if (e < 20) {
                D[e >> 2] |= c << (8 * k);
            } else if (e < 28) {
                const int lo = e < 24 ? 0 : 2;  // D0/D1 or D2/D3
                D[lo] |= (c & 7u) << sh;
                D[lo + 1] |= (c >> 3) << sh;
            } else {
                D[4] |= (c & 7u) << sh;
                D[1] |= ((c >> 3) & 1u) << (sh + 2);
                D[3] |= (c >> 4) << (sh + 2);
            }
        }
        for (int i = 0; i < 4; i++) *(uint32_t*)(pa + p16(b, 0, 1, R, r) + 4 * i) = D[i];
        *(uint32_t*)(pb + ((size_t)b * R + r) * 4) = D[4];
    } else if (type == kQ4_K) {
        const uint8_t* s = src + idx * 144;
        for (int i = 0; i < 16; i++) pb[p16(b, 0, 1, R, r) + i] = s[i];
        for (int i = 0; i < 128; i++) pa[p16(b, i >> 4, 8, R, r) + (i & 15)] = s[16 + i];
    } else if (type == kF32 || type == kF16) {
        // row-major elements: block b of row r is 32 contiguous values
        const int nbytes = type == kF32 ? 128 : 64, C = nbytes / 16;
        const uint8_t* s = src + idx * nbytes;
        for (int i = 0; i < nbytes; i++) pa[p16(b, i >> 4, C, R, r) + (i & 15)] = s[i];
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
            const uint32_t d4 = *(const uint32_t*)(t.pb + ((size_t)b * R + r) * 4);
            for (int e = 0; e < 32; e++) {
                int q = q5_code(qs, d4, e) - 16;
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

// Fit codes (see Q5Blk): for each sub-block of block b of row r, the
// smallest move (dA, dB), |dA|, |dB| <= 3 ulps by growing square rings, for
// which rne(fl(u*A + B)) = g(u) on every code u the sub-block holds; else the
// exact-decode flag.  g(u) is the exact decode's int16: the saturated
// round-half-away of fl(E * row_inv), E the decoder's exact value of u.
// n codes u[] with exact values E = gu(u) and A0, B0(A) as the decoders form them.
template <int N, class GE, class B0>
__device__ __forceinline__ uint32_t fit_search(const int (&u)[N], float a0, float inv, GE&& gu, B0&& b0) {
    int g[N];
#pragma unroll
    for (int i = 0; i < N; i++) g[i] = max(-32768, min(32767, round_away(gu(u[i]) * inv)));
    for (int rad = 0; rad <= 3; rad++)
        for (int da = -rad; da <= rad; da++)
            for (int db = -rad; db <= rad; db++) {
                if (abs(da) != rad && abs(db) != rad) continue;
                const uint32_t code = (uint32_t)(da + 4) | ((uint32_t)(db + 4) << 3);
                const float a = fit_a(a0, code), bb = fit_b(b0(a), code);
                bool ok = true;
#pragma unroll
                for (int i = 0; i < N; i++)
                    ok = ok && fit_biased(fit_rne(__builtin_fmaf((float)u[i], a, bb))) - (int32_t)kFitM == g[i];
                if (ok) return code;
            }
    return 0x80u;
}

template <int FMT>
__global__ __launch_bounds__(256) void fit_kernel(TmqTensorDev t, int all_exact) {
    const int r = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
    if (r >= t.rows_pad) return;
    const size_t R = t.rows_pad, o = (size_t)b * R + r;
    const float inv = t.row_inv[r];
    uint8_t* pe = (uint8_t*)t.pe;
    if (all_exact) {
        const int n = FMT == kQ5_0 ? 1 : FMT == kQ4_K ? 8 : 16;
        for (int i = 0; i < n; i++) pe[o * n + i] = 0x80u;
        return;
    }
    if constexpr (FMT == kQ5_0) {
        const Q5Blk k = q5_load(t, b, r);
        const float d = h2f(k.d);
        int u[32];
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const uint32_t U = q5_codes(k, g);
#pragma unroll
            for (int j = 0; j < 4; j++) u[4 * g + j] = (int)((U >> (8 * j)) & 31u);
        }
        pe[o] = (uint8_t)fit_search(
            u, d * inv, inv, [&](int c) { return d * (float)(c - 16); },
            [](float a) { return -16.0f * a; });
    } else if constexpr (FMT == kQ4_K) {
        const Q4KBlk k = q4k_load(t, b, r);
        const float d = h2f(k.h.x), dmin = h2f(k.h.x >> 16);
#pragma unroll 1
        for (int s = 0; s < 8; s++) {
            int sc, m;
            q4k_scale_min(k.h, s, sc, m);
            const float Ad = d * (float)sc, Bm = dmin * (float)m;
            int u[32];
#pragma unroll
            for (int i = 0; i < 32; i++) {
                const uint32_t by = byte_of(k.qs[(s >> 1) * 2 + (i >> 4)], i & 15);
                u[i] = (int)((s & 1) ? (by >> 4) : (by & 15u));
            }
            const float b0 = -Bm * inv;
            pe[o * 8 + s] = (uint8_t)fit_search(
                u, Ad * inv, inv, [&](int c) { return __builtin_fmaf((float)c, Ad, -Bm); },
                [&](float) { return b0; });
        }
    } else {
        const Q6KBlk k = q6k_load(t, b, r);
        const float ss = h2f(k.d);
#pragma unroll 1
        for (int q = 0; q < 4; q++) {
            const int half = q >> 1, lc = q & 1;
            const uint4 qla = k.ql[half * 4 + lc], qlb = k.ql[half * 4 + 2 + lc], qhc = k.qh[half * 2 + lc];
#pragma unroll 1
            for (int sub = 0; sub < 4; sub++) {
                const int j = half * 8 + lc + 2 * sub;
                const float S = ss * (float)(int8_t)byte_of(k.sc, j);
                int u[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t U = q6_codes(qla, qlb, qhc, sub, i);
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) u[4 * i + jj] = (int)((U >> (8 * jj)) & 63u);
                }
                pe[o * 16 + j] = (uint8_t)fit_search(
                    u, S * inv, inv, [&](int c) { return S * (float)(c - 32); },
                    [](float a) { return -32.0f * a; });
            }
        }
    }
}

// Integer fit codes of the MFMA decoders (see IFit): for block b of row r
// the first (dA, dB) by growing |dA| then |dB| (dA in [-4, 3], dB in
// [-8, 7]) whose fitted weights equal g(u) on every code the block holds,
// else the pair with the fewest differing elements.  Pass 0 writes the code
// and the number of differing codes; pass 1 writes one correction per
// differing code from corr[off[r * nb + b]] on.  force: every block takes
// the code dA = 3, dB = 7 (testing the corrections).
__global__ __launch_bounds__(256) void ifit_kernel(TmqTensorDev t, int pass, int force, uint8_t* cnt,
                                                   const int32_t* off, uint4* corr) {
    const int r = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
    if (r >= t.rows_pad) return;
    const size_t R = t.rows_pad;
    const float inv = t.row_inv[r], ri256 = inv * 256.0f;
    const Q5Blk k = q5_load(t, b, r);
    const float d = h2f(k.d);
    int u[32], gv[32];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const uint32_t U = q5_codes(k, q);
#pragma unroll
        for (int i = 0; i < 4; i++) u[4 * q + i] = (int)((U >> (8 * i)) & 31u);
    }
#pragma unroll
    for (int i = 0; i < 32; i++)
        gv[i] = max(-32768, min(32767, round_away(d * (float)(u[i] - 16) * inv)));
    uint32_t best = 0x7fu;
    if (!force) {
        int best_mis = 33;
        for (int ia = 0; ia < 8 && best_mis; ia++) {
            const int da = (ia & 1) ? -((ia + 1) >> 1) : (ia >> 1);  // 0, -1, 1, -2, 2, -3, 3, -4
            for (int ib = 0; ib < 16 && best_mis; ib++) {
                const int db = (ib & 1) ? -((ib + 1) >> 1) : (ib >> 1);  // 0, -1, 1, ..., 7, -8
                const uint32_t e = (uint32_t)(da + 4) | ((uint32_t)(db + 8) << 3);
                const IFit f = ifit_q5(k.d, ri256, e);
                int mis = 0;
#pragma unroll
                for (int i = 0; i < 32; i++) mis += ifit_w(f, u[i]) != gv[i];
                if (mis < best_mis) {
                    best_mis = mis;
                    best = e;
                }
            }
        }
    }
    const IFit f = ifit_q5(k.d, ri256, best);
    uint32_t bad = 0;  // codes whose fitted weight differs
#pragma unroll
    for (int i = 0; i < 32; i++)
        if (ifit_w(f, u[i]) != gv[i]) bad |= 1u << u[i];
    if (pass == 0) {
        // blocks 4j .. 4j+3 of row r share a dword (plane [b/4][r] x 4 B)
        ((uint8_t*)t.pi)[((size_t)(b >> 2) * R + r) * 4 + (b & 3)] = (uint8_t)best;
        cnt[(size_t)r * t.nb + b] = (uint8_t)__builtin_popcount(bad);
        return;
    }
    if (!bad) return;
    int slot = off[(size_t)r * t.nb + b];
    for (; bad; bad &= bad - 1) {
        const int c = __builtin_ctz(bad);
        uint32_t m = 0;
        int delta = 0;
#pragma unroll
        for (int i = 0; i < 32; i++)
            if (u[i] == c) {
                m |= 1u << i;
                delta = gv[i] - ifit_w(f, c);
            }
        corr[slot++] = make_uint4((uint32_t)r, (uint32_t)(32 * b), m, (uint32_t)delta);
    }
}

// Integer fit codes of the K-quant MFMA decoders (kfit): one thread per
// (row, sub-block).  The sub-block's exact weights g(u) are those of the
// fitted-float decoders' fit (fit_kernel: clamp16(roundf(fl(E(u)*row_inv))),
// E as the reference dequantises); the first (dA, dB) by growing |dA| then
// |dB| (dA in [-4, 3], dB in [-16, 15]) that gives g on every code the
// sub-block holds is kept, else the pair with the fewest differing codes.
// Sub-block k of block b: Q4_K k = s (32 weights, columns 256b + 32s + i),
// quarter q = s >> 1; Q6_K k = 4q + sub for quarter q = 2h + lc (16 weights,
// columns 256b + 128h + 32sub + 16lc + i, scale 8h + lc + 2sub).  Pass 0
// writes the code (plane pi, quarter-major) and the number of differing
// codes at cnt[(r*nb + b)*NSUB + k]; pass 1 writes one correction per
// differing code from corr[off[...]] on.  force: every sub-block takes the
// code dA = 3, dB = 15 (testing the corrections).
template <int FMT>
__global__ __launch_bounds__(256) void ikfit_kernel(TmqTensorDev t, int pass, int force, uint8_t* cnt,
                                                    const int32_t* off, uint4* corr) {
    constexpr int NSUB = FMT == kQ4_K ? 8 : 16, N = FMT == kQ4_K ? 32 : 16, P = FMT == kQ4_K ? 8 : 32;
    const int r = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y / NSUB, k = blockIdx.y % NSUB;
    if (r >= t.rows_pad) return;
    const size_t R = t.rows_pad;
    const float inv = t.row_inv[r], ri256 = inv * 256.0f;
    int u[N], gv[N];
    float an, bn;
    int q, col0;
    size_t po;  // byte of the fit code in plane pi
    if constexpr (FMT == kQ4_K) {
        const Q4KBlk kb = q4k_load(t, b, r);
        const int sidx = k;
        q = sidx >> 1;
        const float d = h2f(kb.h.x), dmin = h2f(kb.h.x >> 16);
        int sc, m;
        q4k_scale_min(kb.h, sidx, sc, m);
        const float Ad = d * (float)sc, Bm = dmin * (float)m;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t by = byte_of(kb.qs[(sidx >> 1) * 2 + (i >> 4)], i & 15);
            u[i] = (int)((sidx & 1) ? (by >> 4) : (by & 15u));
            gv[i] = max(-32768, min(32767, round_away(__builtin_fmaf((float)u[i], Ad, -Bm) * inv)));
        }
        q4k_nom(d * ri256, dmin * ri256, sc, m, an, bn);
        col0 = 256 * b + 32 * sidx;
        po = (((size_t)b * 4 + q) * R + r) * 2 + (sidx & 1);
    } else {
        const Q6KBlk kb = q6k_load(t, b, r);
        q = k >> 2;
        const int sub = k & 3, h = q >> 1, lc = q & 1;
        const float ss = h2f(kb.d);
        const int sc = (int)(int8_t)byte_of(kb.sc, 8 * h + lc + 2 * sub);
        const float S = ss * (float)sc;
        const uint4 qla = kb.ql[h * 4 + lc], qlb = kb.ql[h * 4 + 2 + lc], qhc = kb.qh[h * 2 + lc];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t U = q6_codes(qla, qlb, qhc, sub, i);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                u[4 * i + j] = (int)((U >> (8 * j)) & 63u);
                gv[4 * i + j] = max(-32768, min(32767, round_away(S * (float)(u[4 * i + j] - 32) * inv)));
            }
        }
        an = (ss * ri256) * (float)sc;
        bn = 128.0f;
        col0 = 256 * b + 128 * h + 32 * sub + 16 * lc;
        po = (((size_t)b * 4 + q) * R + r) * 4 + sub;
    }
    uint32_t best = 255u;
    if (!force) {
        int best_mis = N + 1;
        for (int ia = 0; ia < 8 && best_mis; ia++) {
            const int da = (ia & 1) ? -((ia + 1) >> 1) : (ia >> 1);  // 0, -1, 1, -2, 2, -3, 3, -4
            for (int ib = 0; ib < 32 && best_mis; ib++) {
                const int db = (ib & 1) ? -((ib + 1) >> 1) : (ib >> 1);  // 0, -1, 1, ..., 15, -16
                const uint32_t e = (uint32_t)(da + 4) | ((uint32_t)(db + 16) << 3);
                const IFit f = kfit(an, bn, P, e);
                int mis = 0;
#pragma unroll
                for (int i = 0; i < N; i++) mis += ifit_w(f, u[i]) != gv[i];
                if (mis < best_mis) {
                    best_mis = mis;
                    best = e;
                }
            }
        }
    }
    const IFit f = kfit(an, bn, P, best);
    uint64_t bad = 0;  // codes whose fitted weight differs
#pragma unroll
    for (int i = 0; i < N; i++)
        if (ifit_w(f, u[i]) != gv[i]) bad |= 1ull << u[i];
    const size_t ci = ((size_t)r * t.nb + b) * NSUB + k;
    if (pass == 0) {
        ((uint8_t*)t.pi)[po] = (uint8_t)best;
        cnt[ci] = (uint8_t)__builtin_popcountll(bad);
        return;
    }
    if (!bad) return;
    int slot = off[ci];
    for (; bad; bad &= bad - 1) {
        const int c = __builtin_ctzll(bad);
        uint32_t m = 0;
        int delta = 0;
#pragma unroll
        for (int i = 0; i < N; i++)
            if (u[i] == c) {
                m |= 1u << i;
                delta = gv[i] - ifit_w(f, c);
            }
        corr[slot++] = make_uint4((uint32_t)r, (uint32_t)col0, m, (uint32_t)delta);
    }
}

// UQ8.8 combined scale of every (row, block) of a Q8_0 tensor, as
// matmul_fpga_q8 forms them for its tiles (sim/tmac_gguf.cpp:1022-1039);
// out[r * nb + b]
__global__ __launch_bounds__(256) void q8_scales_kernel(TmqTensorDev t, uint16_t* out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)t.rows * t.nb) return;
    const int r = (int)(i / t.nb), b = (int)(i % t.nb);
    out[i] = (uint16_t)q8_cs(h2f(ld2(t.pd + ((size_t)b * t.rows_pad + r) * 2)), t.row_inv[r]);
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

// ------------------------------------------------------ prefill operands
// Weight digits of one tensor (tmq_prefill.h): the int16 weights the decode
// GEMVs multiply -- the same block decoders and normalisation -- stored as
// two int8 planes at rows row0.. of a plane set K columns wide.  One lane
// per row.
template <int FMT>
__global__ __launch_bounds__(64) void pf_wdigits_kernel(TmqTensorDev t, int8_t* planes, int K, int row0) {
    const int r = blockIdx.x * 64 + threadIdx.x;
    if (r >= t.rows) return;
    const WDigits S{planes, row0 + r, K};
    int sh = 0, sl = 0;
    const float inv = t.row_inv[r];
    for (int b = 0; b < t.nb; b++) {
        if constexpr (FMT == kQ8_0) q8_mac(q8_load(t, b, r), S, b, inv, sh, sl);
        else blk_mac<FMT, false>(blk_load<FMT>(t, b, r), S, b, inv, sh, sl);
    }
}

// Per row of a digit plane set: the sums of (v - 128) = 256*hi + lo over
// each 64-column chunk and over the row.  One wave per row.
__global__ __launch_bounds__(64) void pf_rowsums_kernel(TmqPfPlanes p) {
    const int r = blockIdx.x, lane = threadIdx.x, nc = p.K / TMQ_PF_CHUNK;
    int32_t tot = 0;
    for (int c = 0; c < nc; c++) {
        const size_t o = tmq_pf_off(r, c * TMQ_PF_CHUNK + lane, p.K, 0);
        int v = 256 * (int)p.d[o] + (int)p.d[o + 1024];
        for (int k = 32; k > 0; k >>= 1) v += __shfl_xor(v, k);
        if (lane == 0) p.csum[(size_t)r * nc + c] = v;
        tot += v;
    }
    if (lane == 0) p.tsum[r] = tot;
}

// Activation operands of one token (workgroup t of T_pad): the columns'
// values, RMSNorm, x_scale and xq exactly as eng_prologue forms them, then
// xq as digits with its (xq - 128) sums.  Each thread takes groups of four
// consecutive columns (one dword of each digit plane).  Tokens t >= T get
// zero planes.
__device__ __forceinline__ float pf_value(const TmqPfAct& a, int t, int i, int tok) {
    if (a.mode == TMQ_PF_EMBED_NORM) return tensor_elem(a.emb, tok, i);
    if (a.mode == TMQ_PF_RESID_NORM) return a.x[(size_t)t * a.n + i] + tmq_pf_fin(a.d1, t, i);
    return a.x[(size_t)t * a.n + i];
}
template <int G>
__global__ __launch_bounds__(256) void pf_act_kernel(TmqPfAct a) {
    tmq_warm_kernargs<sizeof(TmqPfAct)>();
    extern __shared__ float pf_lds[];
    __shared__ float red[8];
    __shared__ float spec[4 * 64];  // seq_sum_spec<4>
    __shared__ int spec_c[4];
    const int t = blockIdx.x, n = a.n, tid = threadIdx.x, nt = blockDim.x;
    const int wave = tid >> 6, lane = tid & 63, nc = n / TMQ_PF_CHUNK, ng = n >> 2;
    int8_t* dp = a.out.d;
    // the next GU GEMM's per-token sums and token-tile counters (quantising
    // epilogue), for every row
    if (tid == 0 && a.zero_tsum) a.zero_tsum[t] = 0;
    if (t * nt + tid < a.zero_ncnt) a.zero_cnt[32 * (t * nt + tid)] = 0u;
    if (t >= a.T) {
        for (int gi = tid; gi < ng; gi += nt) {
            const size_t o = tmq_pf_off(t, 4 * gi, n, 0);
            *(uint32_t*)(dp + o) = 0u;
            *(uint32_t*)(dp + o + 1024) = 0u;
        }
        for (int c = tid; c < nc; c += nt) a.out.csum[(size_t)t * nc + c] = 0;
        if (tid == 0) {
            a.out.tsum[t] = 0;
            a.xs[t] = 1.0f;
        }
        return;
    }
    float* X = pf_lds;       // values (after x*w for the norm modes)
    float* sq = pf_lds + n;  // squares
    const bool norm = a.mode == TMQ_PF_EMBED_NORM || a.mode == TMQ_PF_RESID_NORM || a.mode == TMQ_PF_NORM;
    const bool wr = a.x_out && (a.mode == TMQ_PF_EMBED_NORM || a.mode == TMQ_PF_RESID_NORM);
    const int tok = a.mode == TMQ_PF_EMBED_NORM ? a.tokens[a.p0 + t] : 0;
    float m = 0.0f;
    // one group of four columns: the value before the norm to x_out, the
    // squares and x*w (norm modes) or x to LDS, the running max |.|
    auto put = [&](int i0, float (&v)[4], float4 w4) {
        if (wr) *(float4*)(a.x_out + (size_t)t * n + i0) = make_float4(v[0], v[1], v[2], v[3]);
        if (norm) {
            const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
            float s4[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                s4[j] = v[j] * v[j];
                v[j] = v[j] * wv[j];
            }
            *(float4*)(sq + i0) = make_float4(s4[0], s4[1], s4[2], s4[3]);
        }
        *(float4*)(X + i0) = make_float4(v[0], v[1], v[2], v[3]);
#pragma unroll
        for (int j = 0; j < 4; j++) m = fmaxf(m, fabsf(v[j]));
    };
    constexpr int SMAX = 4;  // split-K parts summed in registers (RESID_NORM)
    // the batched paths read 16-byte groups
    const uintptr_t al = (uintptr_t)a.x | (uintptr_t)a.w |
                         (a.mode == TMQ_PF_RESID_NORM
                              ? (uintptr_t)a.d1.rw | (uintptr_t)a.d1.row_inv | (uintptr_t)a.d1.bias | (uintptr_t)a.d1.part
                              : 0);
    // (the register-hungry RESID_NORM batch only for up to two groups a thread)
    if (a.mode == TMQ_PF_EMBED_NORM || ng > G * nt || (al & 15) ||
        (a.mode == TMQ_PF_RESID_NORM && (G > 2 || a.d1.split > SMAX || a.d1.ld % 4))) {
        for (int gi = tid; gi < ng; gi += nt) {
            const int i0 = 4 * gi;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = pf_value(a, t, i0 + j, tok);
            put(i0, v, norm ? *(const float4*)(a.w + i0) : make_float4(1.0f, 1.0f, 1.0f, 1.0f));
        }
    } else if (a.mode == TMQ_PF_RESID_NORM) {
      if constexpr (G <= 2) {
        // every load of the thread's groups first (indices clamped into the
        // row), then the arithmetic: x + the finalised split-K sums
        // (tmq_pf_fin), then the norm
        const TmqPfPart& D = a.d1;
        const float* bp = D.bias ? D.bias : D.row_inv;
        const float xs_t = D.xs[t];
        const int64_t corr = 128 * (int64_t)D.tx[t] + 16384 * (int64_t)D.K;
        float4 xv[G], w4[G], ri4[G], bi4[G];
        int4 rw4[G];
        int64_t pp[G][SMAX][4];
#pragma unroll
        for (int g = 0; g < G; g++) {
            const int i0 = 4 * min(tid + g * nt, ng - 1);
            xv[g] = *(const float4*)(a.x + (size_t)t * n + i0);
            w4[g] = *(const float4*)(a.w + i0);
            ri4[g] = *(const float4*)(D.row_inv + i0);
            bi4[g] = *(const float4*)(bp + i0);
            rw4[g] = *(const int4*)(D.rw + i0);
#pragma unroll
            for (int sp = 0; sp < SMAX; sp++) {
                const int64_t* q = D.part + ((size_t)min(sp, D.split - 1) * D.T_pad + t) * D.ld + i0;
#pragma unroll
                for (int j = 0; j < 4; j++) pp[g][sp][j] = q[j];
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            if (tid + g * nt < ng) {
                const int i0 = 4 * (tid + g * nt);
                const float xin[4] = {xv[g].x, xv[g].y, xv[g].z, xv[g].w};
                const float riv[4] = {ri4[g].x, ri4[g].y, ri4[g].z, ri4[g].w};
                const float biv[4] = {bi4[g].x, bi4[g].y, bi4[g].z, bi4[g].w};
                const int rwv[4] = {rw4[g].x, rw4[g].y, rw4[g].z, rw4[g].w};
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int64_t acc = 128 * (int64_t)rwv[j] + corr;
#pragma unroll
                    for (int sp = 0; sp < SMAX; sp++) acc += sp < D.split ? pp[g][sp][j] : 0;
                    float d = (float)(((double)acc * (double)xs_t) / (double)riv[j]);
                    if (D.bias) d = d + biv[j];
                    v[j] = xin[j] + d;
                }
                put(i0, v, w4[g]);
            }
        }
      }
    } else {
        // PLAIN, NORM, SILU: the values (and norm weights) of all the
        // thread's groups first
        const float* wp = norm ? a.w : a.x;
        float4 xv[G], w4[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            const int i0 = 4 * min(tid + g * nt, ng - 1);
            xv[g] = *(const float4*)(a.x + (size_t)t * n + i0);
            w4[g] = *(const float4*)(wp + i0);
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            if (tid + g * nt < ng) {
                float v[4] = {xv[g].x, xv[g].y, xv[g].z, xv[g].w};
                put(4 * (tid + g * nt), v, w4[g]);
            }
        }
    }
    m = tmq_wave_max(m);
    if (lane == 0) red[1 + wave] = m;
    if (tid == 0 && a.zero_bits) a.zero_bits[t] = 0u;
    __syncthreads();
    float s = 1.0f;
    if (norm) {
        const float ss = seq_sum_spec<4>(sq, n, spec, spec_c, a.spec_miss);
        if (tid == 0) red[0] = 1.0f / sqrtf(ss / (float)n + a.eps);
        __syncthreads();
        s = red[0];
    }
    float mm;
    if (a.mode == TMQ_PF_SILU) {
        mm = __builtin_bit_cast(float, a.max_bits[t]);
    } else {
        mm = 0.0f;
        for (int i = 0; i < (nt >> 6); i++) mm = fmaxf(mm, red[1 + i]);
        if (norm) mm = mm * s;
    }
    const float xs = (mm < 1e-10f) ? 1.0f : mm / 32767.0f;
    // 16 threads per 64-column chunk; n/4 groups cover whole chunks
    int32_t tot = 0;
    for (int g0 = 0; g0 < ng; g0 += nt) {
        const int gi = g0 + tid;
        int sum = 0;
        if (gi < ng) {
            const int i0 = 4 * gi;
            const float4 x4 = *(const float4*)(X + i0);
            float u[4] = {x4.x, x4.y, x4.z, x4.w};
            uint32_t hi = 0, lo = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (norm) u[j] = u[j] * s;
                const int q = (int)(int16_t)roundf(u[j] / xs);
                hi |= ((uint32_t)(q >> 8) & 255u) << (8 * j);
                lo |= (((uint32_t)q & 255u) ^ 128u) << (8 * j);
                sum += q - 128;
            }
            const size_t o = tmq_pf_off(t, i0, n, 0);
            *(uint32_t*)(dp + o) = hi;
            *(uint32_t*)(dp + o + 1024) = lo;
        }
        sum = tmq_row_sum(sum);
        if (gi < ng && (gi & 15) == 0) a.out.csum[(size_t)t * nc + (gi >> 4)] = sum;
        tot += ((tid & 15) == 0 && gi < ng) ? sum : 0;
    }
    tot = tmq_wave_sum(tot);
    __syncthreads();
    if (lane == 0) red[1 + wave] = __builtin_bit_cast(float, tot);
    __syncthreads();
    if (tid == 0) {
        int32_t T = 0;
        for (int i = 0; i < (nt >> 6); i++) T += __builtin_bit_cast(int32_t, red[1 + i]);
        a.out.tsum[t] = T;
        a.xs[t] = xs;
    }
}

}  // namespace

// The Q6_K code plane of the MFMA decoder (TmqTensorDev.pq): one thread per
// (row, block, quarter) reads the quarter's ql / qh chunks as the decoder
// read them and stores sub-blocks 0-2 of its codes a byte each, sub-block 3's
// six bits spread over the top two bits of the three (48 bytes for 64
// codes, as ql + qh): the decoder then takes 48 of every 64 codes with one
// mask a dword.
__global__ __launch_bounds__(256) void q6_pack_kernel(TmqTensorDev t) {
    const size_t R = t.rows_pad, total = R * t.nb * 4;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int r = (int)(idx % R);
    const int bq = (int)(idx / R), q = bq & 3, b = bq >> 2;
    const int h = q >> 1, lc = q & 1;
    const uint4 qla = *(const uint4*)(t.pa + (((size_t)b * 8 + 4 * h + lc) * R + r) * 16);
    const uint4 qlb = *(const uint4*)(t.pa + (((size_t)b * 8 + 4 * h + 2 + lc) * R + r) * 16);
    const uint4 qhc = *(const uint4*)(t.pb + (((size_t)b * 4 + 2 * h + lc) * R + r) * 16);
    uint8_t* pq = (uint8_t*)t.pq;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        uint32_t D[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            D[e] = q6_codes(qla, qlb, qhc, k, e) | (((q6_codes(qla, qlb, qhc, 3, e) >> (2 * k)) & 0x03030303u) << 6);
        *(uint4*)(pq + (((size_t)b * 12 + 3 * q + k) * R + r) * 16) = make_uint4(D[0], D[1], D[2], D[3]);
    }
    // the quarter's scales 8h + lc + 2k, k = 0..3, one byte each
    const uint4 sc = *(const uint4*)(t.pc + ((size_t)b * R + r) * 16);
    uint32_t sq = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) sq |= (uint32_t)byte_of(sc, 8 * h + lc + 2 * k) << (8 * k);
    *(uint32_t*)(pq + R * t.nb * 192 + (((size_t)b * 4 + q) * R + r) * 4) = sq;
}

// ---------------------------------------------------------------- launchers
int tmq_launch_act_prep(const TmqActJobs& jobs, hipStream_t s) {
    if (jobs.count <= 0) return 0;
    hipLaunchKernelGGL(act_prep_kernel, dim3(jobs.count), dim3(1024), 0, s, jobs);
    return (int)hipGetLastError();
}

int tmq_launch_q6_pack(const TmqTensorDev& t, hipStream_t s) {
    if (t.type != kQ6_K || !t.pq) return (int)hipErrorInvalidValue;
    const size_t total = (size_t)t.rows_pad * t.nb * 4;
    hipLaunchKernelGGL(q6_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, t);
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

int tmq_launch_fit(const TmqTensorDev& t, int all_exact, hipStream_t s) {
    if (!t.pe || t.clamp) return (int)hipErrorInvalidValue;
    const dim3 grid((t.rows_pad + 255) / 256, t.nb);
    switch (t.type) {
    case kQ5_0: hipLaunchKernelGGL(fit_kernel<kQ5_0>, grid, dim3(256), 0, s, t, all_exact); break;
    case kQ4_K: hipLaunchKernelGGL(fit_kernel<kQ4_K>, grid, dim3(256), 0, s, t, all_exact); break;
    case kQ6_K: hipLaunchKernelGGL(fit_kernel<kQ6_K>, grid, dim3(256), 0, s, t, all_exact); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int tmq_launch_ifit(const TmqTensorDev& t, int pass, uint8_t* cnt, const int32_t* off, uint4* corr,
                    hipStream_t s) {
    if (!t.pi || t.clamp) return (int)hipErrorInvalidValue;
    const char* fe = getenv("TMQ_IFIT_FORCE");
    const int force = fe && atoi(fe) != 0;
    const int ns = tmq_ifit_subs(t.type);
    if (!ns) return (int)hipErrorInvalidValue;
    const dim3 grid((t.rows_pad + 255) / 256, t.nb * ns);
    if (t.type == kQ5_0) hipLaunchKernelGGL(ifit_kernel, grid, dim3(256), 0, s, t, pass, force, cnt, off, corr);
    else if (t.type == kQ4_K) hipLaunchKernelGGL(ikfit_kernel<kQ4_K>, grid, dim3(256), 0, s, t, pass, force, cnt, off, corr);
    else hipLaunchKernelGGL(ikfit_kernel<kQ6_K>, grid, dim3(256), 0, s, t, pass, force, cnt, off, corr);
    return (int)hipGetLastError();
}

template <template <int, bool> class K>
static void* kernel_for(int type, int clamp) {
    switch (type) {
    case kQ5_0M: return clamp ? nullptr : (void*)K<kQ5_0M, false>::fn();
    case kQ4_KM: return clamp ? nullptr : (void*)K<kQ4_KM, false>::fn();
    case kQ6_KM: return clamp ? nullptr : (void*)K<kQ6_KM, false>::fn();
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
    if (w.path != TMQ_WPATH_FPGA) {
        // INT16 / FP32 paths: 4 waves of 64 rows per workgroup
        if (w.path == TMQ_WPATH_INT16 && (!w.t.pw || !w.t.rs16 || !w.act)) return (int)hipErrorInvalidValue;
        if (w.path == TMQ_WPATH_FP32 && !w.xf) return (int)hipErrorInvalidValue;
        const int g = (w.t.rows_pad / 64 + TMQ_WAVES - 1) / TMQ_WAVES;
        if (w.path == TMQ_WPATH_INT16) hipLaunchKernelGGL(i16_gemv_kernel, dim3(g), dim3(64 * TMQ_WAVES), 0, s, w);
        else hipLaunchKernelGGL(f32_gemv_kernel, dim3(g), dim3(64 * TMQ_WAVES), 0, s, w);
        return (int)hipGetLastError();
    }
    const int fmt = tmq_kernel_fmt(w.t);
    void* k = kernel_for<GemvK>(fmt, w.t.clamp);
    if (!k) return (int)hipErrorInvalidValue;
    TmqWork arg = w;
    void* args[] = {&arg};
    return (int)hipLaunchKernel(k, dim3(w.ngroups), dim3(64 * gemv_waves(fmt)), args,
                                tmq_gemv_lds_bytes(fmt, w.t.cols), s);
}

size_t tmq_gemv_lds_bytes(int fmt, int max_cols) {
    const int nbx = min(max_cols, TMQ_MFMA_MAX_COLS) / 32;
    if (fmt == kQ5_0M) return (size_t)mfma_lds_bytes(nbx);
    if (fmt == kQ4_KM) return (size_t)kq_lds_bytes<kQ4_K>(nbx);
    if (fmt == kQ6_KM) return (size_t)kq_lds_bytes<kQ6_K>(nbx);
    return 0;
}

int tmq_launch_chain(int fmt, int clamp, int max_cols, const TmqWork* works_dev, const TmqGroupRef* groups_dev,
                     int total_groups, int split, uint64_t* tail, hipStream_t s) {
    if (total_groups <= 0) return 0;
    void* k = kernel_for<ChainK>(fmt, clamp);
    if (!k) return (int)hipErrorInvalidValue;
    size_t lds = tmq_gemv_lds_bytes(fmt, max_cols);
    if (fmt == kQ8_0 && split) {
        if (max_cols > TMQ_Q8_SPLIT_COLS) return (int)hipErrorInvalidValue;
        lds = (size_t)((max_cols + 63) / 64) * 64 * 8;
    }
    void* args[] = {&works_dev, &groups_dev, &tail};
    return (int)hipLaunchKernel(k, dim3(total_groups), dim3(64 * gemv_waves(fmt)), args, lds, s);
}

int tmq_launch_resid_view(const float* x, const TmqDeferred& d, int n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(resid_view_kernel, dim3((n + 255) / 256), dim3(256), 0, s, x, d, n, out);
    return (int)hipGetLastError();
}

int tmq_launch_zero_acc(int64_t* p, size_t n, hipStream_t s) {
    if (!n) return 0;
    size_t g = (n + 255) / 256;
    if (g > 1024) g = 1024;
    hipLaunchKernelGGL(zero_acc_kernel, dim3((unsigned)g), dim3(256), 0, s, p, n);
    return (int)hipGetLastError();
}

size_t tmq_eng_lds_bytes(int n, int waves, int fa, int fb) {
    const size_t rb = std::max(eng_ring_bytes(fa, waves), eng_ring_bytes(fb, waves));
    const bool mx = fa == kQ5_0M || fa == kQ4_KM || fa == kQ6_KM || fb == kQ5_0M || fb == kQ4_KM || fb == kQ6_KM;
    return eng_base_bytes(n, waves) + rb + (mx && eng_mx_bytes(n) > 4 * (size_t)n ? eng_mx_bytes(n) : 0);
}

template <int NW, bool MULTI>
static void* eng_kernel_for(int fa, int fb) {
#define TMQ_ENG_K(A, B) (void*)eng_gemv_kernel<NW, A, B, MULTI>
    if (fa == kQ5_0 && fb == kQ5_0) return TMQ_ENG_K(kQ5_0, kQ5_0);
    if (fa == kQ5_0 && fb == kQ8_0) return TMQ_ENG_K(kQ5_0, kQ8_0);
    if (fa == kQ5_0M && fb == kQ5_0M) return TMQ_ENG_K(kQ5_0M, kQ5_0M);
    if (fa == kQ5_0M && fb == kQ8_0) return TMQ_ENG_K(kQ5_0M, kQ8_0);
    if constexpr (NW == 4) {
        // the K-quant MFMA decoders take a quarter super-block per wave
        if (fa == kQ4_KM && fb == kQ4_KM) return TMQ_ENG_K(kQ4_KM, kQ4_KM);
        if (fa == kQ6_KM && fb == kQ6_KM) return TMQ_ENG_K(kQ6_KM, kQ6_KM);
    }
    if (fa == kQ4_K && fb == kQ4_K) return TMQ_ENG_K(kQ4_K, kQ4_K);
    if (fa == kQ6_K && fb == kQ6_K) return TMQ_ENG_K(kQ6_K, kQ6_K);
    if (fa == kQ8_0 && fb == kQ8_0) return TMQ_ENG_K(kQ8_0, kQ8_0);
    if (fa == kQ8_DIRECT && fb == kQ8_DIRECT) return TMQ_ENG_K(kQ8_DIRECT, kQ8_DIRECT);
    if constexpr (NW == 4) {
        // the INT16 / FP32 branches (4-wave launches only)
        if (fa == kI16 && fb == kI16) return TMQ_ENG_K(kI16, kI16);
        if (fa == kF32P && fb == kF32P) return TMQ_ENG_K(kF32P, kF32P);
        if constexpr (MULTI) {
            if (fa == kQ5_0 && fb == kI16) return TMQ_ENG_K(kQ5_0, kI16);
            if (fa == kI16 && fb == kQ8_0) return TMQ_ENG_K(kI16, kQ8_0);
        } else {
            if (fa == kI16_DIRECT && fb == kI16_DIRECT) return TMQ_ENG_K(kI16_DIRECT, kI16_DIRECT);
        }
    }
#undef TMQ_ENG_K
    return nullptr;
}

// The kernel and dynamic LDS of an engine launch (checks its shape); the
// kernel opted into its LDS when that is above 64 KiB.
static int eng_resolve(const TmqEngLaunch& l, int waves, void** kernel, size_t* lds) {
    if (l.act.n <= 0 || l.act.n > TMQ_ENG_MAXN || l.act.n % 2 || l.nworks < 1 || l.nworks > TMQ_ENG_MAXW)
        return (int)hipErrorInvalidValue;
    // format of the first and the last work (the others must match the first)
    auto code = [](const TmqWork& w) {
        if (w.path == TMQ_WPATH_INT16) return w.kacc ? kI16 : kI16_DIRECT;
        if (w.path == TMQ_WPATH_FP32) return kF32P;
        if (w.t.type == kQ8_0) return w.kacc ? kQ8_0 : kQ8_DIRECT;
        // the MFMA decoders where the tensor carries their planes
        return tmq_kernel_fmt(w.t);
    };
    const int fa = code(l.w[0]), fb = code(l.w[l.nworks - 1]);
    for (int i = 1; i + 1 < l.nworks; i++)
        if (code(l.w[i]) != fa) return (int)hipErrorInvalidValue;
    // the kernels split a row's units (or Q8_0 tiles) into kc chunks in int32
    for (int i = 0; i < l.nworks; i++) {
        if ((int64_t)l.w[i].t.nb * 4 * (l.w[i].kc > 0 ? l.w[i].kc : 1) >= ((int64_t)1 << 31))
            return (int)hipErrorInvalidValue;
        // MFMA chunks are whole blocks / super-blocks of a row of at most
        // TMQ_MFMA_MAX_COLS columns, the activation's width
        const int f = code(l.w[i]);
        if ((f == kQ5_0M || f == kQ4_KM || f == kQ6_KM) &&
            (l.w[i].kc < 1 || l.w[i].kc > l.w[i].t.nb || l.w[i].t.cols != l.act.n || l.act.n % 32))
            return (int)hipErrorInvalidValue;
        if (l.w[i].path == TMQ_WPATH_INT16 && (!l.w[i].t.pw || !l.w[i].t.rs16)) return (int)hipErrorInvalidValue;
        if (l.w[i].path == TMQ_WPATH_FP32 && l.w[i].t.cols != l.act.n) return (int)hipErrorInvalidValue;
    }
    void* k = nullptr;
    if (l.nworks > 1) k = waves == 16 ? eng_kernel_for<16, true>(fa, fb) : waves == 4 ? eng_kernel_for<4, true>(fa, fb) : nullptr;
    else k = waves == 16 ? eng_kernel_for<16, false>(fa, fb) : waves == 4 ? eng_kernel_for<4, false>(fa, fb) : nullptr;
    if (!k) return (int)hipErrorInvalidValue;
    if (l.rope_out && (!l.rope_src || !l.rope_state || l.rope_max_pos < 1)) return (int)hipErrorInvalidValue;
    *lds = tmq_eng_lds_bytes(l.act.n, waves, fa, fb);
    *kernel = k;
    if (*lds > 64 * 1024) {
        // (once per kernel: dynamic LDS above 64 KiB is opted into)
        static std::mutex mu;
        static std::set<void*> done;
        std::lock_guard<std::mutex> lk(mu);
        if (!done.count(k)) {
            hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            if (e != hipSuccess) return (int)e;
            done.insert(k);
        }
    }
    return 0;
}

int tmq_prepare_eng_gemv(const TmqEngLaunch& l, int waves) {
    void* k = nullptr;
    size_t lds = 0;
    return eng_resolve(l, waves, &k, &lds);
}

int tmq_launch_eng_gemv(const TmqEngLaunch& l, int waves, hipStream_t s) {
    if (l.ngroups <= 0) return 0;
    void* k = nullptr;
    size_t lds = 0;
    const int rc = eng_resolve(l, waves, &k, &lds);
    if (rc) return rc;
    TmqEngLaunch arg = l;
    void* args[] = {&arg};
    return (int)hipLaunchKernel(k, dim3(l.ngroups + (l.rope_out ? 1 : 0)), dim3(64 * waves), args, lds, s);
}

int tmq_launch_silu(const TmqDeferred& g, const TmqDeferred& u, int n, float* x, uint32_t* max_bits,
                    hipStream_t s) {
    hipLaunchKernelGGL(silu_kernel, dim3((n + 255) / 256), dim3(256), 0, s, g, u, n, x, max_bits);
    return (int)hipGetLastError();
}

int tmq_launch_tile_q8(const uint8_t* W, const uint16_t* cs, const int16_t* vec, int64_t* out,
                       hipStream_t s) {
    hipLaunchKernelGGL(tile_q8_kernel, dim3(1), dim3(64), 0, s, W, cs, vec, out);
    return (int)hipGetLastError();
}

int tmq_launch_q8_scales(const TmqTensorDev& t, uint16_t* out, hipStream_t s) {
    if (t.type != kQ8_0) return (int)hipErrorInvalidValue;
    const size_t n = (size_t)t.rows * t.nb;
    hipLaunchKernelGGL(q8_scales_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, t, out);
    return (int)hipGetLastError();
}

int tmq_launch_i16_prep(const TmqTensorDev& t, hipStream_t s) {
    if (!t.pw || !t.rs16) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(i16_prep_kernel, dim3(t.rows_pad / 64), dim3(64), 0, s, t);
    return (int)hipGetLastError();
}

int tmq_launch_check_finite(const TmqTensorDev& t, int* bad, hipStream_t s) {
    hipLaunchKernelGGL(check_finite_kernel, dim3(t.rows_pad / 64), dim3(64), 0, s, t, bad);
    return (int)hipGetLastError();
}

// ------------------------------------------------------ prefill operands
int tmq_launch_pf_wdigits(const TmqTensorDev& t, int8_t* planes, int K, int row0, hipStream_t s) {
    if (t.cols != K || K % TMQ_PF_CHUNK || row0 % 32) return (int)hipErrorInvalidValue;
    const dim3 grid((t.rows + 63) / 64), blk(64);
    switch (t.type) {
    case kQ5_0: hipLaunchKernelGGL(pf_wdigits_kernel<kQ5_0>, grid, blk, 0, s, t, planes, K, row0); break;
    case kQ8_0: hipLaunchKernelGGL(pf_wdigits_kernel<kQ8_0>, grid, blk, 0, s, t, planes, K, row0); break;
    case kQ4_K: hipLaunchKernelGGL(pf_wdigits_kernel<kQ4_K>, grid, blk, 0, s, t, planes, K, row0); break;
    case kQ6_K: hipLaunchKernelGGL(pf_wdigits_kernel<kQ6_K>, grid, blk, 0, s, t, planes, K, row0); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int tmq_launch_pf_rowsums(const TmqPfPlanes& p, hipStream_t s) {
    if (p.rows <= 0 || p.rows % 32 || p.K % TMQ_PF_CHUNK) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(pf_rowsums_kernel, dim3(p.rows), dim3(64), 0, s, p);
    return (int)hipGetLastError();
}

int tmq_launch_pf_act(const TmqPfAct& a, hipStream_t s) {
    if (a.n % TMQ_PF_CHUNK || a.n > TMQ_ENG_MAXN || a.out.rows < a.T || a.out.rows % 32 || a.out.K != a.n)
        return (int)hipErrorInvalidValue;
    // groups of four columns per thread: 1, 2, 5 or 8 (wider rows take the
    // kernel's one-group-at-a-time path)
    const int groups = (a.n / 4 + 255) / 256;
    const dim3 grid(a.out.rows), blk(256);
    const size_t lds = 8 * (size_t)a.n;
    if (groups <= 1) hipLaunchKernelGGL(pf_act_kernel<1>, grid, blk, lds, s, a);
    else if (groups <= 2) hipLaunchKernelGGL(pf_act_kernel<2>, grid, blk, lds, s, a);
    else if (groups <= 5) hipLaunchKernelGGL(pf_act_kernel<5>, grid, blk, lds, s, a);
    else hipLaunchKernelGGL(pf_act_kernel<8>, grid, blk, lds, s, a);
    return (int)hipGetLastError();
}
