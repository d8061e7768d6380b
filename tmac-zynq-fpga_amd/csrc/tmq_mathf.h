// tmq_mathf.h -- fp32 transcendental functions matching the reference host.
//
// The reference engine calls glibc's expf/logf (sim/tmac_gguf.cpp:460,
// :1650-1654).  glibc 2.35 implements expf with the table-driven method of
// Szabolcs Nagy (Arm optimized-routines, "expf.c", MIT/Apache-2.0): with
// N = 32, x*N/ln2 = k + r, exp(x) = 2^(k/N) * p(r) where p is a cubic
// evaluated in double.  The x86-64 build used on FMA-capable hosts contracts
// every multiply-add into an fma.  tmq_expf restates that method; the table
// is the correctly rounded 2^(i/32) minus (i << 47) (derivable from first
// principles).  It agrees with the host's expf on all 2^32 inputs.
//
// logf: glibc 2.35 implements logf with the same author's method (Arm
// optimized-routines "logf.c"): x = 2^k z with z in [0x3f330000, 2x that),
// the top 4 mantissa bits of z - 0x3f330000 pick a pair (1/c, log c) with c
// near the centre of the subinterval, r = z/c - 1 exactly in double, and
// log x = k ln2 + log c + r + A0 r^4 + (A1 r + A2) r^2 in double, rounded
// once to float (0.82 ulp at most).  tmq_logf restates it with that
// published table and polynomial; it agrees with the host's logf on all
// 2^32 inputs, in the fma form used here and in the separate form alike.
#pragma once
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define TMQ_HD __host__ __device__
#else
#define TMQ_HD
#endif

namespace tmq_math {

TMQ_HD inline double as_double(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}
TMQ_HD inline uint64_t as_u64(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}
TMQ_HD inline uint32_t as_u32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// 2^(i/32), correctly rounded, with i<<47 subtracted from the bit pattern so
// that adding k<<47 for k = i + 32*m scales it by 2^m.  A table in constant
// memory on the device (lanes index it independently).
#define TMQ_EXP2_TAB                                                                       \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}
#if defined(__HIPCC__)
static __constant__ uint64_t tmq_exp2_tab_dev[32] = TMQ_EXP2_TAB;
#endif
static const uint64_t tmq_exp2_tab_host[32] = TMQ_EXP2_TAB;

TMQ_HD inline uint64_t exp2_tab(int i) {
#if defined(__HIP_DEVICE_COMPILE__)
    return tmq_exp2_tab_dev[i];
#else
    return tmq_exp2_tab_host[i];
#endif
}

// The table read through a functor, so that a kernel can keep a copy in LDS.
struct Exp2TabConst {
    TMQ_HD uint64_t operator()(int i) const { return exp2_tab(i); }
};

template <class Tab>
TMQ_HD inline float tmq_expf_tab(float x, const Tab& tab) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double Shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const uint32_t abstop = (as_u32(x) >> 20) & 0x7ffu;
    if (abstop >= (as_u32(88.0f) >> 20)) {
        if (as_u32(x) == 0xff800000u) return 0.0f;          // -inf
        if (abstop >= (0x7f800000u >> 20)) return x + x;     // +inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();      // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                 // underflow
    }
    const double xd = (double)x;
    double kd = __builtin_fma(InvLn2N, xd, Shift);
    const uint64_t ki = as_u64(kd);
    kd -= Shift;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    const uint64_t t = tab((int)(ki % 32)) + (ki << 47);
    const double s = as_double(t);
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

TMQ_HD inline float tmq_expf(float x) { return tmq_expf_tab(x, Exp2TabConst{}); }

// (1/c, log c) of the 16 subintervals of logf's reduced argument
#define TMQ_LOGF_TAB                                                                                   \
    {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2, 0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2,     \
     0x1.49539f0f010bp+0,  -0x1.01eae7f513a67p-2, 0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3,     \
     0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3, 0x1.25e227b0b8eap+0,  -0x1.1aa2bc79c81p-3,       \
     0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4, 0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4,     \
     0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5, 0x1p+0,               0x0p+0,                    \
     0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5,  0x1.ca4b31f026aap-1,  0x1.c5e53aa362eb4p-4,      \
     0x1.b2036576afce6p-1, 0x1.526e57720db08p-3,  0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3,       \
     0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2,  0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2}
#if defined(__HIPCC__)
static __constant__ double tmq_logf_tab_dev[32] = TMQ_LOGF_TAB;
#endif
static const double tmq_logf_tab_host[32] = TMQ_LOGF_TAB;

TMQ_HD inline double logf_tab(int j) {
#if defined(__HIP_DEVICE_COMPILE__)
    return tmq_logf_tab_dev[j];
#else
    return tmq_logf_tab_host[j];
#endif
}

TMQ_HD inline float tmq_logf(float x) {
    const double Ln2 = 0x1.62e42fefa39efp-1;
    const double A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2, A2 = -0x1.ffffef20a4123p-2;
    uint32_t ix = as_u32(x);
    if (ix == 0x3f800000u) return 0.0f;
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
        if (ix * 2 == 0) return -__builtin_inff();                           // log(+-0)
        if (ix == 0x7f800000u) return x;                                     // log(inf)
        if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u) return __builtin_nanf("");
        ix = as_u32(x * 0x1p23f) - (23u << 23);                              // subnormal
    }
    const uint32_t tmp = ix - 0x3f330000u;
    const int i = (int)((tmp >> 19) % 16);
    const int k = (int32_t)tmp >> 23;
    const uint32_t iz = ix - (tmp & 0xff800000u);
    float zf;
    memcpy(&zf, &iz, 4);
    const double invc = logf_tab(2 * i), logc = logf_tab(2 * i + 1);
    const double r = __builtin_fma((double)zf, invc, -1.0);
    const double y0 = __builtin_fma((double)k, Ln2, logc);
    const double r2 = r * r;
    double y = __builtin_fma(A1, r, A2);
    y = __builtin_fma(A0, r2, y);
    y = __builtin_fma(y, r2, y0 + r);
    return (float)y;
}

// RoPE factors for positions [0, max_pos), as apply_rope forms them on the
// host (sim/tmac_gguf.cpp:1531-1535): theta = 1/powf(base, (float)d/head_dim),
// freq = pos*theta, (cosf(freq), sinf(freq)) from the host libm.  out holds
// max_pos x head_dim/2 (cos, sin) pairs.  base is read through a volatile so
// that powf runs in the libm at run time, never folded at compile time.
// Host code only.
inline void rope_table(float base, int head_dim, int max_pos, float* out) {
    volatile float base_v = base;
    const float b = base_v;
    const int half = head_dim / 2;
    for (int d = 0; d < head_dim; d += 2) {
        const float theta = 1.0f / powf(b, (float)d / head_dim);
        for (int p = 0; p < max_pos; p++) {
            const float freq = p * theta;
            out[2 * ((size_t)p * half + d / 2)] = cosf(freq);
            out[2 * ((size_t)p * half + d / 2) + 1] = sinf(freq);
        }
    }
}

}  // namespace tmq_math
