// tmq_device.h -- device helpers shared by the kernel sources.
#pragma once
#include <hip/hip_runtime.h>

#include "tmq_internal.h"

// The kernel's arguments into the scalar cache in one round trip: one
// s_load_dword per 64-byte line of the argument struct (in one asm statement
// so that nothing is scheduled between them), then one wait.  The compiler
// otherwise loads them where each is first needed, behind the branches that
// depend on earlier ones: a round trip (~0.3 us) each.  The loaded values are
// not used: the destinations are scratch registers the compiler picks (dead
// after the statement), so the kernel's SGPR count, which bounds how many
// waves a SIMD holds, does not grow.
template <int BYTES>
static __device__ __forceinline__ void tmq_warm_kernargs() {
    constexpr int N = (BYTES + 63) / 64;
    static_assert(N >= 1 && N <= 16, "one to sixteen lines");
    const auto p = __builtin_amdgcn_kernarg_segment_ptr();
    int d[16];
    if constexpr (N == 1)
        asm volatile("s_load_dword %0, %1, 0x0\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]) : "s"(p) : "memory");
    else if constexpr (N == 2)
        asm volatile("s_load_dword %0, %2, 0x0\n" "s_load_dword %1, %2, 0x40\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]) : "s"(p) : "memory");
    else if constexpr (N == 3)
        asm volatile("s_load_dword %0, %3, 0x0\n" "s_load_dword %1, %3, 0x40\n" "s_load_dword %2, %3, 0x80\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]) : "s"(p) : "memory");
    else if constexpr (N == 4)
        asm volatile("s_load_dword %0, %4, 0x0\n" "s_load_dword %1, %4, 0x40\n" "s_load_dword %2, %4, 0x80\n" "s_load_dword %3, %4, 0xc0\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]) : "s"(p) : "memory");
    else if constexpr (N == 5)
        asm volatile("s_load_dword %0, %5, 0x0\n" "s_load_dword %1, %5, 0x40\n" "s_load_dword %2, %5, 0x80\n" "s_load_dword %3, %5, 0xc0\n" "s_load_dword %4, %5, 0x100\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]) : "s"(p) : "memory");
    else if constexpr (N == 6)
        asm volatile("s_load_dword %0, %6, 0x0\n" "s_load_dword %1, %6, 0x40\n" "s_load_dword %2, %6, 0x80\n" "s_load_dword %3, %6, 0xc0\n" "s_load_dword %4, %6, 0x100\n" "s_load_dword %5, %6, 0x140\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]) : "s"(p) : "memory");
    else if constexpr (N == 7)
        asm volatile("s_load_dword %0, %7, 0x0\n" "s_load_dword %1, %7, 0x40\n" "s_load_dword %2, %7, 0x80\n" "s_load_dword %3, %7, 0xc0\n" "s_load_dword %4, %7, 0x100\n" "s_load_dword %5, %7, 0x140\n" "s_load_dword %6, %7, 0x180\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]) : "s"(p) : "memory");
    else if constexpr (N == 8)
        asm volatile("s_load_dword %0, %8, 0x0\n" "s_load_dword %1, %8, 0x40\n" "s_load_dword %2, %8, 0x80\n" "s_load_dword %3, %8, 0xc0\n" "s_load_dword %4, %8, 0x100\n" "s_load_dword %5, %8, 0x140\n" "s_load_dword %6, %8, 0x180\n" "s_load_dword %7, %8, 0x1c0\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]) : "s"(p) : "memory");
    else if constexpr (N == 9)
        asm volatile("s_load_dword %0, %9, 0x0\n" "s_load_dword %1, %9, 0x40\n" "s_load_dword %2, %9, 0x80\n" "s_load_dword %3, %9, 0xc0\n" "s_load_dword %4, %9, 0x100\n" "s_load_dword %5, %9, 0x140\n" "s_load_dword %6, %9, 0x180\n" "s_load_dword %7, %9, 0x1c0\n" "s_load_dword %8, %9, 0x200\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]) : "s"(p) : "memory");
    else if constexpr (N == 10)
        asm volatile("s_load_dword %0, %10, 0x0\n" "s_load_dword %1, %10, 0x40\n" "s_load_dword %2, %10, 0x80\n" "s_load_dword %3, %10, 0xc0\n" "s_load_dword %4, %10, 0x100\n" "s_load_dword %5, %10, 0x140\n" "s_load_dword %6, %10, 0x180\n" "s_load_dword %7, %10, 0x1c0\n" "s_load_dword %8, %10, 0x200\n" "s_load_dword %9, %10, 0x240\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]) : "s"(p) : "memory");
    else if constexpr (N == 11)
        asm volatile("s_load_dword %0, %11, 0x0\n" "s_load_dword %1, %11, 0x40\n" "s_load_dword %2, %11, 0x80\n" "s_load_dword %3, %11, 0xc0\n" "s_load_dword %4, %11, 0x100\n" "s_load_dword %5, %11, 0x140\n" "s_load_dword %6, %11, 0x180\n" "s_load_dword %7, %11, 0x1c0\n" "s_load_dword %8, %11, 0x200\n" "s_load_dword %9, %11, 0x240\n" "s_load_dword %10, %11, 0x280\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]), "=&s"(d[10]) : "s"(p) : "memory");
    else if constexpr (N == 12)
        asm volatile("s_load_dword %0, %12, 0x0\n" "s_load_dword %1, %12, 0x40\n" "s_load_dword %2, %12, 0x80\n" "s_load_dword %3, %12, 0xc0\n" "s_load_dword %4, %12, 0x100\n" "s_load_dword %5, %12, 0x140\n" "s_load_dword %6, %12, 0x180\n" "s_load_dword %7, %12, 0x1c0\n" "s_load_dword %8, %12, 0x200\n" "s_load_dword %9, %12, 0x240\n" "s_load_dword %10, %12, 0x280\n" "s_load_dword %11, %12, 0x2c0\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]), "=&s"(d[10]), "=&s"(d[11]) : "s"(p) : "memory");
    else if constexpr (N == 13)
        asm volatile("s_load_dword %0, %13, 0x0\n" "s_load_dword %1, %13, 0x40\n" "s_load_dword %2, %13, 0x80\n" "s_load_dword %3, %13, 0xc0\n" "s_load_dword %4, %13, 0x100\n" "s_load_dword %5, %13, 0x140\n" "s_load_dword %6, %13, 0x180\n" "s_load_dword %7, %13, 0x1c0\n" "s_load_dword %8, %13, 0x200\n" "s_load_dword %9, %13, 0x240\n" "s_load_dword %10, %13, 0x280\n" "s_load_dword %11, %13, 0x2c0\n" "s_load_dword %12, %13, 0x300\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]), "=&s"(d[10]), "=&s"(d[11]), "=&s"(d[12]) : "s"(p) : "memory");
    else if constexpr (N == 14)
        asm volatile("s_load_dword %0, %14, 0x0\n" "s_load_dword %1, %14, 0x40\n" "s_load_dword %2, %14, 0x80\n" "s_load_dword %3, %14, 0xc0\n" "s_load_dword %4, %14, 0x100\n" "s_load_dword %5, %14, 0x140\n" "s_load_dword %6, %14, 0x180\n" "s_load_dword %7, %14, 0x1c0\n" "s_load_dword %8, %14, 0x200\n" "s_load_dword %9, %14, 0x240\n" "s_load_dword %10, %14, 0x280\n" "s_load_dword %11, %14, 0x2c0\n" "s_load_dword %12, %14, 0x300\n" "s_load_dword %13, %14, 0x340\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]), "=&s"(d[10]), "=&s"(d[11]), "=&s"(d[12]), "=&s"(d[13]) : "s"(p) : "memory");
    else if constexpr (N == 15)
        asm volatile("s_load_dword %0, %15, 0x0\n" "s_load_dword %1, %15, 0x40\n" "s_load_dword %2, %15, 0x80\n" "s_load_dword %3, %15, 0xc0\n" "s_load_dword %4, %15, 0x100\n" "s_load_dword %5, %15, 0x140\n" "s_load_dword %6, %15, 0x180\n" "s_load_dword %7, %15, 0x1c0\n" "s_load_dword %8, %15, 0x200\n" "s_load_dword %9, %15, 0x240\n" "s_load_dword %10, %15, 0x280\n" "s_load_dword %11, %15, 0x2c0\n" "s_load_dword %12, %15, 0x300\n" "s_load_dword %13, %15, 0x340\n" "s_load_dword %14, %15, 0x380\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]), "=&s"(d[10]), "=&s"(d[11]), "=&s"(d[12]), "=&s"(d[13]), "=&s"(d[14]) : "s"(p) : "memory");
    else if constexpr (N == 16)
        asm volatile("s_load_dword %0, %16, 0x0\n" "s_load_dword %1, %16, 0x40\n" "s_load_dword %2, %16, 0x80\n" "s_load_dword %3, %16, 0xc0\n" "s_load_dword %4, %16, 0x100\n" "s_load_dword %5, %16, 0x140\n" "s_load_dword %6, %16, 0x180\n" "s_load_dword %7, %16, 0x1c0\n" "s_load_dword %8, %16, 0x200\n" "s_load_dword %9, %16, 0x240\n" "s_load_dword %10, %16, 0x280\n" "s_load_dword %11, %16, 0x2c0\n" "s_load_dword %12, %16, 0x300\n" "s_load_dword %13, %16, 0x340\n" "s_load_dword %14, %16, 0x380\n" "s_load_dword %15, %16, 0x3c0\n" "s_waitcnt lgkmcnt(0)" : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]), "=&s"(d[10]), "=&s"(d[11]), "=&s"(d[12]), "=&s"(d[13]), "=&s"(d[14]), "=&s"(d[15]) : "s"(p) : "memory");
    (void)d;
}

// Wave reductions by DPP lane moves (VALU only; __shfl_xor is a chain of six
// LDS round trips): pairs and quads (quad permutations), rows of 8 and 16
// (half-row and row mirrors), row 0 into row 1 and row 2 into row 3
// (row_bcast15), rows 0-1 into rows 2-3 (row_bcast31); lane 63 then holds
// the whole wave's value.  `old` is what a lane that a move leaves without a
// source reads: the identity of the operation.
template <int CTRL, int ROW_MASK = 0xf>
static __device__ __forceinline__ int tmq_dpp_i32(int v, int old) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xf, false);
}
// fmaxf over the wave, the same value in every lane (a quiet NaN is fmaxf's
// identity; fmaxf picks the same value in any order for the inputs used
// here, which hold no -0)
static __device__ __forceinline__ float tmq_wave_max(float x) {
    const int q = 0x7fc00000;
    x = fmaxf(x, __int_as_float(tmq_dpp_i32<0xb1>(__float_as_int(x), q)));
    x = fmaxf(x, __int_as_float(tmq_dpp_i32<0x4e>(__float_as_int(x), q)));
    x = fmaxf(x, __int_as_float(tmq_dpp_i32<0x141>(__float_as_int(x), q)));
    x = fmaxf(x, __int_as_float(tmq_dpp_i32<0x140>(__float_as_int(x), q)));
    x = fmaxf(x, __int_as_float(tmq_dpp_i32<0x142, 0xa>(__float_as_int(x), q)));
    x = fmaxf(x, __int_as_float(tmq_dpp_i32<0x143, 0xc>(__float_as_int(x), q)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}
// integer sum over each 16-lane row, in every lane of the row
static __device__ __forceinline__ int tmq_row_sum(int x) {
    x += tmq_dpp_i32<0xb1>(x, 0);
    x += tmq_dpp_i32<0x4e>(x, 0);
    x += tmq_dpp_i32<0x141>(x, 0);
    x += tmq_dpp_i32<0x140>(x, 0);
    return x;
}
// integer sum over the wave, the same value in every lane
static __device__ __forceinline__ int tmq_wave_sum(int x) {
    x = tmq_row_sum(x);
    x += tmq_dpp_i32<0x142, 0xa>(x, 0);
    x += tmq_dpp_i32<0x143, 0xc>(x, 0);
    return __builtin_amdgcn_readlane(x, 63);
}

// int64 row sums of a K-split GEMV live at the device coherence point
// (device-scope atomics); reads go there too.
static __device__ __forceinline__ int64_t tmq_ld_acc(const int64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Row i of a K-split GEMV, finalised (TmqDeferred).
static __device__ float tmq_fin(const TmqDeferred& D, int i) {
    const double xs = (double)*D.xs;
    float v;
    if (D.val) {
        v = __hip_atomic_load(D.val + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (D.ntiles == 0) {
        v = (float)(((double)tmq_ld_acc(D.acc + i) * xs) / (double)D.row_inv[i]);
    } else {
        const double rs = (double)D.row_scale[i];
        float y = 0.0f;
        for (int t = 0; t < D.ntiles; t++)
            y = (float)((double)y + ((double)tmq_ld_acc(D.acc + (size_t)i * D.ntiles + t) * xs) * rs);
        v = y;
    }
    if (D.bias) v = v + D.bias[i];
    return v;
}

// tmq_fin split in two, so that a kernel can issue the loads of several
// deferred values before it waits for any of them: fin_load takes the raw
// terms of row i (no branch on the data; Q8 selects the tiled form, up to
// TMQ_FIN_MAXT tiles), fin_finish forms the value as tmq_fin does.
#define TMQ_FIN_MAXT 16
template <bool Q8>
struct TmqFinRaw {
    int64_t p[Q8 ? TMQ_FIN_MAXT : 1];
    float r, b;
};
template <bool Q8>
static __device__ __forceinline__ TmqFinRaw<Q8> fin_load(const TmqDeferred& D, int i) {
    TmqFinRaw<Q8> f;
    if (D.val) {
        // FP32 path: the value itself (its bits in p[0])
#pragma unroll
        for (int t = 0; t < (Q8 ? TMQ_FIN_MAXT : 1); t++) f.p[t] = 0;
        f.p[0] = (int64_t)__float_as_uint(__hip_atomic_load(D.val + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        f.r = 1.0f;
    } else if constexpr (Q8) {
        const int nt = D.ntiles;
#pragma unroll
        for (int t = 0; t < TMQ_FIN_MAXT; t++) f.p[t] = tmq_ld_acc(D.acc + (size_t)i * nt + min(t, nt - 1));
        f.r = D.row_scale[i];
    } else {
        f.p[0] = tmq_ld_acc(D.acc + i);
        f.r = D.row_inv[i];
    }
    // no bias: any valid row vector stands in (the value is not used)
    const float* bp = D.bias ? D.bias : D.val ? D.val : Q8 ? D.row_scale : D.row_inv;
    f.b = bp[i];
    return f;
}
template <bool Q8>
static __device__ __forceinline__ float fin_finish(const TmqDeferred& D, const TmqFinRaw<Q8>& f, double xs) {
    float v;
    if (D.val) {
        v = __uint_as_float((uint32_t)f.p[0]);
    } else if constexpr (Q8) {
        const double rs = (double)f.r;
        float y = 0.0f;
#pragma unroll
        for (int t = 0; t < TMQ_FIN_MAXT; t++)
            if (t < D.ntiles) y = (float)((double)y + ((double)f.p[t] * xs) * rs);
        v = y;
    } else {
        v = (float)(((double)f.p[0] * xs) / (double)f.r);
    }
    if (D.bias) v = v + f.b;
    return v;
}

