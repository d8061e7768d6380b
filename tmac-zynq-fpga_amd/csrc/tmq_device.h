// tmq_device.h -- device helpers shared by the kernel sources.
#pragma once
#include <hip/hip_runtime.h>

#include "tmq_internal.h"

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

