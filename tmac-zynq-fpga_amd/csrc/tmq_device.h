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
    if (D.ntiles == 0) {
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
