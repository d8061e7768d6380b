// tmq_runtime.h -- host-side objects shared by the runtime sources
// (tmq_api.hip: contexts, tensors, chains; tmq_model.hip: the decode engine).
#pragma once
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/tmq.h"
#include "tmq_internal.h"

// Records the message for tmq_last_error() and returns code.
int tmq_fail(int code, const char* fmt, ...);

#define HIP_TRY(expr)                                                                       \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return tmq_fail(TMQ_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));   \
    } while (0)

#define LAUNCH_TRY(expr)                                                                    \
    do {                                                                                    \
        int e_ = (expr);                                                                    \
        if (e_ != 0)                                                                        \
            return tmq_fail(TMQ_ERR_HIP, "%s: %s", #expr, hipGetErrorString((hipError_t)e_)); \
    } while (0)

// growable device buffer
struct TmqDevBuf {
    void* p = nullptr;
    size_t cap = 0;
    int ensure(size_t n) {
        if (n <= cap) return 0;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        hipError_t e = hipMalloc(&p, n);
        if (e != hipSuccess) return tmq_fail(TMQ_ERR_NOMEM, "hipMalloc(%zu): %s", n, hipGetErrorString(e));
        cap = n;
        return 0;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

struct tmq_ctx {
    int device = 0;
    int ncu = 0;  // compute units of the device
    hipStream_t stream = nullptr;
    TmqDevBuf x, y, act, acc, misc, works, gmap;
};

struct tmq_tensor {
    tmq_ctx* ctx = nullptr;
    TmqTensorDev dev{};
    void* alloc = nullptr;  // planes + row_inv + row_scale
    void* i16_alloc = nullptr;  // INT16 path weights + row scales (tmq_tensor_prepare_int16)
    void* corr_alloc = nullptr;  // integer-fit corrections + their group offsets (MFMA decoders)
    uint64_t weight_bytes = 0;
};

int tmq_rt_set_device(tmq_ctx* ctx);
// 64-row groups of a tensor (Q8_0: 256-row groups, one per workgroup)
int tmq_rt_groups_of(const TmqTensorDev& t);
// upload ggml bytes (host or device) into a new tensor; normalisers computed
// on the device (aux = Q8_0 row_max_abs, optional); mfma: also build the
// planes of the standalone / chain GEMVs' MFMA decoders where the tensor
// qualifies (the decode engine's and prefill's kernels do not read them)
int tmq_rt_tensor_create(tmq_ctx* ctx, uint32_t type, uint64_t rows, uint64_t cols, const void* data,
                         bool data_on_device, uint64_t n_bytes, const float* aux, bool aux_on_device,
                         tmq_tensor** out, bool mfma);
TmqWork tmq_rt_make_work(const tmq_tensor* t, const uint8_t* act, float* y, int64_t* acc);
// builds the INT16 path planes of t once (matmul_fpga_int16's weights)
int tmq_rt_prepare_int16(tmq_ctx* ctx, tmq_tensor* t);
