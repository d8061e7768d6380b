// tmq_api.hip -- host runtime behind include/tmq.h.
//
// Owns contexts (device + stream + scratch), uploaded tensors (planes +
// per-row normalisers), descriptor chains, and the PhaseB arena replay.
// Nothing here computes on the CPU: every numeric result comes from the
// kernels in tmq_kernels.hip.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/tmq.h"
#include "tmq_internal.h"
#include "tmq_runtime.h"

namespace {
thread_local std::string g_err;
}  // namespace

// Scratch of tmq_gemv_dev_noalloc: the prepared activation of one GEMV
// (tmq_act_bytes(cols) bytes, cols <= TMQ_NOALLOC_MAX_COLS), in a
// file-scope device array that lives until the process ends.  Host code
// never uses the array's name as an address: tmq_open looks up each
// device's copy once (hipGetSymbolAddress, with that device current) and
// the entry point passes that pointer to the kernels.  Every call on one
// device shares its copy; calls that overlap on one device race on it.
#define TMQ_NOALLOC_SCRATCH_BYTES ((tmq_act_bytes(TMQ_NOALLOC_MAX_COLS) + 255) & ~(size_t)255)
static __device__ __align__(256) uint8_t scratch[TMQ_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// the device's copy of `scratch` (the device is current); once per device
int scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return tmq_fail(TMQ_ERR_ARG, "device %d >= %d", device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return 0;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return tmq_fail(TMQ_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g_scratch_ptr[device] = ptr;
    return 0;
}
void* scratch_of(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return device >= 0 && device < kMaxDevices ? g_scratch_ptr[device] : nullptr;
}
}  // namespace

int tmq_fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

namespace {

int qk_of(uint32_t type) {
    switch (type) {
    case TMQ_TYPE_Q8_0: case TMQ_TYPE_Q5_0: case TMQ_TYPE_F32: case TMQ_TYPE_F16: return 32;
    case TMQ_TYPE_Q4_K: case TMQ_TYPE_Q6_K: return 256;
    default: return 0;
    }
}
int block_bytes(uint32_t type) {
    switch (type) {
    case TMQ_TYPE_Q8_0: return 34;
    case TMQ_TYPE_Q5_0: return 22;
    case TMQ_TYPE_Q4_K: return 144;
    case TMQ_TYPE_Q6_K: return 210;
    case TMQ_TYPE_F32: return 128;  // 32 elements
    case TMQ_TYPE_F16: return 64;
    default: return 0;
    }
}
bool is_float_type(uint32_t type) { return type == TMQ_TYPE_F32 || type == TMQ_TYPE_F16; }
const char* type_name(uint32_t type) {
    switch (type) {
    case TMQ_TYPE_F32: return "F32";
    case TMQ_TYPE_F16: return "F16";
    case TMQ_TYPE_Q5_0: return "Q5_0";
    case TMQ_TYPE_Q8_0: return "Q8_0";
    case TMQ_TYPE_Q4_K: return "Q4_K";
    case TMQ_TYPE_Q6_K: return "Q6_K";
    default: return "?";
    }
}

struct Segment {
    int type, clamp, gmap_off, ngroups, max_cols;  // type: kernel format (tmq_kernel_fmt)
    int split;                                     // holds split groups
};

}  // namespace

struct tmq_chain {
    tmq_ctx* ctx = nullptr;
    std::vector<TmqWork> works;
    TmqActJobs jobs{};
    void* works_dev = nullptr;
    void* gmap_dev = nullptr;
    void* act_dev = nullptr;
    uint64_t* tail_dev = nullptr;  // tail slots of split groups (zero between launches)
    std::vector<Segment> segs;
    uint64_t weight_bytes = 0;
};

int tmq_rt_set_device(tmq_ctx* ctx) {
    HIP_TRY(hipSetDevice(ctx->device));
    return 0;
}

namespace {

int groups_of(const TmqTensorDev& t) {
    int g64 = t.rows_pad / TMQ_ROWS_PER_GROUP;
    if (t.type == TMQ_TYPE_Q8_0) return (g64 + TMQ_WAVES - 1) / TMQ_WAVES;
    return g64;
}

// Whether a tensor gets the MFMA decoders' planes (integer fit codes, and
// for Q6_K the packed code plane): Q5_0 / Q4_K / Q6_K with the row_inv
// computed at upload, at most TMQ_MFMA_MAX_COLS columns and a weight plane
// under 2 GiB (the decoders address the planes with 32-bit buffer offsets),
// unless TMQ_NOMFMA=1 (testing) or the caller does not use them.
bool mfma_eligible(uint32_t type, uint64_t rows, uint64_t cols, bool ext_row_inv, bool want) {
    if (!want || ext_row_inv || !tmq_ifit_codes((int)type) || cols > TMQ_MFMA_MAX_COLS) return false;
    const char* nm = getenv("TMQ_NOMFMA");
    if (nm && atoi(nm) != 0) return false;
    const uint64_t nb = cols / (type == TMQ_TYPE_Q5_0 ? 32 : 256);
    const uint64_t plane = (rows + 63) / 64 * 64 * nb *
                           (type == TMQ_TYPE_Q5_0 ? 16 : type == TMQ_TYPE_Q6_K ? 208 : 128);
    return plane < (1ull << 31);
}

// Allocate planes + normalisers for a rows x cols tensor (zero filled); the
// MFMA decoders' planes only when `mfma` (mfma_eligible).
int tensor_alloc(tmq_ctx* ctx, uint32_t type, uint64_t rows, uint64_t cols, bool mfma, tmq_tensor** out) {
    const int qk = qk_of(type);
    if (!qk) return tmq_fail(TMQ_ERR_ARG, "unsupported tensor type %u", type);
    if (rows == 0 || cols == 0 || cols % qk)
        return tmq_fail(TMQ_ERR_ARG, "shape %llux%llu invalid for type %u (cols %% %d)",
                    (unsigned long long)rows, (unsigned long long)cols, type, qk);
    if (rows > (1u << 30) || cols > (1u << 20))
        return tmq_fail(TMQ_ERR_ARG, "shape %llux%llu too large", (unsigned long long)rows,
                    (unsigned long long)cols);
    if (type == TMQ_TYPE_Q8_0 && cols > 64 * TMQ_Q8_MAX_TILES)
        return tmq_fail(TMQ_ERR_ARG, "Q8_0 cols %llu > %d", (unsigned long long)cols, 64 * TMQ_Q8_MAX_TILES);
    tmq_tensor* t = new tmq_tensor();
    t->ctx = ctx;
    TmqTensorDev& d = t->dev;
    d.type = (int)type;
    d.rows = (int)rows;
    d.cols = (int)cols;
    d.rows_pad = (int)((rows + 63) / 64 * 64);
    d.nb = (int)(cols / qk);
    const size_t R = d.rows_pad, nb = d.nb;
    // integer fit codes: Q5_0 four blocks' codes a dword, [b/4][r] x 4 B
    size_t sa = 0, sb = 0, sc = 0, sd = 0, se = 0, sq = 0,
           si = !mfma ? 0 : type == TMQ_TYPE_Q5_0 ? (nb + 3) / 4 * R * 4 : nb * R * tmq_ifit_codes((int)type);
    switch (type) {
    case TMQ_TYPE_Q8_0: sa = nb * 2 * R * 16; sd = nb * R * 2; break;
    case TMQ_TYPE_Q5_0: sa = nb * R * 16; sb = nb * R * 4; sd = nb * R * 2; se = nb * R; break;
    case TMQ_TYPE_Q4_K: sa = nb * 8 * R * 16; sb = nb * R * 16; se = nb * R * 8; break;
    case TMQ_TYPE_Q6_K:
        sa = nb * 8 * R * 16; sb = nb * 4 * R * 16; sc = nb * R * 16; sd = nb * R * 2; se = nb * R * 16;
        sq = mfma ? nb * 12 * R * 16 + nb * 4 * R * 4 : 0;
        break;
    case TMQ_TYPE_F32: sa = nb * 8 * R * 16; break;
    case TMQ_TYPE_F16: sa = nb * 4 * R * 16; break;
    }
    auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const size_t total = al(sa) + al(sb) + al(sc) + al(sd) + al(se) + al(si) + al(sq) + al(R * 4) * 2;
    hipError_t e = hipMalloc(&t->alloc, total);
    if (e != hipSuccess) {
        delete t;
        return tmq_fail(TMQ_ERR_NOMEM, "hipMalloc(%zu) for tensor: %s", total, hipGetErrorString(e));
    }
    e = hipMemsetAsync(t->alloc, 0, total, ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(t->alloc);
        delete t;
        return tmq_fail(TMQ_ERR_HIP, "hipMemsetAsync: %s", hipGetErrorString(e));
    }
    uint8_t* p = (uint8_t*)t->alloc;
    d.pa = p; p += al(sa);
    d.pb = sb ? p : nullptr; p += al(sb);
    d.pc = sc ? p : nullptr; p += al(sc);
    d.pd = sd ? p : nullptr; p += al(sd);
    d.pe = se ? p : nullptr; p += al(se);
    d.pi = si ? p : nullptr; p += al(si);
    d.pq = sq ? p : nullptr; p += al(sq);
    d.row_inv = (const float*)p; p += al(R * 4);
    d.row_scale = (const float*)p;
    t->weight_bytes = rows * (cols / qk) * (uint64_t)block_bytes(type);
    *out = t;
    return 0;
}

// Integer fit codes and corrections of the MFMA decoders (t->dev.pi):
// codes and per-(row, block, fitted unit) correction counts on the device,
// the offsets of the corrections (rows in order, so each 64-row group's are
// contiguous) on the host, then the corrections themselves.  A tensor
// allocated without the plane (mfma_eligible) stays on the fitted-float
// decoders.
int ifit_build(tmq_ctx* ctx, tmq_tensor* t) {
    TmqTensorDev& d = t->dev;
    if (!d.pi || d.clamp) {
        d.pi = nullptr;
        return 0;
    }
    const int subs = tmq_ifit_subs(d.type);
    const size_t n = (size_t)d.rows_pad * d.nb * subs;
    uint8_t* cnt = nullptr;
    int32_t* offd = nullptr;
    auto done = [&](int code) {
        if (cnt) (void)hipFree(cnt);
        if (offd) (void)hipFree(offd);
        return code;
    };
    hipError_t e = hipMalloc(&cnt, n);
    if (e != hipSuccess) return done(tmq_fail(TMQ_ERR_NOMEM, "ifit counts: %s", hipGetErrorString(e)));
    int le = tmq_launch_ifit(d, 0, cnt, nullptr, nullptr, ctx->stream);
    if (le) return done(tmq_fail(TMQ_ERR_HIP, "ifit launch: %s", hipGetErrorString((hipError_t)le)));
    std::vector<uint8_t> c(n);
    e = hipMemcpyAsync(c.data(), cnt, n, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return done(tmq_fail(TMQ_ERR_HIP, "ifit counts: %s", hipGetErrorString(e)));
    std::vector<int32_t> off(n);
    const int ng = d.rows_pad / 64;
    std::vector<int32_t> goff(ng + 1);
    int64_t total = 0;
    const size_t per_group = (size_t)64 * d.nb * subs;
    for (size_t i = 0; i < n; i++) {
        if (i % per_group == 0) goff[i / per_group] = (int32_t)total;
        off[i] = (int32_t)total;
        total += c[i];
    }
    goff[ng] = (int32_t)total;
    if (total == 0) return done(0);
    if (total > (1 << 30)) return done(tmq_fail(TMQ_ERR_ARG, "ifit: %lld corrections", (long long)total));
    const size_t cb = ((size_t)total * 16 + 255) & ~(size_t)255;
    e = hipMalloc(&t->corr_alloc, cb + sizeof(int32_t) * (ng + 1));
    if (e == hipSuccess) e = hipMalloc(&offd, sizeof(int32_t) * n);
    if (e != hipSuccess) return done(tmq_fail(TMQ_ERR_NOMEM, "ifit corrections: %s", hipGetErrorString(e)));
    uint4* corr = (uint4*)t->corr_alloc;
    int32_t* go = (int32_t*)((uint8_t*)t->corr_alloc + cb);
    e = hipMemcpyAsync(offd, off.data(), sizeof(int32_t) * n, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(go, goff.data(), sizeof(int32_t) * (ng + 1), hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return done(tmq_fail(TMQ_ERR_HIP, "ifit offsets: %s", hipGetErrorString(e)));
    le = tmq_launch_ifit(d, 1, nullptr, offd, corr, ctx->stream);
    if (le) return done(tmq_fail(TMQ_ERR_HIP, "ifit launch: %s", hipGetErrorString((hipError_t)le)));
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return done(tmq_fail(TMQ_ERR_HIP, "ifit: %s", hipGetErrorString(e)));
    d.corr = corr;
    d.corr_off = go;
    return done(0);
}

// Upload ggml bytes (host or device) into a freshly allocated tensor and
// repack.  When `ext_row_inv` is given (host floats, `rows` of them) it is
// used as the normaliser and the clamp path is enabled; otherwise the
// normalisers are computed on the device.
int tensor_create(tmq_ctx* ctx, uint32_t type, uint64_t rows, uint64_t cols, const void* data,
                  bool data_on_device, uint64_t n_bytes, const float* aux, bool aux_on_device,
                  const float* ext_row_inv, tmq_tensor** out, bool want_mfma = true) {
    if (!ctx || !data || !out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    tmq_tensor* t = nullptr;
    rc = tensor_alloc(ctx, type, rows, cols, mfma_eligible(type, rows, cols, ext_row_inv != nullptr, want_mfma), &t);
    if (rc) return rc;
    if (n_bytes != t->weight_bytes) {
        tmq_tensor_free(t);
        return tmq_fail(TMQ_ERR_ARG, "n_bytes %llu != %llu for %llux%llu type %u",
                    (unsigned long long)n_bytes, (unsigned long long)t->weight_bytes,
                    (unsigned long long)rows, (unsigned long long)cols, type);
    }
    const uint8_t* src = (const uint8_t*)data;
    void* staging = nullptr;
    auto cleanup = [&](int code) {
        if (staging) (void)hipFree(staging);
        if (code) tmq_tensor_free(t);
        return code;
    };
    if (!data_on_device) {
        hipError_t e = hipMalloc(&staging, n_bytes);
        if (e != hipSuccess) return cleanup(tmq_fail(TMQ_ERR_NOMEM, "staging hipMalloc: %s", hipGetErrorString(e)));
        e = hipMemcpyAsync(staging, data, n_bytes, hipMemcpyHostToDevice, ctx->stream);
        if (e != hipSuccess) return cleanup(tmq_fail(TMQ_ERR_HIP, "staging copy: %s", hipGetErrorString(e)));
        src = (const uint8_t*)staging;
    }
    int le = tmq_launch_repack((int)type, src, t->dev, ctx->stream);
    if (le) return cleanup(tmq_fail(TMQ_ERR_HIP, "repack launch: %s", hipGetErrorString((hipError_t)le)));
    if (ext_row_inv) {
        t->dev.clamp = 1;
        t->dev.pi = nullptr;
        std::vector<float> ri(t->dev.rows_pad, 1.0f);
        memcpy(ri.data(), ext_row_inv, sizeof(float) * rows);
        hipError_t e = hipMemcpyAsync((void*)t->dev.row_inv, ri.data(), sizeof(float) * ri.size(),
                                      hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return cleanup(tmq_fail(TMQ_ERR_HIP, "row_inv copy: %s", hipGetErrorString(e)));
        cleanup(0);
        *out = t;
        return 0;
    }
    if (is_float_type(type)) {
        // no normaliser of their own (they only take the INT16 / FP32
        // paths); every element must be finite
        int rcm = ctx->misc.ensure(256);
        if (rcm) return cleanup(rcm);
        int* bad = (int*)ctx->misc.p;
        int badh = 0;
        hipError_t e = hipMemsetAsync(bad, 0, sizeof(int), ctx->stream);
        if (e == hipSuccess) {
            le = tmq_launch_check_finite(t->dev, bad, ctx->stream);
            if (le) e = (hipError_t)le;
        }
        if (e == hipSuccess) e = hipMemcpyAsync(&badh, bad, sizeof(int), hipMemcpyDeviceToHost, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return cleanup(tmq_fail(TMQ_ERR_HIP, "finite check: %s", hipGetErrorString(e)));
        if (badh) return cleanup(tmq_fail(TMQ_ERR_NONFINITE, "non-finite element in %llux%llu %s tensor",
                                          (unsigned long long)rows, (unsigned long long)cols, type_name(type)));
        cleanup(0);
        *out = t;
        return 0;
    }
    // aux row_max_abs (Q8_0) -> device
    const float* aux_dev = nullptr;
    void* aux_tmp = nullptr;
    if (aux && type == TMQ_TYPE_Q8_0) {
        if (aux_on_device) {
            aux_dev = aux;
        } else {
            hipError_t e = hipMalloc(&aux_tmp, sizeof(float) * rows);
            if (e == hipSuccess)
                e = hipMemcpyAsync(aux_tmp, aux, sizeof(float) * rows, hipMemcpyHostToDevice, ctx->stream);
            if (e != hipSuccess) {
                if (aux_tmp) (void)hipFree(aux_tmp);
                return cleanup(tmq_fail(TMQ_ERR_HIP, "aux copy: %s", hipGetErrorString(e)));
            }
            aux_dev = (const float*)aux_tmp;
        }
    }
    int rc2 = ctx->misc.ensure(256);
    if (rc2) return cleanup(rc2);
    int* bad = (int*)ctx->misc.p;
    hipError_t e = hipMemsetAsync(bad, 0, sizeof(int), ctx->stream);
    if (e == hipSuccess) {
        le = tmq_launch_rowstat(t->dev, aux_dev, (float*)t->dev.row_inv, (float*)t->dev.row_scale,
                                bad, ctx->stream);
        if (le) e = (hipError_t)le;
    }
    int badh = 0;
    if (e == hipSuccess && t->dev.pe) {
        // TMQ_NOFIT=1: every sub-block takes the exact decode (testing)
        const char* nf = getenv("TMQ_NOFIT");
        le = tmq_launch_fit(t->dev, nf && atoi(nf) != 0, ctx->stream);
        if (le) e = (hipError_t)le;
    }
    if (e == hipSuccess) e = hipMemcpyAsync(&badh, bad, sizeof(int), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (aux_tmp) (void)hipFree(aux_tmp);
    if (e != hipSuccess) return cleanup(tmq_fail(TMQ_ERR_HIP, "rowstat: %s", hipGetErrorString(e)));
    if (badh) return cleanup(tmq_fail(TMQ_ERR_NONFINITE, "non-finite fp16 block scale in %llux%llu type %u tensor",
                                  (unsigned long long)rows, (unsigned long long)cols, type));
    rc = ifit_build(ctx, t);
    if (rc) return cleanup(rc);
    if (t->dev.pi && t->dev.pq) {
        le = tmq_launch_q6_pack(t->dev, ctx->stream);
        if (le) return cleanup(tmq_fail(TMQ_ERR_HIP, "q6 pack launch: %s", hipGetErrorString((hipError_t)le)));
    }
    cleanup(0);
    *out = t;
    return 0;
}

// host-side preparation of an int16 activation (x_scale unused -> 1)
void act_from_int16(const int16_t* xq, int n, std::vector<uint8_t>& buf) {
    buf.assign(tmq_act_bytes(n), 0);
    float one = 1.0f;
    memcpy(buf.data(), &one, 4);
    memcpy(buf.data() + 4, &n, 4);
    uint32_t* xh = (uint32_t*)(buf.data() + 16);
    uint32_t* xl = xh + n / 2;
    int16_t* q = (int16_t*)(xl + n / 2);
    for (int k = 0; k < n / 2; k++) {
        int a = xq[2 * k], c = xq[2 * k + 1];
        xh[k] = ((uint32_t)(a >> 8) & 0xffffu) | ((uint32_t)(c >> 8) << 16);
        xl[k] = ((uint32_t)a & 0xffu) | (((uint32_t)c & 0xffu) << 16);
    }
    memcpy(q, xq, sizeof(int16_t) * n);
    int32_t* q32 = (int32_t*)(q + n);
    for (int k = 0; k < n; k++) q32[k] = xq[k];
    // MFMA decoders' operand bytes and block sums (tmq_internal.h)
    uint8_t* xa = buf.data() + tmq_act_xa(n);
    int32_t* xs = (int32_t*)(buf.data() + tmq_act_xs(n));
    int32_t* xs16 = (int32_t*)(buf.data() + tmq_act_xs16(n));
    for (int k = 0; k < (int)tmq_act_nbx(n) * 32; k++) {
        const int v = k < n ? xq[k] : 0, b = k >> 5, i = k & 31;
        xa[64 * b + 32 * (i >> 4) + (i & 15)] = (uint8_t)(v >> 8);
        xa[64 * b + 32 * (i >> 4) + 16 + (i & 15)] = (uint8_t)((v & 255) ^ 0x80);
        xs[b] += v;
        xs16[k >> 4] += v;
    }
    memset(xa + 64 * tmq_act_nbx(n) + 16, 1, 16);
}

TmqWork make_work(const tmq_tensor* t, const uint8_t* act, float* y, int64_t* acc) {
    TmqWork w{};
    w.t = t->dev;
    w.act = act;
    w.y = y;
    w.acc = acc;
    w.first_group = 0;
    w.ngroups = groups_of(t->dev);
    return w;
}

// run a GEMV with an int16 activation given on the host; int64 per-row
// results returned on the host (tile API and PhaseB replay share this)
int run_int16(tmq_ctx* ctx, const tmq_tensor* t, const int16_t* xq, std::vector<int64_t>& acc) {
    std::vector<uint8_t> act;
    act_from_int16(xq, t->dev.cols, act);
    int rc = ctx->act.ensure(act.size());
    if (!rc) rc = ctx->acc.ensure(sizeof(int64_t) * (size_t)t->dev.rows);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->act.p, act.data(), act.size(), hipMemcpyHostToDevice, ctx->stream));
    TmqWork w = make_work(t, (const uint8_t*)ctx->act.p, nullptr, (int64_t*)ctx->acc.p);
    LAUNCH_TRY(tmq_launch_gemv(w, ctx->stream));
    acc.resize(t->dev.rows);
    HIP_TRY(hipMemcpyAsync(acc.data(), ctx->acc.p, sizeof(int64_t) * acc.size(), hipMemcpyDeviceToHost,
                           ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

// Descriptors of one format (and clamp mode) form a segment that runs as one
// launch of that format's kernel; `works` is reordered by segment and
// first_group made relative to the segment's first workgroup.
//
// A launch's workgroups run in rounds of one per CU, so a segment of W
// whole-row groups takes ceil(W / ncu) group times even when its last round
// holds a few.  With ncu > 0, a segment whose last round holds T <= ncu / 2
// groups splits those T groups so that the last round takes a fraction of a
// group time:
//  - K-quant MFMA segments: each group into up to ncu / T workgroups over
//    disjoint super-block ranges (at least one each); each split group gets
//    a tail slot (`nslots` of them) where its pieces add their row sums;
//  - Q8_0 segments (256-row groups, one wave per 64 rows) of at most
//    TMQ_Q8_SPLIT_COLS columns: each group into its four 64-row quarters,
//    whose four waves split the row's 64-column tiles (no slot: the tiles'
//    sums meet in the workgroup's LDS).
void plan_segments(std::vector<TmqWork>& works, std::vector<TmqGroupRef>& gmap, std::vector<Segment>& segs,
                   int ncu, int& nslots) {
    std::stable_sort(works.begin(), works.end(), [](const TmqWork& a, const TmqWork& b) {
        const int fa = tmq_kernel_fmt(a.t), fb = tmq_kernel_fmt(b.t);
        return fa != fb ? fa < fb : a.t.clamp < b.t.clamp;
    });
    gmap.clear();
    segs.clear();
    nslots = 0;
    auto close = [&]() {
        if (segs.empty() || ncu <= 0) return;
        Segment& sg = segs.back();
        const bool kq = sg.type == TMQ_FMT_Q4_K_MFMA || sg.type == TMQ_FMT_Q6_K_MFMA;
        const bool q8 = sg.type == TMQ_TYPE_Q8_0 && sg.max_cols <= TMQ_Q8_SPLIT_COLS;
        if (!kq && !q8) return;
        const int tcount = sg.ngroups % ncu;
        if (tcount == 0 || ncu / tcount < 2) return;
        std::vector<TmqGroupRef> last(gmap.end() - tcount, gmap.end());
        gmap.resize(gmap.size() - tcount);
        sg.split = 1;
        if (q8) {
            for (const TmqGroupRef& e : last)
                for (int k = 0; k < TMQ_WAVES; k++) {
                    // quarters past the tensor's padded rows are left out
                    if ((e.group * TMQ_WAVES + k) * 64 >= works[e.work].t.rows_pad) break;
                    TmqGroupRef p = e;
                    p.b0 = (uint16_t)k;
                    p.pieces = TMQ_WAVES;
                    gmap.push_back(p);
                }
            sg.ngroups = (int)gmap.size() - sg.gmap_off;
            return;
        }
        for (const TmqGroupRef& e : last) {
            const int nb = works[e.work].t.nb;
            const int pieces = std::min(std::min(ncu / tcount, nb), 32767);
            if (pieces < 2 || nslots >= 32767) {
                gmap.push_back(e);
                continue;
            }
            const int slot = nslots++;
            for (int k = 0; k < pieces; k++) {
                TmqGroupRef p = e;
                p.b0 = (uint16_t)((int64_t)k * nb / pieces);
                p.b1 = (uint16_t)((int64_t)(k + 1) * nb / pieces);
                p.slot = (int16_t)slot;
                p.pieces = (int16_t)pieces;
                gmap.push_back(p);
            }
        }
        sg.ngroups = (int)gmap.size() - sg.gmap_off;
    };
    for (size_t i = 0; i < works.size(); i++) {
        TmqWork& w = works[i];
        const int fmt = tmq_kernel_fmt(w.t);
        if (segs.empty() || segs.back().type != fmt || segs.back().clamp != w.t.clamp) {
            close();
            segs.push_back(Segment{fmt, w.t.clamp, (int)gmap.size(), 0, 0, 0});
        }
        Segment& sg = segs.back();
        sg.max_cols = std::max(sg.max_cols, w.t.cols);
        w.first_group = sg.ngroups;
        for (int g = 0; g < w.ngroups; g++) gmap.push_back(TmqGroupRef{(int32_t)i, g, 0, 0, 0, 1});
        sg.ngroups += w.ngroups;
    }
    close();
}

int launch_segments(const std::vector<Segment>& segs, const void* works_dev, const void* gmap_dev,
                    uint64_t* tail, hipStream_t s) {
    for (const Segment& sg : segs) {
        int e = tmq_launch_chain(sg.type, sg.clamp, sg.max_cols, (const TmqWork*)works_dev,
                                 (const TmqGroupRef*)gmap_dev + sg.gmap_off, sg.ngroups, sg.split, tail, s);
        if (e) return tmq_fail(TMQ_ERR_HIP, "chain segment launch: %s", hipGetErrorString((hipError_t)e));
    }
    return 0;
}

inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

}  // namespace

int tmq_rt_groups_of(const TmqTensorDev& t) { return groups_of(t); }

int tmq_rt_prepare_int16(tmq_ctx* ctx, tmq_tensor* t) {
    if (t->i16_alloc) return 0;
    const size_t R = t->dev.rows_pad;
    const size_t wb = ((size_t)t->dev.cols / 8) * R * 16, total = ((wb + 255) & ~(size_t)255) + R * 4;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, total);
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_NOMEM, "hipMalloc(%zu) for INT16 planes: %s", total, hipGetErrorString(e));
    TmqTensorDev d = t->dev;
    d.pw = (const uint8_t*)p;
    d.rs16 = (const float*)((uint8_t*)p + ((wb + 255) & ~(size_t)255));
    int le = tmq_launch_i16_prep(d, ctx->stream);
    if (le == 0) le = (int)hipStreamSynchronize(ctx->stream);
    if (le) {
        (void)hipFree(p);
        return tmq_fail(TMQ_ERR_HIP, "INT16 weight preparation: %s", hipGetErrorString((hipError_t)le));
    }
    t->i16_alloc = p;
    t->dev = d;
    return 0;
}

int tmq_rt_tensor_create(tmq_ctx* ctx, uint32_t type, uint64_t rows, uint64_t cols, const void* data,
                         bool data_on_device, uint64_t n_bytes, const float* aux, bool aux_on_device,
                         tmq_tensor** out, bool mfma) {
    return tensor_create(ctx, type, rows, cols, data, data_on_device, n_bytes, aux, aux_on_device,
                         nullptr, out, mfma);
}

TmqWork tmq_rt_make_work(const tmq_tensor* t, const uint8_t* act, float* y, int64_t* acc) {
    return make_work(t, act, y, acc);
}

// =========================================================================
extern "C" {

const char* tmq_last_error(void) { return g_err.c_str(); }
const char* tmq_version(void) { return "tmq 0.1 (gfx950)"; }

int tmq_open(int device, tmq_ctx** out) {
    if (!out) return tmq_fail(TMQ_ERR_ARG, "null out");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) return tmq_fail(TMQ_ERR_NODEV, "no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n) return tmq_fail(TMQ_ERR_ARG, "device %d out of range (%d devices)", device, n);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return tmq_fail(TMQ_ERR_NODEV, "device %d is %s, this library is built for gfx950", device, prop.gcnArchName);
    tmq_ctx* c = new tmq_ctx();
    c->device = device;
    c->ncu = prop.multiProcessorCount;
    e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return tmq_fail(TMQ_ERR_HIP, "stream create: %s", hipGetErrorString(e));
    }
    int rc = scratch_init(device);
    if (rc) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return rc;
    }
    *out = c;
    return 0;
}

int tmq_close(tmq_ctx* ctx) {
    if (!ctx) return 0;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (TmqDevBuf* b : {&ctx->x, &ctx->y, &ctx->act, &ctx->acc, &ctx->misc, &ctx->works, &ctx->gmap}) b->release();
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return 0;
}

void* tmq_stream(tmq_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int tmq_sync(tmq_ctx* ctx) {
    if (!ctx) return tmq_fail(TMQ_ERR_ARG, "null ctx");
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

int tmq_tensor_upload(tmq_ctx* ctx, uint32_t type, uint64_t rows, uint64_t cols, const void* data,
                      uint64_t n_bytes, const float* row_max_abs, tmq_tensor** out) {
    return tensor_create(ctx, type, rows, cols, data, false, n_bytes, row_max_abs, false, nullptr, out);
}

int tmq_tensor_upload_dev(tmq_ctx* ctx, uint32_t type, uint64_t rows, uint64_t cols,
                          const void* data_dev, uint64_t n_bytes, const float* row_max_abs_dev,
                          tmq_tensor** out) {
    return tensor_create(ctx, type, rows, cols, data_dev, true, n_bytes, row_max_abs_dev, true, nullptr, out);
}

int tmq_tensor_free(tmq_tensor* t) {
    if (!t) return 0;
    if (t->alloc || t->i16_alloc || t->corr_alloc) {
        (void)hipSetDevice(t->ctx->device);
        (void)hipStreamSynchronize(t->ctx->stream);
        if (t->alloc) (void)hipFree(t->alloc);
        if (t->i16_alloc) (void)hipFree(t->i16_alloc);
        if (t->corr_alloc) (void)hipFree(t->corr_alloc);
    }
    delete t;
    return 0;
}

int tmq_tensor_info(const tmq_tensor* t, uint32_t* type, uint64_t* rows, uint64_t* cols,
                    uint64_t* weight_bytes) {
    if (!t) return tmq_fail(TMQ_ERR_ARG, "null tensor");
    if (type) *type = (uint32_t)t->dev.type;
    if (rows) *rows = (uint64_t)t->dev.rows;
    if (cols) *cols = (uint64_t)t->dev.cols;
    if (weight_bytes) *weight_bytes = t->weight_bytes;
    return 0;
}

int tmq_tensor_row_norm(tmq_ctx* ctx, const tmq_tensor* t, float* out) {
    if (!ctx || !t || !out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    const float* src = t->dev.type == TMQ_TYPE_Q8_0 ? t->dev.row_scale : t->dev.row_inv;
    HIP_TRY(hipMemcpyAsync(out, src, sizeof(float) * t->dev.rows, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

int tmq_tensor_fit_stats(tmq_ctx* ctx, const tmq_tensor* t, uint64_t* fitted, uint64_t* exact) {
    if (!ctx || !t || !fitted || !exact) return tmq_fail(TMQ_ERR_ARG, "null argument");
    *fitted = *exact = 0;
    const int n = tmq_fit_codes(t->dev.type);
    if (!n || !t->dev.pe || t->dev.clamp) return 0;
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    const size_t R = t->dev.rows_pad, nb = t->dev.nb;
    std::vector<uint8_t> h(nb * R * n);
    HIP_TRY(hipMemcpyAsync(h.data(), t->dev.pe, h.size(), hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    for (size_t b = 0; b < nb; b++)
        for (size_t r = 0; r < (size_t)t->dev.rows; r++)
            for (int i = 0; i < n; i++) (h[(b * R + r) * n + i] & 0x80u ? *exact : *fitted) += 1;
    return 0;
}

int tmq_tensor_ifit_stats(tmq_ctx* ctx, const tmq_tensor* t, uint64_t* blocks, uint64_t* corrections) {
    if (!ctx || !t || !blocks || !corrections) return tmq_fail(TMQ_ERR_ARG, "null argument");
    *blocks = *corrections = 0;
    if (!t->dev.pi) return 0;
    *blocks = (uint64_t)t->dev.rows * t->dev.nb * tmq_ifit_subs(t->dev.type);
    if (!t->dev.corr_off) return 0;
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    int32_t last = 0;
    HIP_TRY(hipMemcpyAsync(&last, t->dev.corr_off + t->dev.rows_pad / 64, sizeof(int32_t), hipMemcpyDeviceToHost,
                           ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    *corrections = (uint64_t)last;
    return 0;
}

int tmq_gemv_dev(tmq_ctx* ctx, const tmq_tensor* t, const float* x_dev, float* y_dev, int64_t* acc_dev) {
    if (!ctx || !t || !x_dev) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (is_float_type((uint32_t)t->dev.type))
        return tmq_fail(TMQ_ERR_ARG, "%s tensor: no matmul_fpga_* of its own (the reference sends it to "
                        "matmul_fpga_int16 or the FP32 loop: tmq_gemv_dev_path)", type_name((uint32_t)t->dev.type));
    int rc = tmq_rt_set_device(ctx);
    if (!rc) rc = ctx->act.ensure(tmq_act_bytes(t->dev.cols));
    if (rc) return rc;
    TmqActJobs jobs{};
    jobs.count = 1;
    jobs.j[0].x = x_dev;
    jobs.j[0].act = (uint8_t*)ctx->act.p;
    jobs.j[0].n = t->dev.cols;
    LAUNCH_TRY(tmq_launch_act_prep(jobs, ctx->stream));
    TmqWork w = make_work(t, (const uint8_t*)ctx->act.p, y_dev, acc_dev);
    LAUNCH_TRY(tmq_launch_gemv(w, ctx->stream));
    return 0;
}

int tmq_gemv_dev_noalloc(tmq_ctx* ctx, const tmq_tensor* t, const float* x_dev, float* y_dev, int64_t* acc_dev) {
    if (!ctx || !t || !x_dev) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (is_float_type((uint32_t)t->dev.type))
        return tmq_fail(TMQ_ERR_ARG, "%s tensor: no matmul_fpga_* of its own", type_name((uint32_t)t->dev.type));
    if (t->dev.cols > TMQ_NOALLOC_MAX_COLS)
        return tmq_fail(TMQ_ERR_ARG, "tmq_gemv_dev_noalloc: cols %d above its scratch limit of %d columns",
                        t->dev.cols, TMQ_NOALLOC_MAX_COLS);
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    uint8_t* act = (uint8_t*)scratch_of(ctx->device);
    if (!act) return tmq_fail(TMQ_ERR_HIP, "tmq_gemv_dev_noalloc: no scratch for device %d", ctx->device);
    TmqActJobs jobs{};
    jobs.count = 1;
    jobs.j[0].x = x_dev;
    jobs.j[0].act = act;
    jobs.j[0].n = t->dev.cols;
    LAUNCH_TRY(tmq_launch_act_prep(jobs, ctx->stream));
    TmqWork w = make_work(t, act, y_dev, acc_dev);
    LAUNCH_TRY(tmq_launch_gemv(w, ctx->stream));
    return 0;
}

int tmq_matmul(tmq_ctx* ctx, const tmq_tensor* t, const float* x, float* y, int rows, int cols) {
    if (!ctx || !t || !x || !y) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (rows != t->dev.rows || cols != t->dev.cols)
        return tmq_fail(TMQ_ERR_ARG, "shape %dx%d does not match tensor %dx%d", rows, cols, t->dev.rows, t->dev.cols);
    int rc = tmq_rt_set_device(ctx);
    if (!rc) rc = ctx->x.ensure(sizeof(float) * cols);
    if (!rc) rc = ctx->y.ensure(sizeof(float) * rows);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->x.p, x, sizeof(float) * cols, hipMemcpyHostToDevice, ctx->stream));
    rc = tmq_gemv_dev(ctx, t, (const float*)ctx->x.p, (float*)ctx->y.p, nullptr);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(y, ctx->y.p, sizeof(float) * rows, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

int tmq_quantize_act(tmq_ctx* ctx, const float* x, int n, int16_t* xq, float* x_scale) {
    if (!ctx || !x || n <= 0 || n % 2) return tmq_fail(TMQ_ERR_ARG, "bad activation arguments");
    int rc = tmq_rt_set_device(ctx);
    if (!rc) rc = ctx->x.ensure(sizeof(float) * n);
    if (!rc) rc = ctx->act.ensure(tmq_act_bytes(n));
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->x.p, x, sizeof(float) * n, hipMemcpyHostToDevice, ctx->stream));
    TmqActJobs jobs{};
    jobs.count = 1;
    jobs.j[0].x = (const float*)ctx->x.p;
    jobs.j[0].act = (uint8_t*)ctx->act.p;
    jobs.j[0].n = n;
    LAUNCH_TRY(tmq_launch_act_prep(jobs, ctx->stream));
    // layout of the prepared activation: x_scale at 0, int16 values at 16 + 4n
    if (x_scale) HIP_TRY(hipMemcpyAsync(x_scale, ctx->act.p, sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    if (xq)
        HIP_TRY(hipMemcpyAsync(xq, (const uint8_t*)ctx->act.p + 16 + 4 * (size_t)n, sizeof(int16_t) * n,
                               hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

int tmq_tensor_q8_scales(tmq_ctx* ctx, const tmq_tensor* t, uint16_t* out) {
    if (!ctx || !t || !out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (t->dev.type != TMQ_TYPE_Q8_0) return tmq_fail(TMQ_ERR_ARG, "not a Q8_0 tensor");
    int rc = tmq_rt_set_device(ctx);
    const size_t n = (size_t)t->dev.rows * t->dev.nb;
    if (!rc) rc = ctx->misc.ensure(sizeof(uint16_t) * n);
    if (rc) return rc;
    LAUNCH_TRY(tmq_launch_q8_scales(t->dev, (uint16_t*)ctx->misc.p, ctx->stream));
    HIP_TRY(hipMemcpyAsync(out, ctx->misc.p, sizeof(uint16_t) * n, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

int tmq_route(uint32_t type, uint32_t flags) {
    if (!qk_of(type)) return tmq_fail(TMQ_ERR_ARG, "unsupported tensor type %u", type);
    if (!(flags & TMQ_FLAG_FPGA)) return TMQ_PATH_FP32;
    const bool own = (type == TMQ_TYPE_Q5_0 && (flags & TMQ_FLAG_Q5_0)) ||
                     (type == TMQ_TYPE_Q6_K && (flags & TMQ_FLAG_Q6_K)) ||
                     (type == TMQ_TYPE_Q4_K && (flags & TMQ_FLAG_Q4_K)) ||
                     (type == TMQ_TYPE_Q8_0 && (flags & TMQ_FLAG_Q8_0));
    return own ? TMQ_PATH_FPGA : TMQ_PATH_INT16;
}

// Tiles of one matmul in the reference's tilings, as its matmul_fpga_*
// count them into g_timing.total_tiles: 64x64 for Q8_0 and INT16
// (sim/tmac_gguf.cpp:901-934, :965-1078), 8-row x 896 Q5_0 tiles
// (:1267-1300), 56-row x 256-column Q4_K tiles (:1154-1188) and 32-row x
// 256-column Q6_K tiles (:1442-1497); rows*cols MACs (:899, :963, :1109,
// :1233, :1379).  The FP32 loop counts nothing.
int tmq_matmul_tiles(uint32_t type, uint32_t flags, uint64_t rows, uint64_t cols, int64_t* tiles, int64_t* macs) {
    if (!tiles || !macs) return tmq_fail(TMQ_ERR_ARG, "null argument");
    const int path = tmq_route(type, flags);
    if (path < 0) return path;
    auto cdiv = [](uint64_t a, uint64_t b) { return (int64_t)((a + b - 1) / b); };
    *tiles = 0;
    *macs = 0;
    if (path == TMQ_PATH_FP32) return TMQ_OK;
    *macs = (int64_t)(rows * cols);
    if (path == TMQ_PATH_INT16 || type == TMQ_TYPE_Q8_0) *tiles = cdiv(rows, 64) * cdiv(cols, 64);
    else if (type == TMQ_TYPE_Q5_0) *tiles = cdiv(rows, 8);
    else if (type == TMQ_TYPE_Q4_K) *tiles = cdiv(rows, 56) * cdiv(cols, 256);
    else *tiles = cdiv(rows, 32) * cdiv(cols, 256);
    return TMQ_OK;
}

int tmq_tensor_prepare_int16(tmq_ctx* ctx, tmq_tensor* t) {
    if (!ctx || !t) return tmq_fail(TMQ_ERR_ARG, "null argument");
    int rc = tmq_rt_set_device(ctx);
    return rc ? rc : tmq_rt_prepare_int16(ctx, t);
}

int tmq_gemv_dev_path(tmq_ctx* ctx, const tmq_tensor* t, int path, const float* x_dev, float* y_dev,
                      int64_t* acc_dev) {
    if (path == TMQ_PATH_FPGA) return tmq_gemv_dev(ctx, t, x_dev, y_dev, acc_dev);
    if (!ctx || !t || !x_dev) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (path != TMQ_PATH_INT16 && path != TMQ_PATH_FP32) return tmq_fail(TMQ_ERR_ARG, "unknown matmul path %d", path);
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    TmqWork w = make_work(t, nullptr, y_dev, nullptr);
    if (path == TMQ_PATH_FP32) {
        if (acc_dev) return tmq_fail(TMQ_ERR_ARG, "the FP32 path has no integer partials (acc_dev must be NULL)");
        w.path = TMQ_WPATH_FP32;
        w.xf = x_dev;
        LAUNCH_TRY(tmq_launch_gemv(w, ctx->stream));
        return 0;
    }
    // INT16: weights quantised once per tensor, activation as every path does
    rc = tmq_rt_prepare_int16(ctx, const_cast<tmq_tensor*>(t));
    if (!rc) rc = ctx->act.ensure(tmq_act_bytes(t->dev.cols));
    if (rc) return rc;
    TmqActJobs jobs{};
    jobs.count = 1;
    jobs.j[0].x = x_dev;
    jobs.j[0].act = (uint8_t*)ctx->act.p;
    jobs.j[0].n = t->dev.cols;
    LAUNCH_TRY(tmq_launch_act_prep(jobs, ctx->stream));
    w = make_work(t, (const uint8_t*)ctx->act.p, y_dev, acc_dev);
    w.path = TMQ_WPATH_INT16;
    LAUNCH_TRY(tmq_launch_gemv(w, ctx->stream));
    return 0;
}

int tmq_matmul_path(tmq_ctx* ctx, const tmq_tensor* t, int path, const float* x, float* y, int rows, int cols) {
    if (!ctx || !t || !x || !y) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (rows != t->dev.rows || cols != t->dev.cols)
        return tmq_fail(TMQ_ERR_ARG, "shape %dx%d does not match tensor %dx%d", rows, cols, t->dev.rows, t->dev.cols);
    int rc = tmq_rt_set_device(ctx);
    if (!rc) rc = ctx->x.ensure(sizeof(float) * cols);
    if (!rc) rc = ctx->y.ensure(sizeof(float) * rows);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->x.p, x, sizeof(float) * cols, hipMemcpyHostToDevice, ctx->stream));
    rc = tmq_gemv_dev_path(ctx, t, path, (const float*)ctx->x.p, (float*)ctx->y.p, nullptr);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(y, ctx->y.p, sizeof(float) * rows, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

int tmq_matmul_flags(tmq_ctx* ctx, const tmq_tensor* t, uint32_t flags, const float* x, float* y, int rows,
                     int cols) {
    if (!t) return tmq_fail(TMQ_ERR_ARG, "null tensor");
    const int path = tmq_route((uint32_t)t->dev.type, flags);
    if (path < 0) return path;
    return tmq_matmul_path(ctx, t, path, x, y, rows, cols);
}

int tmq_gemv_partials_path(tmq_ctx* ctx, const tmq_tensor* t, int path, const float* x, int64_t* acc,
                           uint64_t acc_len, float* x_scale) {
    if (path == TMQ_PATH_FPGA) return tmq_gemv_partials(ctx, t, x, acc, acc_len, x_scale);
    if (path != TMQ_PATH_INT16) return tmq_fail(TMQ_ERR_ARG, "path %d has no integer partials", path);
    if (!ctx || !t || !x || !acc) return tmq_fail(TMQ_ERR_ARG, "null argument");
    const uint64_t need = (uint64_t)t->dev.rows * ((t->dev.cols + 63) / 64);
    if (acc_len < need) return tmq_fail(TMQ_ERR_ARG, "acc_len %llu < %llu", (unsigned long long)acc_len,
                                        (unsigned long long)need);
    int rc = tmq_rt_set_device(ctx);
    if (!rc) rc = ctx->x.ensure(sizeof(float) * t->dev.cols);
    if (!rc) rc = ctx->acc.ensure(sizeof(int64_t) * need);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->x.p, x, sizeof(float) * t->dev.cols, hipMemcpyHostToDevice, ctx->stream));
    rc = tmq_gemv_dev_path(ctx, t, TMQ_PATH_INT16, (const float*)ctx->x.p, nullptr, (int64_t*)ctx->acc.p);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(acc, ctx->acc.p, sizeof(int64_t) * need, hipMemcpyDeviceToHost, ctx->stream));
    if (x_scale) HIP_TRY(hipMemcpyAsync(x_scale, ctx->act.p, sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

int tmq_gemv_partials(tmq_ctx* ctx, const tmq_tensor* t, const float* x, int64_t* acc,
                      uint64_t acc_len, float* x_scale) {
    if (!ctx || !t || !x || !acc) return tmq_fail(TMQ_ERR_ARG, "null argument");
    const uint64_t need = t->dev.type == TMQ_TYPE_Q8_0
                              ? (uint64_t)t->dev.rows * ((t->dev.cols + 63) / 64)
                              : (uint64_t)t->dev.rows;
    if (acc_len < need) return tmq_fail(TMQ_ERR_ARG, "acc_len %llu < %llu", (unsigned long long)acc_len,
                                    (unsigned long long)need);
    int rc = tmq_rt_set_device(ctx);
    if (!rc) rc = ctx->x.ensure(sizeof(float) * t->dev.cols);
    if (!rc) rc = ctx->acc.ensure(sizeof(int64_t) * need);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->x.p, x, sizeof(float) * t->dev.cols, hipMemcpyHostToDevice, ctx->stream));
    rc = tmq_gemv_dev(ctx, t, (const float*)ctx->x.p, nullptr, (int64_t*)ctx->acc.p);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(acc, ctx->acc.p, sizeof(int64_t) * need, hipMemcpyDeviceToHost, ctx->stream));
    if (x_scale) HIP_TRY(hipMemcpyAsync(x_scale, ctx->act.p, sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

// ---------------------------------------------------------------- tiles
int tmq_vecmul_tile_q8(tmq_ctx* ctx, const uint8_t* q8_W, const uint16_t* cs, const int16_t* vec,
                       int64_t* result) {
    if (!ctx || !q8_W || !cs || !vec || !result) return tmq_fail(TMQ_ERR_ARG, "null argument");
    int rc = tmq_rt_set_device(ctx);
    if (!rc) rc = ctx->misc.ensure(4096 + 256 + 128 + 512);
    if (rc) return rc;
    uint8_t* p = (uint8_t*)ctx->misc.p;
    HIP_TRY(hipMemcpyAsync(p, q8_W, 4096, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipMemcpyAsync(p + 4096, cs, 256, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipMemcpyAsync(p + 4352, vec, 128, hipMemcpyHostToDevice, ctx->stream));
    LAUNCH_TRY(tmq_launch_tile_q8(p, (const uint16_t*)(p + 4096), (const int16_t*)(p + 4352),
                                  (int64_t*)(p + 4480), ctx->stream));
    HIP_TRY(hipMemcpyAsync(result, p + 4480, 512, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return 0;
}

int tmq_vecmul_tile_q5_0_8x896(tmq_ctx* ctx, const uint8_t* blocks, const int16_t* act,
                               const float* row_inv, int64_t* result, int row_base) {
    if (!ctx || !blocks || !act || !row_inv || !result) return tmq_fail(TMQ_ERR_ARG, "null argument");
    tmq_tensor* t = nullptr;
    int rc = tensor_create(ctx, TMQ_TYPE_Q5_0, 8, 896, blocks, false, 224 * 22, nullptr, false, row_inv, &t);
    if (rc) return rc;
    std::vector<int64_t> acc;
    rc = run_int16(ctx, t, act, acc);
    tmq_tensor_free(t);
    if (rc) return rc;
    for (int i = 0; i < 8; i++) result[row_base + i] += acc[i];
    return 0;
}

int tmq_vecmul_tile_q5_0_4x896(tmq_ctx* ctx, const uint8_t* blocks56, const int16_t* act,
                               const float* row_norm, int64_t* result, int row_base) {
    if (!ctx || !blocks56 || !act || !row_norm || !result) return tmq_fail(TMQ_ERR_ARG, "null argument");
    // the 56 interleaved 48-byte pairs (core 0 block, core 1 block, 4 bytes
    // of padding) as 4 rows of 28 ggml blocks: pair bi holds column block
    // bi % 28 of row bi / 28 (core 0) and of row 2 + bi / 28 (core 1)
    // (sim/fpga_sim.hpp:1215-1222); the weight is the same (d*q)*row_norm
    // rounded and clamped to int16 as the 8-row tile's (d*q)*row_inv
    std::vector<uint8_t> rows((size_t)4 * 28 * 22);
    for (int bi = 0; bi < 56; bi++) {
        const int r = bi / 28, cb = bi % 28;
        memcpy(&rows[((size_t)r * 28 + cb) * 22], blocks56 + (size_t)bi * 48, 22);
        memcpy(&rows[((size_t)(r + 2) * 28 + cb) * 22], blocks56 + (size_t)bi * 48 + 22, 22);
    }
    tmq_tensor* t = nullptr;
    int rc = tensor_create(ctx, TMQ_TYPE_Q5_0, 4, 896, rows.data(), false, rows.size(), nullptr, false, row_norm, &t);
    if (rc) return rc;
    std::vector<int64_t> acc;
    rc = run_int16(ctx, t, act, acc);
    tmq_tensor_free(t);
    if (rc) return rc;
    for (int i = 0; i < 4; i++) result[row_base + i] += acc[i];
    return 0;
}

static int tile_kquant(tmq_ctx* ctx, uint32_t type, const uint8_t* blocks, int nblocks,
                       const int16_t* act, int ncols, const float* row_inv, int64_t* result,
                       int row_base) {
    if (!ctx || !blocks || !act || !row_inv || !result) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (nblocks <= 0 || ncols < 0) return tmq_fail(TMQ_ERR_ARG, "nblocks %d ncols %d", nblocks, ncols);
    tmq_tensor* t = nullptr;
    int rc = tensor_create(ctx, type, (uint64_t)nblocks, 256, blocks, false,
                           (uint64_t)nblocks * block_bytes(type), nullptr, false, row_inv + row_base, &t);
    if (rc) return rc;
    // columns past ncols do not contribute (the reference stops at wi >= ncols)
    std::vector<int16_t> a(256, 0);
    for (int i = 0; i < ncols && i < 256; i++) a[i] = act[i];
    std::vector<int64_t> acc;
    rc = run_int16(ctx, t, a.data(), acc);
    tmq_tensor_free(t);
    if (rc) return rc;
    for (int bi = 0; bi < nblocks; bi++)
        if (row_base + bi < 896) result[row_base + bi] += acc[bi];
    return 0;
}

int tmq_vecmul_tile_q6_k(tmq_ctx* ctx, const uint8_t* blocks, int nblocks, const int16_t* act,
                         int ncols, const float* row_inv, int64_t* result, int row_base) {
    return tile_kquant(ctx, TMQ_TYPE_Q6_K, blocks, nblocks, act, ncols, row_inv, result, row_base);
}

int tmq_vecmul_tile_q4k(tmq_ctx* ctx, const uint8_t* blocks, int nblocks, const int16_t* act,
                        int ncols, const float* row_inv, int64_t* result, int row_base) {
    return tile_kquant(ctx, TMQ_TYPE_Q4_K, blocks, nblocks, act, ncols, row_inv, result, row_base);
}

// ---------------------------------------------------------------- chains
int tmq_chain_create(tmq_ctx* ctx, const tmq_desc* descs, int n, tmq_chain** out) {
    if (!ctx || !descs || n <= 0 || !out) return tmq_fail(TMQ_ERR_ARG, "bad chain arguments");
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    tmq_chain* ch = new tmq_chain();
    ch->ctx = ctx;
    std::map<const float*, int> xs;  // distinct activations
    std::vector<int> act_of(n);
    std::vector<int> ncols_of;
    for (int i = 0; i < n; i++) {
        const tmq_desc& d = descs[i];
        const tmq_tensor* t = d.weight;
        if (!t || !d.x_dev) {
            delete ch;
            return tmq_fail(TMQ_ERR_DESC, "descriptor %d: null weight or x", i);
        }
        const TmqTensorDev& td = t->dev;
        if (is_float_type((uint32_t)td.type)) {
            delete ch;
            return tmq_fail(TMQ_ERR_DESC, "descriptor %d: %s tensors have no descriptor type", i, type_name((uint32_t)td.type));
        }
        long rows;
        if (td.type == TMQ_TYPE_Q4_K || td.type == TMQ_TYPE_Q6_K) {
            if (d.num_col_groups == 0 || d.num_tiles % d.num_col_groups || d.num_col_groups * 256 != td.cols) {
                delete ch;
                return tmq_fail(TMQ_ERR_DESC, "descriptor %d: num_col_groups %d / num_tiles %d inconsistent with cols %d",
                            i, d.num_col_groups, d.num_tiles, td.cols);
            }
            rows = (long)(d.num_tiles / d.num_col_groups) * d.tile_res_rows;
        } else {
            rows = (long)d.num_tiles * d.tile_res_rows;
        }
        if (rows != td.rows) {
            delete ch;
            return tmq_fail(TMQ_ERR_DESC, "descriptor %d: tiles give %ld rows, tensor has %d", i, rows, td.rows);
        }
        auto it = xs.find(d.x_dev);
        if (it == xs.end()) {
            if ((int)xs.size() >= TMQ_MAX_ACT) {
                delete ch;
                return tmq_fail(TMQ_ERR_DESC, "more than %d distinct activations in one chain", TMQ_MAX_ACT);
            }
            int id = (int)xs.size();
            xs[d.x_dev] = id;
            ncols_of.push_back(td.cols);
            act_of[i] = id;
        } else {
            act_of[i] = it->second;
            if (ncols_of[it->second] != td.cols) {
                delete ch;
                return tmq_fail(TMQ_ERR_DESC, "descriptor %d: activation shared with a different width", i);
            }
        }
    }
    // activation buffers
    std::vector<size_t> act_off(xs.size());
    size_t act_total = 0;
    for (size_t a = 0; a < xs.size(); a++) {
        act_off[a] = act_total;
        act_total += (tmq_act_bytes(ncols_of[a]) + 255) & ~(size_t)255;
    }
    hipError_t e = hipMalloc(&ch->act_dev, act_total);
    if (e != hipSuccess) {
        delete ch;
        return tmq_fail(TMQ_ERR_NOMEM, "chain act alloc: %s", hipGetErrorString(e));
    }
    ch->jobs.count = (int)xs.size();
    for (auto& kv : xs) {
        TmqActJob& j = ch->jobs.j[kv.second];
        j.x = kv.first;
        j.act = (uint8_t*)ch->act_dev + act_off[kv.second];
        j.n = ncols_of[kv.second];
    }
    // work list, one segment per format
    std::vector<TmqGroupRef> gmap;
    for (int i = 0; i < n; i++) {
        const tmq_desc& d = descs[i];
        ch->works.push_back(make_work(d.weight, (const uint8_t*)ch->act_dev + act_off[act_of[i]], d.y_dev, d.acc_dev));
        ch->weight_bytes += d.weight->weight_bytes;
    }
    // TMQ_NOSPLIT=1 (testing): no split groups
    const char* nsp = getenv("TMQ_NOSPLIT");
    int nslots = 0;
    plan_segments(ch->works, gmap, ch->segs, nsp && atoi(nsp) != 0 ? 0 : ctx->ncu, nslots);
    e = hipMalloc(&ch->works_dev, sizeof(TmqWork) * ch->works.size());
    if (e == hipSuccess) e = hipMalloc(&ch->gmap_dev, sizeof(TmqGroupRef) * gmap.size());
    if (e == hipSuccess && nslots) e = hipMalloc(&ch->tail_dev, sizeof(uint64_t) * TMQ_TAIL_SLOT_WORDS * nslots);
    if (e == hipSuccess && nslots) e = hipMemset(ch->tail_dev, 0, sizeof(uint64_t) * TMQ_TAIL_SLOT_WORDS * nslots);
    if (e == hipSuccess)
        e = hipMemcpy(ch->works_dev, ch->works.data(), sizeof(TmqWork) * ch->works.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(ch->gmap_dev, gmap.data(), sizeof(TmqGroupRef) * gmap.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        tmq_chain_free(ch);
        return tmq_fail(TMQ_ERR_NOMEM, "chain alloc: %s", hipGetErrorString(e));
    }
    *out = ch;
    return 0;
}

int tmq_chain_prepare(tmq_ctx* ctx, tmq_chain* ch) {
    if (!ctx || !ch) return tmq_fail(TMQ_ERR_ARG, "null argument");
    LAUNCH_TRY(tmq_launch_act_prep(ch->jobs, ctx->stream));
    return 0;
}

int tmq_chain_launch(tmq_ctx* ctx, tmq_chain* ch) {
    if (!ctx || !ch) return tmq_fail(TMQ_ERR_ARG, "null argument");
    return launch_segments(ch->segs, ch->works_dev, ch->gmap_dev, ch->tail_dev, ctx->stream);
}

int tmq_chain_run(tmq_ctx* ctx, tmq_chain* ch) {
    int rc = tmq_chain_prepare(ctx, ch);
    return rc ? rc : tmq_chain_launch(ctx, ch);
}

int tmq_chain_free(tmq_chain* ch) {
    if (!ch) return 0;
    if (ch->ctx) {
        (void)hipSetDevice(ch->ctx->device);
        (void)hipStreamSynchronize(ch->ctx->stream);
    }
    if (ch->works_dev) (void)hipFree(ch->works_dev);
    if (ch->gmap_dev) (void)hipFree(ch->gmap_dev);
    if (ch->tail_dev) (void)hipFree(ch->tail_dev);
    if (ch->act_dev) (void)hipFree(ch->act_dev);
    delete ch;
    return 0;
}

uint64_t tmq_chain_weight_bytes(const tmq_chain* ch) { return ch ? ch->weight_bytes : 0; }

// ---------------------------------------------------------------- PhaseB
// Walks the chain on the host (descriptors are 32 bytes each), rebuilds
// each matmul descriptor's weights as device tensors and runs them in chain
// launches; results land in the arena at result_addr, as phaseb_verify
// writes them (sim/tmac_gguf.cpp:851-852).  Descriptors run in chain order
// as far as the hardware would see: one whose activation or weights read a
// result range still pending (an OP->OP chain, :551-561) first waits for
// the pending ones to land in the arena.
namespace {
struct PbPart {
    tmq_tensor* t = nullptr;
    std::vector<uint8_t> act;
};
struct PbItem {
    std::vector<PbPart> parts;  // one tensor, or one per column group
    uint32_t result_addr = 0;
    int nrows = 0;
    bool kquant = false;
};
void pb_free(std::vector<PbItem>& items) {
    for (PbItem& it : items)
        for (PbPart& p : it.parts) tmq_tensor_free(p.t);
    items.clear();
}
// every pending descriptor in one launch per format, results into the arena
int pb_flush(tmq_ctx* ctx, std::vector<PbItem>& items, uint8_t* arena, uint32_t arena_base) {
    if (items.empty()) return 0;
    size_t act_total = 0, acc_total = 0;
    std::vector<size_t> aoff, coff;
    for (PbItem& it : items)
        for (PbPart& p : it.parts) {
            aoff.push_back(act_total);
            act_total += (p.act.size() + 255) & ~(size_t)255;
            coff.push_back(acc_total);
            acc_total += (size_t)p.t->dev.rows;
        }
    int rc = ctx->act.ensure(act_total);
    if (!rc) rc = ctx->acc.ensure(sizeof(int64_t) * acc_total);
    if (rc) return rc;
    std::vector<TmqWork> works;
    std::vector<TmqGroupRef> gmap;
    std::vector<Segment> segs;
    size_t k = 0;
    for (PbItem& it : items)
        for (PbPart& p : it.parts) {
            HIP_TRY(hipMemcpyAsync((uint8_t*)ctx->act.p + aoff[k], p.act.data(), p.act.size(), hipMemcpyHostToDevice,
                                   ctx->stream));
            works.push_back(make_work(p.t, (const uint8_t*)ctx->act.p + aoff[k], nullptr, (int64_t*)ctx->acc.p + coff[k]));
            k++;
        }
    // (no split groups: the arena's descriptors are one-off launches)
    int nslots = 0;
    plan_segments(works, gmap, segs, 0, nslots);
    rc = ctx->works.ensure(sizeof(TmqWork) * works.size());
    if (!rc) rc = ctx->gmap.ensure(sizeof(TmqGroupRef) * gmap.size());
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->works.p, works.data(), sizeof(TmqWork) * works.size(), hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipMemcpyAsync(ctx->gmap.p, gmap.data(), sizeof(TmqGroupRef) * gmap.size(), hipMemcpyHostToDevice,
                           ctx->stream));
    rc = launch_segments(segs, ctx->works.p, ctx->gmap.p, nullptr, ctx->stream);
    if (rc) return rc;
    std::vector<int64_t> acc(acc_total);
    HIP_TRY(hipMemcpyAsync(acc.data(), ctx->acc.p, sizeof(int64_t) * acc_total, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    k = 0;
    for (PbItem& it : items) {
        // column-group parts add up per row, as the tiles accumulate (:815-817)
        std::vector<int64_t> rows(it.nrows, 0);
        for (PbPart& p : it.parts) {
            for (int r = 0; r < it.nrows && r < p.t->dev.rows; r++) rows[r] += acc[coff[k] + r];
            k++;
        }
        uint8_t* dst = arena + (it.result_addr - arena_base);
        for (int r = 0; r < it.nrows; r++) {
            // K-quant tiles only accumulate rows < 896 (sim/fpga_sim.hpp:1112, :779)
            const int64_t v = (it.kquant && r >= 896) ? 0 : rows[r];
            memcpy(dst + (size_t)r * 8, &v, 8);
        }
    }
    pb_free(items);
    return 0;
}
}  // namespace

int tmq_phaseb_run(tmq_ctx* ctx, uint8_t* arena, uint64_t arena_bytes, uint32_t arena_base,
                   uint32_t head_off, uint32_t* rows_out, int max_desc) {
    if (!ctx || !arena) return tmq_fail(TMQ_ERR_ARG, "null argument");
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    auto in_arena = [&](uint64_t off, uint64_t len) {
        return off >= arena_base && off - arena_base + len <= arena_bytes;
    };
    std::vector<PbItem> items;  // pending
    std::vector<uint32_t> rows_list;
    auto cleanup = [&](int code) {
        pb_free(items);
        return code;
    };
    // does [a, a+len) read a result range that is still pending?
    auto reads_pending = [&](uint64_t a, uint64_t len) {
        for (const PbItem& it : items)
            if (a < (uint64_t)it.result_addr + 8ull * it.nrows && (uint64_t)it.result_addr < a + len) return true;
        return false;
    };
    uint32_t off = head_off;
    int walked = 0;
    while (off) {
        if (walked >= (1 << 16)) return cleanup(tmq_fail(TMQ_ERR_DESC, "descriptor chain longer than 65536 (cycle?)"));
        if (!in_arena(off, 32)) return cleanup(tmq_fail(TMQ_ERR_DESC, "descriptor at 0x%x outside arena", off));
        const uint8_t* d = arena + (off - arena_base);
        const uint32_t next = rd32(d), wa = rd32(d + 4), aa = rd32(d + 8), ra = rd32(d + 12);
        const int nt = rd16(d + 0x10), tb = rd16(d + 0x12), type = d[0x14], tr = d[0x15];
        const int cg = d[0x19];
        int nrows = 0;
        if (type == TMQ_TYPE_Q5_0) {
            // sim tile: 8 rows x 896 (224 blocks) + row_inv section; replay
            // recomputes row_inv per tile (sim/tmac_gguf.cpp:766-777)
            if (tr != 8 || tb < 224 * 22)
                return cleanup(tmq_fail(TMQ_ERR_DESC, "Q5_0 descriptor at 0x%x: tile_res_rows %d / tile_bytes %d not the 8x896 tile", off, tr, tb));
            nrows = nt * tr;
            if (!in_arena(wa, (uint64_t)nt * tb) || !in_arena(aa, 896 * 2) || !in_arena(ra, (uint64_t)nrows * 8))
                return cleanup(tmq_fail(TMQ_ERR_DESC, "Q5_0 descriptor at 0x%x: address out of arena", off));
            if (reads_pending(wa, (uint64_t)nt * tb) || reads_pending(aa, 896 * 2))
                if ((rc = pb_flush(ctx, items, arena, arena_base))) return cleanup(rc);
            std::vector<uint8_t> w((size_t)nt * 224 * 22);
            for (int ti = 0; ti < nt; ti++)
                memcpy(w.data() + (size_t)ti * 224 * 22, arena + (wa - arena_base) + (size_t)ti * tb, 224 * 22);
            PbItem it;
            it.parts.resize(1);
            int rc2 = tensor_create(ctx, TMQ_TYPE_Q5_0, (uint64_t)nrows, 896, w.data(), false, w.size(), nullptr,
                                    false, nullptr, &it.parts[0].t);
            if (rc2) return cleanup(rc2);
            it.parts[0].t->dev.clamp = 1;
            act_from_int16((const int16_t*)(arena + (aa - arena_base)), 896, it.parts[0].act);
            it.result_addr = ra;
            it.nrows = nrows;
            items.push_back(std::move(it));
        } else if (type == TMQ_TYPE_Q6_K || type == TMQ_TYPE_Q4_K) {
            const bool k6 = type == TMQ_TYPE_Q6_K;
            const int bb = k6 ? 210 : 144, blk_bytes = k6 ? 32 * 210 : 56 * 144;
            if (cg == 0 || tr == 0 || nt % cg)
                return cleanup(tmq_fail(TMQ_ERR_DESC, "K-quant descriptor at 0x%x: num_col_groups %d tile_res_rows %d num_tiles %d", off, cg, tr, nt));
            if (tb < blk_bytes + tr * 4 || tr * bb > blk_bytes)
                return cleanup(tmq_fail(TMQ_ERR_DESC, "K-quant descriptor at 0x%x: tile_bytes %d too small", off, tb));
            nrows = (nt / cg) * tr;
            const int cols = cg * 256;
            if (!in_arena(wa, (uint64_t)nt * tb) || !in_arena(aa, (uint64_t)cols * 2) || !in_arena(ra, (uint64_t)nrows * 8))
                return cleanup(tmq_fail(TMQ_ERR_DESC, "K-quant descriptor at 0x%x: address out of arena", off));
            if (reads_pending(wa, (uint64_t)nt * tb) || reads_pending(aa, (uint64_t)cols * 2))
                if ((rc = pb_flush(ctx, items, arena, arena_base))) return cleanup(rc);
            // row_inv of every (row, column group): the tile's UQ24.8 value (:791-795)
            std::vector<float> ri((size_t)nrows * cg, 0.0f);
            bool uniform = true;
            for (int ti = 0; ti < nt; ti++) {
                const int cgi = ti % cg, row0 = (ti / cg) * tr;
                const uint8_t* tile = arena + (wa - arena_base) + (size_t)ti * tb;
                for (int i = 0; i < tr; i++) {
                    ri[(size_t)(row0 + i) * cg + cgi] = (float)rd32(tile + blk_bytes + i * 4) / 256.0f;
                    if (cgi > 0 && ri[(size_t)(row0 + i) * cg + cgi] != ri[(size_t)(row0 + i) * cg]) uniform = false;
                }
            }
            // one tensor when every row has one row_inv, else one per column
            // group (each tile's own value applies to its columns)
            const int np = uniform ? 1 : cg, pcols = uniform ? cols : 256;
            PbItem it;
            it.parts.resize(np);
            const int16_t* act = (const int16_t*)(arena + (aa - arena_base));
            for (int p = 0; p < np; p++) {
                const int ncg = uniform ? cg : 1;
                std::vector<uint8_t> w((size_t)nrows * ncg * bb);
                std::vector<float> pri(nrows);
                for (int ti = 0; ti < nt; ti++) {
                    const int cgi = ti % cg, row0 = (ti / cg) * tr;
                    if (!uniform && cgi != p) continue;
                    const int dcol = uniform ? cgi : 0;
                    const uint8_t* tile = arena + (wa - arena_base) + (size_t)ti * tb;
                    for (int i = 0; i < tr; i++) {
                        memcpy(w.data() + ((size_t)(row0 + i) * ncg + dcol) * bb, tile + (size_t)i * bb, bb);
                        pri[row0 + i] = ri[(size_t)(row0 + i) * cg + (uniform ? 0 : p)];
                    }
                }
                int rc2 = tensor_create(ctx, (uint32_t)type, (uint64_t)nrows, (uint64_t)pcols, w.data(), false,
                                        w.size(), nullptr, false, pri.data(), &it.parts[p].t);
                if (rc2) return cleanup(rc2);
                act_from_int16(act + (uniform ? 0 : 256 * p), pcols, it.parts[p].act);
            }
            it.result_addr = ra;
            it.nrows = nrows;
            it.kquant = true;
            items.push_back(std::move(it));
        } else {
            nrows = 0;  // CPU_OP and unsupported types: no matmul rows (:823-829)
        }
        rows_list.push_back((uint32_t)nrows);
        walked++;
        off = next;
    }
    if ((rc = pb_flush(ctx, items, arena, arena_base))) return cleanup(rc);
    if (rows_out)
        for (int i = 0; i < (int)rows_list.size() && i < max_desc; i++) rows_out[i] = rows_list[i];
    return walked;
}

}  // extern "C"
