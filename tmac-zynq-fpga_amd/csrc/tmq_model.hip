// tmq_model.hip -- batch-1 decode engine: a .tmac model resident in HBM and
// the launch sequence of one decode step, optionally captured as a HIP graph.
//
// Mirrors the reference engine (sim/tmac_gguf.cpp): load_tmac (:1894),
// reset_cache/process_prompt (:1950, :1969), forward_layer_with_cache
// (:1559), get_logits_q8 (:1820) and generate (:2001) with greedy selection.
// The host only orders launches; every number is computed on the GPU, except
// the RoPE cos/sin table, which is filled once per model from the host libm
// exactly as apply_rope (:1527-1554) computes its factors.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <map>
#include <string>
#include <vector>

#include "../../include/tmq.h"
#include "tmq_engine.h"
#include "tmq_internal.h"
#include "tmq_mathf.h"
#include "tmq_prefill.h"
#include "tmq_runtime.h"

namespace {

struct Entry {
    std::string name;
    uint64_t rows, cols, n_bytes;
    uint32_t type;
    const uint8_t* data;
};

// one engine GEMV launch (passed by value) and its workgroup size
struct Launch {
    TmqEngLaunch P{};
    int waves = 4;
};

struct Layer {
    tmq_tensor *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    tmq_tensor *gate = nullptr, *up = nullptr, *down = nullptr;
    tmq_tensor* gu_t = nullptr;  // gate and up rows interleaved by 32 (fused SwiGLU GEMV), or null
    size_t attn_norm = 0, ffn_norm = 0;  // offsets into fvec (floats)
    long bq = -1, bk = -1, bv = -1;      // bias offsets or -1
    Launch qkv, o_l, gu, dn;
    bool fused_gu = false;  // gate+up+SwiGLU in one launch (gu_t) under the current flags
    // K-split results of this layer's GEMVs, finalised by their consumers
    TmqDeferred dq{}, dk{}, dv{}, dout{}, dg{}, du{}, dd{};
};

inline uint64_t rd64(const uint8_t* p) {
    uint64_t v;
    memcpy(&v, p, 8);
    return v;
}
inline uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

// Parse the .tmac container (scripts/extract_tmac.py:6-24): "TMAC", u64
// count, then per tensor u64 name_len, name, u64 rows, u64 cols, u32 type,
// u64 n_bytes, data.  Every field is bounds checked.
int parse_tmac(const uint8_t* base, uint64_t size, std::vector<Entry>& out) {
    if (size < 12 || memcmp(base, "TMAC", 4) != 0) return tmq_fail(TMQ_ERR_ARG, "not a .tmac file (magic)");
    const uint64_t n = rd64(base + 4);
    uint64_t off = 12;
    if (n > (1u << 20)) return tmq_fail(TMQ_ERR_ARG, ".tmac: implausible tensor count %llu", (unsigned long long)n);
    for (uint64_t i = 0; i < n; i++) {
        if (size - off < 8) return tmq_fail(TMQ_ERR_ARG, ".tmac: truncated at tensor %llu", (unsigned long long)i);
        const uint64_t nl = rd64(base + off);
        off += 8;
        if (nl == 0 || nl > 4096 || size - off < nl + 28)
            return tmq_fail(TMQ_ERR_ARG, ".tmac: bad name length %llu at tensor %llu", (unsigned long long)nl,
                            (unsigned long long)i);
        Entry e;
        e.name.assign((const char*)base + off, (size_t)nl);
        off += nl;
        e.rows = rd64(base + off);
        e.cols = rd64(base + off + 8);
        e.type = rd32(base + off + 16);
        e.n_bytes = rd64(base + off + 20);
        off += 28;
        if (e.n_bytes > size - off)
            return tmq_fail(TMQ_ERR_ARG, ".tmac: tensor %s data (%llu B) past end of file", e.name.c_str(),
                            (unsigned long long)e.n_bytes);
        e.data = base + off;
        off += e.n_bytes;
        out.push_back(e);
    }
    return 0;
}

uint64_t ggml_bytes(uint32_t type, uint64_t rows, uint64_t cols) {
    switch (type) {
    case TMQ_TYPE_Q8_0: return cols % 32 ? 0 : rows * (cols / 32) * 34;
    case TMQ_TYPE_Q5_0: return cols % 32 ? 0 : rows * (cols / 32) * 22;
    case TMQ_TYPE_Q4_K: return cols % 256 ? 0 : rows * (cols / 256) * 144;
    case TMQ_TYPE_Q6_K: return cols % 256 ? 0 : rows * (cols / 256) * 210;
    default: return 0;
    }
}

int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

}  // namespace

// Batched prefill (tmq_prefill.h): weight digit planes of every layer,
// built on first use, and the activation buffers of one chunk of tokens.
struct PfLayer {
    TmqPfPlanes qkv{}, o{}, gu{}, dn{};
};
struct Prefill {
    bool built = false;
    void* wmem = nullptr;  // all layers' weight planes
    void* amem = nullptr;  // chunk buffers
    int chunk = 0;         // tokens per chunk the buffers hold (multiple of 128)
    std::vector<PfLayer> layers;
    float *x0 = nullptr, *x1 = nullptr, *qb = nullptr, *ctx = nullptr, *s = nullptr;
    TmqPfPlanes in[4]{};   // activation planes: QKV, O, GU, DN inputs
    float* xs[4] = {nullptr, nullptr, nullptr, nullptr};
    int64_t* part = nullptr;
    uint32_t* max_bits = nullptr;
    uint32_t* gq_cnt = nullptr;  // the quantising GU epilogue's counters and release flags (TmqPfGemm.gq_cnt)
    int dn_split = 4;
    int o_split = 2;   // attn_output GEMM split over K (finalised by the ffn_norm input)
    int qkv_split = 1; // q/k/v GEMM split over K (finished by pf_qkv_fin)
    int tile[4] = {4, 4, 3, 1};  // GEMM workgroup tiles: qkv, o, gate/up, down (tmq_launch_pf_gemm)
    // captured prefills, by prompt length, chunk and the settings the
    // launches read (a capture holds the chunk buffers' addresses: dropped
    // with them)
    struct Graph {
        int lim, chunk, guq, spin;
        hipGraphExec_t g;
    };
    std::vector<Graph> graphs;
    int cap_lim = 0, cap_chunk = 0;  // what the capture in progress runs
};

struct tmq_model {
    tmq_ctx* ctx = nullptr;
    tmq_model_config cfg{};
    tmq_tensor* emb = nullptr;
    std::vector<Layer> layers;
    long out_norm = -1;
    std::vector<tmq_tensor*> owned;
    // device memory (one allocation)
    void* dmem = nullptr;
    // residual stream, double buffered: hid[1] = after the attention block's
    // input materialisation (embedding / + down), hid[0] = after + attn_output
    float* hid[2] = {nullptr, nullptr};
    float *ctxv = nullptr, *logits = nullptr, *fvec = nullptr, *dump = nullptr, *view = nullptr;
    int64_t* kacc = nullptr;  // all K-split accumulators of a step
    size_t kacc_n = 0;        // used by the current flags (zeroed per step)
    size_t kacc_cap = 0;      // allocated
    uint32_t flags = TMQ_FLAGS_ALL;  // the reference's --fpga* globals (TMQ_FLAG_*)
    float* xs = nullptr;      // x_scale slots, 4 per layer
    uint64_t* cand = nullptr;  // logits argmax candidates, one per 64 rows
    int n_cand = 0;
    float *kc = nullptr, *vc = nullptr;
    float2* rope = nullptr;
    float2* rope_cur = nullptr;  // the current position's RoPE row (written by every qkv launch)
    TmqEngState* state = nullptr;
    int32_t* tokens = nullptr;
    float* silu_x = nullptr;      // SiLU(gate) * up of the current layer
    uint32_t* max_bits = nullptr; // per layer TMQ_MAX_SLOTS slots of max |silu_x| (in the zeroed accumulator range)
    Launch logits_l;
    uint64_t weight_bytes = 0;
    int pos = -1;  // host mirror of state.pos
    bool use_graphs = true;
    hipGraphExec_t g_feed = nullptr, g_decode = nullptr;
    // tmq_model_profile: an event before and after every launch
    std::vector<std::pair<const char*, hipEvent_t>>* prof = nullptr;
    int prefill_chunk = 512;  // 0: prompts run one token at a time
    int spec_miss = 0;        // TMQ_SPEC_MISS=1: every RMSNorm sum segment re-runs (testing)
    const char* prefill_off = nullptr;  // why the model cannot use the batched prefill
    Prefill pf;
};

namespace {

void model_release(tmq_model* m) {
    if (!m) return;
    if (m->ctx) {
        (void)hipSetDevice(m->ctx->device);
        (void)hipStreamSynchronize(m->ctx->stream);
    }
    if (m->g_feed) (void)hipGraphExecDestroy(m->g_feed);
    if (m->g_decode) (void)hipGraphExecDestroy(m->g_decode);
    for (tmq_tensor* t : m->owned) tmq_tensor_free(t);
    if (m->dmem) (void)hipFree(m->dmem);
    for (auto& g : m->pf.graphs) (void)hipGraphExecDestroy(g.g);
    if (m->pf.wmem) (void)hipFree(m->pf.wmem);
    if (m->pf.amem) (void)hipFree(m->pf.amem);
    delete m;
}

// ---------------------------------------------------------------- launches
// Profiling (tmq_model_profile, eager launches only): an event on the
// stream, tagged with the launch it opens (name) or closes (null).
int prof_mark(tmq_model* m, const char* name) {
    if (!m->prof) return 0;
    hipEvent_t e = nullptr;
    HIP_TRY(hipEventCreate(&e));
    m->prof->push_back({name, e});
    HIP_TRY(hipEventRecord(e, m->ctx->stream));
    return 0;
}
#define PROF(name, call)                          \
    do {                                          \
        int prc_ = prof_mark(m, name);            \
        if (prc_) return prc_;                    \
        call;                                     \
        if ((prc_ = prof_mark(m, nullptr))) return prc_; \
    } while (0)

int launch_gemv(tmq_model* m, const Launch& l) {
    LAUNCH_TRY(tmq_launch_eng_gemv(l.P, l.waves, m->ctx->stream));
    return 0;
}

// all layers at the current position (forward_all_layers); layer 0's QKV
// launch also performs process_embedding of tokens[pos].  The step's K-split
// accumulators are zeroed first.  With dump, the residual stream after the
// embedding and after every layer is copied to dump[(l+1)*H].
// With cap (eager launches only), the fp32 input of every matmul is stored
// per layer at cap + l*(3*hidden + ffn): the attn_norm output (q, k, v),
// the attention context (attn_output), the ffn_norm output (gate, up) and
// SiLU(gate)*up (ffn_down).
int launch_layers(tmq_model* m, bool dump, float* cap = nullptr) {
    hipStream_t s = m->ctx->stream;
    const tmq_model_config& c = m->cfg;
    const int H = c.hidden, KV = c.n_kv_heads * TMQ_HEAD_DIM;
    const size_t per = 3 * (size_t)H + c.inter;
    PROF("zero_acc", LAUNCH_TRY(tmq_launch_zero_acc(m->kacc, m->kacc_n, s)));
    for (int l = 0; l < c.n_layers; l++) {
        const Layer& L0 = m->layers[l];
        Layer Lc;
        if (cap) {
            Lc = L0;
            Lc.qkv.P.act.act_out = cap + l * per;
            Lc.gu.P.act.act_out = cap + l * per + 2 * (size_t)H;
        }
        const Layer& L = cap ? Lc : L0;
        int rc = 0;
        PROF(l == 0 ? "embedding+attn_norm+qkv" : "attn_norm+qkv", rc = launch_gemv(m, L.qkv));
        if (rc) return rc;
        if (dump && l == 0) HIP_TRY(hipMemcpyAsync(m->dump, m->hid[1], sizeof(float) * H, hipMemcpyDeviceToDevice, s));
        TmqAttnArgs aa{};
        aa.q = L.dq;
        aa.k = L.dk;
        aa.v = L.dv;
        aa.kc = m->kc + (size_t)l * c.max_seq * KV;
        aa.vc = m->vc + (size_t)l * c.max_seq * KV;
        aa.rope_cur = m->rope_cur;
        aa.state = m->state;
        aa.ctx = m->ctxv;
        aa.n_heads = c.n_heads;
        aa.n_kv = c.n_kv_heads;
        aa.max_pos = c.max_seq;
        PROF("rope+attention", LAUNCH_TRY(tmq_launch_attn(aa, s)));
        if (cap) HIP_TRY(hipMemcpyAsync(cap + l * per + H, m->ctxv, sizeof(float) * H, hipMemcpyDeviceToDevice, s));
        PROF("attn_output", rc = launch_gemv(m, L.o_l));
        if (rc) return rc;
        PROF(L.fused_gu ? "ffn_norm+gate+up+silu_x_up" : "ffn_norm+gate+up", rc = launch_gemv(m, L.gu));
        if (rc) return rc;
        if (!L.fused_gu)
            PROF("silu_x_up", LAUNCH_TRY(tmq_launch_silu(L.dg, L.du, c.inter, m->silu_x,
                                                         m->max_bits + TMQ_MAX_SLOTS * l, s)));
        if (cap)
            HIP_TRY(hipMemcpyAsync(cap + l * per + 3 * (size_t)H, m->silu_x, sizeof(float) * c.inter,
                                   hipMemcpyDeviceToDevice, s));
        PROF("ffn_down", rc = launch_gemv(m, L.dn));
        if (rc) return rc;
        if (dump) LAUNCH_TRY(tmq_launch_resid_view(m->hid[0], L.dd, H, m->dump + (size_t)(l + 1) * H, s));
    }
    return 0;
}

// one position whose token the host stored at tokens[pos+1]
int launch_feed_impl(tmq_model* m, bool dump, float* cap = nullptr) {
    LAUNCH_TRY(tmq_launch_advance(m->state, m->cfg.max_seq, m->ctx->stream));
    return launch_layers(m, dump, cap);
}
int launch_feed(tmq_model* m) { return launch_feed_impl(m, false); }

// get_logits_q8: output_norm (when present) of the residual stream + the
// Q8_0 logits GEMV, which also leaves per-wave argmax candidates
int launch_logits(tmq_model* m) { return launch_gemv(m, m->logits_l); }

// one greedy generate() iteration: logits, argmax -> tokens[pos+1] (and
// pos+1), then all layers of that token
int launch_decode(tmq_model* m) {
    int rc = 0;
    PROF("output_norm+logits", rc = launch_logits(m));
    if (rc) return rc;
    PROF("argmax", LAUNCH_TRY(tmq_launch_argmax(m->cand, m->n_cand, m->state, m->tokens, m->cfg.max_seq,
                                                m->ctx->stream)));
    return launch_layers(m, false);
}

int capture(tmq_model* m, int (*fn)(tmq_model*), hipGraphExec_t* out) {
    hipStream_t s = m->ctx->stream;
    HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int rc = fn(m);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_HIP, "graph capture: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_HIP, "graph instantiate: %s", hipGetErrorString(e));
    return 0;
}

int run_feed(tmq_model* m) {
    if (m->use_graphs) {
        if (!m->g_feed) {
            int rc = capture(m, launch_feed, &m->g_feed);
            if (rc) return rc;
        }
        HIP_TRY(hipGraphLaunch(m->g_feed, m->ctx->stream));
        return 0;
    }
    return launch_feed(m);
}
int run_decode(tmq_model* m) {
    if (m->use_graphs) {
        if (!m->g_decode) {
            int rc = capture(m, launch_decode, &m->g_decode);
            if (rc) return rc;
        }
        HIP_TRY(hipGraphLaunch(m->g_decode, m->ctx->stream));
        return 0;
    }
    return launch_decode(m);
}

int check_state(tmq_model* m) {
    TmqEngState st{};
    HIP_TRY(hipMemcpyAsync(&st, m->state, sizeof st, hipMemcpyDeviceToHost, m->ctx->stream));
    HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    if (st.err) return tmq_fail(TMQ_ERR_ARG, "decode step failed on the device (token or position out of range)");
    if (st.pf_err) return tmq_fail(TMQ_ERR_HIP, "prefill: a gate/up workgroup's wait for its token tile ran out of polls");
    if (st.pos != m->pos) return tmq_fail(TMQ_ERR_HIP, "device position %d != expected %d", st.pos, m->pos);
    return 0;
}

// ---------------------------------------------------------------- prefill
// Weight digit planes of every layer (once per model).  q, k, v share one
// plane set (rows q | k | v), gate and up another (rows gate | up).
int pf_build_weights(tmq_model* m) {
    Prefill& P = m->pf;
    P.dn_split = std::max(1, env_int("TMQ_PF_SPLIT_DN", P.dn_split));
    P.o_split = std::max(1, env_int("TMQ_PF_SPLIT_O", P.o_split));
    P.qkv_split = std::max(1, env_int("TMQ_PF_SPLIT_QKV", P.qkv_split));
    if (const char* e = getenv("TMQ_PF_TILES")) {
        int t[4];
        if (sscanf(e, "%d,%d,%d,%d", &t[0], &t[1], &t[2], &t[3]) == 4)
            for (int i = 0; i < 4; i++) P.tile[i] = t[i];
    }
    const tmq_model_config& c = m->cfg;
    const int H = c.hidden, KV = c.n_kv_heads * TMQ_HEAD_DIM, I = c.inter;
    auto bytes = [](int rows, int K) { return 2 * (size_t)rows * K + 4 * (size_t)rows * (K / TMQ_PF_CHUNK + 1); };
    const size_t per = bytes(H + 2 * KV, H) + bytes(H, H) + bytes(2 * I, H) + bytes(H, I);
    const size_t total = per * c.n_layers + 256 * 16 * (size_t)c.n_layers;
    hipError_t e = hipMalloc(&P.wmem, total);
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_NOMEM, "prefill weight planes (%zu B): %s", total, hipGetErrorString(e));
    hipStream_t s = m->ctx->stream;
    HIP_TRY(hipMemsetAsync(P.wmem, 0, total, s));
    uint8_t* B = (uint8_t*)P.wmem;
    size_t off = 0;
    auto carve = [&](int rows, int K) {
        TmqPfPlanes pl{};
        auto take = [&](size_t n) {
            uint8_t* p = B + off;
            off += (n + 255) & ~(size_t)255;
            return p;
        };
        pl.d = (int8_t*)take(2 * (size_t)rows * K);
        pl.csum = (int32_t*)take(4 * (size_t)rows * (K / TMQ_PF_CHUNK));
        pl.tsum = (int32_t*)take(4 * (size_t)rows);
        pl.rows = rows;
        pl.K = K;
        return pl;
    };
    P.layers.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        const Layer& Y = m->layers[l];
        PfLayer& Q = P.layers[l];
        Q.qkv = carve(H + 2 * KV, H);
        Q.o = carve(H, H);
        Q.gu = carve(2 * I, H);
        Q.dn = carve(H, I);
        struct Job {
            const tmq_tensor* t;
            const TmqPfPlanes* pl;
            int row0;
        } jobs[] = {{Y.q, &Q.qkv, 0}, {Y.k, &Q.qkv, H}, {Y.v, &Q.qkv, H + KV}, {Y.o, &Q.o, 0},
                    {Y.gate, &Q.gu, 0}, {Y.up, &Q.gu, I}, {Y.down, &Q.dn, 0}};
        for (const Job& j : jobs) LAUNCH_TRY(tmq_launch_pf_wdigits(j.t->dev, j.pl->d, j.pl->K, j.row0, s));
        for (const TmqPfPlanes* pl : {&Q.qkv, &Q.o, &Q.gu, &Q.dn}) LAUNCH_TRY(tmq_launch_pf_rowsums(*pl, s));
    }
    if (off > total) return tmq_fail(TMQ_ERR_HIP, "prefill plane layout overflow");
    P.built = true;
    return 0;
}

// Buffers of a chunk of up to `chunk` tokens (a multiple of 128: whole
// GEMM token tiles).
int pf_build_buffers(tmq_model* m, int chunk) {
    Prefill& P = m->pf;
    if (P.amem && P.chunk == chunk) return 0;
    if (P.amem) {
        HIP_TRY(hipStreamSynchronize(m->ctx->stream));
        for (auto& g : P.graphs) (void)hipGraphExecDestroy(g.g);
        P.graphs.clear();
        (void)hipFree(P.amem);
        P.amem = nullptr;
    }
    const tmq_model_config& c = m->cfg;
    const int H = c.hidden, I = c.inter, T = chunk;
    std::vector<std::pair<void**, size_t>> parts;
    parts.push_back({(void**)&P.x0, 4 * (size_t)T * H});
    parts.push_back({(void**)&P.x1, 4 * (size_t)T * H});
    parts.push_back({(void**)&P.qb, 4 * (size_t)T * H});
    parts.push_back({(void**)&P.ctx, 4 * (size_t)T * H});
    parts.push_back({(void**)&P.s, 4 * (size_t)T * I});
    // split-K sums of the down projection and attn_output, or those of q/k/v
    // followed by the Q8_0 V tiles
    const int KV = c.n_kv_heads * TMQ_HEAD_DIM;
    const size_t part_n = std::max((size_t)std::max(P.dn_split, P.o_split) * T * H,
                                   (size_t)P.qkv_split * T * (H + 2 * KV) + (size_t)T * KV * (H / TMQ_PF_CHUNK));
    parts.push_back({(void**)&P.part, 8 * part_n});
    parts.push_back({(void**)&P.max_bits, 4 * (size_t)T});
    // the GU epilogue's counters and flags: 128 bytes each, per token tile
    // one counter and one flag a workgroup (row tile)
    parts.push_back({(void**)&P.gq_cnt, 128 * (size_t)(T / 32) * (I / 32 + 1)});
    for (int i = 0; i < 4; i++) {
        const int K = i == 3 ? I : H;
        P.in[i].rows = T;
        P.in[i].K = K;
        parts.push_back({(void**)&P.in[i].d, 2 * (size_t)T * K});
        parts.push_back({(void**)&P.in[i].csum, 4 * (size_t)T * (K / TMQ_PF_CHUNK)});
        parts.push_back({(void**)&P.in[i].tsum, 4 * (size_t)T});
        parts.push_back({(void**)&P.xs[i], 4 * (size_t)T});
    }
    size_t total = 0;
    for (auto& pr : parts) total += (pr.second + 255) & ~(size_t)255;
    hipError_t e = hipMalloc(&P.amem, total);
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_NOMEM, "prefill buffers (%zu B): %s", total, hipGetErrorString(e));
    size_t off = 0;
    for (auto& pr : parts) {
        *pr.first = (uint8_t*)P.amem + off;
        off += (pr.second + 255) & ~(size_t)255;
    }
    P.chunk = chunk;
    return 0;
}

// Whether the model's layers fit the prefill kernels: 64-aligned widths,
// and Q8_0 only among q/k/v (whose GEMM folds Q8_0 tiles).
const char* pf_unsupported(const tmq_model* m) {
    const tmq_model_config& c = m->cfg;
    const int KV = c.n_kv_heads * TMQ_HEAD_DIM;
    if (c.hidden % 64 || KV % 64 || c.inter % 64) return "hidden, KV and FFN widths must be multiples of 64";
    if (c.n_heads / c.n_kv_heads > 8) return "more than 8 query heads per KV head";
    for (const Layer& Y : m->layers) {
        for (const tmq_tensor* t : {Y.o, Y.gate, Y.up, Y.down})
            if (t->dev.type == TMQ_TYPE_Q8_0) return "Q8_0 attn_output / FFN weights";
        for (const tmq_tensor* t : {Y.q, Y.k})
            if (t->dev.type == TMQ_TYPE_Q8_0) return "Q8_0 attn_q / attn_k weights";
    }
    return nullptr;
}

TmqPfSeg pf_seg(const tmq_tensor* t, int row0, const float* bias) {
    TmqPfSeg sg{};
    sg.row0 = row0;
    sg.rows = t->dev.rows;
    sg.q8 = t->dev.type == TMQ_TYPE_Q8_0;
    sg.row_inv = t->dev.row_inv;
    sg.row_scale = t->dev.row_scale;
    sg.bias = bias;
    return sg;
}

// GEMM tile (tmq_launch_pf_gemm) for a plane set of K columns whose tensors
// start at the given rows: the preferred one if its row tile (128 for tiles
// 0 and 2, 64 for tiles 1, 3 and 4; gate/up pairs: 64 / 32 per tensor)
// divides every boundary and its stage (128 columns for tile 4, else 64)
// divides K, else the 64-row tile.
// columns per stage of a GEMM tile: the most splits over K it takes is K / this
int pf_stage_cols(int tile) { return tile == 4 ? 128 : 64; }

int pf_tile(int want, int K, std::initializer_list<int> bounds) {
    const int rt = want == 1 || want == 3 || want == 4 ? 64 : 128;
    if (K % pf_stage_cols(want)) return 1;
    for (int b : bounds)
        if (b % rt) return 1;
    return want;
}

// One chunk: positions [p0, p0+T) through every layer.  With `last`, the
// decode engine's residual state is set from the chunk's last token.
int pf_run_chunk(tmq_model* m, int p0, int T, bool last) {
    Prefill& P = m->pf;
    const tmq_model_config& c = m->cfg;
    const int H = c.hidden, KV = c.n_kv_heads * TMQ_HEAD_DIM, I = c.inter, L = c.n_layers;
    const int tile_qkv = pf_tile(P.tile[0], H, {H, KV}), tile_o = pf_tile(P.tile[1], H, {H});
    const int tile_gu = pf_tile(P.tile[2], H, {2 * I}), tile_dn = pf_tile(P.tile[3], I, {H});
    const int T_pad = (T + 127) & ~127;  // whole 128-token GEMM tiles
    hipStream_t s = m->ctx->stream;
    // gate/up quantises the SwiGLU rows itself where all its workgroups are
    // resident at once (TMQ_PF_GUQ=0: the separate act kernel); its wait
    // gives up after TMQ_PF_GUQ_SPIN polls
    int gq_tiles = 0;
    const bool gq = env_int("TMQ_PF_GUQ", 1) != 0 &&
                    tmq_pf_gu_quant_fits(tile_gu, T_pad, I, m->ctx->ncu, &gq_tiles) && gq_tiles <= P.chunk / 32;
    const int gq_words = gq_tiles * (I / 32 + 1);  // (row tiles of any GU tile: at most I / 32)
    const int gq_spin = std::max(0, env_int("TMQ_PF_GUQ_SPIN", 1 << 20));
    auto fv = [&](long o) -> const float* { return o < 0 ? nullptr : m->fvec + o; };
    auto act = [&](int mode, int set, const float* x, const float* w, int n) {
        TmqPfAct a{};
        a.mode = mode;
        a.n = n;
        a.T = T;
        a.p0 = p0;
        a.x = x;
        a.w = w;
        a.eps = c.norm_eps;
        a.spec_miss = m->spec_miss;
        a.out = P.in[set];
        a.out.rows = T_pad;
        a.xs = P.xs[set];
        return a;
    };
    auto gemm = [&](int mode, const TmqPfPlanes& W, int set) {
        TmqPfGemm g{};
        g.mode = mode;
        g.K = W.K;
        g.T = T;
        g.T_pad = T_pad;
        g.p0 = p0;
        g.split = 1;
        g.rows = W.rows;
        g.w = W.d;
        g.rw_c = W.csum;
        g.rw_t = W.tsum;
        g.x = P.in[set].d;
        g.tx_c = P.in[set].csum;
        g.tx_t = P.in[set].tsum;
        g.xs = P.xs[set];
        g.H = H;
        g.KV = KV;
        return g;
    };
    auto dn_part = [&](int l) {
        TmqPfPart d{};
        d.part = P.part;
        d.rw = P.layers[l].dn.tsum;
        d.tx = P.in[3].tsum;
        d.xs = P.xs[3];
        d.row_inv = m->layers[l].down->dev.row_inv;
        d.bias = nullptr;
        d.split = std::min(P.dn_split, I / pf_stage_cols(tile_dn));
        d.ld = H;
        d.K = I;
        d.T_pad = T_pad;
        return d;
    };
    for (int l = 0; l < L; l++) {
        const Layer& Y = m->layers[l];
        const PfLayer& W = P.layers[l];
        // attn_norm + quantisation of the layer input (embedding at layer 0)
        TmqPfAct a0 = act(l == 0 ? TMQ_PF_EMBED_NORM : TMQ_PF_RESID_NORM, 0, P.x1, m->fvec + Y.attn_norm, H);
        if (l == 0) {
            a0.tokens = m->tokens;
            a0.emb = m->emb->dev;
        } else {
            a0.d1 = dn_part(l - 1);
        }
        a0.x_out = P.x0;
        LAUNCH_TRY(tmq_launch_pf_act(a0, s));
        // q, k, v -> RoPE -> q buffer and this layer's caches; split over K,
        // finished by pf_qkv_fin (which also folds Q8_0 V tiles)
        const int qkv_split = std::min(P.qkv_split, H / pf_stage_cols(tile_qkv));
        TmqPfGemm g = gemm(qkv_split > 1 ? TMQ_PF_QKVS : TMQ_PF_QKV, W.qkv, 0);
        g.split = qkv_split;
        g.nseg = 3;
        g.seg[0] = pf_seg(Y.q, 0, fv(Y.bq));
        g.seg[1] = pf_seg(Y.k, H, fv(Y.bk));
        g.seg[2] = pf_seg(Y.v, H + KV, fv(Y.bv));
        g.q_out = P.qb;
        g.kc = m->kc + (size_t)l * c.max_seq * KV;
        g.vc = m->vc + (size_t)l * c.max_seq * KV;
        g.rope = m->rope;
        // (the down projection's sums were consumed above)
        g.part = P.part;
        g.tpart = P.part + (qkv_split > 1 ? (size_t)qkv_split * T_pad * (H + 2 * KV) : 0);
        LAUNCH_TRY(tmq_launch_pf_gemm(g, tile_qkv, s));
        if (qkv_split > 1 || Y.v->dev.type == TMQ_TYPE_Q8_0) {
            TmqPfQkvFin f{};
            f.part = qkv_split > 1 ? P.part : nullptr;
            f.tpart = g.tpart;
            f.rw_t = W.qkv.tsum;
            f.rw_c = W.qkv.csum;
            f.tx_t = P.in[0].tsum;
            f.tx_c = P.in[0].csum;
            f.xs = P.xs[0];
            for (int i = 0; i < 3; i++) f.seg[i] = g.seg[i];
            f.q_out = g.q_out;
            f.kc = g.kc;
            f.vc = g.vc;
            f.rope = g.rope;
            f.split = qkv_split;
            f.K = H;
            f.T = T;
            f.T_pad = T_pad;
            f.p0 = p0;
            f.H = H;
            f.KV = KV;
            LAUNCH_TRY(tmq_launch_pf_qkv_fin(f, s));
        }
        // attention over positions 0 .. p0+t
        TmqPfAttn at{};
        at.q = P.qb;
        at.kc = g.kc;
        at.vc = g.vc;
        at.ctx = P.ctx;
        at.T = T;
        at.p0 = p0;
        at.n_heads = c.n_heads;
        at.n_kv = c.n_kv_heads;
        at.ncu = m->ctx->ncu;
        LAUNCH_TRY(tmq_launch_pf_attn(at, s));
        // attn_output, split over K; the residual and the finalisation go
        // with the ffn_norm input
        LAUNCH_TRY(tmq_launch_pf_act(act(TMQ_PF_PLAIN, 1, P.ctx, nullptr, H), s));
        const int o_split = std::min(P.o_split, H / pf_stage_cols(tile_o));  // at most one split per stage
        g = gemm(TMQ_PF_PART, W.o, 1);
        g.split = o_split;
        g.part = P.part;
        LAUNCH_TRY(tmq_launch_pf_gemm(g, tile_o, s));
        // residual + attn_output, ffn_norm, gate/up + SwiGLU
        TmqPfAct a2 = act(TMQ_PF_RESID_NORM, 2, P.x0, m->fvec + Y.ffn_norm, H);
        a2.d1.part = P.part;
        a2.d1.rw = W.o.tsum;
        a2.d1.tx = P.in[1].tsum;
        a2.d1.xs = P.xs[1];
        a2.d1.row_inv = Y.o->dev.row_inv;
        a2.d1.bias = nullptr;
        a2.d1.split = o_split;
        a2.d1.ld = H;
        a2.d1.K = H;
        a2.d1.T_pad = T_pad;
        a2.x_out = P.x1;
        a2.zero_bits = P.max_bits;
        if (gq) {
            a2.zero_tsum = P.in[3].tsum;
            a2.zero_cnt = P.gq_cnt;
            a2.zero_ncnt = gq_words;
        }
        LAUNCH_TRY(tmq_launch_pf_act(a2, s));
        g = gemm(TMQ_PF_GU, W.gu, 2);
        g.nseg = 2;
        g.gu_rows = I;
        g.seg[0] = pf_seg(Y.gate, 0, nullptr);
        g.seg[1] = pf_seg(Y.up, I, nullptr);
        g.s_out = P.s;
        g.max_bits = P.max_bits;
        if (gq) {
            // the SwiGLU rows quantised for the down projection in the epilogue
            g.gq_d = P.in[3].d;
            g.gq_tsum = P.in[3].tsum;
            g.gq_xs = P.xs[3];
            g.gq_cnt = P.gq_cnt;
            g.gq_err = &m->state->pf_err;
            g.gq_spin = gq_spin;
            g.gq_ntiles = gq_tiles;
        }
        LAUNCH_TRY(tmq_launch_pf_gemm(g, tile_gu, s));
        if (!gq) {
            TmqPfAct a3 = act(TMQ_PF_SILU, 3, P.s, nullptr, I);
            a3.max_bits = P.max_bits;
            LAUNCH_TRY(tmq_launch_pf_act(a3, s));
        }
        // down projection, split over K; finalised by the next layer's input
        g = gemm(TMQ_PF_PART, W.dn, 3);
        g.split = std::min(P.dn_split, I / pf_stage_cols(tile_dn));
        g.part = P.part;
        LAUNCH_TRY(tmq_launch_pf_gemm(g, tile_dn, s));
    }
    if (last) {
        const Layer& Z = m->layers[L - 1];
        TmqPfHandoff h{};
        h.dn = dn_part(L - 1);
        h.x1 = P.x1;
        h.t = T - 1;
        h.H = H;
        h.hid = m->hid[0];
        h.kacc = const_cast<int64_t*>(Z.dd.acc);
        h.xs_slot = const_cast<float*>(Z.dd.xs);
        LAUNCH_TRY(tmq_launch_pf_handoff(h, s));
    }
    return 0;
}

// Every chunk of positions [0, lim).
int pf_run_all(tmq_model* m, int lim, int chunk) {
    for (int p0 = 0; p0 < lim; p0 += chunk) {
        const int T = std::min(chunk, lim - p0);
        const int rc = pf_run_chunk(m, p0, T, p0 + T >= lim);
        if (rc) return rc;
    }
    return 0;
}

// Positions [0, n) of a prompt whose tokens are on the device: as many as
// the prefill's attention can hold go through in chunks; returns how many.
int pf_prompt(tmq_model* m, int n, int* done) {
    *done = 0;
    const int qpk = m->cfg.n_heads / m->cfg.n_kv_heads;
    int lim = std::min(n, TMQ_PF_ATTN_MAXPOS);
    while (lim > 0 && tmq_pf_attn_lds(qpk, lim) > TMQ_PF_ATTN_LDS_MAX) lim--;
    if (lim < 2) return 0;
    int rc;
    if (!m->pf.built && (rc = pf_build_weights(m))) return rc;
    const int chunk = std::min(m->prefill_chunk, lim);
    if ((rc = pf_build_buffers(m, (chunk + 127) & ~127))) return rc;
    Prefill& P = m->pf;
    // one HIP graph per prompt length (TMQ_PF_GRAPH=0: launched one by one)
    if (!m->use_graphs || env_int("TMQ_PF_GRAPH", 1) == 0) {
        if ((rc = pf_run_all(m, lim, chunk))) return rc;
        *done = lim;
        return 0;
    }
    const int guq = env_int("TMQ_PF_GUQ", 1), spin = env_int("TMQ_PF_GUQ_SPIN", 1 << 20);
    hipGraphExec_t ge = nullptr;
    for (const auto& g : P.graphs)
        if (g.lim == lim && g.chunk == chunk && g.guq == guq && g.spin == spin) ge = g.g;
    if (!ge) {
        // the launches' one-time set-up (kernel attributes) before the capture
        if ((rc = tmq_pf_prepare())) return tmq_fail(TMQ_ERR_HIP, "prefill set-up: %s", hipGetErrorString((hipError_t)rc));
        if (P.graphs.size() >= 8) {
            HIP_TRY(hipStreamSynchronize(m->ctx->stream));
            for (auto& g : P.graphs) (void)hipGraphExecDestroy(g.g);
            P.graphs.clear();
        }
        P.cap_lim = lim;
        P.cap_chunk = chunk;
        if ((rc = capture(m, [](tmq_model* mm) { return pf_run_all(mm, mm->pf.cap_lim, mm->pf.cap_chunk); }, &ge)))
            return rc;
        P.graphs.push_back({lim, chunk, guq, spin, ge});
    }
    HIP_TRY(hipGraphLaunch(ge, m->ctx->stream));
    *done = lim;
    return 0;
}

// ------------------------------------------------------------------ build
// The launch lists of one decode step under the model's flags (the
// reference's command-line globals, sim/tmac_gguf.cpp:2085-2091): every
// projection takes the branch `matmul` takes for its tensor type
// (:473-493, tmq_route) -- its own quantized kernel, the INT16 fallback or
// the FP32 loop -- and the logits are get_logits_q8 under --fpga-q8, else
// get_logits, i.e. `matmul` of token_embd (:1852-1866, :2033-2037).
int build_launches(tmq_model* m) {
    const tmq_model_config& c = m->cfg;
    // the attention's dynamic LDS limit, set before any capture
    if (const int e = tmq_attn_prepare()) return tmq_fail(TMQ_ERR_HIP, "attention set-up: %s", hipGetErrorString((hipError_t)e));
    const int L = c.n_layers, H = c.hidden, I = c.inter;
    const uint32_t flags = m->flags;
    auto path_of = [&](const tmq_tensor* t) {
        const int p = tmq_route((uint32_t)t->dev.type, flags);
        return p == TMQ_PATH_INT16 ? (int)TMQ_WPATH_INT16 : p == TMQ_PATH_FP32 ? (int)TMQ_WPATH_FP32 : (int)TMQ_WPATH_FPGA;
    };
    const int logits_path = (flags & TMQ_FLAG_Q8_0) ? (int)TMQ_WPATH_FPGA : path_of(m->emb);
    // INT16 weights of every tensor routed there, built once per tensor
    int rc = 0;
    for (Layer& Y : m->layers)
        for (tmq_tensor* t : {Y.q, Y.k, Y.v, Y.o, Y.gate, Y.up, Y.down})
            if (path_of(t) == TMQ_WPATH_INT16 && (rc = tmq_rt_prepare_int16(m->ctx, t))) return rc;
    if (logits_path == TMQ_WPATH_INT16 && (rc = tmq_rt_prepare_int16(m->ctx, m->emb))) return rc;

    // accumulator slots of this flag set (FP32 rows hold final floats)
    auto slot = [&](const tmq_tensor* t) -> size_t {
        const int p = path_of(t);
        const size_t n = (p == TMQ_WPATH_FPGA && t->dev.type != TMQ_TYPE_Q8_0) || p == TMQ_WPATH_FP32
                             ? (size_t)t->dev.rows
                             : (size_t)t->dev.rows * ((t->dev.cols + 63) / 64);
        return (n + 31) & ~(size_t)31;
    };
    std::vector<size_t> acc_off(L);
    size_t acc_n = 0;
    for (int l = 0; l < L; l++) {
        const Layer& Y = m->layers[l];
        acc_off[l] = acc_n;
        for (const tmq_tensor* t : {Y.q, Y.k, Y.v, Y.o, Y.gate, Y.up, Y.down}) acc_n += slot(t);
    }
    const size_t slots64 = TMQ_MAX_SLOTS / 2;  // int64 words holding a layer's max slots
    if (acc_n + slots64 * L > m->kacc_cap) return tmq_fail(TMQ_ERR_HIP, "accumulator layout exceeds its buffer");
    m->kacc_n = acc_n + slots64 * L;  // + the max slots of every layer
    m->max_bits = (uint32_t*)(m->kacc + acc_n);  // layer l's slots at max_bits + TMQ_MAX_SLOTS * l
    auto fv_ptr = [&](long o) -> const float* { return o < 0 ? nullptr : m->fvec + o; };

    // Work lists.  Every launch is one engine GEMV: per layer qkv / o /
    // gate+up / down, each split over K (kc workgroups per 64-row group) into
    // int64 accumulators that the next launch finalises; then the logits
    // (one wave per 64 rows, direct).  The INT16 and FP32 branches run in
    // 4-wave launches; FP32 rows are not split (their sums are sequential).
    // (attn_output over 14 K chunks: 196 workgroups, 0.45 % faster per step than 7)
    const int kc_qkv = env_int("TMQ_KC_QKV", 7), kc_o = env_int("TMQ_KC_O", 14);
    const int kc_gu = env_int("TMQ_KC_GU", 1), kc_dn = env_int("TMQ_KC_DN", 19);
    auto nw_env = [](const char* n, int d) { return env_int(n, d) == 4 ? 4 : env_int(n, d) == 16 ? 16 : d; };
    const int nw_qkv = nw_env("TMQ_NW_QKV", 4), nw_o = nw_env("TMQ_NW_O", 4);
    const int nw_gu = nw_env("TMQ_NW_GU", 16), nw_dn = nw_env("TMQ_NW_DN", 4);
    auto add_work = [&](Launch& ln, const tmq_tensor* t, int64_t* kacc, float* xs_out, int kc) {
        TmqWork w = tmq_rt_make_work(t, nullptr, nullptr, nullptr);
        w.path = path_of(t);
        const int g64 = t->dev.rows_pad / 64;
        if (w.path == TMQ_WPATH_FP32) {
            w.kc = 1;
            w.y = (float*)kacc;
            w.ngroups = (g64 + ln.waves - 1) / ln.waves;
        } else {
            // (the MFMA decoders split a row by whole blocks / super-blocks)
            const int units = (t->dev.type == TMQ_TYPE_Q8_0 || w.path == TMQ_WPATH_INT16) ? (t->dev.cols + 63) / 64
                              : tmq_kernel_fmt(t->dev) != t->dev.type
                                  ? t->dev.nb
                                  : t->dev.nb * (t->dev.type == TMQ_TYPE_Q5_0 ? 1 : 4);
            if (kc > units) kc = units;
            if (kc < 1) kc = 1;
            w.kc = kc;
            w.kacc = kacc;
            w.xs_out = xs_out;
            w.ngroups = g64 * kc;
        }
        w.first_group = ln.P.ngroups;
        ln.P.ngroups += w.ngroups;
        ln.P.w[ln.P.nworks++] = w;
    };
    auto deferred = [&](const tmq_tensor* t, int64_t* acc, float* xs, const float* bias) {
        TmqDeferred d{};
        const int p = path_of(t);
        d.acc = acc;
        d.xs = xs;
        d.bias = bias;
        if (p == TMQ_WPATH_FP32) {
            d.val = (const float*)acc;
            d.row_inv = d.row_scale = (const float*)acc;
        } else if (p == TMQ_WPATH_INT16) {
            d.row_inv = d.row_scale = t->dev.rs16;
            d.ntiles = (t->dev.cols + 63) / 64;
        } else {
            d.row_inv = t->dev.row_inv;
            d.row_scale = t->dev.row_scale;
            d.ntiles = t->dev.type == TMQ_TYPE_Q8_0 ? (t->dev.cols + 63) / 64 : 0;
        }
        return d;
    };
    auto recipe = [&](int mode, const float* x, const float* w, int n) {
        TmqEngAct a{};
        a.mode = mode;
        a.n = n;
        a.x = x;
        a.w = w;
        a.eps = c.norm_eps;
        a.spec_miss = m->spec_miss;
        a.state = m->state;
        return a;
    };
    auto all_fpga = [&](std::initializer_list<const tmq_tensor*> ts) {
        for (const tmq_tensor* t : ts)
            if (path_of(t) != TMQ_WPATH_FPGA) return false;
        return true;
    };
    for (int l = 0; l < L; l++) {
        Layer& Y = m->layers[l];
        Y.qkv = Launch{};
        Y.o_l = Launch{};
        Y.gu = Launch{};
        Y.dn = Launch{};
        int64_t* A = m->kacc + acc_off[l];
        int64_t *aq = A, *ak = aq + slot(Y.q), *av = ak + slot(Y.k);
        int64_t *ao = av + slot(Y.v), *ag = ao + slot(Y.o);
        int64_t *au = ag + slot(Y.gate), *ad = au + slot(Y.up);
        float* xs = m->xs + 4 * l;
        Y.dq = deferred(Y.q, aq, xs + 0, fv_ptr(Y.bq));
        Y.dk = deferred(Y.k, ak, xs + 0, fv_ptr(Y.bk));
        Y.dv = deferred(Y.v, av, xs + 0, fv_ptr(Y.bv));
        Y.dout = deferred(Y.o, ao, xs + 1, nullptr);
        Y.dg = deferred(Y.gate, ag, xs + 2, nullptr);
        Y.du = deferred(Y.up, au, xs + 2, nullptr);
        Y.dd = deferred(Y.down, ad, xs + 3, nullptr);
        if (l == 0) {
            Y.qkv.P.act = recipe(TMQ_ACT_EMBED_NORM, nullptr, m->fvec + Y.attn_norm, H);
            Y.qkv.P.act.tokens = m->tokens;
            Y.qkv.P.act.emb = m->emb->dev;
        } else {
            Y.qkv.P.act = recipe(TMQ_ACT_RESID_NORM, m->hid[0], m->fvec + Y.attn_norm, H);
            Y.qkv.P.act.d1 = m->layers[l - 1].dd;
        }
        Y.qkv.P.act.hidden_out = m->hid[1];
        Y.qkv.waves = all_fpga({Y.q, Y.k, Y.v}) ? nw_qkv : 4;
        add_work(Y.qkv, Y.q, aq, xs + 0, kc_qkv);
        add_work(Y.qkv, Y.k, ak, nullptr, kc_qkv);
        add_work(Y.qkv, Y.v, av, nullptr, kc_qkv);
        Y.qkv.P.rope_src = m->rope;
        Y.qkv.P.rope_out = m->rope_cur;
        Y.qkv.P.rope_state = m->state;
        Y.qkv.P.rope_max_pos = c.max_seq;
        Y.o_l.P.act = recipe(TMQ_ACT_PLAIN, m->ctxv, nullptr, H);
        Y.o_l.waves = all_fpga({Y.o}) ? nw_o : 4;
        add_work(Y.o_l, Y.o, ao, xs + 1, kc_o);
        Y.gu.P.act = recipe(TMQ_ACT_RESID_NORM, m->hid[1], m->fvec + Y.ffn_norm, H);
        Y.gu.P.act.d1 = Y.dout;
        Y.gu.P.act.hidden_out = m->hid[0];
        Y.fused_gu = Y.gu_t && all_fpga({Y.gate, Y.up});
        Y.gu.waves = all_fpga({Y.gate, Y.up}) ? nw_gu : 4;
        if (Y.fused_gu) {
            add_work(Y.gu, Y.gu_t, nullptr, nullptr, 1);
            Y.gu.P.w[0].silu = m->silu_x;
            Y.gu.P.w[0].silu_max = m->max_bits + TMQ_MAX_SLOTS * l;
            if (Y.gu.P.w[0].ngroups > TMQ_MAX_SLOTS) return tmq_fail(TMQ_ERR_ARG, "ffn too wide for the max slots");
        } else {
            add_work(Y.gu, Y.gate, ag, xs + 2, kc_gu);
            add_work(Y.gu, Y.up, au, nullptr, kc_gu);
        }
        Y.dn.P.act = recipe(TMQ_ACT_PRESCALED, m->silu_x, nullptr, I);
        Y.dn.P.act.max_bits = m->max_bits + TMQ_MAX_SLOTS * l;
        // fused gate/up: one slot per workgroup; silu_kernel: one atomic slot
        Y.dn.P.act.max_n = Y.fused_gu ? Y.gu.P.w[0].ngroups : 1;
        Y.dn.waves = all_fpga({Y.down}) ? nw_dn : 4;
        if (Y.dn.P.act.max_n > 64 * Y.dn.waves || Y.dn.P.act.max_n > TMQ_MAX_SLOTS)
            return tmq_fail(TMQ_ERR_ARG, "more max slots than down threads");
        add_work(Y.dn, Y.down, ad, xs + 3, kc_dn);
    }
    // logits: the residual stream (hid[0] + the last down projection),
    // output_norm when present, direct GEMV with argmax candidates
    m->logits_l = Launch{};
    m->logits_l.waves = 4;
    m->logits_l.P.act = recipe(TMQ_ACT_RESID_NORM, m->hid[0], m->out_norm >= 0 ? m->fvec + m->out_norm : nullptr, H);
    m->logits_l.P.act.d1 = m->layers[L - 1].dd;
    {
        TmqWork w = tmq_rt_make_work(m->emb, nullptr, m->logits, nullptr);
        const int g64 = m->emb->dev.rows_pad / 64;
        w.path = logits_path;
        w.kc = 1;
        w.cand = m->cand;
        w.ngroups = (g64 + m->logits_l.waves - 1) / m->logits_l.waves;
        w.first_group = 0;
        m->logits_l.P.w[0] = w;
        m->logits_l.P.nworks = 1;
        m->logits_l.P.ngroups = w.ngroups;
    }
    // every launch checked, and its kernel's LDS opted into, before any
    // graph capture
    for (int l = 0; l < L; l++) {
        const Layer& Y = m->layers[l];
        for (const Launch* ln : {&Y.qkv, &Y.o_l, &Y.gu, &Y.dn}) {
            const int e = tmq_prepare_eng_gemv(ln->P, ln->waves);
            if (e) return tmq_fail(TMQ_ERR_HIP, "layer %d engine launch: %s", l, hipGetErrorString((hipError_t)e));
        }
    }
    {
        const int e = tmq_prepare_eng_gemv(m->logits_l.P, m->logits_l.waves);
        if (e) return tmq_fail(TMQ_ERR_HIP, "logits launch: %s", hipGetErrorString((hipError_t)e));
    }
    // captured step graphs hold the old launches
    if (m->g_feed) (void)hipGraphExecDestroy(m->g_feed);
    if (m->g_decode) (void)hipGraphExecDestroy(m->g_decode);
    m->g_feed = m->g_decode = nullptr;
    return 0;
}

int build_model(tmq_model* m, const std::vector<Entry>& ents, int max_seq) {
    tmq_ctx* ctx = m->ctx;
    std::map<std::string, const Entry*> by;
    for (const Entry& e : ents) by[e.name] = &e;
    auto get = [&](const std::string& n) -> const Entry* {
        auto it = by.find(n);
        return it == by.end() ? nullptr : it->second;
    };
    const Entry* emb = get("token_embd.weight");
    if (!emb) return tmq_fail(TMQ_ERR_ARG, "model has no token_embd.weight");
    if (emb->type != TMQ_TYPE_Q8_0)
        return tmq_fail(TMQ_ERR_ARG, "token_embd.weight is type %u; the Q8_0 logits path needs Q8_0", emb->type);
    tmq_model_config& c = m->cfg;
    c.vocab = (int)emb->rows;
    c.hidden = (int)emb->cols;
    int L = 0;
    while (get("blk." + std::to_string(L) + ".attn_q.weight")) L++;
    if (L == 0) return tmq_fail(TMQ_ERR_ARG, "model has no blk.0.attn_q.weight");
    c.n_layers = L;
    const Entry* k0 = get("blk.0.attn_k.weight");
    const Entry* g0 = get("blk.0.ffn_gate.weight");
    if (!k0 || !g0) return tmq_fail(TMQ_ERR_ARG, "model lacks blk.0.attn_k / ffn_gate");
    c.head_dim = TMQ_HEAD_DIM;
    c.n_heads = c.hidden / TMQ_HEAD_DIM;
    c.n_kv_heads = (int)(k0->rows / TMQ_HEAD_DIM);
    c.inter = (int)g0->rows;
    c.max_seq = max_seq;
    c.rope_base = 1000000.0f;
    c.norm_eps = 1e-6f;
    const int H = c.hidden, KV = c.n_kv_heads * TMQ_HEAD_DIM, I = c.inter;
    if (H % TMQ_HEAD_DIM || H % 32 || c.n_kv_heads <= 0 || (int)k0->rows % TMQ_HEAD_DIM ||
        c.n_heads % c.n_kv_heads || I <= 0 || I > 65536 || I % 2)
        return tmq_fail(TMQ_ERR_ARG, "unsupported model shape hidden %d, kv rows %llu, ffn %d", H,
                        (unsigned long long)k0->rows, I);
    if (c.vocab <= 0) return tmq_fail(TMQ_ERR_ARG, "empty vocabulary");
    if (H > TMQ_ENG_MAXN || I > TMQ_ENG_MAXN)
        return tmq_fail(TMQ_ERR_ARG, "hidden %d / ffn %d above the engine's %d", H, I, TMQ_ENG_MAXN);

    // fp32 vectors: norms and biases
    std::vector<float> fv;
    auto add_vec = [&](const std::string& n, int count, bool required, long* off) -> int {
        const Entry* e = get(n);
        if (!e) {
            if (required) return tmq_fail(TMQ_ERR_ARG, "model lacks %s", n.c_str());
            *off = -1;
            return 0;
        }
        if (e->type != 0 || e->n_bytes != (uint64_t)count * 4 || e->rows * e->cols != (uint64_t)count)
            return tmq_fail(TMQ_ERR_ARG, "%s: expected %d F32 values (type %u, %llu bytes)", n.c_str(), count,
                            e->type, (unsigned long long)e->n_bytes);
        *off = (long)fv.size();
        const size_t at = fv.size();
        fv.resize(at + ((count + 63) / 64) * 64, 0.0f);
        memcpy(fv.data() + at, e->data, (size_t)count * 4);
        return 0;
    };
    // TMQ_ENG_MFMA=1: the engine's Q5_0 / K-quant projections run on the
    // MFMA decoders (their tensors carry the integer-fit planes).  Off by
    // default: a decode launch gives each wave one or two blocks, where the
    // fitted-float decoders finish sooner (the MFMA path's correction loads,
    // barriers and accumulator read-out sit on the launch's critical path).
    const bool eng_mfma = env_int("TMQ_ENG_MFMA", 0) != 0;
    auto upload = [&](const std::string& n, uint64_t rows, uint64_t cols, tmq_tensor** out) -> int {
        const Entry* e = get(n);
        if (!e) return tmq_fail(TMQ_ERR_ARG, "model lacks %s", n.c_str());
        if (e->rows != rows || e->cols != cols)
            return tmq_fail(TMQ_ERR_ARG, "%s: shape %llux%llu, expected %llux%llu", n.c_str(),
                            (unsigned long long)e->rows, (unsigned long long)e->cols, (unsigned long long)rows,
                            (unsigned long long)cols);
        const uint64_t need = ggml_bytes(e->type, rows, cols);
        if (!need) return tmq_fail(TMQ_ERR_ARG, "%s: type %u unsupported for %llux%llu", n.c_str(), e->type,
                                   (unsigned long long)rows, (unsigned long long)cols);
        if (e->n_bytes != need)
            return tmq_fail(TMQ_ERR_ARG, "%s: %llu bytes, expected %llu", n.c_str(), (unsigned long long)e->n_bytes,
                            (unsigned long long)need);
        const float* aux = nullptr;
        if (e->type == TMQ_TYPE_Q8_0) {  // sim/matmul_q8.cpp:24-30
            const Entry* a = get(n + "_row_max_abs");
            if (a && a->type == 0 && a->cols == 1 && a->rows == rows && a->n_bytes == rows * 4)
                aux = (const float*)a->data;
        }
        int rc = tmq_rt_tensor_create(ctx, e->type, rows, cols, e->data, false, e->n_bytes, aux, false, out, eng_mfma);
        if (rc) return tmq_fail(rc, "%s: %s", n.c_str(), tmq_last_error());
        m->owned.push_back(*out);
        m->weight_bytes += e->n_bytes;
        return 0;
    };
    int rc = upload("token_embd.weight", c.vocab, H, &m->emb);
    if (rc) return rc;
    m->layers.resize(L);
    for (int l = 0; l < L; l++) {
        Layer& Y = m->layers[l];
        const std::string p = "blk." + std::to_string(l) + ".";
        long off;
        if ((rc = add_vec(p + "attn_norm.weight", H, true, &off))) return rc;
        Y.attn_norm = (size_t)off;
        if ((rc = add_vec(p + "ffn_norm.weight", H, true, &off))) return rc;
        Y.ffn_norm = (size_t)off;
        if ((rc = add_vec(p + "attn_q.bias", H, false, &Y.bq))) return rc;
        if ((rc = add_vec(p + "attn_k.bias", KV, false, &Y.bk))) return rc;
        if ((rc = add_vec(p + "attn_v.bias", KV, false, &Y.bv))) return rc;
        if ((rc = upload(p + "attn_q.weight", H, H, &Y.q))) return rc;
        if ((rc = upload(p + "attn_k.weight", KV, H, &Y.k))) return rc;
        if ((rc = upload(p + "attn_v.weight", KV, H, &Y.v))) return rc;
        if ((rc = upload(p + "attn_output.weight", H, H, &Y.o))) return rc;
        if ((rc = upload(p + "ffn_gate.weight", I, H, &Y.gate))) return rc;
        if ((rc = upload(p + "ffn_up.weight", I, H, &Y.up))) return rc;
        if ((rc = upload(p + "ffn_down.weight", H, I, &Y.down))) return rc;
        // the decode GEMV's copy of gate and up, rows interleaved in groups
        // of 32, so that one workgroup finishes SwiGLU (TmqWork.silu)
        const Entry* eg = get(p + "ffn_gate.weight");
        const Entry* eu = get(p + "ffn_up.weight");
        if (env_int("TMQ_FUSED_SWIGLU", 1) && eg->type == eu->type && eg->type != TMQ_TYPE_Q8_0 && I % 32 == 0) {
            const uint64_t rb = ggml_bytes(eg->type, 1, H);
            std::vector<uint8_t> buf(2 * (size_t)I * rb);
            for (int q = 0; q < I / 32; q++) {
                memcpy(buf.data() + (size_t)(64 * q) * rb, eg->data + (size_t)(32 * q) * rb, 32 * rb);
                memcpy(buf.data() + (size_t)(64 * q + 32) * rb, eu->data + (size_t)(32 * q) * rb, 32 * rb);
            }
            rc = tmq_rt_tensor_create(ctx, eg->type, 2 * (uint64_t)I, H, buf.data(), false, buf.size(), nullptr, false,
                                      &Y.gu_t, eng_mfma);
            if (rc) return tmq_fail(rc, "%sffn_gate/up: %s", p.c_str(), tmq_last_error());
            m->owned.push_back(Y.gu_t);
        }
    }
    if ((rc = add_vec("output_norm.weight", H, false, &m->out_norm))) return rc;

    // K-split accumulators: per layer q, k, v, o, gate, up, down, each
    // sized for its largest use (INT16 / Q8_0: rows x 64-column tiles), plus
    // one max slot per layer; build_launches lays out the slots the current
    // flags use at the front
    auto acc_cap = [](const tmq_tensor* t) -> size_t {
        return (((size_t)t->dev.rows * ((t->dev.cols + 63) / 64)) + 31) & ~(size_t)31;
    };
    size_t acc_cap_n = 0;
    for (int l = 0; l < L; l++) {
        const Layer& Y = m->layers[l];
        for (const tmq_tensor* t : {Y.q, Y.k, Y.v, Y.o, Y.gate, Y.up, Y.down}) acc_cap_n += acc_cap(t);
    }
    // device buffer layout
    auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const int n_cand = (int)((c.vocab + 63) / 64);
    size_t off = 0;
    std::map<std::string, size_t> lay;
    auto place = [&](const char* n, size_t bytes) {
        lay[n] = off;
        off += al(bytes);
    };
    place("state", sizeof(TmqEngState));
    place("tokens", sizeof(int32_t) * (size_t)(max_seq + 1));
    place("hid0", 4 * (size_t)H);
    place("hid1", 4 * (size_t)H);
    place("view", 4 * (size_t)H);
    place("ctx", 4 * (size_t)H);
    place("logits", 4 * (size_t)c.vocab);
    place("cand", 8 * (size_t)n_cand);
    place("dump", 4 * (size_t)H * (L + 1));
    place("xs", 4 * 4 * (size_t)L);
    place("kacc", 8 * (acc_cap_n + (size_t)(TMQ_MAX_SLOTS / 2) * L));
    place("silu", 4 * (size_t)I);
    place("fvec", 4 * fv.size() + 4);
    place("rope", sizeof(float2) * 32 * (size_t)max_seq);
    place("rope_cur", sizeof(float2) * 32);
    place("kc", 4 * (size_t)L * max_seq * KV);
    place("vc", 4 * (size_t)L * max_seq * KV);
    hipError_t e = hipMalloc(&m->dmem, off);
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_NOMEM, "model buffers (%zu B): %s", off, hipGetErrorString(e));
    uint8_t* B = (uint8_t*)m->dmem;
    m->state = (TmqEngState*)(B + lay["state"]);
    m->tokens = (int32_t*)(B + lay["tokens"]);
    m->hid[0] = (float*)(B + lay["hid0"]);
    m->hid[1] = (float*)(B + lay["hid1"]);
    m->view = (float*)(B + lay["view"]);
    m->ctxv = (float*)(B + lay["ctx"]);
    m->logits = (float*)(B + lay["logits"]);
    m->cand = (uint64_t*)(B + lay["cand"]);
    m->n_cand = n_cand;
    m->dump = (float*)(B + lay["dump"]);
    m->xs = (float*)(B + lay["xs"]);
    m->kacc = (int64_t*)(B + lay["kacc"]);
    m->kacc_cap = acc_cap_n + (size_t)(TMQ_MAX_SLOTS / 2) * L;
    m->silu_x = (float*)(B + lay["silu"]);
    m->fvec = (float*)(B + lay["fvec"]);
    m->rope = (float2*)(B + lay["rope"]);
    m->rope_cur = (float2*)(B + lay["rope_cur"]);
    m->kc = (float*)(B + lay["kc"]);
    m->vc = (float*)(B + lay["vc"]);

    hipStream_t s = ctx->stream;
    HIP_TRY(hipMemcpyAsync(m->fvec, fv.data(), 4 * fv.size(), hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemsetAsync(m->xs, 0, 4 * 4 * (size_t)L, s));
    HIP_TRY(hipMemsetAsync(m->hid[0], 0, 4 * (size_t)H, s));
    HIP_TRY(hipMemsetAsync(m->hid[1], 0, 4 * (size_t)H, s));
    LAUNCH_TRY(tmq_launch_zero_acc(m->kacc, m->kacc_cap, s));
    HIP_TRY(hipMemsetAsync(m->kc, 0, 4 * (size_t)L * max_seq * KV, s));
    HIP_TRY(hipMemsetAsync(m->vc, 0, 4 * (size_t)L * max_seq * KV, s));
    // RoPE factors exactly as apply_rope forms them (sim/tmac_gguf.cpp:1531-1535)
    std::vector<float2> rope((size_t)max_seq * 32);
    tmq_math::rope_table(c.rope_base, TMQ_HEAD_DIM, max_seq, (float*)rope.data());
    HIP_TRY(hipMemcpyAsync(m->rope, rope.data(), sizeof(float2) * rope.size(), hipMemcpyHostToDevice, s));
    TmqEngState st{-1, 0, 0, 0};
    HIP_TRY(hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s));
    HIP_TRY(hipStreamSynchronize(s));
    m->use_graphs = env_int("TMQ_GRAPHS", 1) != 0;
    // read before the work lists: every launch's recipe copies it
    m->spec_miss = env_int("TMQ_SPEC_MISS", 0) != 0;
    m->prefill_chunk = env_int("TMQ_PREFILL", 512);
    m->prefill_off = pf_unsupported(m);
    m->flags = TMQ_FLAGS_ALL;
    return build_launches(m);
}

int reset(tmq_model* m) {
    hipStream_t s = m->ctx->stream;
    TmqEngState st{-1, 0, 0, 0};
    HIP_TRY(hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s));
    m->pos = -1;
    return 0;
}

int load_common(tmq_ctx* ctx, const uint8_t* data, uint64_t n, int max_seq, tmq_model** out) {
    if (!ctx || !data || !out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (max_seq <= 0) max_seq = 512;
    if (max_seq > TMQ_MAX_POS) return tmq_fail(TMQ_ERR_ARG, "max_seq %d > %d", max_seq, TMQ_MAX_POS);
    int rc = tmq_rt_set_device(ctx);
    if (rc) return rc;
    std::vector<Entry> ents;
    rc = parse_tmac(data, n, ents);
    if (rc) return rc;
    tmq_model* m = new tmq_model();
    m->ctx = ctx;
    rc = build_model(m, ents, max_seq);
    if (rc) {
        std::string msg = tmq_last_error();
        model_release(m);
        return tmq_fail(rc, "%s", msg.c_str());
    }
    *out = m;
    return 0;
}

}  // namespace

extern "C" {

int tmq_model_load_mem(tmq_ctx* ctx, const void* data, uint64_t n_bytes, int max_seq, tmq_model** out) {
    return load_common(ctx, (const uint8_t*)data, n_bytes, max_seq, out);
}

int tmq_model_load(tmq_ctx* ctx, const char* path, int max_seq, tmq_model** out) {
    if (!path) return tmq_fail(TMQ_ERR_ARG, "null path");
    FILE* f = fopen(path, "rb");
    if (!f) return tmq_fail(TMQ_ERR_ARG, "cannot open %s", path);
    std::vector<uint8_t> buf;
    if (fseek(f, 0, SEEK_END) == 0) {
        long sz = ftell(f);
        if (sz > 0) {
            buf.resize((size_t)sz);
            (void)fseek(f, 0, SEEK_SET);
            if (fread(buf.data(), 1, buf.size(), f) != buf.size()) buf.clear();
        }
    }
    fclose(f);
    if (buf.empty()) return tmq_fail(TMQ_ERR_ARG, "cannot read %s", path);
    return load_common(ctx, buf.data(), buf.size(), max_seq, out);
}

int tmq_model_free(tmq_model* m) {
    model_release(m);
    return 0;
}

int tmq_model_get_config(const tmq_model* m, tmq_model_config* out) {
    if (!m || !out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    *out = m->cfg;
    return 0;
}

uint64_t tmq_model_weight_bytes(const tmq_model* m) { return m ? m->weight_bytes : 0; }

int tmq_model_position(const tmq_model* m) { return m ? m->pos + 1 : -1; }

int tmq_model_set_graphs(tmq_model* m, int enable) {
    if (!m) return tmq_fail(TMQ_ERR_ARG, "null model");
    m->use_graphs = enable != 0;
    return 0;
}

int tmq_model_prompt(tmq_model* m, const int32_t* tokens, int n) {
    if (!m || !tokens || n <= 0) return tmq_fail(TMQ_ERR_ARG, "bad prompt arguments");
    if (n > m->cfg.max_seq) return tmq_fail(TMQ_ERR_ARG, "prompt of %d tokens exceeds max_seq %d", n, m->cfg.max_seq);
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab)
            return tmq_fail(TMQ_ERR_ARG, "token %d at %d outside [0, %d)", tokens[i], i, m->cfg.vocab);
    int rc = tmq_rt_set_device(m->ctx);
    if (!rc) rc = reset(m);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(m->tokens, tokens, sizeof(int32_t) * n, hipMemcpyHostToDevice, m->ctx->stream));
    int done = 0;
    // the batched prefill reproduces the all-flags arithmetic only
    if (m->prefill_chunk > 0 && !m->prefill_off && m->flags == TMQ_FLAGS_ALL && n >= 2) {
        if ((rc = pf_prompt(m, n, &done))) return rc;
        if (done > 0) {
            // pos and err only: pf_err keeps what the prefill left
            TmqEngState st{done - 1, 0, 0, 0};
            HIP_TRY(hipMemcpyAsync(m->state, &st, 2 * sizeof(int32_t), hipMemcpyHostToDevice, m->ctx->stream));
            m->pos = done - 1;
        }
    }
    for (int i = done; i < n; i++) {
        if ((rc = run_feed(m))) return rc;
        m->pos++;
    }
    return check_state(m);
}

int tmq_model_set_flags(tmq_model* m, uint32_t flags) {
    if (!m) return tmq_fail(TMQ_ERR_ARG, "null model");
    if (flags & ~TMQ_FLAGS_ALL) return tmq_fail(TMQ_ERR_ARG, "unknown flag bits 0x%x", flags & ~TMQ_FLAGS_ALL);
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    const uint32_t old = m->flags;
    m->flags = flags;
    rc = build_launches(m);
    if (rc) {
        m->flags = old;
        (void)build_launches(m);
    }
    return rc;
}

uint32_t tmq_model_get_flags(const tmq_model* m) { return m ? m->flags : 0u; }

int tmq_model_reset(tmq_model* m) {
    if (!m) return tmq_fail(TMQ_ERR_ARG, "null model");
    int rc = tmq_rt_set_device(m->ctx);
    if (!rc) rc = reset(m);
    if (!rc) HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    return rc;
}

int tmq_model_set_prefill(tmq_model* m, int chunk) {
    if (!m || chunk < 0) return tmq_fail(TMQ_ERR_ARG, "bad prefill arguments");
    if (chunk > 0 && m->prefill_off) return tmq_fail(TMQ_ERR_ARG, "batched prefill unavailable: %s", m->prefill_off);
    m->prefill_chunk = chunk;
    return 0;
}

int tmq_model_feed(tmq_model* m, int32_t token) {
    if (!m) return tmq_fail(TMQ_ERR_ARG, "null model");
    if (token < 0 || token >= m->cfg.vocab) return tmq_fail(TMQ_ERR_ARG, "token %d outside [0, %d)", token, m->cfg.vocab);
    if (m->pos + 1 >= m->cfg.max_seq) return tmq_fail(TMQ_ERR_ARG, "context full (max_seq %d)", m->cfg.max_seq);
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(m->tokens + m->pos + 1, &token, 4, hipMemcpyHostToDevice, m->ctx->stream));
    if ((rc = run_feed(m))) return rc;
    m->pos++;
    return check_state(m);
}

int tmq_model_logits(tmq_model* m, float* logits) {
    if (!m || !logits) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (m->pos < 0) return tmq_fail(TMQ_ERR_ARG, "no position processed yet");
    int rc = tmq_rt_set_device(m->ctx);
    if (!rc) rc = launch_logits(m);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(logits, m->logits, sizeof(float) * m->cfg.vocab, hipMemcpyDeviceToHost, m->ctx->stream));
    return check_state(m);
}

int tmq_model_generate(tmq_model* m, int n, int32_t* out_tokens) {
    if (!m || n < 0 || (n > 0 && !out_tokens)) return tmq_fail(TMQ_ERR_ARG, "bad generate arguments");
    if (m->pos < 0) return tmq_fail(TMQ_ERR_ARG, "no prompt processed");
    if (m->pos + n >= m->cfg.max_seq)
        return tmq_fail(TMQ_ERR_ARG, "%d more positions exceed max_seq %d", n, m->cfg.max_seq);
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    const int first = m->pos + 1;
    for (int i = 0; i < n; i++) {
        if ((rc = run_decode(m))) return rc;
        m->pos++;
    }
    if (n > 0)
        HIP_TRY(hipMemcpyAsync(out_tokens, m->tokens + first, sizeof(int32_t) * n, hipMemcpyDeviceToHost,
                               m->ctx->stream));
    return check_state(m);
}

int tmq_model_generate_async(tmq_model* m, int n) {
    if (!m || n < 0) return tmq_fail(TMQ_ERR_ARG, "bad generate arguments");
    if (m->pos < 0) return tmq_fail(TMQ_ERR_ARG, "no prompt processed");
    if (m->pos + n >= m->cfg.max_seq)
        return tmq_fail(TMQ_ERR_ARG, "%d more positions exceed max_seq %d", n, m->cfg.max_seq);
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    for (int i = 0; i < n; i++) {
        if ((rc = run_decode(m))) return rc;
        m->pos++;
    }
    return 0;
}

int tmq_model_tokens(tmq_model* m, int first, int n, int32_t* out) {
    if (!m || !out || first < 0 || n < 0 || first + n > m->pos + 1)
        return tmq_fail(TMQ_ERR_ARG, "token range [%d, %d) outside the %d processed positions", first, first + n,
                        m ? m->pos + 1 : 0);
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(out, m->tokens + first, sizeof(int32_t) * n, hipMemcpyDeviceToHost, m->ctx->stream));
    return check_state(m);
}

int tmq_model_hidden(tmq_model* m, float* out) {
    if (!m || !out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    if (m->pos < 0) return tmq_fail(TMQ_ERR_ARG, "no position processed yet");
    // the residual stream: hid[0] + the last layer's pending down projection
    LAUNCH_TRY(tmq_launch_resid_view(m->hid[0], m->layers.back().dd, m->cfg.hidden, m->view, m->ctx->stream));
    HIP_TRY(hipMemcpyAsync(out, m->view, sizeof(float) * m->cfg.hidden, hipMemcpyDeviceToHost, m->ctx->stream));
    return check_state(m);
}

int tmq_model_profile(tmq_model* m, int n, tmq_launch_time* out, int max, int* count) {
    if (!m || n <= 0 || !out || max <= 0 || !count) return tmq_fail(TMQ_ERR_ARG, "bad profile arguments");
    if (m->pos < 0) return tmq_fail(TMQ_ERR_ARG, "no prompt processed");
    if (m->pos + n >= m->cfg.max_seq)
        return tmq_fail(TMQ_ERR_ARG, "%d more positions exceed max_seq %d", n, m->cfg.max_seq);
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    std::vector<std::pair<const char*, hipEvent_t>> ev;
    m->prof = &ev;
    for (int i = 0; i < n && !rc; i++) {
        if (!(rc = launch_decode(m))) m->pos++;
    }
    m->prof = nullptr;
    hipError_t e = hipStreamSynchronize(m->ctx->stream);
    int k = 0;
    if (!rc && e == hipSuccess && !ev.empty()) {
        for (size_t i = 0; i + 1 < ev.size() && k < max; i += 2) {
            float a = 0.0f, b = 0.0f;
            if (hipEventElapsedTime(&a, ev[0].second, ev[i].second) != hipSuccess ||
                hipEventElapsedTime(&b, ev[0].second, ev[i + 1].second) != hipSuccess) {
                rc = tmq_fail(TMQ_ERR_HIP, "profile events");
                break;
            }
            out[k].name = ev[i].first;
            out[k].start_ms = a;
            out[k].end_ms = b;
            k++;
        }
    }
    for (auto& pe : ev) (void)hipEventDestroy(pe.second);
    *count = k;
    if (rc) return rc;
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_HIP, "profile: %s", hipGetErrorString(e));
    return check_state(m);
}

int tmq_model_feed_dump(tmq_model* m, int32_t token, float* layers_out) {
    if (!m || !layers_out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (token < 0 || token >= m->cfg.vocab) return tmq_fail(TMQ_ERR_ARG, "token %d outside [0, %d)", token, m->cfg.vocab);
    if (m->pos + 1 >= m->cfg.max_seq) return tmq_fail(TMQ_ERR_ARG, "context full (max_seq %d)", m->cfg.max_seq);
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(m->tokens + m->pos + 1, &token, 4, hipMemcpyHostToDevice, m->ctx->stream));
    if ((rc = launch_feed_impl(m, true))) return rc;
    m->pos++;
    const size_t nb = sizeof(float) * m->cfg.hidden * (size_t)(m->cfg.n_layers + 1);
    HIP_TRY(hipMemcpyAsync(layers_out, m->dump, nb, hipMemcpyDeviceToHost, m->ctx->stream));
    return check_state(m);
}

int tmq_model_feed_capture(tmq_model* m, int32_t token, float* acts_out) {
    if (!m || !acts_out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (token < 0 || token >= m->cfg.vocab) return tmq_fail(TMQ_ERR_ARG, "token %d outside [0, %d)", token, m->cfg.vocab);
    if (m->pos + 1 >= m->cfg.max_seq) return tmq_fail(TMQ_ERR_ARG, "context full (max_seq %d)", m->cfg.max_seq);
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    const size_t n = (size_t)m->cfg.n_layers * (3 * (size_t)m->cfg.hidden + m->cfg.inter);
    void* cap = nullptr;
    HIP_TRY(hipMalloc(&cap, sizeof(float) * n));
    hipStream_t s = m->ctx->stream;
    hipError_t e = hipMemcpyAsync(m->tokens + m->pos + 1, &token, 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && (rc = launch_feed_impl(m, false, (float*)cap)) == 0)
        e = hipMemcpyAsync(acts_out, cap, sizeof(float) * n, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(cap);
    if (rc) return rc;
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_HIP, "feed_capture: %s", hipGetErrorString(e));
    m->pos++;
    return check_state(m);
}

int tmq_model_logits_capture(tmq_model* m, float* logits, float* x_out) {
    if (!m || !x_out) return tmq_fail(TMQ_ERR_ARG, "null argument");
    if (m->pos < 0) return tmq_fail(TMQ_ERR_ARG, "no position processed yet");
    int rc = tmq_rt_set_device(m->ctx);
    if (rc) return rc;
    hipStream_t s = m->ctx->stream;
    const int H = m->cfg.hidden;
    void* cap = nullptr;
    HIP_TRY(hipMalloc(&cap, sizeof(float) * H));
    Launch l = m->logits_l;
    l.P.act.act_out = (float*)cap;
    rc = launch_gemv(m, l);
    hipError_t e = hipSuccess;
    if (!rc && m->out_norm < 0) {
        // no output_norm: the logits read the residual stream itself
        int le = tmq_launch_resid_view(m->hid[0], m->layers.back().dd, H, (float*)cap, s);
        if (le) e = (hipError_t)le;
    }
    if (!rc && e == hipSuccess && logits)
        e = hipMemcpyAsync(logits, m->logits, sizeof(float) * m->cfg.vocab, hipMemcpyDeviceToHost, s);
    if (!rc && e == hipSuccess) e = hipMemcpyAsync(x_out, cap, sizeof(float) * H, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(cap);
    if (rc) return rc;
    if (e != hipSuccess) return tmq_fail(TMQ_ERR_HIP, "logits_capture: %s", hipGetErrorString(e));
    return 0;
}

const tmq_tensor* tmq_model_tensor(const tmq_model* m, const char* name) {
    if (!m || !name) {
        tmq_fail(TMQ_ERR_ARG, "null argument");
        return nullptr;
    }
    const std::string n(name);
    if (n == "token_embd.weight") return m->emb;
    for (int l = 0; l < (int)m->layers.size(); l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        if (n.compare(0, p.size(), p) != 0) continue;
        const std::string r = n.substr(p.size());
        const Layer& Y = m->layers[l];
        if (r == "attn_q.weight") return Y.q;
        if (r == "attn_k.weight") return Y.k;
        if (r == "attn_v.weight") return Y.v;
        if (r == "attn_output.weight") return Y.o;
        if (r == "ffn_gate.weight") return Y.gate;
        if (r == "ffn_up.weight") return Y.up;
        if (r == "ffn_down.weight") return Y.down;
    }
    tmq_fail(TMQ_ERR_ARG, "model has no matmul tensor %s", name);
    return nullptr;
}

}  // extern "C"
