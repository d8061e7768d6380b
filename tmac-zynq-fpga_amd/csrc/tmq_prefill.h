// tmq_prefill.h -- batched prefill: the prompt's tokens pushed through each
// layer together, with every projection as one int8 MFMA GEMM.
//
// The reference processes a prompt one token at a time (process_prompt,
// sim/tmac_gguf.cpp:1992-1997).  Every per-token quantity of a layer --
// the norms, the int16 activation, the projections' int64 row sums, RoPE,
// the cache rows -- depends only on that token and on earlier positions'
// cache rows, so a layer can take all the prompt's tokens at once and give
// the same bits, provided each operation is the same.  The projections are
// exact integer sums; attention keeps each chain's order per query.
//
// Exact int16 x int16 products from int8 MFMA ("digits"):
//   w = 256*a + b + 128   a = w >> 8,  b = (w & 255) - 128,  both in [-128, 127]
//   x = 256*c + e + 128   (same split of the activation's xq)
//   sum_k w*x = 65536*S(a,c) + 256*(S(a,e) + S(b,c)) + S(b,e)
//             + 128*sum_k (w-128) + 128*sum_k (x-128) + 16384*K
// where S(.,.) are int8 dot products over K (each within int32 for
// K <= 65536: |a*c| <= 2^14).  The weights' digit planes are a function of
// the weights only (the int16 w of each format's normalisation), built once;
// the per-row and per-token sums of (w-128), (x-128) are kept per 64-column
// chunk, which is also the Q8_0 tile of the reference's fold.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tmq_internal.h"

#define TMQ_PF_CHUNK 64  // columns per correction chunk (= one Q8_0 tile)

// Digit operand planes of one matrix of `rows` rows (weight rows or
// tokens, a multiple of 32) and K columns (a multiple of 64), stored
// fragment-major: the MFMA operand of 32 rows x 32 columns for one digit is
// 1 KiB contiguous, lane l's 16 bytes at l*16 holding row 32b + (l & 31),
// columns 32s + 16*(l >> 5) .. +15.  Fragment (b, s, d) (d = 0: hi, 1: lo)
// starts at ((b * K/32 + s) * 2 + d) * 1024, so the 2*KC fragments of
// KC consecutive column steps of one block are contiguous.  Plus the
// chunk and total sums of (v - 128) per row.
struct TmqPfPlanes {
    int8_t* d;       // rows * K * 2 bytes
    int32_t* csum;   // [rows][K/64]
    int32_t* tsum;   // [rows]
    int32_t rows, K;
};
#if defined(__HIPCC__)
__host__ __device__ __forceinline__ size_t tmq_pf_off(int row, int col, int K, int digit) {
    const int b = row >> 5, s = col >> 5, lane = (row & 31) + 32 * ((col >> 4) & 1);
    return ((((size_t)b * (K >> 5) + s) * 2 + digit) * 64 + lane) * 16 + (col & 15);
}
#endif

// Split-K digit sums of one GEMM, finalised by the consumer:
//   acc = sum_s part[s][t][row] + 128*(rw[row] + tx[t]) + 16384*K
//   v   = (float)((double)acc * xs[t] / (double)row_inv[row])  (+ bias)
struct TmqPfPart {
    const int64_t* part;   // [split][T_pad][ld]
    const int32_t* rw;     // per row of the plane set: sum (w - 128)
    const int32_t* tx;     // per token: sum (x - 128)
    const float* xs;       // per token x_scale
    const float* row_inv;  // per row of the tensor
    const float* bias;     // per row of the tensor, or null
    int32_t split, ld, K, T_pad;
};

// Activation operands of a layer step for T tokens (one workgroup each):
// the value of every column, then RMSNorm / quantisation exactly as the
// decode engine's prologues (sim/tmac_gguf.cpp:447-453, :1225-1231).
enum {
    TMQ_PF_EMBED_NORM = 0,  // embedding of tokens[p0 + t], then the norm
    TMQ_PF_RESID_NORM = 1,  // x[t] + finalise(d1), then the norm
    TMQ_PF_NORM = 2,        // x[t], then the norm
    TMQ_PF_PLAIN = 3,       // x[t]
    TMQ_PF_SILU = 4         // x[t] with the max |x| given per token (max_bits)
};
struct TmqPfAct {
    int32_t mode, n, T, p0;
    const float* x;            // [T][n]
    const float* w;            // RMSNorm weight (norm modes)
    float eps;
    int32_t spec_miss;         // as TmqEngAct::spec_miss
    const uint32_t* max_bits;  // SILU: per token
    TmqPfPart d1;              // RESID_NORM
    float* x_out;              // EMBED/RESID: the value before the norm, [T][n]
    uint32_t* zero_bits;       // NORM: per-token max slots cleared for the next GU GEMM (or null)
    int32_t* zero_tsum;        // per token (all T_pad rows): cleared for a quantising GU GEMM (or null)
    uint32_t* zero_cnt;        // words 32 i, i < zero_ncnt: its counters and flags, cleared
    int32_t zero_ncnt, pad_;
    const int32_t* tokens;     // EMBED: token ids by position
    TmqTensorDev emb;          // EMBED: quantised embedding
    TmqPfPlanes out;           // digit planes [T_pad][n]
    float* xs;                 // [T_pad] x_scale per token
};

// One tensor's rows inside a GEMM's plane set.
struct TmqPfSeg {
    int32_t row0, rows;
    int32_t q8;                // Q8_0: fold 64-column tiles (sim/tmac_gguf.cpp:1075-1076)
    int32_t pad_;
    const float* row_inv;      // Q5_0/K-quants: row_inv; Q8_0: unused
    const float* row_scale;    // Q8_0
    const float* bias;         // may be null
};

enum {
    TMQ_PF_QKV = 0,   // q -> RoPE -> q_out; k -> RoPE -> kc; v -> vc
    TMQ_PF_GU = 2,    // s_out = silu(gate) * up, max |s| per token
    TMQ_PF_PART = 3,  // int64 digit sums per split
    TMQ_PF_QKVS = 4   // q, k, v split over K: int64 sums per split; pf_qkv_fin finishes
};
struct TmqPfGemm {
    int32_t mode, K, T, T_pad, p0, split, gu_rows, nseg;
    int32_t rows, pad_;        // rows of the plane set (GU: 2 * gu_rows)
    const int8_t* w;           // weight digit planes (fragment-major)
    const int32_t* rw_c;       // [rows][K/64]
    const int32_t* rw_t;       // [rows]
    const int8_t* x;           // activation digit planes (fragment-major, T_pad rows)
    const int32_t* tx_c;       // [T_pad][K/64]
    const int32_t* tx_t;       // [T_pad]
    const float* xs;           // [T_pad]
    TmqPfSeg seg[3];
    // QKV
    float* q_out;              // [T][H]
    float* kc;                 // this layer's caches [max_pos][KV]
    float* vc;
    const float2* rope;        // [max_pos][32]
    int32_t H, KV;
    // GU
    float* s_out;              // [T][gu_rows]
    uint32_t* max_bits;        // [T]
    // PART, QKVS (rows of the Q8_0 segment excepted)
    int64_t* part;             // [split][T_pad][rows]
    // QKV, QKVS: the Q8_0 segment's per-tile sums
    int64_t* tpart;            // [K/64][seg rows][T_pad]
    // GU with gq_d set: the SwiGLU rows quantised in the epilogue, as
    // pf_act_kernel's SILU mode would (digit planes of T_pad rows, the sums
    // of q - 128 per token, x_scale per token; the per-chunk sums are not
    // formed: only a Q8_0 weight reads them, and no down projection is Q8_0
    // here).  The workgroups of a token tile meet in gq_cnt[tile] once their
    // max atomics are in, which needs every workgroup of the launch resident
    // at once (tmq_pf_gu_quant_fits); a wait past gq_spin polls sets *gq_err
    // and goes on.  gq_cnt and gq_tsum start at zero (the ffn_norm act
    // kernel clears them).
    int8_t* gq_d;
    int32_t* gq_tsum;
    float* gq_xs;
    uint32_t* gq_cnt;          // words 32 i: the tiles' counters, then per tile one flag a workgroup
    int32_t* gq_err;
    int32_t gq_spin, gq_ntiles;
};

// q, k, v rows finished from the int64 sums a QKV / QKVS GEMM left: the split
// sums of the Q5_0 / K-quant rows finalised (sim/tmac_gguf.cpp:1303-1305),
// the Q8_0 V rows' tile sums folded (:1075-1076), + bias (:1595-1597), RoPE
// on q and k (:1537-1539), stored to q_out and this layer's caches.  With
// `part` null (a QKV GEMM, which finished the other rows) only the Q8_0 rows.
struct TmqPfQkvFin {
    const int64_t* part;       // [split][T_pad][H + 2 KV] or null
    const int64_t* tpart;      // [K/64][KV][T_pad] when seg[2] is Q8_0
    const int32_t* rw_t;       // plane-set rows: sum (w - 128)
    const int32_t* rw_c;       // [H + 2 KV][K/64]
    const int32_t* tx_t;       // [T_pad]
    const int32_t* tx_c;       // [T_pad][K/64]
    const float* xs;           // [T_pad]
    TmqPfSeg seg[3];           // q, k, v
    float* q_out;              // [T][H]
    float* kc;                 // this layer's caches [max_pos][KV]
    float* vc;
    const float2* rope;        // [max_pos][32]
    int32_t split, K, T, T_pad, p0, H, KV, pad_;
};

// Attention of T consecutive positions p0.. (one workgroup per token and KV
// head): the sequential chains of the decode engine's attention, per query.
struct TmqPfAttn {
    const float* q;            // [T][H] after RoPE
    const float* kc;           // this layer's caches, positions 0 .. p0+T-1 written
    const float* vc;
    float* ctx;                // [T][H]
    int32_t T, p0, n_heads, n_kv;
    int32_t ncu;               // compute units of the device (0: unknown)
    int32_t deal;              // set by the launch: workgroups dealt over the CUs in rounds
};

// The decode engine's state after the last token of a prefill: the
// residual before the last layer's down projection, that projection's int64
// row sums and x_scale (TmqDeferred form), so logits and the next step run
// exactly as after a sequential prompt.
struct TmqPfHandoff {
    TmqPfPart dn;              // last layer's down projection
    const float* x1;           // [T][H]
    int32_t t, H;              // token index (T-1)
    float* hid;                // engine residual buffer
    int64_t* kacc;             // engine K-split sums of the last down projection
    float* xs_slot;
};

#if defined(__HIPCC__)
// int64 row sum of row r, token t of a split-K GEMM (TmqPfPart).
__device__ __forceinline__ int64_t tmq_pf_acc(const TmqPfPart& D, int t, int r) {
    int64_t acc = 0;
    for (int s = 0; s < D.split; s++) acc += D.part[((size_t)s * D.T_pad + t) * D.ld + r];
    return acc + 128 * ((int64_t)D.rw[r] + D.tx[t]) + 16384 * (int64_t)D.K;
}
// ... finalised as the decode engine's K-split rows (sim/tmac_gguf.cpp:1303-1305,
// bias :1595-1597)
__device__ __forceinline__ float tmq_pf_fin(const TmqPfPart& D, int t, int r) {
    float v = (float)(((double)tmq_pf_acc(D, t, r) * (double)D.xs[t]) / (double)D.row_inv[r]);
    if (D.bias) v = v + D.bias[r];
    return v;
}
#endif

// Launchers: tmq_kernels.hip (operand planes) and tmq_prefill.hip.
int tmq_launch_pf_wdigits(const TmqTensorDev& t, int8_t* planes, int K, int row0, hipStream_t s);
int tmq_launch_pf_rowsums(const TmqPfPlanes& p, hipStream_t s);
int tmq_launch_pf_act(const TmqPfAct& a, hipStream_t s);
// tile: 0 = 128 rows x 128 tokens per workgroup, 1 = 64 x 128, 2 = 128 x 64,
// 3 = 64 x 128 with two stage buffers (three workgroups per CU), 4 = 64 x 64
// with K split in halves between the workgroup's waves (K a multiple of 128)
int tmq_launch_pf_gemm(const TmqPfGemm& g, int tile, hipStream_t s);
// Whether every workgroup of a GU launch over T_pad tokens (tile, gu_rows)
// is resident at once on ncu CUs (the quantising epilogue's wait needs it);
// the token tiles of the launch in *ntiles.
bool tmq_pf_gu_quant_fits(int tile, int T_pad, int gu_rows, int ncu, int* ntiles);
int tmq_launch_pf_attn(const TmqPfAttn& a, hipStream_t s);
// One-time set-up of the prefill launches (the attention kernels' dynamic
// LDS limit), so that a stream capture of them makes no such call.
int tmq_pf_prepare();
int tmq_launch_pf_handoff(const TmqPfHandoff& h, hipStream_t s);
int tmq_launch_pf_qkv_fin(const TmqPfQkvFin& f, hipStream_t s);
size_t tmq_pf_attn_lds(int qpk, int npos);
// dynamic LDS the attention kernel may take beside its ~19 KiB of static
// buffers (160 KiB per workgroup in all), and the positions it attends over
// at most (its scores are held in registers, 512 positions per pass)
#define TMQ_PF_ATTN_LDS_MAX (120 * 1024)
#define TMQ_PF_ATTN_MAXPOS 4096
