// tmq_internal.h -- device data layout shared by the kernels and the host runtime.
//
// Weights live in HBM in a row-interleaved "plane" layout built once at
// upload from the ggml bytes (same byte count, no decoding):
//
//   for every block column b (QK weights wide) and every 16-byte chunk c of
//   a block's field, the chunks of all rows are contiguous:
//       plane16(p, b, c, C, r) = p + ((b*C + c)*rows_pad + r) * 16
//   so the 64 lanes of a wave (one row each) read 1 KiB contiguous per load.
//
//   Q8_0  A: q    [b][2][r] x16B     D: d [b][r] u16
//   Q5_0  A: D0-D3 [b][r]   x16B     B: D4  [b][r] u32     D: d [b][r] u16
//         (the 32 5-bit codes repacked into five dwords, tmq_kernels.hip
//         q5_codes; fit codes E: pe [b][r], integer fit codes pi [b/4][r]
//         x 4 B, block b's code in byte b % 4)
//   Q4_K  A: qs   [b][8][r] x16B     B: hdr (d,dmin,scales[12]) [b][r] x16B
//   Q6_K  A: ql   [b][8][r] x16B     B: qh [b][4][r] x16B   C: sc [b][r] x16B
//         D: d [b][r] u16
//   F32   A: 32 floats [b][8][r] x16B        (b = 32-column block)
//   F16   A: 32 halves [b][4][r] x16B
//
// rows_pad = rows rounded up to 64; padding rows are zero (they compute 0).
//
// INT16 path (matmul_fpga_int16, sim/tmac_gguf.cpp:887-940), built on first
// use by tmq_tensor_prepare_int16: the rounded int16 weights of every row,
// W: [c/8][r] x16B (8 consecutive columns per chunk), and the per-row
// row_scale max|E|/32767 (rs16).
#pragma once
#include <stdint.h>

#define TMQ_ROWS_PER_GROUP 64
#define TMQ_WAVES 4
#define TMQ_WG (64 * TMQ_WAVES)
// waves per workgroup of the standalone / chain GEMVs of a type (Q6_K: 8,
// its long rows split into shorter waves; measured 4 % faster for Q6_K and
// 4 % slower for Q4_K on the 896x4864 BASELINE shapes)
// Kernel format of a standalone / chain GEMV: the tensor's type, or
// TMQ_FMT_*_MFMA for a Q5_0 / Q4_K / Q6_K tensor on the MFMA decoders (its
// integer fit built at upload).
#define TMQ_FMT_Q5_0_MFMA 106
#define TMQ_FMT_Q4_K_MFMA 112
#define TMQ_FMT_Q6_K_MFMA 114
constexpr int gemv_waves(int fmt) { return fmt == 14 ? 8 : TMQ_WAVES; }
#define TMQ_Q8_MAX_TILES 256  // cols <= 16384 for Q8_0

struct TmqTensorDev {
    int32_t type;
    int32_t rows, cols, rows_pad;
    int32_t nb;        // blocks per row: cols/32 (Q8_0, Q5_0) or cols/256 (K-quants)
    int32_t clamp;     // 1: clamp before rounding (externally supplied row_inv)
    const uint8_t* pa;
    const uint8_t* pb;
    const uint8_t* pc;
    const uint8_t* pd;
    const uint8_t* pe;       // fit codes (Q5_0: 1 B, Q4_K: 8 B, Q6_K: 16 B per block and row)
    const uint8_t* pi;       // integer fit codes of the MFMA decoders: Q5_0 [b/4][r] 4 B (block b in byte b%4); Q4_K [b][q][r] 2 B
                             // (sub-blocks 2q, 2q+1); Q6_K [b][q][r] 4 B (the quarter's four sub-blocks)
    const uint8_t* pq;       // Q6_K codes for the MFMA decoder: chunk 3q+k (k < 3) of block b, [b][12][r] 16 B,
                             // holds sub-block k of quarter q (a code in the low 6 bits of each byte) and, in
                             // the top 2 bits, bits 2k, 2k+1 of sub-block 3's codes; then, at 192 B per
                             // (row, block), the quarter's four sub-block scales, [b][q][r] 4 B
    const uint4* corr;       // their corrections (TmqCorr), grouped by 64-row group
    const int32_t* corr_off; // [rows_pad/64 + 1] first correction of each group (null: none)
    const float* row_inv;    // Q5_0/K-quants: row_inv; Q8_0: 1/row_scale (guarded)
    const float* row_scale;  // Q8_0 only
    const uint8_t* pw;       // INT16 path weights (null until prepared)
    const float* rs16;       // INT16 path row scales
};

static inline int tmq_kernel_fmt(const TmqTensorDev& t) {
    if (!t.pi || t.clamp) return t.type;
    return t.type == 6 ? TMQ_FMT_Q5_0_MFMA : t.type == 12 ? TMQ_FMT_Q4_K_MFMA : t.type == 14 ? TMQ_FMT_Q6_K_MFMA
                                                                                       : t.type;
}

// matmul branch a work takes (sim/tmac_gguf.cpp:473-493)
enum { TMQ_WPATH_FPGA = 0, TMQ_WPATH_INT16 = 1, TMQ_WPATH_FP32 = 2 };

// Prepared activation, written by act_prep (or by the host for int16 input):
//   +0  float x_scale   +4 int32 n   +16 u32 XH[n/2]   +16+2n u32 XL[n/2]
//   +16+4n int16 xq[n]   +16+6n int32 xq[n] (the fitted decoders' int64 sums)
//   +XA  (tmq_act_xa) the MFMA decoders' operand bytes, 64 B per 32-element
//        block b: int8 xh of elements 0-15, int8 xl-128 of 0-15, xh of
//        16-31, xl-128 of 16-31; then 16 zero bytes and 16 bytes of 1
//   +XS  (XA + 64*nbx + 32) int32 sum of xq over each block, padded to 16 B
//   +XS16 (tmq_act_xs16) int32 sum of xq over each 16 elements, padded to 16 B
// XH/XL hold (xq >> 8, xq & 255) as int16 pairs (elements 2k, 2k+1), so that
// sum w*xq = 256*sum w*xh + sum w*xl with every partial inside int32.
constexpr uint64_t tmq_act_nbx(int n) { return ((uint64_t)n + 31) / 32; }
constexpr uint64_t tmq_act_xa(int n) { return (16 + (uint64_t)n * 10 + 15) & ~(uint64_t)15; }
constexpr uint64_t tmq_act_xs(int n) { return tmq_act_xa(n) + 64 * tmq_act_nbx(n) + 32; }
constexpr uint64_t tmq_act_xs16(int n) { return tmq_act_xs(n) + ((4 * tmq_act_nbx(n) + 15) & ~(uint64_t)15); }
constexpr uint64_t tmq_act_bytes(int n) { return tmq_act_xs16(n) + ((8 * tmq_act_nbx(n) + 15) & ~(uint64_t)15) + 16; }

// One correction of the MFMA decoders' integer fit (uint4): the block's
// fitted weights differ from the exact ones by `delta` on the elements
// col0 + i, i in `mask` (all holding one code), so the row sum takes
// delta * sum of xq over them.  x = row, y = col0, z = mask, w = delta.

// One GEMV of a chain.  The output epilogue of row r is
//     v = finalize(acc_r);  if (bias) v = v + bias[r];  if (resid) v = y[r] + v;
//     y[r] = v
// (bias: sim/tmac_gguf.cpp:1595-1597; residual: :1670, :1710).
//
// Engine GEMVs may instead split K over `kc` workgroups per 64-row group
// and leave int64 row sums in `kacc` (accumulated with device-scope atomics:
// integer addition is associative, so the sums are exact in any order;
// Q8_0: one int64 per row and 64-column tile, [rows][ntiles]) plus the
// activation's x_scale in `xs_out`; the next launch finalises the rows (see
// TmqDeferred).
struct TmqWork {
    TmqTensorDev t;
    const uint8_t* act;
    float* y;            // may be null
    int64_t* acc;        // may be null; Q8_0: [rows][ntiles]
    const float* bias;   // may be null
    uint64_t* cand;      // Q8_0, engine GEMV: per-wave argmax candidate keys (may be null)
    int64_t* kacc;       // engine K-split: int64 row sums (zero before the launch)
    float* xs_out;       // engine K-split: x_scale of the launch's activation
    int32_t first_group;
    int32_t ngroups;     // workgroups of this GEMV (row groups x kc)
    int32_t kc;          // engine K-split: workgroups per row group (>= 1)
    int32_t resid;
    int32_t path;        // TMQ_WPATH_*: the type's own kernel, INT16 or FP32
    const float* xf;     // FP32 path: the fp32 activation (act unused)
    // engine, kc = 1: fused SwiGLU.  The tensor holds ffn_gate and ffn_up
    // rows interleaved in groups of 32 (rows 64q..64q+31 = gate rows
    // 32q..32q+31, the next 32 = the same up rows); row j of the result,
    // silu(gate_j) * up_j, goes to silu[j] and max |silu| to *silu_max.
    float* silu;
    uint32_t* silu_max;
};

// Rows of a K-split engine GEMV finalised by the consumer:
//   Q5_0 / K-quants  v = (float)((double)acc[i] * xs / (double)row_inv[i])
//                    (sim/tmac_gguf.cpp:1303-1305)
//   Q8_0             v = fold over tiles t of (float)((double)v + (double)P*xs*row_scale[i])
//                    (:1075-1076)
//   then v = v + bias[i] when a bias is given (:1595-1597).
//   FP32 path        v = val[i], the rows as the FP32 loop left them
//   INT16 path       as Q8_0, the tiles of matmul_fpga_int16 with its row
//                    scales (:930-931)
struct TmqDeferred {
    const int64_t* acc;
    const float* xs;
    const float* row_inv;
    const float* row_scale;
    const float* bias;
    const float* val;      // FP32 path: final row values (acc, row_* unused)
    int32_t ntiles;        // 0: Q5_0 / K-quants; > 0: Q8_0 / INT16 tiles per row
    int32_t pad_;
};

// Decode-engine state in device memory.  pos = the position being processed
// (-1 after a reset); it is advanced by the first kernel of a step, so a
// captured step replays without host involvement.  err != 0 stops the step.
// pf_err != 0: a wait of the prefill's gate/up workgroups for the rest of
// their token tile ran out of polls (the prompt then fails).
struct TmqEngState {
    int32_t pos;
    int32_t err;
    int32_t pf_err;
    int32_t pad_;
};

// Activation recipe of an engine GEMV launch: every workgroup computes the
// int16 activation of its launch into LDS before its row groups (the
// reference's rms_norm / silu / matmul quantisation, sim/tmac_gguf.cpp:447-461,
// :1225-1231), so no separate normalisation launch is needed.
//   EMBED_NORM  x = embedding row of tokens[pos] (process_embedding, :1955)
//   RESID_NORM  x = x_in + d1 (the residual adds, :1670, :1710)
//   PLAIN       x = x_in (the attention context)
//   PRESCALED   x = x_in with max|x| given (SiLU*up from tmq_launch_silu)
// then, for the two NORM modes, x = rms_norm(x, w) (:447-453) when w is
// set.  x before the norm is stored to hidden_out by workgroup 0 when
// hidden_out is set.
enum { TMQ_ACT_RESID_NORM = 0, TMQ_ACT_PLAIN = 1, TMQ_ACT_PRESCALED = 2, TMQ_ACT_EMBED_NORM = 3 };
#define TMQ_ENG_MAXN 6144
struct TmqEngAct {
    int32_t mode;
    int32_t n;
    const float* x;            // RESID_NORM / PLAIN / PRESCALED input
    const float* w;            // NORM modes: RMSNorm weight (null: no norm)
    const uint32_t* max_bits;  // PRESCALED: max|x| as the largest of max_n slots (bits of non-negative floats)
    int32_t max_n;             // PRESCALED: slots in max_bits (1 .. TMQ_MAX_SLOTS)
    float eps;
    int32_t spec_miss;         // nonzero: the norm's segmented sum re-runs every segment (testing)
    TmqDeferred d1;            // RESID_NORM: the residual term
    float* hidden_out;
    float* act_out;            // NORM modes: workgroup 0 stores the fp32 norm output (capture)
    TmqEngState* state;        // EMBED_NORM: token = tokens[state->pos]
    const int32_t* tokens;
    TmqTensorDev emb;          // EMBED_NORM: quantized embedding
};

// max |x| slots of a PRESCALED activation: each producing workgroup stores
// its own (no contended atomic); the consumer's prologue takes the largest
#define TMQ_MAX_SLOTS 256

// One engine GEMV launch, passed by value: the activation recipe and up to
// TMQ_ENG_MAXW works whose workgroups follow each other (first_group).
#define TMQ_ENG_MAXW 3
struct TmqEngLaunch {
    TmqEngAct act;
    TmqWork w[TMQ_ENG_MAXW];
    int32_t nworks;
    int32_t ngroups;   // total workgroups
    // qkv launches (rope_out set): one more workgroup copies the RoPE row of
    // the current position (rope_src[state->pos], 32 (cos, sin) pairs) to
    // rope_out, so that the attention after the launch reads it without
    // waiting for the position first
    const float2* rope_src;
    float2* rope_out;
    const TmqEngState* rope_state;
    int32_t rope_max_pos;
    int32_t pad_;
};

// Activation-quantisation jobs: one workgroup each, at most TMQ_MAX_ACT per launch.
#define TMQ_MAX_ACT 16
struct TmqActJob {
    const float* x;
    uint8_t* act;
    int32_t n;
    int32_t pad_;
};
struct TmqActJobs {
    int32_t count;
    int32_t pad_;
    TmqActJob j[TMQ_MAX_ACT];
};

// Launchers (tmq_kernels.hip); all asynchronous on `stream`, return a
// hipError_t value (0 = success).
struct ihipStream_t;
typedef struct ihipStream_t* hipStream_t;
int tmq_launch_act_prep(const TmqActJobs& jobs, hipStream_t s);
int tmq_launch_repack(int type, const uint8_t* src, const TmqTensorDev& t, hipStream_t s);
// Q6_K: the MFMA decoder's code plane (TmqTensorDev.pq) from the ql / qh planes
int tmq_launch_q6_pack(const TmqTensorDev& t, hipStream_t s);
// fit codes (plane pe) of a Q5_0 / Q4_K / Q6_K tensor from its planes and
// row_inv; all_exact: every sub-block flagged for the exact decode
int tmq_launch_fit(const TmqTensorDev& t, int all_exact, hipStream_t s);
// bytes of fit codes per block and row (0: no fitted decode)
static inline int tmq_fit_codes(int type) { return type == 6 ? 1 : type == 12 ? 8 : type == 14 ? 16 : 0; }
// integer fit codes (plane pi) of the MFMA decoders.  pass 0: the codes and
// the number of corrections of each (row, block, fitted unit) into
// cnt[(r * nb + b) * subs + k] (subs = tmq_ifit_subs); pass 1: the
// corrections of each from corr[off[...]] on.
int tmq_launch_ifit(const TmqTensorDev& t, int pass, uint8_t* cnt, const int32_t* off, uint4* corr,
                    hipStream_t s);
// bytes of integer fit codes per block and row (0: type without the MFMA decoder)
static inline int tmq_ifit_codes(int type) { return type == 6 ? 1 : type == 12 ? 8 : type == 14 ? 16 : 0; }
// fitted units per block of the MFMA decoders (Q5_0 block, K-quant sub-block)
static inline int tmq_ifit_subs(int type) { return type == 6 ? 1 : type == 12 ? 8 : type == 14 ? 16 : 0; }
// widest activation the MFMA decoders keep in LDS (wider rows take the
// fitted-float decoders)
#define TMQ_MFMA_MAX_COLS 8192
int tmq_launch_rowstat(const TmqTensorDev& t, const float* aux_max_abs, float* row_inv,
                       float* row_scale, int* bad_flag, hipStream_t s);
int tmq_launch_gemv(const TmqWork& w, hipStream_t s);
// One workgroup of a chain launch: row group `group` of works[work] over
// super-blocks [b0, b1) (b1 = 0: the whole row).  A K-quant MFMA group split
// into `pieces` > 1 workgroups adds its int64 row sums into tail slot
// `slot`; the piece completing the slot's count finalises the rows and
// clears the slot for the next launch.  A Q8_0 group split into pieces = 4
// runs as four workgroups, one per 64-row quarter b0.
struct TmqGroupRef {
    int32_t work, group;
    uint16_t b0, b1;
    int16_t slot, pieces;
};
// int64 words of a tail slot: 64 row sums, the piece count, padding to 640 B
#define TMQ_TAIL_SLOT_WORDS 80
// one launch per chain segment (descriptors of one kernel format
// (tmq_kernel_fmt) and clamp mode, max_cols = the widest of them); `tail`:
// zeroed slots of the segment's split groups (null when none)
// split: the segment holds split groups (Q8_0 quarters take dynamic LDS)
int tmq_launch_chain(int fmt, int clamp, int max_cols, const TmqWork* works_dev, const TmqGroupRef* groups_dev,
                     int total_groups, int split, uint64_t* tail, hipStream_t s);
// widest Q8_0 rows whose chain groups split into quarters (the quarters'
// 64-column tile sums, 512 B a tile, meet in LDS)
#define TMQ_Q8_SPLIT_COLS 4096
// dynamic LDS of a standalone / chain GEMV launch of a kernel format
size_t tmq_gemv_lds_bytes(int fmt, int max_cols);
// engine GEMV: activation recipe + works of any formats; waves = 16 or 4
int tmq_launch_eng_gemv(const TmqEngLaunch& l, int waves, hipStream_t s);
// the checks of tmq_launch_eng_gemv and the kernel's LDS opt-in, without a
// launch (before stream capture)
int tmq_prepare_eng_gemv(const TmqEngLaunch& l, int waves);
// x = silu(g) * u over n rows of two K-split GEMVs; *max_bits = max over
// the bits of |x| (atomic; zero before)
int tmq_launch_silu(const TmqDeferred& g, const TmqDeferred& u, int n, float* x, uint32_t* max_bits,
                    hipStream_t s);
// dynamic LDS of an engine launch whose works use kernel formats fa / fb
size_t tmq_eng_lds_bytes(int n, int waves, int fa, int fb);
// out[i] = x[i] + finalise(d, i), i < n
int tmq_launch_resid_view(const float* x, const TmqDeferred& d, int n, float* out, hipStream_t s);
// zero n int64 K-split accumulators
int tmq_launch_zero_acc(int64_t* p, size_t n, hipStream_t s);
int tmq_launch_tile_q8(const uint8_t* W, const uint16_t* cs, const int16_t* vec, int64_t* out,
                       hipStream_t s);
// UQ8.8 combined scales of a Q8_0 tensor, out[r * nb + b]
int tmq_launch_q8_scales(const TmqTensorDev& t, uint16_t* out, hipStream_t s);
// INT16 path weights and row scales of a tensor (t.pw, t.rs16 allocated)
int tmq_launch_i16_prep(const TmqTensorDev& t, hipStream_t s);
// F32 / F16 tensors: flags non-finite elements
int tmq_launch_check_finite(const TmqTensorDev& t, int* bad, hipStream_t s);
