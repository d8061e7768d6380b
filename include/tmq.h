/*
 * tmq.h -- C ABI of the MI355X (gfx950) quantized-GEMV library (libtmq.so).
 *
 * Drop-in for the quantized matrix-vector path of liuwantao3/tmac-zynq-fpga
 * that the reference offloads to its FPGA cores.  Each entry point names the
 * reference interface it replaces (paths relative to that repository).
 * Plain C types only: pointers, sizes, status codes.  Nothing aborts; every
 * call returns TMQ_OK or a negative status and records a message that
 * tmq_last_error() returns (per host thread).
 *
 * Arithmetic contract (identical to the reference's --fpga-* CPU path):
 *   x_scale = max|x|/32767 (1 if max|x| < 1e-10), xq = (int16)roundf(x/x_scale)
 *   Q5_0/Q4_K/Q6_K: w = clamp16(roundf(E * row_inv)), row_inv = 32767/max_row|E|
 *                   acc = sum w*xq (int64), y = (float)((double)acc*x_scale/row_inv)
 *   Q8_0:           deq = (q8 * cs) >> 8 with cs the UQ8.8 block/row scale,
 *                   per-64-column-tile int64 partials folded in double, in order.
 * The int64 partials and the fp32 outputs are bit-identical to the reference.
 */
#ifndef TMQ_H
#define TMQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define TMQ_OK 0
#define TMQ_ERR_ARG (-1)       /* null pointer, bad type, unsupported shape   */
#define TMQ_ERR_HIP (-2)       /* HIP runtime error (message has the detail)  */
#define TMQ_ERR_NONFINITE (-3) /* an fp16 block scale is Inf or NaN           */
#define TMQ_ERR_NOMEM (-4)     /* device allocation failed                    */
#define TMQ_ERR_DESC (-5)      /* malformed descriptor / chain                */
#define TMQ_ERR_NODEV (-6)     /* no usable gfx950 device                     */

/* ggml tensor types, same codes as sim/tmac_gguf.cpp:154-159 and the PhaseB
 * DESC_TYPE_* constants of sim/fpga_sim.hpp:1272-1279.  F32 and F16 tensors
 * have no matmul_fpga_* of their own: the reference's `matmul` sends them to
 * matmul_fpga_int16 or the FP32 loop (TMQ_PATH_INT16 / TMQ_PATH_FP32). */
#define TMQ_TYPE_F32 0
#define TMQ_TYPE_F16 1
#define TMQ_TYPE_Q5_0 6
#define TMQ_TYPE_Q8_0 8
#define TMQ_TYPE_Q4_K 12
#define TMQ_TYPE_Q6_K 14
#define TMQ_TYPE_CPU_OP 15

typedef struct tmq_ctx tmq_ctx;
typedef struct tmq_tensor tmq_tensor;
typedef struct tmq_chain tmq_chain;

/* Last error message of the calling host thread ("" if none). */
const char* tmq_last_error(void);

/* Library version string. */
const char* tmq_version(void);

/* ---- context ---------------------------------------------------------
 * One context per device (and per host thread that issues work).  Owns a
 * non-blocking HIP stream at default priority.  Replaces the accelerator
 * singleton fpga_sim::accel() (sim/fpga_sim.hpp:431-434) and its
 * register/DDR model. */
int tmq_open(int device, tmq_ctx** out);
int tmq_close(tmq_ctx* ctx);
/* hipStream_t of the context, as void* */
void* tmq_stream(tmq_ctx* ctx);
int tmq_sync(tmq_ctx* ctx);

/* ---- tensors ---------------------------------------------------------
 * Upload one ggml tensor (rows = ne[1] outputs, cols = ne[0] inputs; the
 * Tensor of sim/tmac_gguf.cpp:163-169 as filled by load_tmac :1894-1947).
 * `data` holds rows*cols/QK ggml blocks, row-major.  The bytes are repacked
 * into a row-interleaved device layout and the per-row normaliser (row_inv;
 * Q8_0: row_scale) is computed once here, on the device, instead of on every
 * call as matmul_fpga_* do (sim/tmac_gguf.cpp:1242-1263 etc.).  For Q8_0,
 * `row_max_abs` may carry the `<name>_row_max_abs` aux tensor
 * (sim/matmul_q8.cpp:24-30); NULL computes it from the weights (the two are
 * identical, scripts/extract_tmac.py:231-259).  Requires cols % QK == 0
 * (QK = 32 for Q8_0/Q5_0, 256 for K-quants) and, for Q8_0, cols <= 16384.
 * Returns TMQ_ERR_NONFINITE if any fp16 scale is Inf/NaN.  F32 / F16
 * tensors (row-major elements, cols % 32 == 0, every element finite) are
 * accepted for the INT16 and FP32 paths. */
int tmq_tensor_upload(tmq_ctx* ctx, uint32_t type, uint64_t rows, uint64_t cols,
                      const void* data, uint64_t n_bytes, const float* row_max_abs,
                      tmq_tensor** out);
/* Same, from device memory (ggml bytes already resident in HBM). */
int tmq_tensor_upload_dev(tmq_ctx* ctx, uint32_t type, uint64_t rows, uint64_t cols,
                          const void* data_dev, uint64_t n_bytes, const float* row_max_abs_dev,
                          tmq_tensor** out);
int tmq_tensor_free(tmq_tensor* t);
/* type/rows/cols and ggml weight bytes of an uploaded tensor */
int tmq_tensor_info(const tmq_tensor* t, uint32_t* type, uint64_t* rows, uint64_t* cols,
                    uint64_t* weight_bytes);
/* Per-row normaliser as computed at upload: row_inv (Q5_0/K-quants) or
 * row_scale (Q8_0); host array of `rows` floats. */
int tmq_tensor_row_norm(tmq_ctx* ctx, const tmq_tensor* t, float* out);
/* Decode fits made at upload (no counterpart in the reference; diagnostics
 * for tests and profiling).  Within one sub-block (Q5_0: a block, Q4_K: 32
 * weights, Q6_K: 16 weights) of a row the int16 weight of code u is the
 * integer nearest to fl(u*A + B) for a pair (A, B) checked against the
 * exact decode on every code the sub-block holds; sub-blocks without such
 * a pair take the exact decode.  Counts over the tensor's rows; both 0 for Q8_0 and for
 * tensors uploaded with an external row_inv.  TMQ_NOFIT=1 in the
 * environment at upload sends every sub-block to the exact decode. */
int tmq_tensor_fit_stats(tmq_ctx* ctx, const tmq_tensor* t, uint64_t* fitted, uint64_t* exact);
/* Integer fit of the MFMA decoders (no counterpart in the reference;
 * diagnostics).  Q5_0, Q4_K and Q6_K tensors of at most 8192 columns: within
 * each fitted unit of a row (Q5_0 block, Q4_K 32-weight sub-block, Q6_K
 * 16-weight sub-block) the int16 weight of code u is floor((AN*u + BN)/256)
 * for integers AN, BN fixed at upload; the codes no such pair reproduces
 * are listed as corrections, applied exactly after the fitted sums.
 * *blocks = fitted units with a code (0: the tensor takes the fitted-float
 * decoders), *corrections = listed codes.  TMQ_NOMFMA=1 at upload keeps the
 * tensor on the fitted-float decoders; TMQ_IFIT_FORCE=1 gives every unit
 * one fixed, mostly wrong pair (testing the corrections). */
int tmq_tensor_ifit_stats(tmq_ctx* ctx, const tmq_tensor* t, uint64_t* blocks, uint64_t* corrections);

/* ---- GEMV (boundary 1) -------------------------------------------------
 * Drop-in for the --fpga-* dispatch of `matmul` (sim/tmac_gguf.cpp:473-493):
 * matmul_fpga_q8 (:948, logits via q8_logits_matmul_with_tensor,
 * sim/matmul_q8.cpp:22), matmul_fpga_q5_0 (:1221), matmul_fpga_q4_k (:1097),
 * matmul_fpga_q6_k (:1367).  Host x[cols] in, host y[rows] overwritten,
 * synchronous.  rows/cols must equal the tensor's. */
int tmq_matmul(tmq_ctx* ctx, const tmq_tensor* t, const float* x, float* y, int rows, int cols);

/* ---- the three branches of `matmul` (sim/tmac_gguf.cpp:473-493) --------
 * TMQ_PATH_FPGA   the tensor type's own matmul_fpga_* (tmq_matmul above)
 * TMQ_PATH_INT16  matmul_fpga_int16 (:887-940): exact element values
 *                 (read_tensor, :398-411), per row row_scale = max|E|/32767,
 *                 w = (int16)roundf(E/row_scale), 64x64 int16 tiles whose
 *                 int64 results fold as y += (double)P*x_scale*row_scale in
 *                 column-tile order.  The rounded weights depend on the
 *                 weights only and are built once per tensor
 *                 (tmq_tensor_prepare_int16, 2 bytes per weight).
 * TMQ_PATH_FP32   the loop without any --fpga flag (:488-492):
 *                 y_r = sum_j read_tensor(r,j)*x[j] in fp32, j ascending.
 * Flags mirror the reference globals set by its command line (:2085-2091):
 * TMQ_FLAG_FPGA = g_use_fpga (--fpga, --fpga-int16, or any --fpga-<type>),
 * TMQ_FLAG_<type> = g_fpga_<type>. */
#define TMQ_PATH_FPGA 0
#define TMQ_PATH_INT16 1
#define TMQ_PATH_FP32 2
#define TMQ_FLAG_FPGA 1u
#define TMQ_FLAG_Q8_0 2u
#define TMQ_FLAG_Q5_0 4u
#define TMQ_FLAG_Q4_K 8u
#define TMQ_FLAG_Q6_K 16u
#define TMQ_FLAGS_ALL (TMQ_FLAG_FPGA | TMQ_FLAG_Q8_0 | TMQ_FLAG_Q5_0 | TMQ_FLAG_Q4_K | TMQ_FLAG_Q6_K)
/* The branch `matmul` takes for a tensor type under flags (:474-492):
 * TMQ_PATH_* or a negative status for an unknown type. */
int tmq_route(uint32_t type, uint32_t flags);
/* Tiles and MACs one matmul adds to the reference's [FPGA TIMING SUMMARY]
 * counters (fpga_sim::g_timing, sim/fpga_sim.hpp:148-174) under flags: the
 * branch tmq_route picks, tiled as its matmul_fpga_* tiles (Q8_0 and INT16
 * 64x64, Q5_0 8 rows, Q4_K 56x256, Q6_K 32x256; rows*cols MACs; the FP32
 * loop 0 and 0).  Host only. */
int tmq_matmul_tiles(uint32_t type, uint32_t flags, uint64_t rows, uint64_t cols, int64_t* tiles,
                     int64_t* macs);
/* `matmul` itself: routes by type and flags, host x/y, synchronous. */
int tmq_matmul_flags(tmq_ctx* ctx, const tmq_tensor* t, uint32_t flags, const float* x, float* y,
                     int rows, int cols);
/* one branch, chosen by the caller (host x/y, synchronous) */
int tmq_matmul_path(tmq_ctx* ctx, const tmq_tensor* t, int path, const float* x, float* y, int rows,
                    int cols);
/* device-pointer form; acc_dev (INT16: int64 [rows][ceil(cols/64)] tile
 * results, FP32: must be NULL) may be NULL */
int tmq_gemv_dev_path(tmq_ctx* ctx, const tmq_tensor* t, int path, const float* x_dev, float* y_dev,
                      int64_t* acc_dev);
/* host form returning the integer partials of TMQ_PATH_FPGA / _INT16 */
int tmq_gemv_partials_path(tmq_ctx* ctx, const tmq_tensor* t, int path, const float* x, int64_t* acc,
                           uint64_t acc_len, float* x_scale);
/* builds the INT16 path's rounded weights now (otherwise on first use) */
int tmq_tensor_prepare_int16(tmq_ctx* ctx, tmq_tensor* t);

/* The activation quantisation every matmul_fpga_* performs first
 * (sim/tmac_gguf.cpp:955-961, :1101-1107, :1225-1231, :1371-1377), on the
 * GPU: host x[n] in, host xq[n] and *x_scale out (either may be NULL). */
int tmq_quantize_act(tmq_ctx* ctx, const float* x, int n, int16_t* xq, float* x_scale);
/* The UQ8.8 combined scale matmul_fpga_q8 forms for every (row, 32-column
 * block) of a Q8_0 tensor (sim/tmac_gguf.cpp:1022-1039), on the GPU:
 * out[r * (cols/32) + b]. */
int tmq_tensor_q8_scales(tmq_ctx* ctx, const tmq_tensor* t, uint16_t* out);

/* Device-pointer, stream-ordered form of tmq_matmul: x_dev fp32[cols],
 * y_dev fp32[rows] (may be NULL), acc_dev optional int64 partials: per row
 * (Q5_0/K-quants) or per row and 64-column tile, [rows][ceil(cols/64)]
 * (Q8_0, the tile results of sim/fpga_sim.hpp:466-491). */
int tmq_gemv_dev(tmq_ctx* ctx, const tmq_tensor* t, const float* x_dev, float* y_dev,
                 int64_t* acc_dev);

/* tmq_gemv_dev without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as tmq_gemv_dev; the
 * prepared activation lives in a fixed per-device scratch array of the
 * library (about 160 KiB, held until the process ends) instead of a buffer
 * the context allocates on first use.  Tensors wider than
 * TMQ_NOALLOC_MAX_COLS columns are rejected with TMQ_ERR_ARG.  Every call
 * on one device shares that array: calls that overlap on one device (two
 * streams, two contexts) race and must be ordered by the caller. */
#define TMQ_NOALLOC_MAX_COLS 16384
int tmq_gemv_dev_noalloc(tmq_ctx* ctx, const tmq_tensor* t, const float* x_dev, float* y_dev,
                         int64_t* acc_dev);

/* Host form returning the integer partials (layout as acc_dev above) and
 * x_scale; used by parity tests. */
int tmq_gemv_partials(tmq_ctx* ctx, const tmq_tensor* t, const float* x, int64_t* acc,
                      uint64_t acc_len, float* x_scale);

/* ---- tile primitives (boundary 2) ----------------------------------------
 * Mirror the fpga_sim tile calls, executed on the GPU; host pointers,
 * synchronous.  Same accumulate/overwrite behaviour as the reference. */
/* axi_vecmul_tile_q8 (sim/fpga_sim.hpp:466): q8_W 64x64 int8 column-major
 * [k][n], cs u16[128] UQ8.8 at [n*2+k/32], vec int16[64]; result int64[64]
 * overwritten. */
int tmq_vecmul_tile_q8(tmq_ctx* ctx, const uint8_t* q8_W, const uint16_t* cs,
                       const int16_t* vec, int64_t* result);
/* axi_vecmul_tile_q5_0_8x896_axilite (sim/fpga_sim.hpp:1004): 224 blocks
 * (8 rows x 896), act int16[896], row_inv[8]; result[row_base+i] += acc_i. */
int tmq_vecmul_tile_q5_0_8x896(tmq_ctx* ctx, const uint8_t* blocks, const int16_t* act,
                               const float* row_inv, int64_t* result, int row_base);
/* axi_vecmul_tile_q5_0_4x896_axilite (sim/fpga_sim.hpp:1194): the hp_fsm
 * 4x896 tile, 56 interleaved 48-byte pairs (core 0 block, core 1 block, 4
 * bytes of padding; pair bi: column block bi % 28 of rows bi / 28 and
 * 2 + bi / 28), act int16[896], row_norm[4]; result[row_base+i] += acc_i. */
int tmq_vecmul_tile_q5_0_4x896(tmq_ctx* ctx, const uint8_t* blocks56, const int16_t* act,
                               const float* row_norm, int64_t* result, int row_base);
/* axi_vecmul_tile_q6_k_axilite (sim/fpga_sim.hpp:1058) and
 * axi_vecmul_tile_q4k_axilite (sim/fpga_sim.hpp:821): nblocks one-row blocks,
 * act int16[ncols] (ncols <= 256 columns of each block are used), row_inv
 * indexed by absolute row; result[row_base+bi] += acc (rows < 896 only). */
int tmq_vecmul_tile_q6_k(tmq_ctx* ctx, const uint8_t* blocks, int nblocks, const int16_t* act,
                         int ncols, const float* row_inv, int64_t* result, int row_base);
int tmq_vecmul_tile_q4k(tmq_ctx* ctx, const uint8_t* blocks, int nblocks, const int16_t* act,
                        int ncols, const float* row_inv, int64_t* result, int row_base);

/* ---- descriptor chains (boundary 3) ---------------------------------------
 * Replay of a PhaseB descriptor chain held in a byte arena
 * (struct PhaseBDescriptor, sim/fpga_sim.hpp:1254-1270; replay semantics of
 * phaseb_run_descriptor, sim/tmac_gguf.cpp:761-831).  `arena` holds the
 * reference DDR arena from offset `arena_base` (descriptor addresses are
 * arena offsets).  Every matmul descriptor of the chain starting at
 * `head_off` runs in one kernel launch; its int64 row results are written
 * into the arena at result_addr, as the hardware would, and its row count
 * into rows_out[i] (up to max_desc entries).  Returns the number of
 * descriptors walked, or a negative status. */
int tmq_phaseb_run(tmq_ctx* ctx, uint8_t* arena, uint64_t arena_bytes, uint32_t arena_base,
                   uint32_t head_off, uint32_t* rows_out, int max_desc);

/* Device-resident chain over uploaded tensors: the GPU equivalent of a
 * descriptor chain built by phaseb_add_descriptor (sim/tmac_gguf.cpp:533-574).
 * num_tiles/tile_res_rows/num_col_groups keep the PhaseB meaning: output rows
 * = num_tiles*tile_res_rows (Q5_0, Q8_0) or (num_tiles/num_col_groups)*
 * tile_res_rows (Q4_K, Q6_K), and must match the tensor.  All descriptors run
 * in one kernel launch (plus one activation-quantisation launch). */
typedef struct {
    const tmq_tensor* weight;
    const float* x_dev;   /* fp32 activation, device */
    float* y_dev;         /* fp32 output rows, device (may be NULL) */
    int64_t* acc_dev;     /* int64 partials, device (may be NULL) */
    uint16_t num_tiles;
    uint8_t tile_res_rows;
    uint8_t num_col_groups;
} tmq_desc;

int tmq_chain_create(tmq_ctx* ctx, const tmq_desc* descs, int n, tmq_chain** out);
/* tmq_chain_run = tmq_chain_prepare (quantise the chain's activations, one
 * launch) + tmq_chain_launch (all matmul descriptors, one launch).  The two
 * halves are exposed so a caller can re-run the matmuls on activations that
 * have not changed. */
int tmq_chain_run(tmq_ctx* ctx, tmq_chain* chain);
int tmq_chain_prepare(tmq_ctx* ctx, tmq_chain* chain);
int tmq_chain_launch(tmq_ctx* ctx, tmq_chain* chain);
int tmq_chain_free(tmq_chain* chain);
/* total ggml weight bytes streamed by one run of the chain */
uint64_t tmq_chain_weight_bytes(const tmq_chain* chain);

/* ------------------------------------------------------------------------
 * Decode engine: a .tmac model resident on the GPU, run one position at a
 * time.  Replaces the reference engine's host loop around the matmuls
 * (sim/tmac_gguf.cpp:1559-1711 forward_layer_with_cache, :1820 get_logits_q8,
 * :1950-2045 reset_cache / process_embedding / process_prompt / generate) run
 * with --fpga-q8 --fpga-q5-0 --fpga-q4k --fpga-q6-k.  Results follow that
 * path's arithmetic (fp32 operations in the reference's order); the token
 * choice is greedy (first index of the largest logit) where the reference
 * samples top-k with rand() (:1974-1990).
 * ------------------------------------------------------------------------ */
typedef struct tmq_model tmq_model;

typedef struct {
    int32_t n_layers, hidden, inter, vocab;
    int32_t n_heads, n_kv_heads, head_dim, max_seq;
    float rope_base, norm_eps;
} tmq_model_config;

/* load_tmac (sim/tmac_gguf.cpp:1894-1947): the .tmac container of
 * scripts/extract_tmac.py:6-24, uploaded and checked (shapes, types, sizes).
 * Shapes are taken from the tensors (head_dim 64, RoPE base 1e6, RMSNorm eps
 * 1e-6 as the reference's constants, :136-148, :451, :1528).  max_seq <= 3072
 * positions of KV cache (0: 512); the reference fixes 256 (:148). */
int tmq_model_load(tmq_ctx* ctx, const char* path, int max_seq, tmq_model** out);
int tmq_model_load_mem(tmq_ctx* ctx, const void* data, uint64_t n_bytes, int max_seq, tmq_model** out);
int tmq_model_free(tmq_model* m);
int tmq_model_get_config(const tmq_model* m, tmq_model_config* out);
/* ggml weight bytes streamed per generated token (all layers + logits) */
uint64_t tmq_model_weight_bytes(const tmq_model* m);
/* number of positions processed since the last prompt */
int tmq_model_position(const tmq_model* m);
/* capture the step sequences as HIP graphs (default on; TMQ_GRAPHS=0 off) */
int tmq_model_set_graphs(tmq_model* m, int enable);
/* reset_cache + process_prompt (sim/tmac_gguf.cpp:1950-1997) */
int tmq_model_prompt(tmq_model* m, const int32_t* tokens, int n);
/* The reference's --fpga* flags (TMQ_FLAG_*, default TMQ_FLAGS_ALL = the
 * four --fpga-<type> paths): every projection then takes the branch that
 * `matmul` takes for its type under these flags (sim/tmac_gguf.cpp:473-493:
 * its own quantized kernel, matmul_fpga_int16, or the FP32 loop without
 * any flag), and the logits are get_logits_q8 under TMQ_FLAG_Q8_0, else
 * get_logits (:1852-1866, :2033-2037).  Tensors routed to INT16 get their
 * rounded weights built here (2 bytes per weight).  The batched prefill
 * covers the all-flags arithmetic only: other flag sets run prompts one
 * token at a time.  Captured step graphs are rebuilt. */
int tmq_model_set_flags(tmq_model* m, uint32_t flags);
uint32_t tmq_model_get_flags(const tmq_model* m);
/* How tmq_model_prompt runs the prompt: chunk > 0 (default 512; env
 * TMQ_PREFILL) pushes up to `chunk` tokens through each layer together
 * (int8-MFMA GEMMs, the same bits as one token at a time); 0 processes one
 * token at a time like process_prompt (:1992-1997).  Fails if the model's
 * shapes or formats do not fit the batched kernels. */
int tmq_model_set_prefill(tmq_model* m, int chunk);
/* reset_cache (:1951-1955): the next fed token is position 0 */
int tmq_model_reset(tmq_model* m);
/* process_embedding + forward_all_layers of one more token (:1958-1972) */
int tmq_model_feed(tmq_model* m, int32_t token);
/* as tmq_model_feed, also returning the hidden state after the embedding
 * and after every layer ((n_layers+1) x hidden floats; --dump-layers, :2001-2018) */
int tmq_model_feed_dump(tmq_model* m, int32_t token, float* layers_out);
/* as tmq_model_feed, also returning the fp32 input of every matmul of the
 * position, per layer l at acts_out + l*(3*hidden + ffn): the attn_norm
 * output (attn_q/k/v), the attention context (attn_output), the ffn_norm
 * output (ffn_gate/up) and SiLU(gate)*up (ffn_down) -- what the reference's
 * matmul calls of forward_layer_with_cache receive (:1583-1707).  Used to
 * rebuild the reference's per-matmul artefacts (PhaseB chains, tile dumps). */
int tmq_model_feed_capture(tmq_model* m, int32_t token, float* acts_out);
/* get_logits_q8 / get_logits of the last processed position as
 * tmq_model_logits (logits may be NULL), also returning the fp32 input of
 * the logits matmul (the output_norm of the residual stream, hidden floats) */
int tmq_model_logits_capture(tmq_model* m, float* logits, float* x_out);
/* the uploaded tensor of a matmul weight by its .tmac name
 * ("token_embd.weight", "blk.N.attn_q.weight", ...); NULL if absent */
const tmq_tensor* tmq_model_tensor(const tmq_model* m, const char* name);
/* get_logits_q8 (:1820-1845) of the last processed position -> vocab floats */
int tmq_model_logits(tmq_model* m, float* logits);
/* generate (:2025-2045) with greedy choice: n x (logits, argmax, feed);
 * the chosen tokens are returned in out_tokens[n] */
int tmq_model_generate(tmq_model* m, int n, int32_t* out_tokens);
/* the same, queued without waiting; read the tokens with tmq_model_tokens */
int tmq_model_generate_async(tmq_model* m, int n);
/* tokens of positions [first, first+n) (prompt and generated) */
int tmq_model_tokens(tmq_model* m, int first, int n, int32_t* out);
/* current hidden state (hidden floats) */
int tmq_model_hidden(tmq_model* m, float* out);

/* The --perf pipeline profile (sim/tmac_gguf.cpp:17-134, the PROFILE_SCOPE
 * spans of forward_layer_with_cache and get_logits_q8, :1578-1865): n greedy
 * generate() steps launched one by one with a GPU event before and after
 * every launch.  out[k] = one launch: its operation name (a static string:
 * the reference's scope names, joined with '+' where one launch does
 * several) and its start/end in ms from the first event.  *count = launches
 * recorded (at most max).  Advances the position by n like
 * tmq_model_generate. */
typedef struct {
    const char* name;
    float start_ms, end_ms;
} tmq_launch_time;
int tmq_model_profile(tmq_model* m, int n, tmq_launch_time* out, int max, int* count);

#ifdef __cplusplus
}
#endif
#endif /* TMQ_H */
