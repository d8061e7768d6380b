/*
 * tmq_oracle.h -- CPU restatement of the reference's quantized-GEMV arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the GPU path is
 * compared against (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).
 * The product (libtmq.so) never links, loads or calls it.
 *
 * Every function states the reference file:line it restates.  All reference
 * paths are relative to liuwantao3/tmac-zynq-fpga.
 */
#ifndef TMQ_ORACLE_H
#define TMQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type codes, sim/tmac_gguf.cpp:154-159 */
#define TMQO_F32 0
#define TMQO_F16 1
#define TMQO_Q5_0 6
#define TMQO_Q8_0 8
#define TMQO_Q4_K 12
#define TMQO_Q6_K 14

/* IEEE half -> float, sim/tmac_gguf.cpp:216-228, sim/fpga_sim.hpp:113-123 */
float tmqo_f16_to_f32(uint16_t h);

/* Activation quantisation inlined in every matmul_fpga_*:
 * sim/tmac_gguf.cpp:955-961 (Q8), :1101-1107 (Q4_K), :1225-1231 (Q5_0),
 * :1371-1377 (Q6_K).  Writes xq[n], returns x_scale. */
float tmqo_quantize_act(const float* x, int n, int16_t* xq);

/* Per-row normalisation (row_inv = 32767/max|E|), computed per call by the
 * reference: Q5_0 sim/tmac_gguf.cpp:1242-1263, Q4_K :1116-1136,
 * Q6_K :1381-1424. */
void tmqo_row_inv_q5_0(const uint8_t* w, int rows, int cols, float* row_inv);
void tmqo_row_inv_q4_k(const uint8_t* w, int rows, int cols, float* row_inv);
void tmqo_row_inv_q6_k(const uint8_t* w, int rows, int cols, float* row_inv);
/* Q8_0 row max |q*d|, sim/tmac_gguf.cpp:987-1002 and the offline aux tensor
 * scripts/extract_tmac.py:231-259 (same value). */
void tmqo_row_max_abs_q8_0(const uint8_t* w, int rows, int cols, float* max_abs);
/* Q8_0 row_scale from max_abs, sim/tmac_gguf.cpp:981-1003 */
float tmqo_q8_row_scale(float max_abs);
/* Q8_0 UQ8.8 combined scale for one (row, block), sim/tmac_gguf.cpp:1022-1039 */
uint16_t tmqo_q8_combined_scale(uint16_t d_bits, float row_scale);

/* Per-row int64 accumulators of the dispatch path (row_inv supplied):
 * Q5_0 sim/fpga_sim.hpp:1004-1052 as driven by sim/tmac_gguf.cpp:1265-1280,
 * Q4_K sim/fpga_sim.hpp:730-788 as driven by sim/tmac_gguf.cpp:1154-1190,
 * Q6_K sim/fpga_sim.hpp:1058-1115 as driven by sim/tmac_gguf.cpp:1442-1499. */
void tmqo_acc_q5_0(const uint8_t* w, int rows, int cols, const int16_t* xq,
                   const float* row_inv, int64_t* acc);
void tmqo_acc_q4_k(const uint8_t* w, int rows, int cols, const int16_t* xq,
                   const float* row_inv, int64_t* acc);
void tmqo_acc_q6_k(const uint8_t* w, int rows, int cols, const int16_t* xq,
                   const float* row_inv, int64_t* acc);
/* Q8_0 per-row, per-64-column-tile int64 partials P[r*ntiles + t],
 * sim/tmac_gguf.cpp:1005-1072 with sim/fpga_sim.hpp:316-349 + :45-54. */
void tmqo_tiles_q8_0(const uint8_t* w, int rows, int cols, const int16_t* xq,
                     const float* row_scale, int64_t* P);

/* Finalisation.  K-quants/Q5_0: sim/tmac_gguf.cpp:1192-1194,1303-1305,1501-1503.
 * Q8_0 sequential fold: sim/tmac_gguf.cpp:1075-1076. */
float tmqo_finalize_rowinv(int64_t acc, float x_scale, float row_inv);
float tmqo_finalize_q8(const int64_t* P, int ntiles, float x_scale, float row_scale);

/* Whole matmul_fpga_* (dispatch semantics, per-call row scan).
 * sim/tmac_gguf.cpp:948 (Q8_0, with optional row_max_abs aux tensor as in
 * sim/matmul_q8.cpp:22-35), :1097 (Q4_K), :1221 (Q5_0), :1367 (Q6_K). */
void tmqo_matmul_q8_0(const uint8_t* w, const float* x, float* y, int rows, int cols,
                      const float* row_max_abs);
void tmqo_matmul_q5_0(const uint8_t* w, const float* x, float* y, int rows, int cols);
void tmqo_matmul_q4_k(const uint8_t* w, const float* x, float* y, int rows, int cols);
void tmqo_matmul_q6_k(const uint8_t* w, const float* x, float* y, int rows, int cols);

/* read_tensor (sim/tmac_gguf.cpp:398-411): exact element (r, j), F32/F16/
 * Q8_0/Q5_0/Q4_K/Q6_K. */
float tmqo_read_tensor(uint32_t type, const uint8_t* w, int cols, int r, int j);
/* matmul_fpga_int16 (sim/tmac_gguf.cpp:887-940), the branch of `matmul`
 * for a type whose --fpga-* flag is off.  tiles (int64 [rows][ceil(cols/64)])
 * and row_scale ([rows]) may be NULL. */
void tmqo_matmul_int16(uint32_t type, const uint8_t* w, const float* x, float* y, int rows, int cols,
                       int64_t* tiles, float* row_scale);
/* the FP32 loop of `matmul` without any --fpga flag (sim/tmac_gguf.cpp:488-492) */
void tmqo_matmul_fp32(uint32_t type, const uint8_t* w, const float* x, float* y, int rows, int cols);

/* fpga_sim tile primitives./* fpga_sim tile primitives.
 * axi_vecmul_tile_q8              sim/fpga_sim.hpp:466-491 (+ :316-349, :45-54)
 * axi_vecmul_tile_q5_0_8x896      sim/fpga_sim.hpp:1004-1052  (accumulates)
 * axi_vecmul_tile_q6_k_axilite    sim/fpga_sim.hpp:1058-1115  (accumulates)
 * axi_vecmul_tile_q4k_axilite     sim/fpga_sim.hpp:821-839 -> :730-788 (accumulates)
 * axi_vecmul_tile_q5_0_4x896      sim/fpga_sim.hpp:1194-1249  (accumulates) */
void tmqo_tile_q8(const uint8_t* q8_W, const uint16_t* cs, const int16_t* vec, int64_t* result);
void tmqo_tile_q5_0_8x896(const uint8_t* blocks, const int16_t* act, const float* row_inv,
                          int64_t* result, int row_base);
void tmqo_tile_q6_k(const uint8_t* blocks, int nblocks, const int16_t* act, int ncols,
                    const float* row_inv, int64_t* result, int row_base);
void tmqo_tile_q4_k(const uint8_t* blocks, int nblocks, const int16_t* act, int ncols,
                    const float* row_inv, int64_t* result, int row_base);
void tmqo_tile_q5_0_4x896(const uint8_t* blocks56, const int16_t* act, const float* row_norm,
                          int64_t* result, int row_base);

/* PhaseB descriptor replay, sim/tmac_gguf.cpp:761-831 (Q5_0 row_inv recomputed
 * per tile :712-734; K-quant row_inv read back as UQ24.8 :791-795,:816-820).
 * arena = bytes of the reference DDR arena starting at offset arena_base
 * (descriptor addresses are arena offsets).  Returns rows written (0 for
 * CPU_OP and for unsupported types). */
int tmqo_phaseb_run(const uint8_t* arena, uint32_t arena_base, uint32_t desc_off, int64_t* acc);

#ifdef __cplusplus
}
#endif
#endif
