// ref_harness.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Compiles the reference's own simulation engine (sim/tmac_gguf.cpp, which
// pulls in sim/fpga_sim.hpp) in place from the reference tree, with its
// main() renamed, and exposes the file-static functions the quantized-GEMV
// path is made of through extern "C" wrappers.  Used in this container only,
// to cross-check the CPU restatement (tmq_oracle.c) and to write the golden
// vectors under tests/golden/.  No reference source is copied here: the
// #include below reads it from the reference tree at build time.
#define main tmac_ref_main
#include "tmac_gguf.cpp"
#undef main

#include <cstdlib>

static Tensor ref_make_tensor(uint32_t type, uint64_t rows, uint64_t cols,
                              const uint8_t* data, uint64_t n_bytes) {
    Tensor t;
    memset(&t, 0, sizeof(t));
    snprintf(t.name, sizeof(t.name), "harness");
    t.rows = rows;
    t.cols = cols;
    t.type = type;
    t.n_bytes = n_bytes;
    t.data = const_cast<uint8_t*>(data);
    return t;
}

extern "C" {

float ref_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
float ref_read_f16(const uint8_t* p) { return fpga_sim::read_f16(p); }

void ref_dequant_q4k_block_to_float(const uint8_t* blk, float* out) {
    fpga_sim::dequant_q4k_block_to_float(blk, out);
}

// matmul_fpga_{q8,q5_0,q4_k,q6_k} (sim/tmac_gguf.cpp:948,1221,1097,1367)
int ref_matmul(uint32_t type, const uint8_t* data, uint64_t n_bytes, int rows, int cols,
               const float* x, float* y, const float* row_max_abs) {
    Tensor t = ref_make_tensor(type, (uint64_t)rows, (uint64_t)cols, data, n_bytes);
    switch (type) {
    case TENSOR_Q8_0: matmul_fpga_q8(&t, x, y, rows, cols, row_max_abs); return 0;
    case TENSOR_Q5_0: matmul_fpga_q5_0(&t, x, y, rows, cols); return 0;
    case TENSOR_Q4_K: matmul_fpga_q4_k(&t, x, y, rows, cols); return 0;
    case TENSOR_Q6_K: matmul_fpga_q6_k(&t, x, y, rows, cols); return 0;
    default: return -1;
    }
}

// The no-flag FP32 path of `matmul` (sim/tmac_gguf.cpp:488-492)
void ref_matmul_fp32(uint32_t type, const uint8_t* data, uint64_t n_bytes, int rows, int cols,
                     const float* x, float* y) {
    Tensor t = ref_make_tensor(type, (uint64_t)rows, (uint64_t)cols, data, n_bytes);
    bool saved = g_use_fpga;
    g_use_fpga = false;
    matmul(&t, x, y, rows, cols);
    g_use_fpga = saved;
}

// matmul_fpga_int16 (sim/tmac_gguf.cpp:887-940), any tensor type
void ref_matmul_int16(uint32_t type, const uint8_t* data, uint64_t n_bytes, int rows, int cols,
                      const float* x, float* y) {
    Tensor t = ref_make_tensor(type, (uint64_t)rows, (uint64_t)cols, data, n_bytes);
    matmul_fpga_int16(&t, x, y, rows, cols);
}

// fpga_sim tile primitives
void ref_tile_q8(const uint8_t* q8_W, const uint16_t* cs, const int16_t* vec, int64_t* result) {
    fpga_sim::axi_vecmul_tile_q8(q8_W, cs, vec, result);
}
void ref_tile_q5_0_8x896(const uint8_t* blocks, const int16_t* act, const float* row_inv,
                         int64_t* result, int row_base) {
    fpga_sim::axi_vecmul_tile_q5_0_8x896_axilite(blocks, act, row_inv, result, row_base);
}
void ref_tile_q6_k(const uint8_t* blocks, int nblocks, const int16_t* act, int ncols,
                   const float* row_inv, int64_t* result, int row_base) {
    fpga_sim::axi_vecmul_tile_q6_k_axilite(blocks, nblocks, act, ncols, row_inv, result, row_base);
}
void ref_tile_q4_k(const uint8_t* blocks, int nblocks, const int16_t* act, int ncols,
                   const float* row_inv, int64_t* result, int row_base) {
    fpga_sim::axi_vecmul_tile_q4k_axilite(blocks, nblocks, act, ncols, row_inv, result, row_base);
}
void ref_tile_q5_0_4x896(const uint8_t* blocks56, const int16_t* act, const float* row_norm,
                         int64_t* result, int row_base) {
    fpga_sim::axi_vecmul_tile_q5_0_4x896_axilite(blocks56, act, row_norm, result, row_base);
}
// Q4_K 16-block constant KAT entry (sim/fpga_sim.hpp:844-855)
void ref_tile_q4k_16(const uint8_t* blocks, const int16_t* vec, int64_t* result) {
    fpga_sim::axi_vecmul_tile_q4k_axilite(blocks, vec, result);
}

// PhaseB descriptor chain (sim/tmac_gguf.cpp:513-880).  begin() turns on
// descriptor building inside the matmul_fpga_* calls that follow.
int ref_phaseb_begin(void) {
    if (!g_ddr) {
        g_ddr = (uint8_t*)calloc(DDR_SIZE, 1);
        if (!g_ddr) return -1;
    }
    phaseb_init();
    g_fpga_phaseb = true;
    return 0;
}
void ref_phaseb_end(void) { g_fpga_phaseb = false; }
uint32_t ref_phaseb_head(void) { return g_phaseb.head; }
uint32_t ref_phaseb_next_off(void) { return g_phaseb.next_off; }
int ref_phaseb_count(void) { return (int)g_phaseb.slots.size(); }
const uint8_t* ref_ddr(void) { return g_ddr; }
int ref_phaseb_run(uint32_t desc_off, int64_t* acc) { return phaseb_run_descriptor(desc_off, acc); }
uint32_t ref_phaseb_alloc(uint32_t bytes) { return phaseb_alloc(bytes); }
uint32_t ref_phaseb_add_descriptor(uint32_t w, uint32_t a, uint32_t r, uint16_t nt, uint16_t tb,
                                   uint8_t type, uint8_t trr, uint8_t flags, uint16_t atb,
                                   uint8_t ncg) {
    return phaseb_add_descriptor(w, a, r, nt, tb, type, trr, flags, atb, ncg);
}

// Cosimulation tile dumps as main() opens them (sim/tmac_gguf.cpp:2095-2130):
// which 0 = --dump-tiles (Q8), 1 = --dump-tiles-q5-0, 2 = --dump-tiles-q6-k
int ref_dump_tiles_open(int which, int n, const char* path) {
    FILE* f = fopen(path, "wb");
    if (!f) return -1;
    uint32_t header[4] = {(uint32_t)n, 0, 0, 0};
    fwrite(header, 4, 4, f);
    if (which == 0) { g_dump_file = f; g_dump_tiles_remaining = n; }
    else if (which == 1) { g_dump_q5_0_file = f; g_dump_q5_0_tiles_remaining = n; }
    else { g_dump_q6k_file = f; g_dump_q6k_tiles_remaining = n; }
    return 0;
}
void ref_dump_tiles_close(void) {
    for (FILE** f : {&g_dump_file, &g_dump_q5_0_file, &g_dump_q6k_file})
        if (*f) { fclose(*f); *f = nullptr; }
    g_dump_tiles_remaining = g_dump_q5_0_tiles_remaining = g_dump_q6k_tiles_remaining = 0;
}
// phaseb_verify (:834-880) and phaseb_dump_files (:609-708, writes
// /tmp/tb_phaseb.bin and /tmp/tb_phaseb.hdr)
int ref_phaseb_verify(void) { return phaseb_verify(); }
void ref_phaseb_dump_files(void) { phaseb_dump_files(); }

// Whole-model engine, run as `tmac_gguf model.tmac --fpga-q8 --fpga-q5-0
// --fpga-q4k --fpga-q6-k` would (sim/tmac_gguf.cpp:2066-2091): load_tmac
// into the arena, then process_prompt / get_logits_q8 / one generate step.
int ref_model_load(const char* path) {
    if (!g_ddr) {
        g_ddr = (uint8_t*)calloc(DDR_SIZE, 1);
        if (!g_ddr) return -1;
    }
    if (load_tmac(path) != 0) return -1;
    g_use_fpga = g_fpga_q8 = g_fpga_q4k = g_fpga_q5_0 = g_fpga_q6_k = true;
    return 0;
}
// the command line's flag globals (sim/tmac_gguf.cpp:2085-2091): bit 0
// g_use_fpga, 1 g_fpga_q8, 2 g_fpga_q5_0, 3 g_fpga_q4k, 4 g_fpga_q6_k
void ref_model_set_flags(unsigned flags) {
    g_use_fpga = (flags & 1u) != 0;
    g_fpga_q8 = (flags & 2u) != 0;
    g_fpga_q5_0 = (flags & 4u) != 0;
    g_fpga_q4k = (flags & 8u) != 0;
    g_fpga_q6_k = (flags & 16u) != 0;
}
// the logits as generate() / main() choose them (:2033-2037, :2151-2155)
void ref_model_logits_auto(const float* hidden, float* logits) {
    if (g_fpga_q8) get_logits_q8(logits, hidden);
    else get_logits(logits, hidden);
}
int ref_model_prompt(const int* tokens, int n, float* hidden) {
    std::vector<int> v(tokens, tokens + n);
    return process_prompt(hidden, v, false);
}
void ref_model_reset(void) { reset_cache(); }
void ref_model_logits(const float* hidden, float* logits) { get_logits_q8(logits, hidden); }
// generate()'s body after sampling (sim/tmac_gguf.cpp:2020-2021)
void ref_model_step(float* hidden, int token, int pos) {
    process_embedding(hidden, token);
    forward_all_layers(hidden, pos);
}
// the same with the hidden state after the embedding and after each layer
void ref_model_step_dump(float* hidden, int token, int pos, float* dump) {
    process_embedding(hidden, token);
    memcpy(dump, hidden, sizeof(float) * HIDDEN_DIM);
    for (int l = 0; l < NUM_LAYERS; l++) {
        forward_layer_with_cache(hidden, l, pos);
        memcpy(dump + (size_t)(l + 1) * HIDDEN_DIM, hidden, sizeof(float) * HIDDEN_DIM);
    }
}
// the counters of the [FPGA TIMING SUMMARY] (sim/fpga_sim.hpp:148-174):
// tiles and MACs every matmul_fpga_* adds (sim/tmac_gguf.cpp:899, :934 ...)
void ref_timing_reset(void) { fpga_sim::g_timing.reset(); }
void ref_timing_counts(int64_t* tiles, int64_t* macs) {
    *tiles = fpga_sim::g_timing.total_tiles;
    *macs = fpga_sim::g_timing.total_mac_ops;
}
// apply_rope (sim/tmac_gguf.cpp:1527): q [14*64], k [2*64] rotated in place
void ref_apply_rope(float* q, float* k, int pos) { apply_rope(q, k, pos); }

}  // extern "C"
