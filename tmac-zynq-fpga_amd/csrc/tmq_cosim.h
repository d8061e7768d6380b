// tmq_cosim.h -- the reference CLI's per-matmul artefacts, rebuilt by
// tmq_gguf from the GPU engine's results: the cosimulation tile dumps
// (--dump-tiles, --dump-tiles-q5-0, --dump-tiles-q6-k; sim/tmac_gguf.cpp:
// 1046-1065, 1282-1298, 1478-1495, 2095-2130) and the PhaseB descriptor
// chain (--fpga-phaseb, --dump-phaseb; :505-880).
//
// Host code over the C ABI: every number in these files comes from the GPU
// (activation quantisation, row normalisers, UQ8.8 scales, tile and row
// int64 sums, the chain replay); the host only arranges bytes in the
// reference's file and arena layouts.
#pragma once
#include <stdint.h>

#include <cstdio>
#include <map>
#include <string>
#include <vector>

#include "../../include/tmq.h"

namespace tmq_cli {

// One tensor of a .tmac file (scripts/extract_tmac.py:6-24).
struct TmacTensor {
    uint64_t rows = 0, cols = 0;
    uint32_t type = 0;
    const uint8_t* data = nullptr;
    uint64_t n_bytes = 0;
};

// The .tmac container read into memory (bounds-checked).
struct TmacFile {
    std::vector<uint8_t> bytes;
    std::map<std::string, TmacTensor> tensors;
    bool load(const char* path, std::string* err);
    const TmacTensor* get(const std::string& name) const;
};

// One matmul call of the reference engine: the weight and the fp32 input
// it receives (forward_layer_with_cache :1583-1707, get_logits_q8 :1843).
struct MatmulCall {
    std::string name;
    const float* x;
};

// The per-matmul recorders of one run.  Each call is offered in the
// reference's order; a recorder takes the calls its flags route to the
// matching matmul_fpga_* and stops when its tile count (or the PhaseB
// arena) is exhausted.
class Recorder {
public:
    Recorder(tmq_ctx* ctx, const tmq_model* m, const TmacFile* f, uint32_t flags);
    ~Recorder();
    // --dump-tiles N (Q8_0), --dump-tiles-q5-0 N, --dump-tiles-q6-k N
    bool open_tiles(int which, int n, const std::string& path);
    // --fpga-phaseb
    void enable_phaseb();
    // more calls wanted
    bool active() const;
    int offer(const MatmulCall& c);
    // the calls of one position, from tmq_model_feed_capture's layout
    int offer_position(const float* acts, int n_layers, int hidden, int inter);
    // phaseb_verify (:834-880): replay on the GPU, compare with the
    // outputs of the dispatch path; returns the error count (< 0: failure)
    int phaseb_verify();
    // phaseb_dump_files (:609-708) into dir/tb_phaseb.bin and .hdr
    int phaseb_dump(const std::string& dir);
    bool phaseb_enabled() const { return pb_on_; }

private:
    enum { kQ8 = 0, kQ5 = 1, kQ6 = 2 };
    struct TileDump {
        FILE* f = nullptr;
        int remaining = 0;
        std::string path;
    };
    struct Slot {
        uint32_t result_addr = 0;
        int nrows = 0;
        float x_scale = 0.0f;
        std::vector<float> row_inv, expected;
    };
    tmq_ctx* ctx_;
    const tmq_model* m_;
    const TmacFile* f_;
    uint32_t flags_;
    TileDump dump_[3];
    // PhaseB arena: the reference DDR from kBase on (1 GiB DDR)
    bool pb_on_ = false, pb_full_ = false;
    std::vector<uint8_t> mem_;
    uint32_t next_off_ = 0, head_ = 0, tail_ = 0, prev_res_ = 0;
    uint8_t prev_rows_ = 0;
    std::vector<Slot> slots_;

    int dump_q8(const MatmulCall& c, const TmacTensor& t, const tmq_tensor* g);
    int dump_q5(const MatmulCall& c, const TmacTensor& t, const tmq_tensor* g);
    int dump_q6(const MatmulCall& c, const TmacTensor& t, const tmq_tensor* g);
    int phaseb_record(const MatmulCall& c, const TmacTensor& t, const tmq_tensor* g);
    uint32_t alloc(uint32_t bytes);
    uint8_t* at(uint32_t addr) { return mem_.data() + (addr - kBase); }
    uint32_t add_descriptor(uint32_t w, uint32_t a, uint32_t r, uint16_t nt, uint16_t tb, uint8_t type,
                            uint8_t trr, uint8_t flags, uint16_t atb, uint8_t ncg);
    void close_tile(int which);

public:
    static constexpr uint32_t kBase = 0x18000000u;   // phaseb_init (:516)
    static constexpr uint64_t kDdrSize = 1ull << 30;  // DDR_SIZE (:150)
};

}  // namespace tmq_cli
