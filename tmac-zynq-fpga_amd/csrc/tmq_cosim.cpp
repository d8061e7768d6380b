// tmq_cosim.cpp -- tile dumps and PhaseB chains of tmq_gguf (see tmq_cosim.h).
#include "tmq_cosim.h"

#include <cmath>
#include <cstdlib>
#include <cstring>

namespace tmq_cli {

namespace {

template <class T>
T rd(const uint8_t* p) {
    T v;
    memcpy(&v, p, sizeof v);
    return v;
}
template <class T>
void wr(uint8_t* p, T v) {
    memcpy(p, &v, sizeof v);
}

// x86 float -> unsigned narrowing the reference's casts compile to
// (truncate to int32, keep the low bits): (uint16_t)(ri * 256.0f + 0.5f)
uint16_t uq16(float ri) { return (uint16_t)(int32_t)(ri * 256.0f + 0.5f); }
uint32_t uq32(float ri) { return (uint32_t)(int64_t)(ri * 256.0f + 0.5f); }

int fail(const char* what) {
    fprintf(stderr, "[ERROR] %s: %s\n", what, tmq_last_error());
    return -1;
}

}  // namespace

// ------------------------------------------------------------------ .tmac
bool TmacFile::load(const char* path, std::string* err) {
    FILE* f = fopen(path, "rb");
    if (!f) {
        *err = std::string("cannot open ") + path;
        return false;
    }
    fseek(f, 0, SEEK_END);
    const long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    bytes.resize(n > 0 ? (size_t)n : 0);
    const bool ok = n > 0 && fread(bytes.data(), 1, bytes.size(), f) == bytes.size();
    fclose(f);
    if (!ok || bytes.size() < 12 || memcmp(bytes.data(), "TMAC", 4) != 0) {
        *err = "not a .tmac file";
        return false;
    }
    const uint64_t size = bytes.size(), count = rd<uint64_t>(bytes.data() + 4);
    uint64_t off = 12;
    for (uint64_t i = 0; i < count; i++) {
        if (size - off < 8) return *err = "truncated .tmac", false;
        const uint64_t nl = rd<uint64_t>(bytes.data() + off);
        off += 8;
        if (nl == 0 || nl > 4096 || size - off < nl + 28) return *err = "bad tensor name in .tmac", false;
        std::string name((const char*)bytes.data() + off, (size_t)nl);
        off += nl;
        TmacTensor t;
        t.rows = rd<uint64_t>(bytes.data() + off);
        t.cols = rd<uint64_t>(bytes.data() + off + 8);
        t.type = rd<uint32_t>(bytes.data() + off + 16);
        t.n_bytes = rd<uint64_t>(bytes.data() + off + 20);
        off += 28;
        if (t.n_bytes > size - off) return *err = "tensor data past the end of the .tmac", false;
        t.data = bytes.data() + off;
        off += t.n_bytes;
        tensors[name] = t;
    }
    return true;
}

const TmacTensor* TmacFile::get(const std::string& name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : &it->second;
}

// --------------------------------------------------------------- recorder
Recorder::Recorder(tmq_ctx* ctx, const tmq_model* m, const TmacFile* f, uint32_t flags)
    : ctx_(ctx), m_(m), f_(f), flags_(flags) {}

Recorder::~Recorder() {
    for (int i = 0; i < 3; i++) close_tile(i);
}

bool Recorder::open_tiles(int which, int n, const std::string& path) {
    if (n <= 0) return true;
    TileDump& d = dump_[which];
    d.f = fopen(path.c_str(), "wb");
    if (!d.f) return false;
    // 16-byte header: tile count, three zero words (:2101-2103)
    const uint32_t header[4] = {(uint32_t)n, 0, 0, 0};
    fwrite(header, 4, 4, d.f);
    d.remaining = n;
    d.path = path;
    static const char* kind[3] = {"Q8", "Q5_0", "Q6_K"};
    fprintf(stderr, "[COSIM] Dumping first %d %s tiles to %s\n", n, kind[which], path.c_str());
    return true;
}

void Recorder::close_tile(int which) {
    TileDump& d = dump_[which];
    if (d.f) fclose(d.f);
    d.f = nullptr;
}

void Recorder::enable_phaseb() {
    pb_on_ = true;
    next_off_ = kBase;
}

bool Recorder::active() const {
    for (const TileDump& d : dump_)
        if (d.f && d.remaining > 0) return true;
    return pb_on_ && !pb_full_;
}

int Recorder::offer_position(const float* acts, int n_layers, int hidden, int inter) {
    const size_t per = 3 * (size_t)hidden + inter;
    for (int l = 0; l < n_layers && active(); l++) {
        const float* a = acts + l * per;
        const std::string p = "blk." + std::to_string(l) + ".";
        // forward_layer_with_cache's matmul order (:1583-1707)
        const MatmulCall calls[7] = {{p + "attn_q.weight", a},        {p + "attn_k.weight", a},
                                     {p + "attn_v.weight", a},        {p + "attn_output.weight", a + hidden},
                                     {p + "ffn_gate.weight", a + 2 * (size_t)hidden},
                                     {p + "ffn_up.weight", a + 2 * (size_t)hidden},
                                     {p + "ffn_down.weight", a + 3 * (size_t)hidden}};
        for (const MatmulCall& c : calls) {
            int rc = offer(c);
            if (rc) return rc;
        }
    }
    return 0;
}

int Recorder::offer(const MatmulCall& c) {
    const TmacTensor* t = f_->get(c.name);
    const tmq_tensor* g = tmq_model_tensor(m_, c.name.c_str());
    if (!t || !g) return fail(c.name.c_str());
    // only the calls `matmul` sends to the type's own matmul_fpga_* (:474-483)
    if (tmq_route(t->type, flags_) != TMQ_PATH_FPGA) return 0;
    int rc = 0;
    switch (t->type) {
    case TMQ_TYPE_Q8_0:
        if (dump_[kQ8].f && dump_[kQ8].remaining > 0) rc = dump_q8(c, *t, g);
        break;
    case TMQ_TYPE_Q5_0:
        if (dump_[kQ5].f && dump_[kQ5].remaining > 0) rc = dump_q5(c, *t, g);
        if (!rc && pb_on_ && !pb_full_) rc = phaseb_record(c, *t, g);
        break;
    case TMQ_TYPE_Q6_K:
        if (dump_[kQ6].f && dump_[kQ6].remaining > 0) rc = dump_q6(c, *t, g);
        if (!rc && pb_on_ && !pb_full_) rc = phaseb_record(c, *t, g);
        break;
    case TMQ_TYPE_Q4_K:
        if (pb_on_ && !pb_full_) rc = phaseb_record(c, *t, g);
        break;
    default:
        break;
    }
    return rc;
}

// --dump-tiles (matmul_fpga_q8, :1005-1065): per 64x64 tile, in row-group
// then column-tile order, the int8 weights column-major [k][n], the UQ8.8
// combined scales [n*2 + blk], the int16 activation slice and the tile's
// int64 results.
int Recorder::dump_q8(const MatmulCall& c, const TmacTensor& t, const tmq_tensor* g) {
    const int R = (int)t.rows, C = (int)t.cols, nt = (C + 63) / 64, nb = C / 32;
    std::vector<int16_t> xq(C);
    std::vector<int64_t> acc((size_t)R * nt);
    std::vector<uint16_t> cs((size_t)R * nb);
    float xs = 0.0f;
    if (tmq_quantize_act(ctx_, c.x, C, xq.data(), &xs) != TMQ_OK) return fail("quantize_act");
    if (tmq_gemv_partials(ctx_, g, c.x, acc.data(), acc.size(), &xs) != TMQ_OK) return fail("gemv_partials");
    if (tmq_tensor_q8_scales(ctx_, g, cs.data()) != TMQ_OK) return fail("q8_scales");
    TileDump& d = dump_[kQ8];
    for (int r = 0; r < R && d.remaining > 0; r += 64) {
        const int rs = std::min(64, R - r);
        for (int c0 = 0; c0 < C && d.remaining > 0; c0 += 64) {
            const int csz = std::min(64, C - c0);
            uint8_t w[64][64] = {{0}};
            uint16_t sc[128] = {0};
            int16_t vec[64] = {0};
            int64_t res[64] = {0};
            for (int i = 0; i < rs; i++)
                for (int k = 0; k < csz; k++) {
                    const uint64_t idx = (uint64_t)(r + i) * C + c0 + k;
                    w[k][i] = t.data[(idx / 32) * 34 + 2 + idx % 32];
                }
            for (int i = 0; i < rs; i++)
                for (int blk = 0; blk < 2; blk++) {
                    const int fc = c0 + blk * 32;
                    sc[i * 2 + blk] = fc < C ? cs[(size_t)(r + i) * nb + fc / 32] : 0;
                }
            for (int k = 0; k < csz; k++) vec[k] = xq[c0 + k];
            for (int i = 0; i < rs; i++) res[i] = acc[(size_t)(r + i) * nt + c0 / 64];
            fwrite(w, 1, sizeof w, d.f);
            fwrite(sc, 2, 128, d.f);
            fwrite(vec, 2, 64, d.f);
            fwrite(res, 8, 64, d.f);
            if (--d.remaining == 0) {
                close_tile(kQ8);
                fprintf(stderr, "[COSIM] Dumped all tiles to %s\n", d.path.c_str());
            }
        }
    }
    return 0;
}

// --dump-tiles-q5-0 (matmul_fpga_q5_0, :1282-1298): per 8-row tile the 224
// blocks, the int16 activation (896), the 8 row_inv and the tile's 8 int64
// results.  The reference passes an 8-entry result array with row_base =
// row0, so every tile after the first dumps zeros; here each tile dumps
// its own rows' sums.
int Recorder::dump_q5(const MatmulCall& c, const TmacTensor& t, const tmq_tensor* g) {
    const int R = (int)t.rows, C = (int)t.cols;
    if (C != 896) {
        fprintf(stderr, "[COSIM] %s: Q5_0 tiles need 896 columns, skipped\n", c.name.c_str());
        return 0;
    }
    std::vector<int16_t> xq(C);
    std::vector<int64_t> acc(R);
    std::vector<float> ri(R);
    float xs = 0.0f;
    if (tmq_quantize_act(ctx_, c.x, C, xq.data(), &xs) != TMQ_OK) return fail("quantize_act");
    if (tmq_gemv_partials(ctx_, g, c.x, acc.data(), acc.size(), &xs) != TMQ_OK) return fail("gemv_partials");
    if (tmq_tensor_row_norm(ctx_, g, ri.data()) != TMQ_OK) return fail("row_norm");
    TileDump& d = dump_[kQ5];
    const size_t row_bytes = 28 * 22;
    for (int row0 = 0; row0 < R && d.remaining > 0; row0 += 8) {
        uint8_t blocks[224 * 22] = {0};
        const int rs = std::min(8, R - row0);
        memcpy(blocks, t.data + (size_t)row0 * row_bytes, rs * row_bytes);
        float rinv[8] = {0};
        int64_t res[8] = {0};
        for (int i = 0; i < rs; i++) {
            rinv[i] = ri[row0 + i];
            res[i] = acc[row0 + i];
        }
        fwrite(blocks, 1, sizeof blocks, d.f);
        fwrite(xq.data(), 2, 896, d.f);
        fwrite(rinv, 4, 8, d.f);
        fwrite(res, 8, 8, d.f);
        if (--d.remaining == 0) {
            close_tile(kQ5);
            fprintf(stderr, "[COSIM] Dumped all Q5_0 tiles to %s\n", d.path.c_str());
        }
    }
    return 0;
}

// --dump-tiles-q6-k (matmul_fpga_q6_k, :1478-1495): per 32-row x 256-column
// tile (column group outer), the 32 blocks, the activation slice (256), the
// 32 row_inv and the 32 int64 results of that column group.  Blocks past
// the last row are written as zeros (the reference writes whatever its
// stack held), and every tile dumps its own sums (the reference's result
// array overflows past the first tile).
int Recorder::dump_q6(const MatmulCall& c, const TmacTensor& t, const tmq_tensor* g) {
    const int R = (int)t.rows, C = (int)t.cols, nbr = C / 256;
    if (R > 896) {
        fprintf(stderr, "[COSIM] %s: Q6_K tiles need rows <= 896, skipped\n", c.name.c_str());
        return 0;
    }
    std::vector<int16_t> xq(C);
    std::vector<float> ri(896, 0.0f);
    float xs = 0.0f;
    if (tmq_quantize_act(ctx_, c.x, C, xq.data(), &xs) != TMQ_OK) return fail("quantize_act");
    if (tmq_tensor_row_norm(ctx_, g, ri.data()) != TMQ_OK) return fail("row_norm");
    TileDump& d = dump_[kQ6];
    for (int c0 = 0; c0 < C && d.remaining > 0; c0 += 256) {
        for (int row0 = 0; row0 < R && d.remaining > 0; row0 += 32) {
            const int nblocks = std::min(32, R - row0);
            uint8_t blocks[32 * 210] = {0};
            for (int bi = 0; bi < nblocks; bi++)
                memcpy(blocks + bi * 210, t.data + ((size_t)(row0 + bi) * nbr + c0 / 256) * 210, 210);
            std::vector<int64_t> res896(896, 0);
            if (tmq_vecmul_tile_q6_k(ctx_, blocks, nblocks, xq.data() + c0, 256, ri.data(), res896.data(), row0) !=
                TMQ_OK)
                return fail("vecmul_tile_q6_k");
            float rinv[32] = {0};
            int64_t res[32] = {0};
            for (int i = 0; i < 32 && row0 + i < 896; i++) {
                rinv[i] = ri[row0 + i];
                res[i] = res896[row0 + i];
            }
            fwrite(blocks, 1, sizeof blocks, d.f);
            fwrite(xq.data() + c0, 2, 256, d.f);
            fwrite(rinv, 4, 32, d.f);
            fwrite(res, 8, 32, d.f);
            if (--d.remaining == 0) {
                close_tile(kQ6);
                fprintf(stderr, "[COSIM] Dumped all Q6_K tiles to %s\n", d.path.c_str());
            }
        }
    }
    return 0;
}

// ----------------------------------------------------------------- PhaseB
// phaseb_alloc (:522-530): bump allocation in the DDR from 0x18000000; past
// the 1 GiB DDR every later allocation fails.
uint32_t Recorder::alloc(uint32_t bytes) {
    const uint64_t off = next_off_;
    const uint64_t end = off + bytes;
    next_off_ = (uint32_t)end;
    if (end > kDdrSize) {
        fprintf(stderr, "[PHASEB] DDR full at %llu\n", (unsigned long long)end);
        pb_full_ = true;
        return 0;
    }
    mem_.resize((size_t)(end - kBase), 0);
    return (uint32_t)off;
}

// phaseb_add_descriptor (:533-574): the 32-byte PhaseBDescriptor of
// sim/fpga_sim.hpp:1254-1270, linked to the previous one; an activation
// address equal to the previous result address (OP->OP chain) takes
// act_total_bytes = previous tile_res_rows * 8.
uint32_t Recorder::add_descriptor(uint32_t w, uint32_t a, uint32_t r, uint16_t nt, uint16_t tb, uint8_t type,
                                  uint8_t trr, uint8_t flags, uint16_t atb, uint8_t ncg) {
    const uint32_t off = alloc(32);
    if (!off) return 0;
    uint8_t* d = at(off);
    memset(d, 0, 32);
    wr<uint32_t>(d + 0x04, w);
    wr<uint32_t>(d + 0x08, a);
    wr<uint32_t>(d + 0x0C, r);
    wr<uint16_t>(d + 0x10, nt);
    wr<uint16_t>(d + 0x12, tb);
    d[0x14] = type;
    d[0x15] = trr;
    d[0x16] = flags;
    if (a == prev_res_ && prev_res_ != 0) {
        const uint16_t derived = (uint16_t)(prev_rows_ * 8u);
        fprintf(stderr, "[PHASEB] Chain detected: act_addr=0x%04x matches prev result, auto-derive act_total_bytes=%u "
                        "(prev rows=%u)\n", a, derived, prev_rows_);
        wr<uint16_t>(d + 0x17, derived);
    } else {
        wr<uint16_t>(d + 0x17, atb);
    }
    d[0x19] = ncg;
    if (tail_) wr<uint32_t>(at(tail_), off);
    else head_ = off;
    tail_ = off;
    prev_res_ = r;
    prev_rows_ = trr;
    return off;
}

// The PhaseB part of matmul_fpga_q5_0 (:1307-1355), _q4_k (:1140-1211) and
// _q6_k (:1430-1516): the tiles (blocks + row_inv, UQ16.8 for Q5_0, UQ24.8
// for the K-quants), the int16 activation, a result slot, the descriptor,
// and the verify slot (x_scale, row_inv, the dispatch path's outputs).
int Recorder::phaseb_record(const MatmulCall& c, const TmacTensor& t, const tmq_tensor* g) {
    const int R = (int)t.rows, C = (int)t.cols;
    const bool q5 = t.type == TMQ_TYPE_Q5_0, q4 = t.type == TMQ_TYPE_Q4_K;
    if (q5 && C != 896) return 0;  // the reference's Q5_0 tiles are 8 x 896
    if (!q5 && R > 896) return 0;  // its K-quant tiles hold rows < 896
    std::vector<int16_t> xq(C);
    std::vector<float> ri(R), y(R);
    float xs = 0.0f;
    if (tmq_quantize_act(ctx_, c.x, C, xq.data(), &xs) != TMQ_OK) return fail("quantize_act");
    if (tmq_tensor_row_norm(ctx_, g, ri.data()) != TMQ_OK) return fail("row_norm");
    if (tmq_matmul(ctx_, g, c.x, y.data(), R, C) != TMQ_OK) return fail("matmul");
    uint32_t wa, aa, ra, ntiles, tile_bytes, tr, ncg;
    if (q5) {
        tr = 8, ntiles = (R + 7) / 8, tile_bytes = 4944, ncg = 1;
    } else {
        tr = q4 ? 56 : 32, tile_bytes = q4 ? 8288 : 6848, ncg = (C + 255) / 256;
        ntiles = ncg * ((R + tr - 1) / tr);
    }
    // weights, activation, results, in that order (:1144-1150, :1315-1317, :1433-1439)
    wa = alloc(ntiles * tile_bytes);
    aa = alloc(C * 2);
    ra = alloc(R * 8);
    // (the reference goes on with a zero activation or result address when
    // only those allocations fail; no descriptor is built here then)
    if (!wa || !aa || !ra) return 0;
    if (q5) {
        const size_t row_bytes = 28 * 22;
        for (int row0 = 0; row0 < R; row0 += 8) {
            uint8_t* tile = at(wa + (row0 / 8) * tile_bytes);
            const int rs = std::min(8, R - row0);
            memcpy(tile, t.data + (size_t)row0 * row_bytes, rs * row_bytes);
            for (int i = 0; i < 8; i++) wr<uint16_t>(tile + 4928 + 2 * i, i < rs ? uq16(ri[row0 + i]) : 0);
        }
    } else {
        const int bb = q4 ? 144 : 210, blk_bytes = (int)tr * bb, nbr = C / 256;
        for (int cgi = 0; cgi < (int)ncg; cgi++)
            for (int row0 = 0; row0 < R; row0 += tr) {
                const int nblocks = std::min((int)tr, R - row0);
                uint8_t* tile = at(wa + ((row0 / tr) * ncg + cgi) * tile_bytes);
                for (int bi = 0; bi < nblocks; bi++)
                    memcpy(tile + bi * bb, t.data + ((size_t)(row0 + bi) * nbr + cgi) * bb, bb);
                for (int i = 0; i < (int)tr; i++) wr<uint32_t>(tile + blk_bytes + 4 * i, i < nblocks ? uq32(ri[row0 + i]) : 0);
            }
    }
    memcpy(at(aa), xq.data(), (size_t)C * 2);
    if (!add_descriptor(wa, aa, ra, (uint16_t)ntiles, (uint16_t)tile_bytes, (uint8_t)t.type, (uint8_t)tr, 0,
                        (uint16_t)(C * 2), (uint8_t)ncg))
        return 0;
    Slot s;
    s.result_addr = ra;
    s.nrows = R;
    s.x_scale = xs;
    s.row_inv = ri;
    s.expected = y;
    slots_.push_back(std::move(s));
    return 0;
}

int Recorder::phaseb_verify() {
    if (slots_.empty()) return 0;
    fprintf(stderr, "\n[PHASEB] Verifying %zu descriptors, chain head 0x%x...\n", slots_.size(), head_);
    fprintf(stderr, "\n[PHASEB] Descriptor chain (%d descriptors, head 0x%x):\n", (int)slots_.size(), head_);
    int idx = 0;
    for (uint32_t off = head_; off; off = rd<uint32_t>(at(off)), idx++) {
        const uint8_t* d = at(off);
        fprintf(stderr, "  [%d] @0x%04x: next=0x%04x wt=0x%04x act=0x%04x res=0x%04x ntiles=%d tileB=%d type=%d "
                        "rowsPerTile=%d flags=0x%x actB=%d cg=%d\n",
                idx, off, rd<uint32_t>(d), rd<uint32_t>(d + 4), rd<uint32_t>(d + 8), rd<uint32_t>(d + 12),
                rd<uint16_t>(d + 0x10), rd<uint16_t>(d + 0x12), d[0x14], d[0x15], d[0x16], rd<uint16_t>(d + 0x17),
                d[0x19]);
    }
    // the whole chain replayed on the GPU; results land at result_addr
    std::vector<uint32_t> rows(slots_.size(), 0);
    const int walked = tmq_phaseb_run(ctx_, mem_.data(), mem_.size(), kBase, head_, rows.data(), (int)rows.size());
    if (walked < 0) return fail("phaseb_run");
    int errors = 0;
    const double max_err = 2.0;  // :842
    const char* dbg = getenv("TMQ_PHASEB_DEBUG");  // descriptor index: print its rows
    if (dbg) {
        const int di = atoi(dbg);
        if (di >= 0 && di < (int)slots_.size())
            for (int r = 0; r < slots_[di].nrows && r < 128; r++) {
                const Slot& s = slots_[di];
                const int64_t acc = rd<int64_t>(at(s.result_addr + 8 * r));
                fprintf(stderr, "[PHASEB-DBG] desc %d row %d acc %lld xs %.9g ri %.9g expected %.9g computed %.9g\n", di, r,
                        (long long)acc, s.x_scale, s.row_inv[r], s.expected[r], (double)acc * s.x_scale / s.row_inv[r]);
            }
    }
    for (int i = 0; i < walked && i < (int)slots_.size(); i++) {
        const Slot& s = slots_[i];
        for (int r = 0; r < (int)rows[i] && r < s.nrows; r++) {
            const int64_t acc = rd<int64_t>(at(s.result_addr + 8 * r));
            const double computed = (double)acc * s.x_scale / s.row_inv[r];
            const double diff = std::fabs(computed - s.expected[r]);
            if (diff > max_err) {
                if (errors < 20)
                    fprintf(stderr, "[PHASEB] desc %d row %d: expected %.6f got %.6f (err %.6f)\n", i, r, s.expected[r],
                            (float)computed, diff);
                errors++;
            }
        }
    }
    fprintf(stderr, "[PHASEB] %d descriptors verified, %d errors\n", std::min(walked, (int)slots_.size()), errors);
    return errors;
}

// phaseb_dump_files (:609-708): the descriptors copied into one contiguous
// array after everything allocated (next = 0xFFFFFFFF, the last 0), the
// DDR image from 0x18000000 to its end as tb_phaseb.bin, and tb_phaseb.hdr:
// "PHBD", ndesc, array base, total rows, per descriptor (result_addr, rows,
// act_total_bytes, previous result_addr, offset into the expected array),
// then the replayed int64 results.
int Recorder::phaseb_dump(const std::string& dir) {
    if (slots_.empty()) {
        fprintf(stderr, "[PHASEB] Nothing to dump\n");
        return 0;
    }
    std::vector<uint32_t> offs;
    for (uint32_t off = head_; off; off = rd<uint32_t>(at(off))) offs.push_back(off);
    const uint32_t nd = (uint32_t)offs.size();
    const uint32_t base = (next_off_ + 31) & ~31u, end = base + nd * 32;
    if (end > next_off_) mem_.resize((size_t)(end - kBase), 0);
    for (uint32_t i = 0; i < nd; i++) {
        memcpy(at(base + 32 * i), at(offs[i]), 32);
        wr<uint32_t>(at(base + 32 * i), i + 1 < nd ? 0xFFFFFFFFu : 0u);
    }
    const std::string bin = dir + "/tb_phaseb.bin", hdr = dir + "/tb_phaseb.hdr";
    FILE* fb = fopen(bin.c_str(), "wb");
    if (!fb) return fprintf(stderr, "[PHASEB] Cannot write %s\n", bin.c_str()), -1;
    fwrite(mem_.data(), 1, (size_t)(end - kBase), fb);
    fclose(fb);
    fprintf(stderr, "[PHASEB] Wrote %u bytes to %s (0x%08x-0x%08x)\n", end - kBase, bin.c_str(), kBase, end);
    std::vector<uint32_t> nrows(nd);
    uint32_t total = 0;
    for (uint32_t i = 0; i < nd; i++) {
        const uint8_t* d = at(offs[i]);
        const int t = d[0x14], nt = rd<uint16_t>(d + 0x10), tr = d[0x15], cg = d[0x19];
        int r = t == TMQ_TYPE_Q5_0 ? nt * tr : (t == TMQ_TYPE_Q4_K || t == TMQ_TYPE_Q6_K) && cg ? (nt / cg) * tr : 0;
        nrows[i] = (uint32_t)r;
        total += (uint32_t)r;
    }
    FILE* fh = fopen(hdr.c_str(), "wb");
    if (!fh) return fprintf(stderr, "[PHASEB] Cannot write %s\n", hdr.c_str()), -1;
    const uint32_t magic = 0x50484244;
    fwrite(&magic, 4, 1, fh);
    fwrite(&nd, 4, 1, fh);
    fwrite(&base, 4, 1, fh);
    fwrite(&total, 4, 1, fh);
    uint32_t eoff = 0, prev = 0;
    for (uint32_t i = 0; i < nd; i++) {
        const uint8_t* d = at(offs[i]);
        const uint32_t ra = rd<uint32_t>(d + 12), atb = rd<uint16_t>(d + 0x17);
        const uint32_t rec[5] = {ra, nrows[i], atb, prev, eoff};
        fwrite(rec, 4, 5, fh);
        eoff += nrows[i];
        prev = ra;
    }
    for (uint32_t i = 0; i < nd; i++) fwrite(at(rd<uint32_t>(at(offs[i]) + 12)), 8, nrows[i], fh);
    fclose(fh);
    fprintf(stderr, "[PHASEB] Wrote %u descriptors (+%u expected entries) to %s\n", nd, total, hdr.c_str());
    return 0;
}

}  // namespace tmq_cli
