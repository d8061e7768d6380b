/*
 * tmq_oracle.c -- CPU restatement of the reference's quantized-GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never part of
 * it.  Build with plain IEEE semantics (gcc -O2 -ffp-contract=off, no
 * -ffast-math, no -march=native) so that every float operation rounds where
 * the reference's does (the reference is built with g++ -O2 for x86-64,
 * which has no FMA contraction).
 *
 * Pinning (what fixes each function besides this file itself):
 *   f16 decode          exhaustive 65536-value check against numpy float16
 *   quantize_act        closed forms (|xq|<=32767, xq[argmax]=+-32767,
 *                       zero vector -> scale 1) and the compiled reference
 *   row_inv / max_abs   brute-force numpy decode of the ggml layouts and the
 *                       compiled reference
 *   acc_* / tiles_q8    the compiled reference (oracle/_ref), the Q4_K
 *                       constant-block KAT of sim/test_integration.cpp:98-155,
 *                       the Q8 tile KATs of verilog/tb_matmul_q8.v:127-199,
 *                       int64 order independence
 *   matmul_*            the compiled reference and the committed golden
 *                       vectors under tests/golden/
 *   phaseb_run          the compiled reference's phaseb_run_descriptor
 */
#include "tmq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- helpers */

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

float tmqo_f16_to_f32(uint16_t h) {
    /* Exact IEEE binary16 -> binary32.  The reference builds the value as
     * sign * (1 + m/1024) * 2^(e-15) with powf of an integer exponent, which
     * is exact; it maps -0 to +0 and every NaN to the positive quiet NaN
     * (sim/tmac_gguf.cpp:216-228). */
    uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return 0.0f;
        float v = ldexpf((float)m, -24);
        return sign ? -v : v;
    }
    if (e == 31) return m ? NAN : (sign ? -INFINITY : INFINITY);
    float v = ldexpf((float)(1024u + m), (int)e - 25);
    return sign ? -v : v;
}

/* Clamp-then-round to int16 used by every tile primitive
 * (sim/fpga_sim.hpp:770-773, :1036-1041, :1101-1104). */
static inline int16_t clamp_round16(float v) {
    if (v > 32767.0f) return 32767;
    if (v < -32768.0f) return -32768;
    return (int16_t)roundf(v);
}

/* Guarded row normaliser, e.g. sim/tmac_gguf.cpp:1261-1262 */
static inline float row_inv_from_max(float max_abs) {
    max_abs = (max_abs < 1e-10f) ? 1.0f : max_abs;
    return 32767.0f / max_abs;
}

/* ------------------------------------------------------- block decoders */

/* Q5_0 element wi of a 22-byte block: [d f16][qh u32][qs 16B].
 * sim/fpga_sim.hpp:1019-1033, sim/tmac_gguf.cpp:1249-1257 */
static inline int q5_0_q(const uint8_t* blk, int wi) {
    uint32_t qh = rd32(blk + 2);
    uint8_t b = blk[6 + (wi & 15)];
    int nib = (wi < 16) ? (b & 0xf) : (b >> 4);
    return (int)((((qh >> wi) & 1u) << 4) | (uint32_t)nib) - 16;
}

/* Q4_K 6-bit scale/min of sub-block s, sim/fpga_sim.hpp:756-765 */
static inline void q4k_scale_min(const uint8_t* sc12, int s, int* sc, int* m) {
    if (s < 4) {
        *sc = sc12[s] & 63;
        *m = sc12[s + 4] & 63;
    } else {
        *sc = (sc12[s + 4] & 0xf) | ((sc12[s - 4] >> 6) << 4);
        *m = (sc12[s + 4] >> 4) | ((sc12[s] >> 6) << 4);
    }
}

/* Q4_K dequantised value E of element wi of a 144-byte block
 * [d f16][dmin f16][scales 12B][qs 128B]; E = d*sc*q4 - dmin*m, evaluated
 * left to right as in sim/fpga_sim.hpp:1136-1139 and :775. */
static inline float q4k_E(const uint8_t* blk, int wi) {
    float d = tmqo_f16_to_f32(rd16(blk));
    float dmin = tmqo_f16_to_f32(rd16(blk + 2));
    int s = wi >> 5, j = wi & 31, sc, m;
    q4k_scale_min(blk + 4, s, &sc, &m);
    uint8_t b = blk[16 + (s >> 1) * 32 + j];
    int q4 = (s & 1) ? (b >> 4) : (b & 0xf);
    float a = d * (float)sc;
    a = a * (float)q4;
    float bm = dmin * (float)m;
    return a - bm;
}

/* Q6_K element wi of a 210-byte block [ql 128][qh 64][sc i8 16][d f16].
 * Returns q6 in [-32,31]; *scf = (float)sc.  sim/fpga_sim.hpp:1069-1094 */
static inline int q6k_q(const uint8_t* blk, int wi, float* scf) {
    int half = wi >> 7, pos = wi & 127, l = pos & 31, sub = pos >> 5;
    uint8_t qlb = blk[half * 64 + l + (sub & 1) * 32];
    int nib = (sub < 2) ? (qlb & 0xf) : (qlb >> 4);
    int hb = (blk[128 + half * 32 + l] >> (2 * sub)) & 3;
    *scf = (float)(int8_t)blk[192 + half * 8 + (l >> 4) + sub * 2];
    return ((hb << 4) | nib) - 32;
}

/* Q6_K dequantised value: (d * sc) * q6, sim/fpga_sim.hpp:1098 */
static inline float q6k_E(const uint8_t* blk, int wi) {
    float scf;
    int q = q6k_q(blk, wi, &scf);
    float ss = tmqo_f16_to_f32(rd16(blk + 208));
    float a = ss * scf;
    return a * (float)q;
}

/* ----------------------------------------------------------- activation */

float tmqo_quantize_act(const float* x, int n, int16_t* xq) {
    float s = 0.0f;
    for (int j = 0; j < n; j++) s = fmaxf(s, fabsf(x[j]));
    s = (s < 1e-10f) ? 1.0f : s / 32767.0f;
    for (int j = 0; j < n; j++) xq[j] = (int16_t)roundf(x[j] / s);
    return s;
}

/* ------------------------------------------------------------ row scans */

void tmqo_row_inv_q5_0(const uint8_t* w, int rows, int cols, float* row_inv) {
    int nb = cols / 32;
    for (int r = 0; r < rows; r++) {
        float mx = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)r * nb + b) * 22;
            float d = tmqo_f16_to_f32(rd16(blk));
            for (int wi = 0; wi < 32; wi++) {
                float ab = fabsf(d * (float)q5_0_q(blk, wi));
                if (ab > mx) mx = ab;
            }
        }
        row_inv[r] = row_inv_from_max(mx);
    }
}

void tmqo_row_inv_q4_k(const uint8_t* w, int rows, int cols, float* row_inv) {
    int nb = cols / 256;
    for (int r = 0; r < rows; r++) {
        float mx = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)r * nb + b) * 144;
            for (int wi = 0; wi < 256; wi++) {
                float ab = fabsf(q4k_E(blk, wi));
                if (ab > mx) mx = ab;
            }
        }
        row_inv[r] = row_inv_from_max(mx);
    }
}

void tmqo_row_inv_q6_k(const uint8_t* w, int rows, int cols, float* row_inv) {
    int nb = cols / 256;
    for (int r = 0; r < rows; r++) {
        float mx = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)r * nb + b) * 210;
            for (int wi = 0; wi < 256; wi++) {
                float ab = fabsf(q6k_E(blk, wi));
                if (ab > mx) mx = ab;
            }
        }
        row_inv[r] = row_inv_from_max(mx);
    }
}

void tmqo_row_max_abs_q8_0(const uint8_t* w, int rows, int cols, float* max_abs) {
    int nb = cols / 32;
    for (int r = 0; r < rows; r++) {
        float mx = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)r * nb + b) * 34;
            float d = tmqo_f16_to_f32(rd16(blk));
            for (int k = 0; k < 32; k++) {
                float a = fabsf((float)(int8_t)blk[2 + k] * d);
                if (a > mx) mx = a;
            }
        }
        max_abs[r] = mx;
    }
}

float tmqo_q8_row_scale(float max_abs) {
    return (max_abs < 1e-10f) ? 1.0f : max_abs / 32767.0f;
}

uint16_t tmqo_q8_combined_scale(uint16_t d_bits, float row_scale) {
    float bs = tmqo_f16_to_f32(d_bits);
    float ri = (row_scale < 1e-10f) ? 1.0f : (1.0f / row_scale);
    float c = bs * ri;
    if (c >= 256.0f) c = 255.996f;
    if (c < 0.0f) c = 0.0f;
    /* (uint16_t)(float) on x86-64 g++: truncating conversion to int32
     * (cvttss2si) and the low 16 bits kept.  c*256+0.5 can round up to
     * 65536.0f for c in [255.998, 256) and then gives 0; NaN gives 0. */
    float t = c * 256.0f + 0.5f;
    int32_t i = (t != t) ? INT32_MIN : (int32_t)t;
    return (uint16_t)((uint32_t)i & 0xffffu);
}

/* ---------------------------------------------------- int64 accumulators */

void tmqo_acc_q5_0(const uint8_t* w, int rows, int cols, const int16_t* xq,
                   const float* row_inv, int64_t* acc) {
    int nb = cols / 32;
    for (int r = 0; r < rows; r++) {
        int64_t a = 0;
        float inv = row_inv[r];
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)r * nb + b) * 22;
            float d = tmqo_f16_to_f32(rd16(blk));
            for (int wi = 0; wi < 32; wi++) {
                float e = d * (float)q5_0_q(blk, wi);
                float nrm = e * inv;
                a += (int64_t)clamp_round16(nrm) * (int64_t)xq[b * 32 + wi];
            }
        }
        acc[r] = a;
    }
}

void tmqo_acc_q4_k(const uint8_t* w, int rows, int cols, const int16_t* xq,
                   const float* row_inv, int64_t* acc) {
    int nb = cols / 256;
    for (int r = 0; r < rows; r++) {
        int64_t a = 0;
        float inv = row_inv[r];
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)r * nb + b) * 144;
            for (int wi = 0; wi < 256; wi++) {
                float v = q4k_E(blk, wi) * inv;
                a += (int64_t)xq[b * 256 + wi] * (int64_t)clamp_round16(v);
            }
        }
        acc[r] = a;
    }
}

void tmqo_acc_q6_k(const uint8_t* w, int rows, int cols, const int16_t* xq,
                   const float* row_inv, int64_t* acc) {
    int nb = cols / 256;
    for (int r = 0; r < rows; r++) {
        int64_t a = 0;
        float inv = row_inv[r];
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)r * nb + b) * 210;
            for (int wi = 0; wi < 256; wi++) {
                float v = q6k_E(blk, wi) * inv;
                a += (int64_t)xq[b * 256 + wi] * (int64_t)clamp_round16(v);
            }
        }
        acc[r] = a;
    }
}

/* Q8_0: dequant inside the tile is deq = (q8 * cs) >> 8 with cs the UQ8.8
 * combined scale of (row, 32-block); result = sum_k vec[k]*deq over the
 * 64-column tile.  Columns past `cols` contribute 0 (zero-padded tile). */
void tmqo_tiles_q8_0(const uint8_t* w, int rows, int cols, const int16_t* xq,
                     const float* row_scale, int64_t* P) {
    int nb = cols / 32, nt = (cols + 63) / 64;
    for (int r = 0; r < rows; r++) {
        for (int t = 0; t < nt; t++) {
            int64_t a = 0;
            for (int b = 2 * t; b < 2 * t + 2 && b < nb; b++) {
                const uint8_t* blk = w + ((size_t)r * nb + b) * 34;
                uint16_t cs = tmqo_q8_combined_scale(rd16(blk), row_scale[r]);
                for (int k = 0; k < 32; k++) {
                    int32_t prod = (int32_t)(int8_t)blk[2 + k] * (int32_t)cs;
                    int16_t deq = (int16_t)(prod >> 8);
                    a += (int64_t)xq[b * 32 + k] * (int64_t)deq;
                }
            }
            P[(size_t)r * nt + t] = a;
        }
    }
}

/* --------------------------------------------------------- finalisation */

float tmqo_finalize_rowinv(int64_t acc, float x_scale, float row_inv) {
    float y = 0.0f;
    y += (double)acc * x_scale / (double)row_inv;
    return y;
}

float tmqo_finalize_q8(const int64_t* P, int ntiles, float x_scale, float row_scale) {
    float y = 0.0f;
    for (int t = 0; t < ntiles; t++) y += (double)P[t] * x_scale * row_scale;
    return y;
}

/* ------------------------------------------------------ whole matmuls */

void tmqo_matmul_q5_0(const uint8_t* w, const float* x, float* y, int rows, int cols) {
    int16_t* xq = (int16_t*)malloc(sizeof(int16_t) * (size_t)cols);
    float* ri = (float*)malloc(sizeof(float) * (size_t)rows);
    int64_t* acc = (int64_t*)malloc(sizeof(int64_t) * (size_t)rows);
    float xs = tmqo_quantize_act(x, cols, xq);
    tmqo_row_inv_q5_0(w, rows, cols, ri);
    tmqo_acc_q5_0(w, rows, cols, xq, ri, acc);
    for (int r = 0; r < rows; r++) y[r] = tmqo_finalize_rowinv(acc[r], xs, ri[r]);
    free(xq); free(ri); free(acc);
}

void tmqo_matmul_q4_k(const uint8_t* w, const float* x, float* y, int rows, int cols) {
    int16_t* xq = (int16_t*)malloc(sizeof(int16_t) * (size_t)cols);
    float* ri = (float*)malloc(sizeof(float) * (size_t)rows);
    int64_t* acc = (int64_t*)malloc(sizeof(int64_t) * (size_t)rows);
    float xs = tmqo_quantize_act(x, cols, xq);
    tmqo_row_inv_q4_k(w, rows, cols, ri);
    tmqo_acc_q4_k(w, rows, cols, xq, ri, acc);
    for (int r = 0; r < rows; r++) y[r] = tmqo_finalize_rowinv(acc[r], xs, ri[r]);
    free(xq); free(ri); free(acc);
}

void tmqo_matmul_q6_k(const uint8_t* w, const float* x, float* y, int rows, int cols) {
    int16_t* xq = (int16_t*)malloc(sizeof(int16_t) * (size_t)cols);
    float* ri = (float*)malloc(sizeof(float) * (size_t)rows);
    int64_t* acc = (int64_t*)malloc(sizeof(int64_t) * (size_t)rows);
    float xs = tmqo_quantize_act(x, cols, xq);
    tmqo_row_inv_q6_k(w, rows, cols, ri);
    tmqo_acc_q6_k(w, rows, cols, xq, ri, acc);
    for (int r = 0; r < rows; r++) y[r] = tmqo_finalize_rowinv(acc[r], xs, ri[r]);
    free(xq); free(ri); free(acc);
}

void tmqo_matmul_q8_0(const uint8_t* w, const float* x, float* y, int rows, int cols,
                      const float* row_max_abs) {
    int nt = (cols + 63) / 64;
    int16_t* xq = (int16_t*)malloc(sizeof(int16_t) * (size_t)cols);
    float* mx = (float*)malloc(sizeof(float) * (size_t)rows);
    float* rs = (float*)malloc(sizeof(float) * (size_t)rows);
    int64_t* P = (int64_t*)malloc(sizeof(int64_t) * (size_t)rows * nt);
    float xs = tmqo_quantize_act(x, cols, xq);
    if (row_max_abs) memcpy(mx, row_max_abs, sizeof(float) * (size_t)rows);
    else tmqo_row_max_abs_q8_0(w, rows, cols, mx);
    for (int r = 0; r < rows; r++) rs[r] = tmqo_q8_row_scale(mx[r]);
    tmqo_tiles_q8_0(w, rows, cols, xq, rs, P);
    for (int r = 0; r < rows; r++) y[r] = tmqo_finalize_q8(P + (size_t)r * nt, nt, xs, rs[r]);
    free(xq); free(mx); free(rs); free(P);
}

/* ------------------------------------ the other branches of `matmul` */

/* read_tensor (sim/tmac_gguf.cpp:398-411): element (r, j) of a row-major
 * tensor as the reference's decoders give it -- F32 as stored, F16 half to
 * float (:216-228), Q8_0 val*scale (:238-248), Q5_0 d*q (:305-323), Q6_K
 * d*scale*q (:325-361), Q4_K d*sc*q4 - dmin*m (:363-393). */
float tmqo_read_tensor(uint32_t type, const uint8_t* w, int cols, int r, int j) {
    uint64_t idx = (uint64_t)j + (uint64_t)r * (uint64_t)cols;
    if (type == TMQO_F32) {
        float v;
        memcpy(&v, w + idx * 4, 4);
        return v;
    }
    if (type == TMQO_F16) return tmqo_f16_to_f32(rd16(w + idx * 2));
    if (type == TMQO_Q8_0) {
        const uint8_t* blk = w + (idx / 32) * 34;
        float d = tmqo_f16_to_f32(rd16(blk));
        return (float)(int8_t)blk[2 + idx % 32] * d;
    }
    if (type == TMQO_Q5_0) {
        const uint8_t* blk = w + (idx / 32) * 22;
        float d = tmqo_f16_to_f32(rd16(blk));
        return d * (float)q5_0_q(blk, (int)(idx % 32));
    }
    if (type == TMQO_Q6_K) return q6k_E(w + (idx / 256) * 210, (int)(idx % 256));
    if (type == TMQO_Q4_K) return q4k_E(w + (idx / 256) * 144, (int)(idx % 256));
    return 0.0f;
}

/* matmul_fpga_int16 (sim/tmac_gguf.cpp:887-940): activation quantised as in
 * every path (:893-899); per group of 64 rows the exact values, per row
 * row_scale = max|E|/32767 (1 below 1e-10, :908-913), and per 64-column tile
 * W_q = (int16)roundf(E / row_scale) (:915-921) times the int16 activation
 * summed in int64 (axi_vecmul_tile_int16 -> vecmul_1x64_int16,
 * sim/fpga_sim.hpp:437-446, :45-54), folded y += (double)P*x_scale*row_scale
 * tile by tile (:930-931).  Optional outputs: the int64 tile results P
 * [rows][ceil(cols/64)] and the row scales. */
void tmqo_matmul_int16(uint32_t type, const uint8_t* w, const float* x, float* y, int rows, int cols,
                       int64_t* tiles, float* row_scale_out) {
    const int N = 64, nt = (cols + N - 1) / N;
    int16_t* xq = (int16_t*)malloc(sizeof(int16_t) * (size_t)cols);
    float* W = (float*)malloc(sizeof(float) * (size_t)N * cols);
    float xs = tmqo_quantize_act(x, cols, xq);
    for (int r = 0; r < rows; r++) y[r] = 0.0f;
    for (int r0 = 0; r0 < rows; r0 += N) {
        int rn = rows - r0 < N ? rows - r0 : N;
        float rs[64];
        for (int i = 0; i < rn; i++)
            for (int j = 0; j < cols; j++) W[(size_t)i * cols + j] = tmqo_read_tensor(type, w, cols, r0 + i, j);
        for (int i = 0; i < rn; i++) {
            float m = 0.0f;
            for (int j = 0; j < cols; j++) m = fmaxf(m, fabsf(W[(size_t)i * cols + j]));
            rs[i] = (m < 1e-10f) ? 1.0f : m / 32767.0f;
            if (row_scale_out) row_scale_out[r0 + i] = rs[i];
        }
        for (int t = 0; t < nt; t++) {
            int c = t * N, cn = cols - c < N ? cols - c : N;
            for (int i = 0; i < rn; i++) {
                int64_t P = 0;
                for (int k = 0; k < cn; k++) {
                    int16_t wq = (int16_t)roundf(W[(size_t)i * cols + c + k] / rs[i]);
                    P += (int64_t)xq[c + k] * (int64_t)wq;
                }
                if (tiles) tiles[(size_t)(r0 + i) * nt + t] = P;
                y[r0 + i] += (double)P * xs * rs[i];
            }
        }
    }
    free(xq);
    free(W);
}

/* The FP32 loop of `matmul` without any --fpga flag (sim/tmac_gguf.cpp:
 * 488-492): y_r = 0 + E(r,0)*x_0 + E(r,1)*x_1 + ..., each product and sum
 * rounded to float, columns ascending. */
void tmqo_matmul_fp32(uint32_t type, const uint8_t* w, const float* x, float* y, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        float sum = 0.0f;
        for (int j = 0; j < cols; j++) sum += tmqo_read_tensor(type, w, cols, r, j) * x[j];
        y[r] = sum;
    }
}

/* ------------------------------------------------------ tile primitives */

void tmqo_tile_q8(const uint8_t* q8_W, const uint16_t* cs, const int16_t* vec, int64_t* result) {
    /* q8_W is column-major [k][n]: k = column in tile, n = row in tile */
    for (int n = 0; n < 64; n++) {
        int64_t a = 0;
        for (int k = 0; k < 64; k++) {
            int32_t prod = (int32_t)(int8_t)q8_W[k * 64 + n] * (int32_t)cs[n * 2 + k / 32];
            a += (int64_t)vec[k] * (int64_t)(int16_t)(prod >> 8);
        }
        result[n] = a;
    }
}

void tmqo_tile_q5_0_8x896(const uint8_t* blocks, const int16_t* act, const float* row_inv,
                          int64_t* result, int row_base) {
    for (int i = 0; i < 8; i++) {
        int64_t a = 0;
        for (int b = 0; b < 28; b++) {
            const uint8_t* blk = blocks + (i * 28 + b) * 22;
            float d = tmqo_f16_to_f32(rd16(blk));
            for (int wi = 0; wi < 32; wi++) {
                float e = d * (float)q5_0_q(blk, wi);
                float nrm = e * row_inv[i];
                a += (int64_t)clamp_round16(nrm) * (int64_t)act[b * 32 + wi];
            }
        }
        result[row_base + i] += a;
    }
}

void tmqo_tile_q6_k(const uint8_t* blocks, int nblocks, const int16_t* act, int ncols,
                    const float* row_inv, int64_t* result, int row_base) {
    for (int bi = 0; bi < nblocks; bi++) {
        const uint8_t* blk = blocks + bi * 210;
        int out_row = row_base + bi;
        float inv = row_inv[out_row];
        int64_t a = 0;
        for (int wi = 0; wi < 256 && wi < ncols; wi++) {
            float v = q6k_E(blk, wi) * inv;
            a += (int64_t)act[wi] * (int64_t)clamp_round16(v);
        }
        if (out_row < 896) result[out_row] += a;
    }
}

void tmqo_tile_q4_k(const uint8_t* blocks, int nblocks, const int16_t* act, int ncols,
                    const float* row_inv, int64_t* result, int row_base) {
    for (int bi = 0; bi < nblocks; bi++) {
        const uint8_t* blk = blocks + bi * 144;
        int out_row = row_base + bi;
        float inv = row_inv[out_row];
        int64_t a = 0;
        for (int wi = 0; wi < 256 && wi < ncols; wi++) {
            float v = q4k_E(blk, wi) * inv;
            a += (int64_t)act[wi] * (int64_t)clamp_round16(v);
        }
        if (out_row < 896) result[out_row] += a;
    }
}

void tmqo_tile_q5_0_4x896(const uint8_t* blocks56, const int16_t* act, const float* row_norm,
                          int64_t* result, int row_base) {
    /* 56 interleaved 48-byte pairs: [core0 block 22B][core1 block 22B][pad 4B];
     * pair bi carries row (bi<28 ? 0 : 1) for core 0 and (bi<28 ? 2 : 3) for
     * core 1, column block bi % 28. */
    int64_t a[4] = {0, 0, 0, 0};
    for (int bi = 0; bi < 56; bi++) {
        const uint8_t* p = blocks56 + bi * 48;
        int r0 = (bi < 28) ? 0 : 1, r1 = (bi < 28) ? 2 : 3, cb = (bi % 28) * 32;
        float d0 = tmqo_f16_to_f32(rd16(p)), d1 = tmqo_f16_to_f32(rd16(p + 22));
        for (int wi = 0; wi < 32; wi++) {
            float n0 = d0 * (float)q5_0_q(p, wi) * row_norm[r0];
            float n1 = d1 * (float)q5_0_q(p + 22, wi) * row_norm[r1];
            a[r0] += (int64_t)clamp_round16(n0) * (int64_t)act[cb + wi];
            a[r1] += (int64_t)clamp_round16(n1) * (int64_t)act[cb + wi];
        }
    }
    for (int i = 0; i < 4; i++) result[row_base + i] += a[i];
}

/* -------------------------------------------------------- PhaseB replay */

/* 32-byte packed descriptor, sim/fpga_sim.hpp:1254-1270 */
typedef struct {
    uint32_t next, weight, act, result;
    uint16_t num_tiles, tile_bytes;
    uint8_t tensor_type, tile_res_rows, flags;
    uint16_t act_total_bytes; /* unaligned at 0x17 */
    uint8_t num_col_groups;
} phb_desc;

static phb_desc phb_read(const uint8_t* p) {
    phb_desc d;
    d.next = rd32(p + 0x00);
    d.weight = rd32(p + 0x04);
    d.act = rd32(p + 0x08);
    d.result = rd32(p + 0x0c);
    d.num_tiles = rd16(p + 0x10);
    d.tile_bytes = rd16(p + 0x12);
    d.tensor_type = p[0x14];
    d.tile_res_rows = p[0x15];
    d.flags = p[0x16];
    d.act_total_bytes = rd16(p + 0x17);
    d.num_col_groups = p[0x19];
    return d;
}

int tmqo_phaseb_run(const uint8_t* arena, uint32_t arena_base, uint32_t desc_off, int64_t* acc) {
    /* every address in the chain is an offset into the reference's DDR
     * arena; `arena` holds that arena from offset `arena_base` on */
    arena -= arena_base;
    phb_desc d = phb_read(arena + desc_off);
    int cg = d.num_col_groups, tr = d.tile_res_rows;
    switch (d.tensor_type) {
    case 6: { /* Q5_0: 8x896 tiles, row_inv recomputed per tile (:712-734) */
        const int16_t* act = (const int16_t*)(arena + d.act);
        for (int ti = 0; ti < d.num_tiles; ti++) {
            const uint8_t* blk = arena + d.weight + (size_t)ti * d.tile_bytes;
            float ri[8];
            tmqo_row_inv_q5_0(blk, 8, 896, ri);
            tmqo_tile_q5_0_8x896(blk, act, ri, acc, ti * tr);
        }
        return d.num_tiles * tr;
    }
    case 14:   /* Q6_K: 32x256 tiles + 32 x u32 UQ24.8 row_inv */
    case 12: { /* Q4_K: 56x256 tiles + 56 x u32 UQ24.8 row_inv */
        int k6 = d.tensor_type == 14;
        int blk_bytes = k6 ? 32 * 210 : 56 * 144;
        float ri_abs[896];
        memset(ri_abs, 0, sizeof(ri_abs));
        for (int ti = 0; ti < d.num_tiles; ti++) {
            int cgi = ti % cg, rg = ti / cg, row0 = rg * tr;
            const uint8_t* blk = arena + d.weight + (size_t)ti * d.tile_bytes;
            const int16_t* act = (const int16_t*)(arena + d.act + cgi * 256 * 2);
            for (int i = 0; i < tr; i++) ri_abs[row0 + i] = (float)rd32(blk + blk_bytes + i * 4) / 256.0f;
            if (k6) tmqo_tile_q6_k(blk, tr, act, 256, ri_abs, acc, row0);
            else tmqo_tile_q4_k(blk, tr, act, 256, ri_abs, acc, row0);
        }
        return (d.num_tiles / cg) * tr;
    }
    case 15: /* CPU_OP: no matmul work */
        return 0;
    default:
        return 0;
    }
}
