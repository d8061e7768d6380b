// tmq_prefill.hip -- gfx950 kernels of the batched prefill (tmq_prefill.h):
// the digit GEMM on int8 MFMA with its fused epilogues, the attention of a
// block of positions, and the hand-over to the decode engine.
//
// GEMM (v_mfma_i32_32x32x32_i8, 32 rows x 32 tokens x 32 columns per
// instruction): both operands are fragment-major digit planes, so every MFMA
// operand is a contiguous 1 KiB block.  A workgroup (4 waves) owns a tile of
// row blocks x token blocks; per stage of KC column steps it copies the
// tile's fragments straight from global memory into LDS (one
// global_load_lds_dwordx4 per fragment and wave, no registers), two stages
// in flight.  Each wave multiplies two row blocks by one or two token
// blocks; per (row block, token block) three int32 accumulators hold
// S(a,c), S(a,e)+S(b,c) and S(b,e).  Accumulator element v of lane l is
// row 8*(v/4) + 4*(l/32) + v%4 of its block, token l & 31.
#include <hip/hip_runtime.h>

#include "tmq_device.h"
#include "tmq_mathf.h"
#include "tmq_prefill.h"

namespace {

typedef int tmq_v4i __attribute__((ext_vector_type(4)));
typedef int tmq_v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) int8_t lds_i8;

// tmq_expf with its 2^(i/32) table in LDS
struct Exp2TabLds {
    const uint64_t* p;
    __device__ uint64_t operator()(int i) const { return p[i]; }
};

__device__ __forceinline__ tmq_v16i mfma(tmq_v4i a, tmq_v4i b, tmq_v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
// 65536*S(a,c) + 256*(S(a,e)+S(b,c)) + S(b,e) + c, formed in fp64: every
// term and partial sum is an integer below 2^53, so the value is exact
__device__ __forceinline__ double digits_f64(int sac, int smid, int sbe, double c) {
    return __builtin_fma((double)sac, 65536.0, __builtin_fma((double)smid, 256.0, (double)sbe + c));
}
// (float)(t / (double)ri) for ri > 0, given rr = 1.0 / (double)ri
// (correctly rounded).  q = t * rr is within 2.5 units in the last place of
// the correctly rounded double quotient (two roundings of relative 2^-53
// each, and that quotient's own half unit), so q and it round to the same
// float unless a midpoint between two floats -- low 29 mantissa bits
// 0x10000000 -- lies within 4 units of q, or q is outside the normal float
// range; those take the division.
__device__ __forceinline__ float div_f32_rr(double t, float ri, double rr) {
    const double q = t * rr;
    const uint64_t b = (uint64_t)__double_as_longlong(q);
    const uint32_t lo = (uint32_t)b & 0x1fffffffu, e = (uint32_t)(b >> 52) & 0x7ffu;
    if (lo - 0x0ffffffcu <= 8u || e - 897u > 253u) return (float)(t / (double)ri);
    return (float)q;
}
// row (within a 32x32 block) of accumulator element v of lane l
__device__ __forceinline__ int blk_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// Workgroup tiles: KG groups of NWR x NWT waves, each wave 2 row blocks x
// WTB token blocks; NBUF stage buffers of KG*KC column steps in a ring,
// NBUF-1 stages in flight (the copies' latency is hidden behind NBUF-1
// stages of MFMA).  With KG > 1 the groups take KC column steps each of
// every stage (a split over K inside the workgroup) and add their integer
// sums in LDS after the loop.
template <int TILE> struct Tile;
template <> struct Tile<0> { static constexpr int NWR = 2, NWT = 2, WTB = 2, NBUF = 4, KG = 1; };  // 128 rows x 128 tokens
template <> struct Tile<1> { static constexpr int NWR = 1, NWT = 4, WTB = 1, NBUF = 3, KG = 1; };  // 64 x 128, 2 per CU
template <> struct Tile<2> { static constexpr int NWR = 2, NWT = 2, WTB = 1, NBUF = 6, KG = 1; };  // 128 x 64
template <> struct Tile<3> { static constexpr int NWR = 1, NWT = 4, WTB = 1, NBUF = 2, KG = 1; };  // 64 x 128, 3 per CU
template <> struct Tile<4> { static constexpr int NWR = 1, NWT = 2, WTB = 1, NBUF = 3, KG = 2; };  // 64 x 64, K in halves
constexpr int KC = 2;  // column steps (of 32) per stage and K group

template <int TILE, bool TR = false>
struct TileGeo {
    static constexpr int KG = Tile<TILE>::KG;
    static constexpr int KS = KC * KG;                                 // column steps per stage
    static constexpr int NRB = 2 * Tile<TILE>::NWR;                    // row blocks per workgroup
    static constexpr int NTB = Tile<TILE>::NWT * Tile<TILE>::WTB;      // token blocks per workgroup
    static constexpr int FRAGS = (NRB + NTB) * KS * 2;                 // 1 KiB fragments per stage
    static constexpr int FPW = FRAGS / 4;                              // memory operations per wave and stage
    static constexpr int NBUF = Tile<TILE>::NBUF;
    static constexpr int GW = Tile<TILE>::NWR * Tile<TILE>::NWT;       // waves per K group
    // TREG (asked for by TR): with one wave row, each wave's token fragments
    // are its own, so the wave loads them into registers (a ring of NBUF
    // stages) and only the weight fragments, which the waves share, go
    // through LDS
    static constexpr bool TREG = TR && Tile<TILE>::NWR == 1;
    static constexpr int LFR = TREG ? NRB * KS * 2 : FRAGS;            // LDS fragments per stage
    static constexpr int LPW = LFR / 4;                                // their copies per wave
    static constexpr int TPW = TREG ? Tile<TILE>::WTB * KC * 2 : 0;    // token loads per wave
    // int32 digit sums a wave holds: 2 x WTB blocks x 3 accumulators x 16
    static constexpr int ACCW = 2 * Tile<TILE>::WTB * 3 * 16;
    // the ring also holds the epilogue's K-group exchange and transposes
    static constexpr int EPI = KG == 2 ? KG * GW * (ACCW / 2) * 64 * 4 : 4 * 32 * 34 * 8;
    static constexpr int STAGE = LFR * 1024 > (EPI + NBUF - 1) / NBUF ? LFR * 1024 : ((EPI + NBUF - 1) / NBUF + 1023) / 1024 * 1024;
    static_assert(GW * KG == 4 && KG <= 2, "four waves, K in one or two groups");
    static_assert(LFR % 4 == 0 && LPW + TPW == FPW, "whole copies per wave; the same operations per stage");
    static_assert((NBUF - 1) * FPW <= 63, "vmcnt holds 6 bits");
    static_assert(KG * GW * (ACCW / 2) * 64 * 4 <= NBUF * STAGE || KG == 1, "the K groups' exchanged sums fit the stage ring");
    static_assert(NBUF * STAGE >= 4 * 32 * 34 * 8, "the epilogue's transpose slices fit the stage ring");
};

template <typename F, int... B>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, B...>) {
    (f(std::integral_constant<int, B>{}), ...);
}
// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>), in order
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// s_waitcnt vmcnt(k * FPW): the copies of the k newest stages may still be
// in flight
template <int FPW, int NBUF>
__device__ __forceinline__ void wait_stages(int k) {
    static_assert(NBUF <= 6, "cases below");
    switch (k) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(FPW) : "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * FPW) : "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NBUF > 3 ? 3 * FPW : 0) : "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NBUF > 4 ? 4 * FPW : 0) : "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NBUF > 5 ? 5 * FPW : 0) : "memory"); break;
    }
}

// The quantising epilogue of a GU launch (TmqPfGemm.gq_d).  Once every max
// atomic of the workgroup is in (vmcnt counts them), the workgroup counts
// itself in its token tile's counter and waits until all gridDim.x *
// gridDim.z workgroups of the tile have (all of them are resident at once:
// the host checked), so that max_bits holds each token's max |s| over its
// whole row.  widx: the workgroup's index in its tile.
// Then, as pf_act_kernel's SILU mode: x_scale = max / 32767 (1 below
// 1e-10), q = (int16)round(s / x_scale) into the digit planes (a high byte,
// and a low byte ^ 128), the sums of q - 128 per token (atomics: each
// workgroup of the tile adds its columns), x_scale per token (one wave per
// token block: xs_writer); rows at or past T get zero digits and x_scale 1.
// The wave holds token blocks tb0 .. tb0 + WTB - 1 and columns [32 s,
// 32 s + 32) of the SwiGLU rows: lane l token l & 31, columns
// 8q + 4 (l >> 5) + k (k < 4) as element 4q + k of gsv.
template <int WTB>
__device__ __forceinline__ void pf_gu_quant(const TmqPfGemm& g, const float (&gsv)[WTB][16], int tile, int widx, int tb0,
                                            int s, bool xs_writer, int lane) {
    // the wait: the tile's counter, then one release flag a workgroup
    // (128 bytes apart), set by the last to arrive; each workgroup polls
    // its own flag only, so the polls queue behind no other atomics
    __shared__ int s_last;
    const int need = gridDim.x * gridDim.z;
    uint32_t* cnt = g.gq_cnt + 32 * tile;
    uint32_t* flag = g.gq_cnt + 32 * (g.gq_ntiles + tile * need);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)need - 1u;
    __syncthreads();
    if (s_last) {
        for (int i = threadIdx.x; i < need; i += blockDim.x)
            __hip_atomic_store(flag + 32 * i, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (threadIdx.x == 0) {
        // (read by a read-modify-write: the value at the coherence point)
        uint32_t* mine = flag + 32 * widx;
        for (int it = 0; __hip_atomic_fetch_or(mine, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u; it++) {
            if (it >= g.gq_spin) {
                __hip_atomic_store(g.gq_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(4);
        }
    }
    __syncthreads();
    const int h = lane >> 5, K32 = g.gu_rows >> 5;
#pragma unroll
    for (int j = 0; j < WTB; j++) {
        const int tb = tb0 + j, t = tb * 32 + (lane & 31);
        const bool live = t < g.T;
        const uint32_t mb =
            live ? __hip_atomic_fetch_or(g.max_bits + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        const float mm = __builtin_bit_cast(float, mb);
        const float xs = (mm < 1e-10f) ? 1.0f : mm / 32767.0f;
        uint32_t hi[4], lo[4];
        int sum = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            hi[q] = lo[q] = 0u;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int v = (int)(int16_t)roundf(gsv[j][4 * q + k] / xs);
                hi[q] |= ((uint32_t)(v >> 8) & 255u) << (8 * k);
                lo[q] |= (((uint32_t)v & 255u) ^ 128u) << (8 * k);
                sum += v - 128;
            }
            if (!live) hi[q] = lo[q] = 0u;
        }
        // a plane row (tmq_pf_off) is 16 columns of one token: half h of the
        // block's columns goes to lane (l & 31) + 32h, whose dwords are runs
        // q = 0, 1 (h = 0) or 2, 3 (h = 1) of lanes l & 31 and (l & 31) + 32
        // in turn
        const uint32_t sh0 = h ? hi[0] : hi[2], sh1 = h ? hi[1] : hi[3];
        const uint32_t sl0 = h ? lo[0] : lo[2], sl1 = h ? lo[1] : lo[3];
        const uint32_t rh0 = __shfl_xor(sh0, 32), rh1 = __shfl_xor(sh1, 32);
        const uint32_t rl0 = __shfl_xor(sl0, 32), rl1 = __shfl_xor(sl1, 32);
        const uint4 vh = h ? make_uint4(rh0, hi[2], rh1, hi[3]) : make_uint4(hi[0], rh0, hi[1], rh1);
        const uint4 vl = h ? make_uint4(rl0, lo[2], rl1, lo[3]) : make_uint4(lo[0], rl0, lo[1], rl1);
        int8_t* dst = g.gq_d + ((((size_t)tb * K32 + s) * 2) * 64 + lane) * 16;
        *(uint4*)dst = vh;
        *(uint4*)(dst + 1024) = vl;
        const int tot = sum + __shfl_xor(sum, 32);
        if (live && lane < 32) __hip_atomic_fetch_add(g.gq_tsum + t, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (xs_writer && lane < 32) g.gq_xs[t] = live ? xs : 1.0f;
    }
}

template <int MODE, int TILE>
__global__ __launch_bounds__(256, TILE == 1 ? 2 : TILE == 3 ? 3 : 1) void pf_gemm_kernel(TmqPfGemm g) {
    tmq_warm_kernargs<sizeof(TmqPfGemm)>();
    typedef Tile<TILE> C;
    // token fragments in registers for gate/up and attn_output (measured:
    // gate/up 35.4 -> 34.2 us, attn_output 8.6 -> 8.3; q/k/v and down were
    // slower that way, 13.4 -> 15.6 and 16.1 -> 17.9)
    constexpr bool TR = MODE == TMQ_PF_GU || (MODE == TMQ_PF_PART && TILE == 4);
    typedef TileGeo<TILE, TR> G;
    constexpr int WTB = C::WTB;
    constexpr bool QKVM = MODE == TMQ_PF_QKV || MODE == TMQ_PF_QKVS;    // q|k|v segments
    constexpr bool PARTM = MODE == TMQ_PF_PART || MODE == TMQ_PF_QKVS;  // int64 sums out
    __shared__ __attribute__((aligned(1024))) int8_t lds[G::NBUF][G::STAGE];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kg = wave / G::GW, wq = wave % G::GW;  // K group, wave within it
    const int wr = wq / C::NWT, wt = wq % C::NWT;
    // XCD-aware tile order: workgroups are dispatched to the 8 XCDs round
    // robin (id % 8); renumber so that consecutive workgroups of one XCD
    // share an operand in its L2 -- the token tiles of one row tile (the
    // weight fragments), or, for the long-K down projection, the row tiles
    // of one token tile (the activation fragments).
    int bx, by, bz;
    {
        const int nx = gridDim.x, ny = gridDim.y, n = nx * ny * gridDim.z;
        const int id = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
        const int per = n >> 3, rem = n & 7, k = id & 7, sl = id >> 3;
        const int v = k * per + min(k, rem) + sl;
        if (MODE == TMQ_PF_PART) {
            bx = v % nx;
            by = (v / nx) % ny;
        } else {
            by = v % ny;
            bx = (v / ny) % nx;
        }
        bz = v / (ny * nx);
    }
    // row block of the workgroup's local row block i; GU: (gate j, up j)
    // pairs, so that wave wr holds gate rows in its first block and the same
    // up rows in its second
    auto rblk = [&](int i) -> int {
        return MODE == TMQ_PF_GU ? (i & 1) * (g.gu_rows >> 5) + bx * (G::NRB / 2) + (i >> 1) : bx * G::NRB + i;
    };
    const int tblk0 = by * G::NTB;
    const int nks = g.K >> 5;
    const int nst_all = nks / G::KS;
    const int st0 = bz * nst_all / g.split;  // (nst_all * split < 2^31)
    const int st1 = (bz + 1) * nst_all / g.split;
    const int nst = st1 - st0;

    // runtime segment (QKV, QKVS): the tile lies inside one tensor
    int si = 0;
    if (QKVM) {
        const int r0 = rblk(0) * 32;
        if (g.nseg > 1 && r0 >= g.seg[1].row0) si = 1;
        if (g.nseg > 2 && r0 >= g.seg[2].row0) si = 2;
    }
    const TmqPfSeg S = si == 0 ? g.seg[0] : si == 1 ? g.seg[1] : g.seg[2];
    const bool q8 = QKVM && S.q8;
    const bool hasb = MODE == TMQ_PF_QKV && S.bias != nullptr;

    // the epilogue's per-row constants of the workgroup's rows -- row_inv
    // (Q8_0: row_scale), sum (w - 128), bias -- one a thread, loaded here
    // (they arrive during the K loop) and put into LDS after it, with the
    // exp table (GU)
    static_assert(G::NRB * 32 <= 256, "one row constant a thread");
    __shared__ float c_inv[G::NRB][32];
    __shared__ int32_t c_rw[G::NRB][32];
    __shared__ float c_bias[G::NRB][32];
    __shared__ double c_rr[G::NRB][32];  // 1 / (double)c_inv
    __shared__ uint64_t c_tab[32];
    float pre_inv = 0.0f, pre_bias = 0.0f;
    int32_t pre_rw = 0;
    if (!PARTM && (int)threadIdx.x < G::NRB * 32) {
        const int i = threadIdx.x >> 5, r = threadIdx.x & 31;
        const TmqPfSeg Sg = MODE == TMQ_PF_GU ? ((i & 1) ? g.seg[1] : g.seg[0]) : S;
        const int row = rblk(i) * 32 + r, rr = row - Sg.row0;
        pre_inv = q8 ? Sg.row_scale[rr] : Sg.row_inv[rr];
        pre_rw = g.rw_t[row];
        pre_bias = hasb ? Sg.bias[rr] : 0.0f;
    }
    // stage st -> buffer b: fragment f of LFR (run f / 2KS = one row or
    // token block, KS column steps x 2 digits contiguous on both sides);
    // wave w issues f = w, w+4, ...  K is a multiple of 32*KS.
    auto issue = [&](int st, int b) {
        const int ks = (st0 + st) * G::KS;
#pragma unroll
        for (int k = 0; k < G::LPW; k++) {
            const int f = wave + 4 * k;  // wave-uniform
            const int run = f / (G::KS * 2), in = f % (G::KS * 2);
            const bool wgt = run < G::NRB;
            const int8_t* base = wgt ? g.w : g.x;
            const int blk = wgt ? rblk(run) : tblk0 + run - G::NRB;
            const int8_t* src = base + ((size_t)blk * nks + ks) * 2048 + (size_t)in * 1024;
            __builtin_amdgcn_global_load_lds((const void*)(src + lane * 16),
                                             (lds_i8*)(lds[b] + (size_t)f * 1024), 16, 0, 0);
        }
    };
    // (column step kc of the wave's K group)
    auto frag = [&](int b, int run, int kc, int d) -> tmq_v4i {
        return *(const tmq_v4i*)(lds[b] + ((size_t)(run * G::KS + kg * KC + kc) * 2 + d) * 1024 + lane * 16);
    };
    // TREG: the wave's token fragments of stage st (its WTB blocks, its K
    // group's KC column steps, both digits), the bytes issue() would have
    // copied for them
    typedef tmq_v4i TokStage[WTB][KC][2];
    auto tload = [&](int st, TokStage& dst) {
        const int ks = (st0 + st) * G::KS + kg * KC;
#pragma unroll
        for (int j = 0; j < WTB; j++) {
            const int8_t* src = g.x + ((size_t)(tblk0 + wt * WTB + j) * nks + ks) * 2048 + lane * 16;
#pragma unroll
            for (int kc = 0; kc < KC; kc++)
#pragma unroll
                for (int d = 0; d < 2; d++) dst[j][kc][d] = *(const tmq_v4i*)(src + (kc * 2 + d) * 1024);
        }
    };

    tmq_v16i acc[2][WTB][3];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < WTB; j++)
#pragma unroll
            for (int d = 0; d < 3; d++) acc[i][j][d] = tmq_v16i{};
    const int tw0 = (tblk0 + wt * WTB) * 32;  // first token of the wave
    // the tokens' x_scale and sum (x - 128): loaded now, converted after the
    // K loop (a conversion here would wait for the loads before the first
    // copies are issued)
    float xs_raw[WTB];
    int32_t tx_raw[WTB];
#pragma unroll
    for (int j = 0; j < WTB; j++) {
        const int t = tw0 + j * 32 + (lane & 31);
        xs_raw[j] = g.xs[t];
        tx_raw[j] = g.tx_t[t];
    }

    // RoPE pairs of the wave's q / k rows (QKV), loaded now: they arrive
    // during the K loop
    float4 rope_cs[WTB][2][4];
    if (MODE == TMQ_PF_QKV && si != 2) {
#pragma unroll
        for (int j = 0; j < WTB; j++) {
            const int pos = g.p0 + min(tw0 + j * 32 + (lane & 31), g.T - 1);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int rr = rblk(2 * wr + i) * 32 + blk_row(4 * q, lane) - S.row0;
                    rope_cs[j][i][q] = *(const float4*)(g.rope + (size_t)pos * 32 + ((rr & 63) >> 1));
                }
        }
    }

    // the token ring (TREG): slot b holds the stage that LDS buffer b holds
    TokStage tk[G::TREG ? G::NBUF : 1];
    static_for<G::NBUF - 1>([&](auto sc) {
        constexpr int st = decltype(sc)::value;
        if (st < nst) {
            issue(st, st);
            if constexpr (G::TREG) tload(st, tk[st]);
        }
    });
    // the K loop, compiled twice: with the Q8_0 tile sums (Q8 true) and
    // without them, so that the common loop carries none of their registers;
    // unrolled by NBUF so that every ring slot is a fixed set of registers
    // (stage st in buffer and slot st % NBUF)
    auto kloop = [&](auto q8c) {
    constexpr bool Q8 = decltype(q8c)::value;
    for (int sb = 0; sb < nst; sb += G::NBUF)
    static_for<G::NBUF>([&](auto bc) {
        constexpr int b = decltype(bc)::value;
        const int st = sb + b;
        if (st >= nst) return;
        // refill the buffer (and slot) the previous iteration finished with
        if (st + G::NBUF - 1 < nst) {
            constexpr int nb = (b + G::NBUF - 1) % G::NBUF;
            issue(st + G::NBUF - 1, nb);
            if constexpr (G::TREG) tload(st + G::NBUF - 1, tk[nb]);
        }
        wait_stages<G::FPW, G::NBUF>(min(G::NBUF - 1, nst - 1 - st));
        // the stage's LDS copies are complete in this wave (vmcnt above);
        // the barrier makes them complete in all.  A plain s_barrier (the
        // workgroup fence of __syncthreads would also wait for the next
        // stage's copies), as asm with a memory clobber so that no LDS
        // access moves across it.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int ks = (st0 + st) * G::KS + kg * KC;  // the group's first column step
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            {
                const tmq_v4i a0 = frag(b, 2 * wr, kc, 0), b0 = frag(b, 2 * wr, kc, 1);
                const tmq_v4i a1 = frag(b, 2 * wr + 1, kc, 0), b1 = frag(b, 2 * wr + 1, kc, 1);
#pragma unroll
                for (int j = 0; j < WTB; j++) {
                    const int tr = G::NRB + wt * WTB + j;
                    tmq_v4i c, e;
                    if constexpr (G::TREG) {
                        c = tk[b][j][kc][0];
                        e = tk[b][j][kc][1];
                    } else {
                        c = frag(b, tr, kc, 0);
                        e = frag(b, tr, kc, 1);
                    }
                    acc[0][j][0] = mfma(a0, c, acc[0][j][0]);
                    acc[1][j][0] = mfma(a1, c, acc[1][j][0]);
                    acc[0][j][1] = mfma(a0, e, acc[0][j][1]);
                    acc[1][j][1] = mfma(a1, e, acc[1][j][1]);
                    acc[0][j][2] = mfma(b0, e, acc[0][j][2]);
                    acc[1][j][2] = mfma(b1, e, acc[1][j][2]);
                    acc[0][j][1] = mfma(b0, c, acc[0][j][1]);
                    acc[1][j][1] = mfma(b1, c, acc[1][j][1]);
                }
            }
            if (Q8 && (kc & 1)) {
                // Q8_0: the 64-column tile just completed, as an int64 digit
                // sum per element, for pf_qkv_fin_kernel
                const int tile = (ks + kc) >> 1;
#pragma unroll
                for (int j = 0; j < WTB; j++) {
                    const int t = tw0 + j * 32 + (lane & 31);
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        // [tile][row][token]: the 32 tokens of a row are contiguous
                        int64_t* out = g.tpart + ((size_t)tile * S.rows + rblk(2 * wr + i) * 32 - S.row0) * g.T_pad + t;
#pragma unroll
                        for (int v = 0; v < 16; v++)
                            out[(size_t)blk_row(v, lane) * g.T_pad] = 65536 * (int64_t)acc[i][j][0][v] +
                                                                       256 * (int64_t)acc[i][j][1][v] +
                                                                       (int64_t)acc[i][j][2][v];
#pragma unroll
                        for (int d = 0; d < 3; d++) acc[i][j][d] = tmq_v16i{};
                    }
                }
            }
        }
        // every wave's reads of buffer b are done (their values fed the
        // MFMAs above) before the next iteration copies a stage into it
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    });
    };
    if (QKVM && q8) kloop(std::integral_constant<bool, true>{});
    else kloop(std::integral_constant<bool, false>{});

    if (QKVM && q8) return;  // pf_qkv_fin_kernel finishes these rows
    double xs_t[WTB], tc_t[WTB];
#pragma unroll
    for (int j = 0; j < WTB; j++) {
        xs_t[j] = (double)xs_raw[j];
        tc_t[j] = (double)(128 * (int64_t)tx_raw[j] + 16384 * (int64_t)g.K);
    }
    if (!PARTM) {
        if ((int)threadIdx.x < G::NRB * 32) {
            const int i = threadIdx.x >> 5, r = threadIdx.x & 31;
            c_inv[i][r] = pre_inv;
            c_rr[i][r] = 1.0 / (double)pre_inv;
            c_rw[i][r] = pre_rw;
            c_bias[i][r] = pre_bias;
        }
        if (MODE == TMQ_PF_GU && threadIdx.x < 32) c_tab[threadIdx.x] = tmq_math::exp2_tab(threadIdx.x);
        __syncthreads();
    }
    // K groups (KG = 2): group g keeps row block g of its waves' two and
    // finishes it; the other block's digit sums go to the wave of the other
    // group that holds the same tile, through the stage ring (free since the
    // loop's last barrier)
    auto mine = [&](int i) { return G::KG == 1 || i == kg; };
    if (G::KG == 2) {
        int* red = (int*)&lds[0][0];
        int* dst = red + (kg * G::GW + wq) * (WTB * 3 * 16) * 64 + lane;
        const int* src = red + ((1 - kg) * G::GW + wq) * (WTB * 3 * 16) * 64 + lane;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            if (mine(i)) continue;
#pragma unroll
            for (int j = 0; j < WTB; j++)
#pragma unroll
                for (int d = 0; d < 3; d++)
#pragma unroll
                    for (int v = 0; v < 16; v++) dst[((j * 3 + d) * 16 + v) * 64] = acc[i][j][d][v];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2; i++) {
            if (!mine(i)) continue;
#pragma unroll
            for (int j = 0; j < WTB; j++)
#pragma unroll
                for (int d = 0; d < 3; d++)
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[i][j][d][v] += src[((j * 3 + d) * 16 + v) * 64];
        }
        // (the epilogue's transposes reuse the ring)
        __syncthreads();
    }
    // the stage ring is free now (the last iteration's barrier): each wave
    // turns its 32x32 blocks to [token][row] in its own slice of it, so that
    // the global stores are whole rows of a token (every wave's LDS accesses
    // execute in order, so no barrier between its writes and reads)
    if (PARTM) {
        // int64 sums, 34 per token (16-byte aligned rows; two lanes a bank
        // at most); stored 256 contiguous bytes a token, four tokens an
        // instruction
        int64_t* tp = (int64_t*)&lds[0][0] + wave * (32 * 34);
#pragma unroll
        for (int j = 0; j < WTB; j++) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                if (!mine(i)) continue;
#pragma unroll
                for (int v = 0; v < 16; v++)
                    tp[(lane & 31) * 34 + blk_row(v, lane)] = 65536 * (int64_t)acc[i][j][0][v] +
                                                               256 * (int64_t)acc[i][j][1][v] +
                                                               (int64_t)acc[i][j][2][v];
                const int r0 = rblk(2 * wr + i) * 32, c = lane & 15;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int tt = (lane >> 4) + 4 * k;
                    const longlong2 val = *(const longlong2*)(tp + tt * 34 + 2 * c);
                    *(longlong2*)(g.part + ((size_t)bz * g.T_pad + tw0 + j * 32 + tt) * g.rows + r0 + 2 * c) = val;
                }
            }
        }
        return;
    }

    // element v of block (i, j), finalised (sim/tmac_gguf.cpp:1303-1305) +
    // bias (:1595-1597)
    auto fin = [&](int i, int j, int v) -> float {
        const int li = 2 * wr + i, rb = blk_row(v, lane);
        const double a = digits_f64(acc[i][j][0][v], acc[i][j][1][v], acc[i][j][2][v],
                                    tc_t[j] + (double)(128 * c_rw[li][rb]));
        float f = div_f32_rr(a * xs_t[j], c_inv[li][rb], c_rr[li][rb]);
        if (hasb) f = f + c_bias[li][rb];
        return f;
    };

    // elements v = 4q .. 4q+3 of a lane are 4 consecutive rows: one float4
    float gsv[MODE == TMQ_PF_GU ? WTB : 1][16];  // GU: the SwiGLU values (quantised after the wait)
#pragma unroll
    for (int j = 0; j < WTB; j++) {
        const int t = tw0 + j * 32 + (lane & 31);
        const bool live = t < g.T;
        if (MODE == TMQ_PF_QKV) {
            if (!live) continue;
            const int pos = g.p0 + t;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                if (!mine(i)) continue;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int rr = rblk(2 * wr + i) * 32 + blk_row(4 * q, lane) - S.row0;  // pairs (rr, rr+1), (rr+2, rr+3)
                    float o[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) o[k] = fin(i, j, 4 * q + k);
                    if (si != 2) {
                        // apply_rope (sim/tmac_gguf.cpp:1537-1539)
                        const float4 cs = rope_cs[j][i][q];
#pragma unroll
                        for (int k = 0; k < 2; k++) {
                            const float y0 = o[2 * k], y1 = o[2 * k + 1];
                            const float c = k ? cs.z : cs.x, sn = k ? cs.w : cs.y;
                            o[2 * k] = y0 * c - y1 * sn;
                            o[2 * k + 1] = y0 * sn + y1 * c;
                        }
                    }
                    float* dst = si == 0   ? g.q_out + (size_t)t * g.H + rr
                                 : si == 1 ? g.kc + (size_t)pos * g.KV + rr
                                           : g.vc + (size_t)pos * g.KV + rr;
                    *(float4*)dst = make_float4(o[0], o[1], o[2], o[3]);
                }
            }
        } else if (MODE == TMQ_PF_GU) {
            // SwiGLU (sim/tmac_gguf.cpp:459-461): gate rows in block 0, the
            // same up rows in block 1
            // (the SwiGLU values through the wave's LDS slice, 36 floats a
            // token; stored 128 contiguous bytes a token, eight tokens an
            // instruction)
            float m = 0.0f;
            const int j0 = rblk(2 * wr) * 32;
            const Exp2TabLds tab{c_tab};
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float gv = fin(0, j, 4 * q + k);
                    const float sv = (gv / (1.0f + tmq_math::tmq_expf_tab(-gv, tab))) * fin(1, j, 4 * q + k);
                    gsv[j][4 * q + k] = sv;
                    m = fmaxf(m, fabsf(sv));
                }
            if (!g.gq_d) {
                float* tp = (float*)&lds[0][0] + wave * (32 * 36);
#pragma unroll
                for (int q = 0; q < 4; q++)
                    *(float4*)(tp + (lane & 31) * 36 + blk_row(4 * q, lane)) =
                        make_float4(gsv[j][4 * q], gsv[j][4 * q + 1], gsv[j][4 * q + 2], gsv[j][4 * q + 3]);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int tt = (lane >> 3) + 8 * k, c = lane & 7, ts = tw0 + j * 32 + tt;
                    const float4 val = *(const float4*)(tp + tt * 36 + 4 * c);
                    if (ts < g.T) *(float4*)(g.s_out + (size_t)ts * g.gu_rows + j0 + 4 * c) = val;
                }
            }
            m = fmaxf(m, __shfl_xor(m, 32));
            if (live && lane < 32)
                __hip_atomic_fetch_max(g.max_bits + t, __builtin_bit_cast(uint32_t, m), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if constexpr (MODE == TMQ_PF_GU) {
        if (g.gq_d) pf_gu_quant<WTB>(g, gsv, by, bx + gridDim.x * bz, tblk0 + wt * WTB, rblk(2 * wr), wr == 0 && bx == 0, lane);
    }
}

// Attention of token t (position P = p0 + t) for the query heads of KV
// head g: the decode engine's chains (attn_kernel) per query -- scores
// summed over d in order and /8, max, exp terms summed over positions in
// order, tmq_logf, weights, the context summed over positions in order.
// The query rows are wave-uniform and read through the scalar cache.  Each
// thread keeps the scores of its positions (tid + 512 k, k < NPASS) in
// registers; LDS holds the exp terms, then the weights, of every position.
typedef __attribute__((address_space(4))) const float cf32;
constexpr int VCH = 32;    // positions per V chunk
// A transposed V chunk: dimension d's VCH positions in 32 floats, float4
// group j of them at group j ^ ((d >> 1) & 7), so that a float4 read by 16
// consecutive dimensions covers all 64 banks once
static __device__ __forceinline__ int vt_idx(int d, int pr) {
    return d * VCH + ((((pr >> 2) ^ ((d >> 1) & 7)) << 2) | (pr & 3));
}
static __device__ __forceinline__ int vt_grp(int d, int j) { return d * VCH + ((j ^ ((d >> 1) & 7)) << 2); }

// acc += w_j * v_j for 16 positions base + j in order, w_j = lane j of the
// lane's 16-lane row of e; with PART, the terms of positions >= nr are added
// as +0 (acc is never -0, so acc + 0 = acc; the V values read there are
// never used)
template <int J>
static __device__ __forceinline__ float row_bcast(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x150 + J, 0xf, 0xf, true));
}
template <bool PART, int... J>
static __device__ __forceinline__ float ctx_half(float acc, float e, const float* v, int base, int nr,
                                                 std::integer_sequence<int, J...>) {
    ((acc += PART ? (base + J < nr ? row_bcast<J>(e) * v[J] : 0.0f) : row_bcast<J>(e) * v[J]), ...);
    return acc;
}
template <int NPASS>
__global__ __launch_bounds__(512, NPASS <= 2 ? 8 : NPASS == 4 ? 6 : 4) void pf_attn_kernel(TmqPfAttn a) {
    tmq_warm_kernargs<sizeof(TmqPfAttn)>();
    extern __shared__ float lds[];
    __shared__ float stat[2][8];
    __shared__ float red[8][8];  // [wave][head] maxima
    __shared__ uint64_t tab[32];
    // V chunks of VCH positions, transposed (dimension-major, vt_idx) so
    // that the lane of dimension d reads four positions at once;
    // double-buffered.  (Under 32 KiB of LDS a workgroup with the exp terms
    // of 512 positions, and at most 64 registers: four workgroups a CU, so
    // that the launch's 2 x T workgroups run in one round.)
    __shared__ __attribute__((aligned(16))) float vb2[2][64 * VCH];
    // Which (token, KV head) this workgroup takes.  Ranked by length (the
    // latest tokens, with the most positions, first), the launch's
    // workgroups go out in that order; with `deal`, when all of them are
    // resident at once (four a CU), the CU that takes workgroup i takes
    // i + ncu, i + 2 ncu, ..., so the ranks are dealt in a snake (forward
    // in even rounds of ncu, backward in odd ones) and every CU gets about
    // the same number of positions.
    int rank = blockIdx.x + a.T * blockIdx.y;
    if (a.deal) {
        const int r = rank / a.ncu, c = rank - r * a.ncu;
        const int n = min(a.ncu, a.T * a.n_kv - r * a.ncu);
        rank = r * a.ncu + ((r & 1) ? n - 1 - c : c);
    }
    const int t = a.T - 1 - rank / a.n_kv, g = rank - (rank / a.n_kv) * a.n_kv, tid = threadIdx.x;
    const int qpk = a.n_heads / a.n_kv, KV = a.n_kv * 64, H = a.n_heads * 64;
    const int np = a.p0 + t + 1, npad = (np + 3) & ~3;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), ln = tid & 63;
    float* ex = lds;  // [qpk][npad]
    const float* kb = a.kc + g * 64;
    const float* vbase = a.vc + g * 64;
    const cf32* qg = (const cf32*)(a.q + (size_t)t * H + g * qpk * 64);
    if (tid < 32) tab[tid] = tmq_math::exp2_tab(tid);
    // scores of positions tid + 512 k; a wave whose 64 positions all lie
    // past the last one computes none (its entries are never read: every
    // later use is guarded by p < np)
    float scr[NPASS][8];
#pragma unroll
    for (int k = 0; k < NPASS; k++) {
        if (k > 0 && k * 512 >= np) break;
        if (k * 512 + wv * 64 >= np) continue;
        const int p = tid + k * 512;
        const float4* kp = (const float4*)(kb + (size_t)min(p, np - 1) * KV);
        // the key row in two halves of 32 dimensions (each head's sum runs
        // over the first half, then on over the second: the same order)
        float s[8];
#pragma unroll
        for (int h = 0; h < 8; h++) s[h] = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            float4 kk[8];
#pragma unroll
            for (int i = 0; i < 8; i++) kk[i] = kp[8 * half + i];
#pragma unroll
            for (int h = 0; h < 8; h++) {
                if (h >= qpk) break;
                const cf32* qh = qg + h * 64 + 32 * half;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    s[h] += qh[4 * i + 0] * kk[i].x;
                    s[h] += qh[4 * i + 1] * kk[i].y;
                    s[h] += qh[4 * i + 2] * kk[i].z;
                    s[h] += qh[4 * i + 3] * kk[i].w;
                }
            }
        }
#pragma unroll
        for (int h = 0; h < 8; h++)
            if (h < qpk) scr[k][h] = s[h] / 8.0f;
    }
    // max per head: the thread's, the wave's, then the workgroup's (fmaxf
    // is exact in any order)
    float mx[8];
#pragma unroll
    for (int h = 0; h < 8; h++) {
        float m = -__builtin_inff();
#pragma unroll
        for (int k = 0; k < NPASS; k++)
            if (h < qpk && tid + k * 512 < np) m = fmaxf(m, scr[k][h]);
        m = tmq_wave_max(m);
        mx[h] = m;
    }
    if (ln == 0)
#pragma unroll
        for (int h = 0; h < 8; h++) red[wv][h] = mx[h];
    __syncthreads();
    if (tid < 8) {
        float m = red[0][tid];
        for (int w = 1; w < 8; w++) m = fmaxf(m, red[w][tid]);
        stat[0][tid] = m;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 8; h++) mx[h] = stat[0][h];
    const Exp2TabLds et{tab};
    // exp terms (scores - max) into LDS
#pragma unroll
    for (int k = 0; k < NPASS; k++) {
        const int p = tid + k * 512;
        if (p >= np) break;
#pragma unroll
        for (int h = 0; h < 8; h++) {
            if (h >= qpk) break;
            ex[h * npad + p] = tmq_math::tmq_expf_tab(scr[k][h] - mx[h], et);
        }
    }
    __syncthreads();
    if (wv == 0 && ln < qpk) {
        // lane h of wave 0 sums head h's terms
        const float* e = ex + ln * npad;
        float es = 0.0f;
        int p = 0;
        // 32 terms per step: eight LDS reads in flight, then the adds in order
        for (; p + 32 <= np; p += 32) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = *(const float4*)(e + p + 4 * j);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                es += v[j].x;
                es += v[j].y;
                es += v[j].z;
                es += v[j].w;
            }
        }
        if (p < np) {
            // the last 1-31 terms: reads clamped into range, the terms past
            // the end added as +0 (es is never -0, so x + 0 = x)
            float v[32];
#pragma unroll
            for (int j = 0; j < 32; j++) v[j] = e[min(p + j, np - 1)];
#pragma unroll
            for (int j = 0; j < 32; j++) es += p + j < np ? v[j] : 0.0f;
        }
        stat[1][ln] = tmq_math::tmq_logf(es) + stat[0][ln];
    }
    __syncthreads();
    // weights (scores - log-sum) over the exp terms
#pragma unroll
    for (int k = 0; k < NPASS; k++) {
        const int p = tid + k * 512;
        if (p >= np) break;
#pragma unroll
        for (int h = 0; h < 8; h++) {
            if (h >= qpk) break;
            ex[h * npad + p] = tmq_math::tmq_expf_tab(scr[k][h] - stat[1][h], et);
        }
    }
    // context, VCH positions per chunk; the next chunk's V rows are loaded
    // into registers while the current one is summed (512 threads x one
    // float4 = one chunk; a wave's lanes take the chunk's 32 positions of two
    // groups of four dimensions)
    auto put_v = [&](float* vt, int pr, int q4, float4 v) {
        vt[vt_idx(4 * q4 + 0, pr)] = v.x;
        vt[vt_idx(4 * q4 + 1, pr)] = v.y;
        vt[vt_idx(4 * q4 + 2, pr)] = v.z;
        vt[vt_idx(4 * q4 + 3, pr)] = v.w;
    };
    static_assert(VCH * 16 == 512, "one float4 a thread per chunk");
    {
        const int nr = min(VCH, np), pr = tid & (VCH - 1), q4 = tid / VCH;
        if (pr < nr) put_v(vb2[0], pr, q4, *(const float4*)(vbase + (size_t)pr * KV + 4 * q4));
    }
    __syncthreads();
    float acc = 0.0f;
    int buf = 0;
    for (int c0 = 0; c0 < np; c0 += VCH) {
        const int nr = min(VCH, np - c0), c1 = c0 + VCH, nr1 = min(VCH, np - c1);
        const int ppr = tid & (VCH - 1), pq4 = tid / VCH;
        float4 pre;
        if (ppr < nr1) pre = *(const float4*)(vbase + (size_t)(c1 + ppr) * KV + 4 * pq4);
        if (wv < qpk) {
            // the chunk's weights in registers: lane i of every 16-lane row
            // holds position h + i of each half h, and each multiply takes
            // its weight by row_newbcast (no broadcast LDS reads); the
            // lane's dimension of the half's V rows in four float4 reads
            const float* e = ex + wv * npad + c0;
            const float* vt = vb2[buf];
            const int r = ln & 15;
#pragma unroll
            for (int h = 0; h < VCH; h += 16) {
                const float eh = e[min(h + r, nr - 1)];
                float4 vv[4];
#pragma unroll
                for (int i = 0; i < 4; i++) vv[i] = *(const float4*)(vt + vt_grp(ln, h / 4 + i));
                if (nr == VCH)
                    acc = ctx_half<false>(acc, eh, (const float*)vv, 0, nr, std::make_integer_sequence<int, 16>{});
                else
                    acc = ctx_half<true>(acc, eh, (const float*)vv, h, nr, std::make_integer_sequence<int, 16>{});
            }
        }
        if (ppr < nr1) put_v(vb2[buf ^ 1], ppr, pq4, pre);
        __syncthreads();
        buf ^= 1;
    }
    if (wv < qpk) a.ctx[(size_t)t * H + (g * qpk + wv) * 64 + ln] = acc;
}

// q, k, v finished (TmqPfQkvFin).  Threads [0, nA): one token and four
// consecutive rows of the q / k and Q5_0 / K-quant v rows, from the split
// sums (rows fastest, one float4 store); threads of the blocks after: one
// token and row of a Q8_0 v segment, from its tile sums (tokens fastest).
__global__ __launch_bounds__(256) void pf_qkv_fin_kernel(TmqPfQkvFin f) {
    tmq_warm_kernargs<sizeof(TmqPfQkvFin)>();
    const bool vq8 = f.seg[2].q8 != 0;
    const int nr = f.part ? f.H + (vq8 ? 1 : 2) * f.KV : 0;  // rows from split sums
    const int g4 = nr >> 2, nA = f.T * g4, nbA = (nA + 255) >> 8;
    if ((int)blockIdx.x < nbA) {
        const int i = blockIdx.x * 256 + threadIdx.x;
        if (i >= nA) return;
        const int t = i / g4, row = (i - t * g4) * 4;
        const int si = row < f.H ? 0 : row < f.H + f.KV ? 1 : 2;
        const int rr = row - (si == 0 ? 0 : si == 1 ? f.H : f.H + f.KV);
        const float* inv = si == 0 ? f.seg[0].row_inv : si == 1 ? f.seg[1].row_inv : f.seg[2].row_inv;
        const float* bias = si == 0 ? f.seg[0].bias : si == 1 ? f.seg[1].bias : f.seg[2].bias;
        const int pos = f.p0 + t;
        const int ld = f.H + 2 * f.KV;
        // every load first
        const int4 rw = *(const int4*)(f.rw_t + row);
        const int64_t tc = 128 * (int64_t)f.tx_t[t] + 16384 * (int64_t)f.K;
        const double xs = (double)f.xs[t];
        float ri[4], bs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 4; k++) ri[k] = inv[rr + k];
        if (bias)
#pragma unroll
            for (int k = 0; k < 4; k++) bs[k] = bias[rr + k];
        float4 cs = make_float4(1.0f, 0.0f, 1.0f, 0.0f);
        if (si != 2) cs = *(const float4*)(f.rope + (size_t)pos * 32 + ((rr & 63) >> 1));
        int64_t a[4] = {tc + 128 * (int64_t)rw.x, tc + 128 * (int64_t)rw.y, tc + 128 * (int64_t)rw.z,
                        tc + 128 * (int64_t)rw.w};
        // the split sums in batches of 8 (loads first; indices clamped, the
        // surplus added as 0)
        for (int s0 = 0; s0 < f.split; s0 += 8) {
            longlong2 u[8], v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const longlong2* p =
                    (const longlong2*)(f.part + ((size_t)min(s0 + j, f.split - 1) * f.T_pad + t) * ld + row);
                u[j] = p[0];
                v[j] = p[1];
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const bool in = s0 + j < f.split;
                a[0] += in ? u[j].x : 0;
                a[1] += in ? u[j].y : 0;
                a[2] += in ? v[j].x : 0;
                a[3] += in ? v[j].y : 0;
            }
        }
        // finalised (sim/tmac_gguf.cpp:1303-1305) + bias (:1595-1597)
        float o[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            o[k] = (float)(((double)a[k] * xs) / (double)ri[k]);
            if (bias) o[k] = o[k] + bs[k];
        }
        if (si != 2) {
            // apply_rope (sim/tmac_gguf.cpp:1537-1539): pairs (rr, rr+1), (rr+2, rr+3)
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const float y0 = o[2 * k], y1 = o[2 * k + 1];
                const float c = k ? cs.z : cs.x, sn = k ? cs.w : cs.y;
                o[2 * k] = y0 * c - y1 * sn;
                o[2 * k + 1] = y0 * sn + y1 * c;
            }
        }
        float* dst = si == 0   ? f.q_out + (size_t)t * f.H + rr
                     : si == 1 ? f.kc + (size_t)pos * f.KV + rr
                               : f.vc + (size_t)pos * f.KV + rr;
        *(float4*)dst = make_float4(o[0], o[1], o[2], o[3]);
        return;
    }
    // Q8_0 v: the tiles folded in order (sim/tmac_gguf.cpp:1075-1076)
    const int i = ((int)blockIdx.x - nbA) * 256 + threadIdx.x;
    if (!vq8 || i >= f.T * f.KV) return;
    const int r = i / f.T, t = i - r * f.T, nt = f.K / TMQ_PF_CHUNK;
    const int32_t* rw = f.rw_c + (size_t)(f.H + f.KV + r) * nt;
    const int32_t* tx = f.tx_c + (size_t)t * nt;
    const double xs = (double)f.xs[t], rs = (double)f.seg[2].row_scale[r];
    float y = 0.0f;
    for (int c0 = 0; c0 < nt; c0 += 8) {
        // 8 tiles' loads first (indices clamped), then the ordered fold
        int64_t p[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int c = min(c0 + j, nt - 1);
            p[j] = f.tpart[((size_t)c * f.KV + r) * f.T_pad + t] + 128 * ((int64_t)rw[c] + tx[c]) +
                   16384 * TMQ_PF_CHUNK;
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (c0 + j < nt) y = (float)((double)y + ((double)p[j] * xs) * rs);
    }
    if (f.seg[2].bias) y = y + f.seg[2].bias[r];
    f.vc[(size_t)(f.p0 + t) * f.KV + r] = y;
}

// The decode engine's residual state after the prefill's last token.
__global__ __launch_bounds__(256) void pf_handoff_kernel(TmqPfHandoff h) {
    for (int r = threadIdx.x; r < h.H; r += blockDim.x) {
        __hip_atomic_store(h.kacc + r, tmq_pf_acc(h.dn, h.t, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        h.hid[r] = h.x1[(size_t)h.t * h.H + r];
    }
    if (threadIdx.x == 0) *h.xs_slot = h.dn.xs[h.t];
}

template <int MODE, int TILE>
int launch_gemm(const TmqPfGemm& g, hipStream_t s) {
    typedef TileGeo<TILE> G;
    const int rt = MODE == TMQ_PF_GU ? g.gu_rows / (16 * G::NRB) : g.rows / (32 * G::NRB);
    const dim3 grid(rt, (g.T_pad + 32 * G::NTB - 1) / (32 * G::NTB), g.split);
    hipLaunchKernelGGL((pf_gemm_kernel<MODE, TILE>), grid, dim3(256), 0, s, g);
    return (int)hipGetLastError();
}
template <int MODE>
int launch_tile(const TmqPfGemm& g, int tile, hipStream_t s) {
    switch (tile) {
    case 0: return launch_gemm<MODE, 0>(g, s);
    case 1: return launch_gemm<MODE, 1>(g, s);
    case 2: return launch_gemm<MODE, 2>(g, s);
    case 3: return launch_gemm<MODE, 3>(g, s);
    case 4: return launch_gemm<MODE, 4>(g, s);
    }
    return (int)hipErrorInvalidValue;
}

}  // namespace

size_t tmq_pf_attn_lds(int qpk, int npos) {
    const size_t npad = ((size_t)npos + 3) & ~(size_t)3;
    return sizeof(float) * (size_t)qpk * npad;
}

namespace {
// resident GU workgroups a CU per tile (0: not known yet), from the first use
int gu_per_cu[4] = {0, 0, 0, 0};
template <int TILE>
bool gu_quant_fits(int T_pad, int gu_rows, int ncu, int* ntiles) {
    typedef TileGeo<TILE> G;
    const long rt = gu_rows / (16 * G::NRB), tt = (T_pad + 32 * G::NTB - 1) / (32 * G::NTB);
    int& per = gu_per_cu[TILE];
    if (per == 0 &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void*)pf_gemm_kernel<TMQ_PF_GU, TILE>, 256, 0) !=
            hipSuccess) {
        per = 0;
        return false;
    }
    *ntiles = (int)tt;
    return rt * tt <= (long)per * ncu;
}
}  // namespace

bool tmq_pf_gu_quant_fits(int tile, int T_pad, int gu_rows, int ncu, int* ntiles) {
    *ntiles = 0;
    if (ncu <= 0 || T_pad <= 0 || gu_rows <= 0) return false;
    switch (tile) {
    case 0: return gu_quant_fits<0>(T_pad, gu_rows, ncu, ntiles);
    case 1: return gu_quant_fits<1>(T_pad, gu_rows, ncu, ntiles);
    case 2: return gu_quant_fits<2>(T_pad, gu_rows, ncu, ntiles);
    case 3: return gu_quant_fits<3>(T_pad, gu_rows, ncu, ntiles);
    }
    return false;  // (tile 4 takes no GU launch)
}

int tmq_launch_pf_gemm(const TmqPfGemm& g, int tile, hipStream_t s) {
    // shapes the kernel assumes: 64-column chunks, whole token tiles of the
    // operand planes, whole row tiles (GU: gate/up tiles of NRB/2 blocks),
    // a split count no larger than the stages, one split for fused epilogues
    if (tile < 0 || tile > 4) return (int)hipErrorInvalidValue;
    const int nrb = tile == 1 || tile == 3 || tile == 4 ? 2 : 4, ntb = tile == 2 || tile == 4 ? 2 : 4;
    const int ks = KC * (tile == 4 ? Tile<4>::KG : 1);  // column steps per stage
    if (g.K <= 0 || g.K % (32 * ks) || g.T_pad % (32 * ntb) || g.T > g.T_pad || g.split < 1 ||
        g.split > g.K / (32 * ks))
        return (int)hipErrorInvalidValue;
    if (g.mode != TMQ_PF_PART && g.mode != TMQ_PF_QKVS && g.split != 1) return (int)hipErrorInvalidValue;
    if (g.gq_d && (g.mode != TMQ_PF_GU || !g.gq_tsum || !g.gq_xs || !g.gq_cnt || !g.gq_err || !g.max_bits))
        return (int)hipErrorInvalidValue;
    if (g.mode == TMQ_PF_GU) {
        // (the SwiGLU epilogue needs both blocks of a wave: no K groups)
        if (tile == 4 || g.gu_rows % (16 * nrb) || g.rows != 2 * g.gu_rows) return (int)hipErrorInvalidValue;
    } else if (g.rows % (32 * nrb)) {
        return (int)hipErrorInvalidValue;
    }
    if (g.mode == TMQ_PF_QKV || g.mode == TMQ_PF_QKVS)
        for (int i = 0; i < g.nseg; i++)
            if (g.seg[i].row0 % (32 * nrb) || (g.seg[i].q8 && !g.tpart)) return (int)hipErrorInvalidValue;
    if ((g.mode == TMQ_PF_PART || g.mode == TMQ_PF_QKVS) && !g.part) return (int)hipErrorInvalidValue;
    switch (g.mode) {
    case TMQ_PF_QKV: return launch_tile<TMQ_PF_QKV>(g, tile, s);
    case TMQ_PF_GU: return launch_tile<TMQ_PF_GU>(g, tile, s);
    case TMQ_PF_PART: return launch_tile<TMQ_PF_PART>(g, tile, s);
    case TMQ_PF_QKVS: return launch_tile<TMQ_PF_QKVS>(g, tile, s);
    }
    return (int)hipErrorInvalidValue;
}

namespace {
bool pf_prepared = false;
template <int NPASS>
int launch_attn(const TmqPfAttn& a, size_t lds, hipStream_t s) {
    if (!pf_prepared) {
        const int e = tmq_pf_prepare();
        if (e) return e;
    }
    hipLaunchKernelGGL((pf_attn_kernel<NPASS>), dim3(a.T, a.n_kv), dim3(512), lds, s, a);
    return (int)hipGetLastError();
}
}  // namespace

int tmq_pf_prepare() {
    if (pf_prepared) return 0;
    for (const void* f : {(const void*)pf_attn_kernel<1>, (const void*)pf_attn_kernel<2>,
                          (const void*)pf_attn_kernel<4>, (const void*)pf_attn_kernel<8>}) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, TMQ_PF_ATTN_LDS_MAX);
        if (e != hipSuccess) return (int)e;
    }
    // (and the GU occupancies the quantising epilogue's check reads)
    int nt = 0;
    for (int tile = 0; tile < 4; tile++) (void)tmq_pf_gu_quant_fits(tile, 128, 64, 1, &nt);
    pf_prepared = true;
    return 0;
}

int tmq_launch_pf_attn(const TmqPfAttn& a, hipStream_t s) {
    const int qpk = a.n_heads / a.n_kv, np = a.p0 + a.T;
    if (qpk < 1 || qpk > 8 || a.n_heads % a.n_kv || a.T < 1 || np > TMQ_PF_ATTN_MAXPOS)
        return (int)hipErrorInvalidValue;
    const size_t lds = tmq_pf_attn_lds(qpk, np);
    if (lds > TMQ_PF_ATTN_LDS_MAX) return (int)hipErrorInvalidValue;
    // registers for the scores of np positions (512 per pass).  Up to 512
    // positions four workgroups fit a CU (64 VGPRs, at most 80 SGPRs, LDS
    // under 40 KiB), and a launch of at most 4 x ncu workgroups is resident
    // at once: dealt in a snake.
    if (np <= 512) {
        TmqPfAttn b = a;
        b.deal = a.ncu > 0 && a.T * a.n_kv <= 4 * a.ncu && a.T * a.n_kv > a.ncu;
        return launch_attn<1>(b, lds, s);
    }
    if (np <= 1024) return launch_attn<2>(a, lds, s);
    if (np <= 2048) return launch_attn<4>(a, lds, s);
    return launch_attn<8>(a, lds, s);
}

int tmq_launch_pf_handoff(const TmqPfHandoff& h, hipStream_t s) {
    hipLaunchKernelGGL(pf_handoff_kernel, dim3(1), dim3(256), 0, s, h);
    return (int)hipGetLastError();
}

int tmq_launch_pf_qkv_fin(const TmqPfQkvFin& f, hipStream_t s) {
    // rows in groups of four inside one segment; split sums of whole rows
    if (f.H % 64 || f.KV % 64 || f.K % TMQ_PF_CHUNK || f.T < 1 || f.T > f.T_pad || f.split < 1 ||
        (f.seg[2].q8 && !f.tpart))
        return (int)hipErrorInvalidValue;
    const int nr = f.part ? f.H + (f.seg[2].q8 ? 1 : 2) * f.KV : 0;
    const int nA = f.T * (nr / 4), nB = f.seg[2].q8 ? f.T * f.KV : 0;
    const int nb = (nA + 255) / 256 + (nB + 255) / 256;
    if (nb == 0) return 0;
    hipLaunchKernelGGL(pf_qkv_fin_kernel, dim3(nb), dim3(256), 0, s, f);
    return (int)hipGetLastError();
}
