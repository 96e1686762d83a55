// Prefill products (M > 8) on the fp16 matrix cores over dequantized tiles: Y = deq(W) . deq(quant(X)), for Q8_0, Q5_K
// and Q6_K weights.
//
// The activations are quantized exactly as ggml-cpu quantizes src1 for the weight's vec_dot (Q8_0 blocks with the
// fp16-rounded d for Q8_0 weights; Q8_K blocks with their fp32 d for the K-quants) and written back as fp16(d * q);
// the weight tiles are dequantized in LDS to fp16(d * q) (Q6_K: fp16(d * sc * q), the exact fp32 product of ggml's
// dequantize_row_q6_K rounded once; Q5_K: fp16(d sc q - dmin m), dequantize_row_q5_K's fp32 value rounded once).
// The weight rounding is a single rounding of ggml's fp32 value, the activation one too for Q8_0 (Q8_K's fp32 d * q
// is rounded to fp32 first, as ggml forms it); relative error <= 2^-11 each. The products accumulate over all of K
// in fp32 inside the MFMA, so there is no per-block epilogue: the VALU work is the weight conversion, once per
// workgroup and element. Against ggml-cpu's per-block integer sums the row-relative error is a few 1e-4.
//
// Tiles: BM x BN per workgroup of WGM x WGN waves, each (BM / WGM) x (BN / WGN) as 32 x 32 v_mfma_f32_32x32x16_f16
// tiles. K advances in stages of 64. Every wave copies its share of each stage straight into LDS with
// global_load_lds, through rings of four stages (three ahead; Q8_0: three stages, two ahead): activations as fp16
// rows; weights as raw bytes (Q8_0: 64 codes and two block scales per row; Q6_K: the 64 ql and 32 qh bytes of the
// stage's half super-block, its four sub-block scales and d; Q5_K: the quarter's 32 qs bytes, the super-block's 32 qh
// bytes, its 12 scale bytes and d | dmin). K-quants: one stage ahead of the matrix cores the workgroup converts the
// stage's raw weights into an fp16 tile (double buffered). Q8_0: each wave converts its own B fragments in registers
// from the raw codes (16 codes per lane and chunk), so there is no fp16 weight tile and a 128 x 128 workgroup needs
// 76 KB: two of them share a CU and cover each other's barrier waits. One barrier per stage. LDS accesses in the loop
// are inline assembly with explicit waits: the compiler cannot see which stage a copy went to, and would otherwise
// wait for every copy in flight.
#include "mx_common.h"
#include "mx_device.h"
#include "mx_dot.h"
#include "mx_dq_act.h"

#include <algorithm>
#include <type_traits>
#include <cstdio>
#include <cstdlib>

namespace mx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

#ifndef MX_DQ_WGN128
#define MX_DQ_WGN128 4  // waves across N in a 128 x 128 tile (4: 64 x 32 per wave; 2: 64 x 64)
#endif
#ifndef MX_DQ_DIRECT_B
#define MX_DQ_DIRECT_B 1  // Q8_0: B fragments converted in registers from the raw codes (0: through an fp16 LDS tile)
#endif
#ifndef MX_DQ_DIRECT_B6
#define MX_DQ_DIRECT_B6 1  // Q6_K likewise, from the raw ql / qh bytes, scales and d (0: through an fp16 LDS tile)
#endif
#ifndef MX_DQ_DIRECT_B5
#define MX_DQ_DIRECT_B5 1  // Q5_K likewise, from the raw qs / qh bytes, scales and d | dmin
#endif
#ifndef MX_DQ_Q8_WGM128
#define MX_DQ_Q8_WGM128 1  // Q8_0 128 x 128 tiles: waves across M (1: four waves of 128 x 32; 2: eight of 64 x 32)
#endif
#ifndef MX_DQ_HALF
#define MX_DQ_HALF 1  // Q8_0 128 x 32 waves: the second half of a stage's A reads overlaps the first half's MFMAs
#endif
constexpr int DQ_KS = 64;  // K per stage
#ifndef MX_DQ_SKINNY_WG
// workgroups the 32 x 128 tile aims for, splitting K (M = 28, N = 2048, K = 6144: 16 splits 17.5 us, 24 splits 19.8;
// the K = 2048 products of the same block move by under 1 % between 256 and 512)
#define MX_DQ_SKINNY_WG 256
#endif
#ifndef MX_DQ_NS_DIRB
#define MX_DQ_NS_DIRB 3  // ring stages of the direct-B (Q8_0) tiles: 76 KB at 128 x 128, two workgroups per CU
#endif

// LDS map of a BM x BN workgroup of NW waves. Row-major fp16 tiles of 64 halves (128 bytes) per row; the 16-byte
// chunk c of row r sits at chunk c ^ ((r ^ (r >> 3)) & 7): any 8 consecutive rows an MFMA fragment read touches use 8
// different chunks (all 32 banks of a 128-byte cycle), and 16 consecutive rows cover all 64 banks of a 256-byte one.
template <int WT, int BM, int BN, int NW, bool RT = false>
struct DqLds {
    static constexpr bool K6 = WT == MX_TYPE_Q6_K, K5 = WT == MX_TYPE_Q5_K;
    // Q8_0 and Q6_K with direct B: each wave converts its B fragments from the raw bytes, so there is no fp16 weight
    // tile
    static constexpr bool DIRB = (MX_DQ_DIRECT_B && !K6 && !K5) || (MX_DQ_DIRECT_B6 && K6) || (MX_DQ_DIRECT_B5 && K5);
    // ring stages: the copies run NS - 1 stages ahead of the matrix cores
    static constexpr int NS = DIRB ? MX_DQ_NS_DIRB : 4;
    // Direct B: bytes that several consecutive stages read alike take a two-slot ring of their own, indexed by
    // g / SHP and copied once per SHP stages (g: the stage along the whole of K). Q6_K: quarters 2 j and 2 j + 1 of a
    // super-block read the same ql and qh bytes (low and high nibbles, qh bit pairs 0-3 and 4-7) and d pair (SHP 2);
    // Q5_K: its four quarters read the super-block's qh, 12 scale bytes and d | dmin (SHP 4). The rest (activations,
    // Q6_K scales, Q5_K qs) keeps the NS-stage ring.
    static constexpr bool SH_RAW = DIRB && K6, SH_QH = DIRB && (K6 || K5), SH_SC = DIRB && K5,
                          SH_DD = DIRB && (K6 || K5), SHARED = SH_RAW || SH_QH || SH_SC || SH_DD;
    static constexpr int SHP = K6 ? 2 : 4;
    static constexpr int N_RAW = SH_RAW ? 2 : NS, N_QH = SH_QH ? 2 : NS, N_SC = SH_SC ? 2 : NS, N_DD = SH_DD ? 2 : NS;
    // raw bytes per weight row and stage: codes (Q8_0 codes, Q6_K ql, Q5_K qs), qh, scales, d
    static constexpr int RB = K5 ? 32 : 64, HB = K6 || K5 ? 32 : 0, SB = K5 ? 12 : 4, DB = K6 || K5 ? 4 : 0;
    static constexpr int A = 0;                            // [stage][BM][128 B] activations
    static constexpr int BH = A + NS * BM * 128;        // [2][BN][128 B] dequantized weights
    static constexpr int RAW = BH + (DIRB ? 0 : 2 * BN * 128);  // [stage][BN][RB] codes
    static constexpr int QH = RAW + N_RAW * BN * RB;    // [slot][BN][HB] qh bytes
    static constexpr int SC = QH + N_QH * BN * HB;      // [slot][BN][SB] scales (Q8_0 two fp16, Q6_K four int8,
                                                           // Q5_K the 12 packed bytes)
    static constexpr int DD = SC + N_SC * BN * SB;      // [slot][BN][DB] Q6_K: the fp16 d pair holding the row's;
                                                           // Q5_K: d | dmin
    // copy instructions per stage (64 lanes each): activation rows (16 B), code rows (16 B), qh rows (16 B), scale
    // words (4 B), d words (4 B), and per wave
    static constexpr int NA = BM / 8, NC = BN * RB / 1024, NH = BN * HB / 1024, NS4 = BN * SB / 256,
                         ND = BN * DB / 256;
    static constexpr int PA = (NA + NW - 1) / NW, PC = (NC + NW - 1) / NW, PH = (NH + NW - 1) / NW;
    static constexpr int PS = (NS4 + NW - 1) / NW, PD = (ND + NW - 1) / NW;
    static constexpr int OPS = PA + PC + PH + PS + PD;  // vector memory ops per wave and stage
    // ... of a stage whose shared bytes an earlier stage brought
    static constexpr int OPS1 = PA + (SH_RAW ? 0 : PC) + (SH_QH ? 0 : PH) + (SH_SC ? 0 : PS) + (SH_DD ? 0 : PD);
    // junk bytes per wave: the largest copy instruction some wave issues beyond the tile's need
    static constexpr int JB = PA * NW > NA || PC * NW > NC || PH * NW > NH ? 1024
                              : PS * NW > NS4 || PD * NW > ND            ? 256
                                                                         : 0;
    static constexpr int JUNK = DD + N_DD * BN * DB;    // [wave][JB] where copies beyond a tile's need land
    static constexpr int RS = JUNK + NW * JB;           // [BM] the tile rows' 2^-e
    static constexpr int YO = RS + BM * 4;              // routed experts: [BM] each tile row's output offset (floats)
    static constexpr int SIZE = YO + (RT ? BM * 8 : 0);
    static_assert(SIZE <= 160 * 1024, "LDS");
};

__device__ __forceinline__ int dq_swz(int row) { return (row ^ (row >> 3)) & 7; }

struct DqProblem {
    WPlanes w;
    int N;
    float *y;
    int64_t ldy;  // floats between consecutive m rows of y
};
struct DqArgs {
    DqProblem prob[4];
    int M, K;
    const _Float16 *xh;  // [M][K] fp16(2^e_m d q) of the quantized activations
    const float *rs;     // [M] 2^-e_m, applied to each row's sums
    int nprob, nsplit;   // dense: grid.x runs over the splits' tiles (below); routed: grid.z = nprob
    int ntot;            // sum of the problems' N: columns of the split partials
    int col0[4];         // first partial column of each problem
    float *ws;           // nsplit > 1: [nsplit][M][ntot] partial sums, added in split order by k_dq_reduce
    // Routed experts (MUL_MAT_ID; the kernel's RT form, one split): grid.y runs over chunks of one expert's (token,
    // slot) pairs -- tiles[3 c] the chunk's first index into pairs, tiles[3 c + 1] its count (<= BM), tiles[3 c + 2]
    // the expert, ntiles[0] the chunks there are. Row i of a chunk is pair p = pairs[first + i] = t n_ids + s: its
    // activation row is xh row t b_ne1 + s % b_ne1, its weights rows expert N .. of each problem's planes, its output
    // row y + s y_nb1 + t y_nb2 (floats).
    const int32_t *tiles, *ntiles, *pairs;
    int n_ids, b_ne1;
    int64_t y_nb1, y_nb2;
};


constexpr int DQ_ACT_NT = 1024;  // threads of an activation-pass workgroup (one row)

// Activation row m (one workgroup) -> Q8_0 blocks -> fp16(2^e d q) (mx_dq_act.h).
__global__ __launch_bounds__(DQ_ACT_NT) void k_dq_act_q8_0(const float *x, int64_t x_stride, int K, int rounding,
                                                            _Float16 *xh, float *rs) {
    __shared__ float red[DQ_ACT_NT / 64];
    const int64_t m = blockIdx.x;
    dq_act_row_q8_0<DQ_ACT_NT>(x + m * x_stride, K, rounding, xh + m * K, rs + m, red);
}

// Activation row m -> Q8_K blocks (the pairing of Q5_K / Q6_K weights) -> fp16(2^e fp32(d q)) (mx_dq_act.h).
__global__ __launch_bounds__(DQ_ACT_NT) void k_dq_act_q8k(const float *x, int64_t x_stride, int K, _Float16 *xh,
                                                           float *rs) {
    __shared__ float red[DQ_ACT_NT / 64];
    const int64_t m = blockIdx.x;
    dq_act_row_q8k<DQ_ACT_NT>(x + m * x_stride, K, xh + m * K, rs + m, red);
}

// Four signed bytes -> four exact fp16 values: (0x64 << 8 | (b ^ 0x80)) is the fp16 of 1152 + b, and 1152 is
// subtracted exactly.
__device__ __forceinline__ void dq_i8x4(uint32_t w, v2h &lo, v2h &hi) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const v2h off = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(v2h, p0) - off;
    hi = __builtin_bit_cast(v2h, p1) - off;
}

// 16 codes of one Q8_0 block times its fp16 d: two 16-byte chunks of fp16(d * q) (one rounding of an exact product).
__device__ __forceinline__ void dq_q8_0_16(v4i c, uint16_t dbits, v4i &o0, v4i &o1) {
    _Float16 d;
    __builtin_memcpy(&d, &dbits, 2);
    const v2h dd = {d, d};
    v2h h[8];
    dq_i8x4((uint32_t)c.x, h[0], h[1]);
    dq_i8x4((uint32_t)c.y, h[2], h[3]);
    dq_i8x4((uint32_t)c.z, h[4], h[5]);
    dq_i8x4((uint32_t)c.w, h[6], h[7]);
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = h[i] * dd;
    o0 = v4i{__builtin_bit_cast(int, h[0]), __builtin_bit_cast(int, h[1]), __builtin_bit_cast(int, h[2]),
             __builtin_bit_cast(int, h[3])};
    o1 = v4i{__builtin_bit_cast(int, h[4]), __builtin_bit_cast(int, h[5]), __builtin_bit_cast(int, h[6]),
             __builtin_bit_cast(int, h[7])};
}

// 16 Q6_K codes of one sub-block: code t = ((ql_t >> ls) & 15) | (((qh_t >> hs) & 3) << 4), value code - 32, times
// d * sc (exact in fp32: 11 + 8 bits) -- (code - 32) * d * sc is exact in fp32 too (<= 24 bits), formed by one fma, and
// rounded once to fp16.
__device__ __forceinline__ void dq_q6_k_16(v4i ql, v4i qh, int hs, int ls, int sc, uint16_t dbits, v4i &o0, v4i &o1) {
    _Float16 dh;
    __builtin_memcpy(&dh, &dbits, 2);
    const float ds = (float)dh * (float)sc, off = -32.0f * ds;
    const uint32_t lw[4] = {(uint32_t)ql.x, (uint32_t)ql.y, (uint32_t)ql.z, (uint32_t)ql.w};
    const uint32_t hw[4] = {(uint32_t)qh.x, (uint32_t)qh.y, (uint32_t)qh.z, (uint32_t)qh.w};
    int r[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t c = ((lw[k] >> ls) & 0x0F0F0F0Fu) | (((hw[k] >> hs) & 0x03030303u) << 4);
        v2h lo, hi;
        lo.x = (_Float16)fmaf((float)(c & 0xFF), ds, off);
        lo.y = (_Float16)fmaf((float)((c >> 8) & 0xFF), ds, off);
        hi.x = (_Float16)fmaf((float)((c >> 16) & 0xFF), ds, off);
        hi.y = (_Float16)fmaf((float)(c >> 24), ds, off);
        r[2 * k] = __builtin_bit_cast(int, lo);
        r[2 * k + 1] = __builtin_bit_cast(int, hi);
    }
    o0 = v4i{r[0], r[1], r[2], r[3]};
    o1 = v4i{r[4], r[5], r[6], r[7]};
}

// 16 Q5_K codes of sub-block `sub`: code t = ((qs_t >> ls) & 15) | (((qh_t >> sub) & 1) << 4), value
// d sc code - dmin m as ggml's dequantize_row_q5_K forms it in fp32 (d sc code and dmin m are exact products, one
// rounding in the difference), then rounded once to fp16.
__device__ __forceinline__ void dq_q5_k_16(v4i qs, v4i qh, int sub, int ls, int sc, int m, uint32_t dm, v4i &o0,
                                           v4i &o1) {
    const float d1 = h2f((uint16_t)(dm & 0xFFFF)) * (float)sc, m1 = h2f((uint16_t)(dm >> 16)) * (float)m;
    const uint32_t lw[4] = {(uint32_t)qs.x, (uint32_t)qs.y, (uint32_t)qs.z, (uint32_t)qs.w};
    const uint32_t hw[4] = {(uint32_t)qh.x, (uint32_t)qh.y, (uint32_t)qh.z, (uint32_t)qh.w};
    int r[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t c = ((lw[k] >> ls) & 0x0F0F0F0Fu) | (((hw[k] >> sub) & 0x01010101u) << 4);
        v2h lo, hi;
        lo.x = (_Float16)(d1 * (float)(c & 0xFF) - m1);
        lo.y = (_Float16)(d1 * (float)((c >> 8) & 0xFF) - m1);
        hi.x = (_Float16)(d1 * (float)((c >> 16) & 0xFF) - m1);
        hi.y = (_Float16)(d1 * (float)(c >> 24) - m1);
        r[2 * k] = __builtin_bit_cast(int, lo);
        r[2 * k + 1] = __builtin_bit_cast(int, hi);
    }
    o0 = v4i{r[0], r[1], r[2], r[3]};
    o1 = v4i{r[4], r[5], r[6], r[7]};
}

// NF fragment reads (4, 6, 8, 12 or 16) and the wait for them.
template <int NF>
__device__ __forceinline__ void dq_read(v8h (&f)[16], const uint32_t (&a)[16]) {
    if constexpr (NF == 16) {
        asm volatile(
            "ds_read_b128 %0, %16\n"
            "ds_read_b128 %1, %17\n"
            "ds_read_b128 %2, %18\n"
            "ds_read_b128 %3, %19\n"
            "ds_read_b128 %4, %20\n"
            "ds_read_b128 %5, %21\n"
            "ds_read_b128 %6, %22\n"
            "ds_read_b128 %7, %23\n"
            "ds_read_b128 %8, %24\n"
            "ds_read_b128 %9, %25\n"
            "ds_read_b128 %10, %26\n"
            "ds_read_b128 %11, %27\n"
            "ds_read_b128 %12, %28\n"
            "ds_read_b128 %13, %29\n"
            "ds_read_b128 %14, %30\n"
            "ds_read_b128 %15, %31\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]), "=&v"(f[7]),
              "=&v"(f[8]), "=&v"(f[9]), "=&v"(f[10]), "=&v"(f[11]), "=&v"(f[12]), "=&v"(f[13]), "=&v"(f[14]),
              "=&v"(f[15])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]), "v"(a[8]),
              "v"(a[9]), "v"(a[10]), "v"(a[11]), "v"(a[12]), "v"(a[13]), "v"(a[14]), "v"(a[15])
            : "memory");
    } else if constexpr (NF == 8) {
        asm volatile(
            "ds_read_b128 %0, %8\n"
            "ds_read_b128 %1, %9\n"
            "ds_read_b128 %2, %10\n"
            "ds_read_b128 %3, %11\n"
            "ds_read_b128 %4, %12\n"
            "ds_read_b128 %5, %13\n"
            "ds_read_b128 %6, %14\n"
            "ds_read_b128 %7, %15\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]), "=&v"(f[7])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7])
            : "memory");
    } else if constexpr (NF == 12) {
        asm volatile(
            "ds_read_b128 %0, %12\n"
            "ds_read_b128 %1, %13\n"
            "ds_read_b128 %2, %14\n"
            "ds_read_b128 %3, %15\n"
            "ds_read_b128 %4, %16\n"
            "ds_read_b128 %5, %17\n"
            "ds_read_b128 %6, %18\n"
            "ds_read_b128 %7, %19\n"
            "ds_read_b128 %8, %20\n"
            "ds_read_b128 %9, %21\n"
            "ds_read_b128 %10, %22\n"
            "ds_read_b128 %11, %23\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]), "=&v"(f[7]),
              "=&v"(f[8]), "=&v"(f[9]), "=&v"(f[10]), "=&v"(f[11])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]), "v"(a[8]),
              "v"(a[9]), "v"(a[10]), "v"(a[11])
            : "memory");
    } else if constexpr (NF == 6) {
        asm volatile(
            "ds_read_b128 %0, %6\n"
            "ds_read_b128 %1, %7\n"
            "ds_read_b128 %2, %8\n"
            "ds_read_b128 %3, %9\n"
            "ds_read_b128 %4, %10\n"
            "ds_read_b128 %5, %11\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5])
            : "memory");
    } else {
        static_assert(NF == 4, "4, 6, 8 or 12 fragments");
        asm volatile(
            "ds_read_b128 %0, %4\n"
            "ds_read_b128 %1, %5\n"
            "ds_read_b128 %2, %6\n"
            "ds_read_b128 %3, %7\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
            : "memory");
    }
}

// Direct B (Q8_0, one 32-column B tile per wave): the wave's 4 TM A fragments, its two 16-byte raw code chunks and
// its row's scale word, and the wait for them.
template <int TM>
__device__ __forceinline__ void dq_read_ab(v8h (&f)[8], v4i (&b)[2], uint32_t &sw, const uint32_t (&a)[8],
                                           uint32_t b0, uint32_t b1, uint32_t sc) {
    if constexpr (TM == 2) {
        asm volatile(
            "ds_read_b128 %8, %11\n"
            "ds_read_b128 %9, %12\n"
            "ds_read_b32 %10, %13\n"
            "ds_read_b128 %0, %14\n"
            "ds_read_b128 %1, %15\n"
            "ds_read_b128 %2, %16\n"
            "ds_read_b128 %3, %17\n"
            "ds_read_b128 %4, %18\n"
            "ds_read_b128 %5, %19\n"
            "ds_read_b128 %6, %20\n"
            "ds_read_b128 %7, %21\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]), "=&v"(f[7]),
              "=&v"(b[0]), "=&v"(b[1]), "=&v"(sw)
            : "v"(b0), "v"(b1), "v"(sc), "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]),
              "v"(a[7])
            : "memory");
    } else {
        static_assert(TM == 1, "wave tiles of 32 or 64 rows");
        asm volatile(
            "ds_read_b128 %4, %7\n"
            "ds_read_b128 %5, %8\n"
            "ds_read_b32 %6, %9\n"
            "ds_read_b128 %0, %10\n"
            "ds_read_b128 %1, %11\n"
            "ds_read_b128 %2, %12\n"
            "ds_read_b128 %3, %13\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(b[0]), "=&v"(b[1]), "=&v"(sw)
            : "v"(b0), "v"(b1), "v"(sc), "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
            : "memory");
    }
}

// Eight fragment reads without their wait, and the wait: dq_wait8's operands tie the registers to it, so that nothing
// reads them before the data has landed.
__device__ __forceinline__ void dq_issue8(v8h (&f)[16], const uint32_t (&a)[8]) {
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %9\n"
        "ds_read_b128 %2, %10\n"
        "ds_read_b128 %3, %11\n"
        "ds_read_b128 %4, %12\n"
        "ds_read_b128 %5, %13\n"
        "ds_read_b128 %6, %14\n"
        "ds_read_b128 %7, %15"
        : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]), "=&v"(f[7])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7])
        : "memory");
}
__device__ __forceinline__ void dq_wait8(v8h (&f)[16]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7])
                 :
                 : "memory");
}

template <int WT, int BM, int BN, int WGM, int WGN, bool RT>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm_dq(DqArgs a) {
    constexpr int NW = WGM * WGN, NT = 64 * NW;
    using L = DqLds<WT, BM, BN, NW, RT>;
    constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
    constexpr int NF = (TM + TN) * 4;  // fragments of the stage's four K steps, read together
    static_assert(L::DIRB ? TN == 1 && (TM == 1 || TM == 2 || TM == 4) : NF == 8 || NF == 12 || NF == 16,
                  "wave tiles of 32 x 32, 64 x 32 or 64 x 64; direct B: 32, 64 or 128 x 32");
    extern __shared__ __align__(16) uint8_t smem[];
    // Dense: grid.x runs over split after split, each the problems' tiles problem after problem, (N_p / BN) x (M / BM)
    // with n fastest; no workgroup of a narrower problem's missing columns is launched (a grid of the widest problem's
    // width per problem launched those, and the launch ran as if it had that many more workgroups). Routed: grid.x the
    // column tiles, grid.y the chunks, grid.z the problems.
    int pi = 0, split = 0, n0, m0 = 0;
    if constexpr (RT) {
        pi = blockIdx.z % a.nprob;  // (one split)
        split = blockIdx.z / a.nprob;
        n0 = blockIdx.x * BN;
    } else {
        const int MT = (a.M + BM - 1) / BM;
        int per = 0;  // tiles of one split
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (i < a.nprob) per += (a.prob[i].N + BN - 1) / BN * MT;
        int t = blockIdx.x;
        split = t / per;
        t -= split * per;
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int ti = (a.prob[i].N + BN - 1) / BN * MT;
            if (pi == i && i + 1 < a.nprob && t >= ti) {
                t -= ti;
                pi = i + 1;
            }
        }
        const int Np = pi == 0 ? a.prob[0].N : (pi == 1 ? a.prob[1].N : (pi == 2 ? a.prob[2].N : a.prob[3].N));
        const int ntp = (Np + BN - 1) / BN;
        n0 = (t % ntp) * BN;
        m0 = (t / ntp) * BM;
    }
    const DqProblem p = pi == 0 ? a.prob[0] : (pi == 1 ? a.prob[1] : (pi == 2 ? a.prob[2] : a.prob[3]));
    if (n0 >= p.N) return;  // routed: uniform, a problem narrower than the grid
    const int M = a.M, N = p.N, K = a.K, nblk = K / 32;
    int mrows = 0, first = 0;  // routed: the chunk's pairs and its first index into pairs
    int64_t wrow0 = 0;         // routed: the expert's first row in the weight planes
    if constexpr (RT) {
        const int c = blockIdx.y;
        if (c >= a.ntiles[0]) return;  // uniform: past the chunks the bucketing wrote
        first = a.tiles[3 * c];
        mrows = a.tiles[3 * c + 1];
        wrow0 = (int64_t)a.tiles[3 * c + 2] * N;
    }
    // the (token, slot) pair of routed tile row i, clamped to the chunk's last (the lambdas capture plain values: a
    // reference to the argument block would move it to private memory)
    const int32_t *pairs = a.pairs;
    const int n_ids = a.n_ids, b_ne1 = a.b_ne1;
    auto pair_of = [=](int i, int &t, int &s) {
        const int pr = pairs[first + min(i, mrows - 1)];
        t = pr / n_ids;
        s = pr - t * n_ids;
    };
    // the activation row of tile row i, clamped to the tile's (routed: the chunk's) last
    auto arow = [=](int i) -> int64_t {
        if constexpr (RT) {
            int t, s;
            pair_of(i, t, s);
            return (int64_t)t * b_ne1 + s % b_ne1;
        } else {
            return min(m0 + i, M - 1);
        }
    };
    // this workgroup's stages: [sb, sb + nst) of K / 64 (the host makes every split non-empty)
    const int per = (K / DQ_KS + a.nsplit - 1) / a.nsplit, sb = split * per;
    const int nst = min(K / DQ_KS - sb, per);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lds = lds_addr(smem);

    // Copy sources of this lane (row bases; issue adds the stage's offset) and LDS destinations (stage 0; a stage adds
    // its slot). Instruction j of a kind is issued by wave j / P (its jj = j % P); instructions past the tile's need
    // copy a valid row again into the wave's junk area.
    //   activations: instruction j covers rows 8 j .. 8 j + 7; lane i brings logical chunk (i & 7) ^ swz(row)
    //   codes / ql: instruction j covers rows 16 j .. 16 j + 15; lane i brings bytes 16 (i & 3) .. of its row
    //   qh: instruction j covers rows 32 j .. 32 j + 31; lane i brings bytes 16 (i & 1) .. of its row
    //   scales, d: instruction j covers rows 64 j .. 64 j + 63; lane i brings its row's four bytes
    const int nsb = K / 256;  // Q6_K super-blocks per row
    const _Float16 *asrc[L::PA];
    uint32_t adst[L::PA];
#pragma unroll
    for (int jj = 0; jj < L::PA; jj++) {
        const int j = wave * L::PA + jj, row = 8 * min(j, L::NA - 1) + (lane >> 3);
        asrc[jj] = a.xh + arow(row) * K + sb * DQ_KS + 8 * ((lane & 7) ^ dq_swz(row));
        adst[jj] = j < L::NA ? L::A + j * 1024 : L::JUNK + wave * L::JB;
    }
    const uint8_t *csrc[L::PC];
    uint32_t cdst[L::PC];
#pragma unroll
    for (int jj = 0; jj < L::PC; jj++) {
        constexpr int LR = L::RB / 16;  // lanes per code row
        const int j = wave * L::PC + jj, row = (64 / LR) * min(j, L::NC - 1) + lane / LR;
        const int64_t grow = wrow0 + min(n0 + row, N - 1);
        // direct B: row r's chunk c lands at chunk c ^ ((r >> 2) & 3) (64-byte rows; 32-byte Q5_K rows: c ^ ((r >> 3)
        // & 1)), so the 16 rows a fragment read's lane group touches cover all 64 banks
        const int cc = !L::DIRB ? lane % LR : L::RB == 64 ? (lane % LR) ^ ((row >> 2) & 3) : (lane % LR) ^ ((row >> 3) & 1);
        csrc[jj] = (L::K6 || L::K5 ? p.w.p0 + grow * nsb * 128 : p.w.p0 + grow * K + sb * DQ_KS) + 16 * cc;
        cdst[jj] = j < L::NC ? L::RAW + j * 1024 : L::JUNK + wave * L::JB;
    }
    const uint8_t *hsrc[L::PH > 0 ? L::PH : 1];
    uint32_t hdst[L::PH > 0 ? L::PH : 1];
#pragma unroll
    for (int jj = 0; jj < L::PH; jj++) {
        const int j = wave * L::PH + jj, row = 32 * min(j, L::NH - 1) + (lane >> 1);
        // direct B: row r's qh chunk c lands at chunk c ^ ((r >> 3) & 1), so the 16 rows of a read's lane group
        // cover all 64 banks
        const int hc = L::DIRB ? (lane & 1) ^ ((row >> 3) & 1) : lane & 1;
        hsrc[jj] = p.w.p1 + (wrow0 + min(n0 + row, N - 1)) * nsb * (L::K5 ? 32 : 64) + 16 * hc;
        hdst[jj] = j < L::NH ? L::QH + j * 1024 : L::JUNK + wave * L::JB;
    }
    const uint8_t *ssrc[L::PS];
    uint32_t sdst[L::PS];
#pragma unroll
    for (int jj = 0; jj < L::PS; jj++) {
        const int j = wave * L::PS + jj, wd = 64 * min(j, L::NS4 - 1) + lane;  // scale word wd of the stage
        if constexpr (L::K5) {  // word c of row wd / 3's 12 bytes
            const int64_t grow = wrow0 + min(n0 + wd / 3, N - 1);
            ssrc[jj] = p.w.p2 + grow * nsb * 12 + 4 * (wd % 3);
        } else {
            const int64_t grow = wrow0 + min(n0 + wd, N - 1);
            ssrc[jj] = L::K6 ? p.w.p2 + grow * nsb * 16 : p.w.p1 + grow * nblk * 2 + sb * 4;
        }
        sdst[jj] = j < L::NS4 ? L::SC + j * 256 : L::JUNK + wave * L::JB;
    }
    int64_t dsb[L::PD > 0 ? L::PD : 1];  // the row's first super-block index in the d plane
    uint32_t ddst[L::PD > 0 ? L::PD : 1];
#pragma unroll
    for (int jj = 0; jj < L::PD; jj++) {
        const int j = wave * L::PD + jj, row = 64 * min(j, L::ND - 1) + lane;
        dsb[jj] = (wrow0 + min(n0 + row, N - 1)) * nsb;
        ddst[jj] = j < L::ND ? L::DD + j * 256 : L::JUNK + wave * L::JB;
    }

    // Returns whether stage t's shared bytes were copied too (the workgroup's first stage and every stage with
    // g % SHP == 0 copy them; with nothing shared, always).
    auto issue = [&](int t) -> bool {
        t = min(t, nst - 1);  // past the end: copy the last stage again into its own slot (identical bytes)
        const int slot = t % L::NS, g = sb + t;  // g: the stage's index along the whole of K
        const bool sh = !L::SHARED || t == 0 || g % L::SHP == 0;
        const int hslot = (g / L::SHP) & 1;
        const int rslot = L::SH_RAW ? hslot : slot, qslot = L::SH_QH ? hslot : slot, sslot = L::SH_SC ? hslot : slot,
                  dslot = L::SH_DD ? hslot : slot;
#pragma unroll
        for (int jj = 0; jj < L::PA; jj++) {
            const uint32_t d = adst[jj] + (adst[jj] < (uint32_t)L::JUNK ? slot * BM * 128 : 0);
            __builtin_amdgcn_global_load_lds((const void *)(asrc[jj] + t * DQ_KS), (lds_void *)(smem + d), 16, 0, 0);
        }
        // K-quants: stage g is quarter g & 3 of super-block g >> 2. Q6_K: both quarters of a half read the half's ql
        // and qh; Q5_K: the quarter's 32 qs bytes and the super-block's 32 qh bytes
        const int coff = L::K6   ? (g >> 2) * 128 + ((g >> 1) & 1) * 64
                         : L::K5 ? (g >> 2) * 128 + (g & 3) * 32
                                 : t * DQ_KS;
        if (!L::SH_RAW || sh) {
#pragma unroll
            for (int jj = 0; jj < L::PC; jj++) {
                const uint32_t d = cdst[jj] + (cdst[jj] < (uint32_t)L::JUNK ? rslot * BN * L::RB : 0);
                __builtin_amdgcn_global_load_lds((const void *)(csrc[jj] + coff), (lds_void *)(smem + d), 16, 0, 0);
            }
        }
        if (!L::SH_QH || sh) {
#pragma unroll
            for (int jj = 0; jj < L::PH; jj++) {
                const uint32_t d = hdst[jj] + (hdst[jj] < (uint32_t)L::JUNK ? qslot * BN * L::HB : 0);
                const int hoff = L::K5 ? (g >> 2) * 32 : (g >> 2) * 64 + ((g >> 1) & 1) * 32;
                __builtin_amdgcn_global_load_lds((const void *)(hsrc[jj] + hoff), (lds_void *)(smem + d), 16, 0, 0);
            }
        }
        const int soff = L::K6 ? (g >> 2) * 16 + (g & 3) * 4 : L::K5 ? (g >> 2) * 12 : t * 4;
        if (!L::SH_SC || sh) {
#pragma unroll
            for (int jj = 0; jj < L::PS; jj++) {
                const uint32_t d = sdst[jj] + (sdst[jj] < (uint32_t)L::JUNK ? sslot * BN * L::SB : 0);
                __builtin_amdgcn_global_load_lds((const void *)(ssrc[jj] + soff), (lds_void *)(smem + d), 4, 0, 0);
            }
        }
        // d: the 4-byte-aligned pair of fp16 d holding this row's (which half: convert). When the plane holds an odd
        // number of d, the last pair runs 2 bytes past them -- inside the plane's padding to 256 bytes, which an odd
        // count of 2-byte values never fills exactly.
        if (!L::SH_DD || sh) {
#pragma unroll
            for (int jj = 0; jj < L::PD; jj++) {
                const uint32_t d = ddst[jj] + (ddst[jj] < (uint32_t)L::JUNK ? dslot * BN * 4 : 0);
                const int64_t e = dsb[jj] + (g >> 2);
                const uint8_t *src = L::K5 ? p.w.p3 + e * 4 : p.w.p3 + (e >> 1) * 4;
                __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(smem + d), 4, 0, 0);
            }
        }
        return sh;
    };

    // Conversion of stage t's raw weights into fp16 tile buffer t & 1, in units of 16 codes: unit u is quarter u & 3
    // of row u >> 2.
    auto convert = [&](int t) {
        const int slot = t % L::NS, g = sb + t;
#pragma unroll
        for (int u = tid; u < BN * 4; u += NT) {
            const int row = u >> 2, q = u & 3;
            const uint32_t raw = lds + L::RAW + slot * BN * L::RB + row * L::RB + 16 * (L::K5 ? (q & 1) : q);
            const uint32_t sc = lds + L::SC + slot * BN * L::SB + row * L::SB;
            v4i o[2];
            if constexpr (L::K5) {  // Q5_K: sub-block 2 (g & 3) + (q >> 1): codes 16 (q & 1) .. of its 32
                const uint32_t qh = lds + L::QH + slot * BN * 32 + row * 32 + 16 * (q & 1);
                const uint32_t dd = lds + L::DD + slot * BN * 4 + row * 4;
                v4i l0, h0;
                uint32_t s0, s1, s2, dw;
                asm volatile(
                    "ds_read_b128 %0, %6\n"
                    "ds_read_b128 %1, %7\n"
                    "ds_read_b32 %2, %8\n"
                    "ds_read_b32 %3, %8 offset:4\n"
                    "ds_read_b32 %4, %8 offset:8\n"
                    "ds_read_b32 %5, %9\n"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(l0), "=&v"(h0), "=&v"(s0), "=&v"(s1), "=&v"(s2), "=&v"(dw)
                    : "v"(raw), "v"(qh), "v"(sc), "v"(dd)
                    : "memory");
                const int sub = 2 * (g & 3) + (q >> 1);
                int scv, mv;
                q4k_scale_min(s0, s1, s2, sub, scv, mv);
                dq_q5_k_16(l0, h0, sub, 4 * (q >> 1), scv, mv, dw, o[0], o[1]);
            } else if constexpr (!L::K6) {  // Q8_0: quarter q is half of block q >> 1
                v4i c0;
                uint32_t sw;
                asm volatile(
                    "ds_read_b128 %0, %2\n"
                    "ds_read_b32 %1, %3\n"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(c0), "=&v"(sw)
                    : "v"(raw), "v"(sc)
                    : "memory");
                dq_q8_0_16(c0, (uint16_t)((q >> 1) ? sw >> 16 : sw & 0xFFFF), o[0], o[1]);
            } else {  // Q6_K: sub-block 4 (g & 3) + q of the super-block
                const uint32_t qh = lds + L::QH + slot * BN * 32 + row * 32 + 16 * (q & 1);
                const uint32_t dd = lds + L::DD + slot * BN * 4 + row * 4;
                v4i l0, h0;
                uint32_t sw, dw;
                asm volatile(
                    "ds_read_b128 %0, %4\n"
                    "ds_read_b128 %1, %5\n"
                    "ds_read_b32 %2, %6\n"
                    "ds_read_b32 %3, %7\n"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(l0), "=&v"(h0), "=&v"(sw), "=&v"(dw)
                    : "v"(raw), "v"(qh), "v"(sc), "v"(dd)
                    : "memory");
                const int64_t e = (wrow0 + min(n0 + row, N - 1)) * nsb + (g >> 2);
                dq_q6_k_16(l0, h0, (g & 1) * 4 + (q >> 1) * 2, (g & 1) * 4, (int8_t)(sw >> (8 * q)),
                           (uint16_t)((e & 1) ? dw >> 16 : dw & 0xFFFF), o[0], o[1]);
            }
            const uint32_t out = lds + L::BH + (t & 1) * BN * 128 + row * 128;
#pragma unroll
            for (int i = 0; i < 2; i++)
                asm volatile("ds_write_b128 %0, %1" ::"v"(out + 16 * ((2 * q + i) ^ dq_swz(row))), "v"(o[i])
                             : "memory");
        }
    };

    const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;
    const int fr = lane & 31, fh = lane >> 5;
    // fragment offsets within a tile: row base plus the swizzled chunk of K step kk: chunk 2 kk + fh; with direct B,
    // chunk 4 (kk >> 1) + 2 fh + (kk & 1), the halves of the 16 codes 16 (2 (kk >> 1) + fh) .. a lane converts at once
    // (any assignment of K to the MFMA's k slots serves, as long as A and B share it)
    uint32_t aoff[TM][4], boff[TN][4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int row = wm + 32 * i + fr, c = L::DIRB ? 4 * (kk >> 1) + 2 * fh + (kk & 1) : 2 * kk + fh;
            aoff[i][kk] = row * 128 + 16 * (c ^ dq_swz(row));
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int row = wn + 32 * j + fr;
            boff[j][kk] = row * 128 + 16 * ((2 * kk + fh) ^ dq_swz(row));
        }
    }
    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // the tile rows' 2^-e (routed: and output offsets), requested ahead of the copies
    float rs_row;
    int64_t yo_row = 0;
    if constexpr (RT) {
        int t, s;
        pair_of(tid < BM ? tid : 0, t, s);
        rs_row = a.rs[(int64_t)t * b_ne1 + s % b_ne1];
        yo_row = s * a.y_nb1 + t * a.y_nb2;
    } else {
        rs_row = a.rs[min(m0 + (tid < BM ? tid : 0), M - 1)];
    }
    bool plast = true;  // whether the latest issue copied the shared bytes too (the ops a stage's wait leaves in flight)
#pragma unroll
    for (int t = 0; t < L::NS - 1; t++) plast = issue(t);
    if constexpr (!L::DIRB) {
        wait_vm<(L::NS - 2) * L::OPS>();  // stage 0 landed (this wave's copies)
        if (tid < BM) {  // read by the epilogue
            *(float *)(smem + L::RS + 4 * tid) = rs_row;
            if constexpr (RT) *(int64_t *)(smem + L::YO + 8 * tid) = yo_row;
        }
        __syncthreads();
        convert(0);
    } else {
        if (tid < BM) {  // visible after the loop's first barrier
            *(float *)(smem + L::RS + 4 * tid) = rs_row;
            if constexpr (RT) *(int64_t *)(smem + L::YO + 8 * tid) = yo_row;
        }
    }
    // direct B: this lane's raw chunk 2 kk2 + fh of row wn + fr, swizzled as the copies placed it, and its scale word
    // (Q6_K: also its qh chunk fh and d pair, and the row's first super-block index in the d plane)
    const int brow = wn + fr;
    // (Q5_K: its one qs chunk fh serves both K-step pairs, as low and high nibbles)
    const uint32_t boffd0 = L::RB == 64 ? brow * L::RB + 16 * ((0 + fh) ^ ((brow >> 2) & 3))
                                        : brow * L::RB + 16 * (fh ^ ((brow >> 3) & 1));
    const uint32_t boffd1 = L::RB == 64 ? brow * L::RB + 16 * ((2 + fh) ^ ((brow >> 2) & 3)) : boffd0;
    const uint32_t hoffd = brow * 32 + 16 * (fh ^ ((brow >> 3) & 1));
    const int64_t erow = (wrow0 + min(n0 + brow, N - 1)) * nsb;

    if constexpr (L::DIRB) {
        // The LDS address of every fragment read, per ring slot: the loop is unrolled over the slots, so a stage runs
        // no address arithmetic (the registers are there to spare: two workgroups of four waves per CU).
        static_assert(L::NS == 3, "the direct-B loop is unrolled over a three-stage ring");
        uint32_t adS[L::NS][8], aeS[L::NS][8], bS0[L::NS], bS1[L::NS], scS[L::NS], hS[L::NS], dS[L::NS];
#pragma unroll
        for (int sl = 0; sl < L::NS; sl++) {
            [[maybe_unused]] const uint32_t at = lds + L::A + sl * BM * 128, rt = lds + L::RAW + sl * BN * L::RB;
#pragma unroll
            for (int x = 0; x < 8; x++) adS[sl][x] = aeS[sl][x] = 0;
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
#pragma unroll
                for (int i = 0; i < TM; i++) {  // A fragment x = kk TM + i: x < 8 in fa, the rest (TM = 4) in fb
                    const int x = kk * TM + i;
                    if (x < 8) adS[sl][x] = at + aoff[i][kk];
                    else aeS[sl][x - 8] = at + aoff[i][kk];
                }
            // (shared bytes: two slots, by g / SHP, below)
            if constexpr (!L::SH_RAW) {
                bS0[sl] = rt + boffd0;
                bS1[sl] = rt + boffd1;
            }
            if constexpr (!L::SH_SC) scS[sl] = lds + L::SC + sl * BN * L::SB + brow * L::SB;
            if constexpr (!L::SH_QH) hS[sl] = lds + L::QH + sl * BN * 32 + hoffd;
            if constexpr (!L::SH_DD) dS[sl] = lds + L::DD + sl * BN * 4 + brow * 4;  // Q6_K: the row's d pair; Q5_K: d | dmin
        }
        [[maybe_unused]] const uint32_t pb0 = lds + L::RAW + boffd0, pb1 = lds + L::RAW + boffd1,
                                        ph = lds + L::QH + hoffd, pdd = lds + L::DD + brow * 4,
                                        psc = lds + L::SC + brow * L::SB;
        auto stage = [&](auto slot, int s) {
            constexpr int SL = decltype(slot)::value;  // == s % L::NS
            // this wave's copies of A(s) and of the raw weights of stage s have landed, and its LDS writes are done;
            // then every wave's. The barrier is the bare instruction: __syncthreads' release fence would wait for
            // every copy in flight (the next stages' too) wherever the compiler can see them pending.
            // (the latest issue, of stage s + 1, copied the shared bytes too or not)
            if (L::SHARED && !plast) wait_vm<(L::NS - 2) * L::OPS1>();
            else wait_vm<(L::NS - 2) * L::OPS>();
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            // this stage's code, qh, scale and d addresses
            const uint32_t hsl = (uint32_t)((sb + s) / L::SHP) & 1u;  // the shared bytes' slot
            const uint32_t b0 = L::SH_RAW ? pb0 + hsl * (BN * L::RB) : bS0[SL];
            const uint32_t b1 = L::SH_RAW ? pb1 + hsl * (BN * L::RB) : bS1[SL];
            const uint32_t hh = L::SH_QH ? ph + hsl * (BN * 32) : hS[SL];
            const uint32_t dd = L::SH_DD ? pdd + hsl * (BN * 4) : dS[SL];
            const uint32_t ss = L::SH_SC ? psc + hsl * (BN * L::SB) : scS[SL];
            v8h fa[8], fb[16];
            v4i braw[2], qh = {0, 0, 0, 0};
            uint32_t sw, dw = 0, s1 = 0, s2 = 0;
            // the K-quants' qh chunk and d word (Q5_K: and scale words 1, 2): landed with the reads below, whose wait
            // covers these
            if constexpr (L::K6)
                asm volatile("ds_read_b128 %0, %2\n\tds_read_b32 %1, %3" : "=&v"(qh), "=&v"(dw) : "v"(hh), "v"(dd)
                             : "memory");
            if constexpr (L::K5)
                asm volatile("ds_read_b128 %0, %4\n\tds_read_b32 %1, %5\n\tds_read_b32 %2, %6 offset:4\n\t"
                             "ds_read_b32 %3, %6 offset:8"
                             : "=&v"(qh), "=&v"(dw), "=&v"(s1), "=&v"(s2)
                             : "v"(hh), "v"(dd), "v"(ss)
                             : "memory");
            dq_read_ab<TM == 4 ? 2 : TM>(fa, braw, sw, adS[SL], b0, b1, ss);
            if constexpr (L::K6 || L::K5) asm volatile("" : "+v"(qh), "+v"(dw), "+v"(s1), "+v"(s2));  // no use before that wait
            // 16 raw values -> two K steps of B fragments: chunk kk2 of the stage (Q8_0: block kk2; Q6_K: values
            // 32 kk2 + 16 fh .. of the quarter, sub-block 4 (g & 3) + 2 kk2 + fh, qh bits 4 (g & 1) + 2 kk2; Q5_K: the
            // same values, sub-block 2 (g & 3) + kk2: qs nibble kk2, qh bit the sub-block)
            const int g = sb + s, gsh = (g & 1) * 4;
            auto conv = [&](int kk2, v4i &o0, v4i &o1) {
                if constexpr (L::K6) {
                    const uint16_t d6 = ((erow + (g >> 2)) & 1) ? (uint16_t)(dw >> 16) : (uint16_t)(dw & 0xFFFF);
                    dq_q6_k_16(braw[kk2], qh, gsh + 2 * kk2, gsh, (int8_t)(sw >> (8 * (2 * kk2 + fh))), d6, o0, o1);
                } else if constexpr (L::K5) {
                    const int sub = 2 * (g & 3) + kk2;
                    int scv, mv;
                    q4k_scale_min(sw, s1, s2, sub, scv, mv);
                    dq_q5_k_16(braw[0], qh, sub, 4 * kk2, scv, mv, dw, o0, o1);
                } else
                    dq_q8_0_16(braw[kk2], (uint16_t)(kk2 ? sw >> 16 : sw & 0xFFFF), o0, o1);
            };
            v4i bq[4];  // K steps 2 kk2 and 2 kk2 + 1 from chunk kk2 (block kk2 of the stage)
            if constexpr (TM == 4 && MX_DQ_HALF) {
                // K steps 2 and 3: their A fragments are read, and chunk 1 converted, while steps 0 and 1 run
                dq_issue8(fb, aeS[SL]);
#pragma unroll
                for (int x = 0; x < 8; x++) asm volatile("" : "+v"(fa[x]));  // steps 0 and 1 stay behind the reads
                conv(0, bq[0], bq[1]);
#pragma unroll
                for (int kk = 0; kk < 2; kk++)
#pragma unroll
                    for (int i = 0; i < TM; i++)
                        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk * TM + i],
                                                                            __builtin_bit_cast(v8h, bq[kk]), acc[i][0],
                                                                            0, 0, 0);
                conv(1, bq[2], bq[3]);
                dq_wait8(fb);
#pragma unroll
                for (int kk = 2; kk < 4; kk++)
#pragma unroll
                    for (int i = 0; i < TM; i++)
                        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[(kk - 2) * TM + i],
                                                                            __builtin_bit_cast(v8h, bq[kk]), acc[i][0],
                                                                            0, 0, 0);
            } else {
                if constexpr (TM == 4) {
                    uint32_t ae16[16];
#pragma unroll
                    for (int x = 0; x < 16; x++) ae16[x] = x < 8 ? aeS[SL][x] : 0;
                    dq_read<8>(fb, ae16);
                }
                conv(0, bq[0], bq[1]);
                conv(1, bq[2], bq[3]);
#pragma unroll
                for (int kk = 0; kk < 4; kk++)
#pragma unroll
                    for (int i = 0; i < TM; i++)
                        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            kk * TM + i < 8 ? fa[kk * TM + i] : fb[kk * TM + i - 8], __builtin_bit_cast(v8h, bq[kk]),
                            acc[i][0], 0, 0, 0);
            }
            plast = issue(s + L::NS - 1);
        };
        int s = 0;
#pragma unroll 1
        for (; s + L::NS <= nst; s += L::NS) {  // whole turns of the ring: no branch between the stages
            stage(std::integral_constant<int, 0>{}, s);
            stage(std::integral_constant<int, 1>{}, s + 1);
            stage(std::integral_constant<int, 2>{}, s + 2);
        }
        if (s < nst) stage(std::integral_constant<int, 0>{}, s);
        if (s + 1 < nst) stage(std::integral_constant<int, 1>{}, s + 1);
    } else {
#pragma unroll 1
    for (int s = 0; s < nst; s++) {
        // this wave's copies of A(s) and of the raw weights of stage s + 1 (direct B: of stage s) have landed, and its
        // LDS writes are done
        wait_vm<(L::NS - 3) * L::OPS>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
        {
        // the stage's fragments, then its MFMAs; the copies three stages ahead and the conversion of the next stage's
        // weights follow while the matrix cores work through them
        const uint32_t at = lds + L::A + (s % L::NS) * BM * 128;
        const uint32_t bt = lds + L::BH + (s & 1) * BN * 128;
        uint32_t ad[16];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
#pragma unroll
            for (int i = 0; i < TM; i++) ad[kk * (TM + TN) + i] = at + aoff[i][kk];
#pragma unroll
            for (int j = 0; j < TN; j++) ad[kk * (TM + TN) + TM + j] = bt + boff[j][kk];
        }
#pragma unroll
        for (int x = NF; x < 16; x++) ad[x] = 0;
        v8h f[16];
        dq_read<NF>(f, ad);
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[kk * (TM + TN) + i], f[kk * (TM + TN) + TM + j],
                                                                        acc[i][j], 0, 0, 0);
        issue(s + L::NS - 1);
        if (s + 1 < nst) convert(s + 1);
        }
    }
    }
    wait_vm<0>();  // the copies of the stages past the end

    // 32 x 32 accumulator layout: lane l, register r holds (row 8 (r / 4) + 4 (l / 32) + r % 4, col l % 32)
    float *y = p.y;
    int64_t ldy = p.ldy;
    if (a.nsplit > 1) {  // this split's partial sums
        y = a.ws + (int64_t)split * M * a.ntot + a.col0[pi];
        ldy = a.ntot;
    }
    const float *rsl = (const float *)(smem + L::RS);  // the rows' 2^-e
    const int64_t *yol = (const int64_t *)(smem + L::YO);  // routed: the rows' output offsets
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn + 32 * j + fr;
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int ml = wm + 32 * i + 8 * (r >> 2) + 4 * fh + (r & 3);  // row within the tile
                if constexpr (RT) {
                    if (ml < mrows) y[yol[ml] + n] = acc[i][j][r] * rsl[ml];
                } else {
                    const int m = m0 + ml;
                    if (m < M) y[(int64_t)m * ldy + n] = acc[i][j][r] * rsl[ml];
                }
            }
        }
}

// y[m][col] = sum of the nsplit partials of (m, col), split 0 first; one thread per VW columns of a row (VW = 4 when
// every problem's width, row stride and base allow 16-byte accesses).
template <int VW>
__global__ __launch_bounds__(256) void k_dq_reduce(DqArgs a) {
    using V = typename std::conditional<VW == 4, float4, float>::type;
    const int c = (blockIdx.x * 256 + threadIdx.x) * VW, m = blockIdx.y;
    if (c >= a.ntot) return;
    const int64_t plane = (int64_t)a.M * a.ntot;
    const float *ws = a.ws + (int64_t)m * a.ntot + c;
    auto add = [](V &s, V v) {
        if constexpr (VW == 4) {
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        } else {
            s += v;
        }
    };
    V v[8], sum{};
    for (int s0 = 0; s0 < a.nsplit; s0 += 8) {  // eight partials' loads in flight at a time
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (s0 + u < a.nsplit) v[u] = *(const V *)(ws + (s0 + u) * plane);
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (s0 + u < a.nsplit) add(sum, v[u]);
    }
    int pi = 0;
    while (pi + 1 < a.nprob && c >= a.col0[pi + 1]) pi++;
    const DqProblem &p = pi == 0 ? a.prob[0] : (pi == 1 ? a.prob[1] : (pi == 2 ? a.prob[2] : a.prob[3]));
    *(V *)(p.y + (int64_t)m * p.ldy + (c - a.col0[pi])) = sum;
}

// ------------------------------------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------------------------------------
bool gemm_dq_supported(int type, int64_t M, int64_t K) {
    return ((type == MX_TYPE_Q8_0 && K % DQ_KS == 0) || ((type == MX_TYPE_Q6_K || type == MX_TYPE_Q5_K) && K % 256 == 0)) &&
           M * K < ((int64_t)1 << 31) && K < (1 << 24);
}

size_t gemm_dq_act_bytes(int64_t M, int64_t K) { return (size_t)M * (size_t)K * 2; }

namespace {

struct DqPlan {
    int bm, bn, nsplit;
    int64_t ntot;
};

// Tile: 128 x 128 when that gives at least 128 workgroups for a group of products, 192 for a single one (measured at
// M = 512, a 128-workgroup grid of 128 x 128 tiles beats a 256-workgroup grid of 128 x 64 ones by 1.3x), else 64 x 64
// (a backend's tile option overrides it: 64 x 64, 128 x 64 or 128 x 128). When 64 x 64 tiles still leave CUs idle
// (few rows: a short prefill block), K is split so that about 512 workgroups stream the weights, each over at least
// four stages (a backend's split option overrides it); the split's reduce pass costs more than it saves on the large
// tiles. A forced tile the kernel lacks gives bm = 0 (refused by the launch).
DqPlan dq_plan(int type, int nprob, const int64_t *N, int64_t M, int64_t K, const Options &o) {
    DqPlan pl{64, 64, 1, 0};
    // The direct-B types also have a 32 x 128 tile of four 32 x 32 waves, for blocks of at most 32 rows (the last,
    // short block of a prompt: half the activation rows of a 64-row tile, so half its fragment reads and MFMAs), and
    // a 64 x 128 one of four 64 x 32 waves
    const bool dirb = (type == MX_TYPE_Q8_0 && MX_DQ_DIRECT_B && MX_DQ_Q8_WGM128 == 1) ||
                      (type == MX_TYPE_Q6_K && MX_DQ_DIRECT_B6) || (type == MX_TYPE_Q5_K && MX_DQ_DIRECT_B5);
    int64_t wg128 = 0;
    for (int i = 0; i < nprob; i++) {
        wg128 += (N[i] + 127) / 128;
        pl.ntot += N[i];
    }
    wg128 *= (M + 127) / 128;
    const int64_t nst = K / DQ_KS;
    // long products (K >= 4096) whose 128 x 128 grid is smaller still keep the large tile and split K instead (at
    // M = 512, N = 2048, K = 6144: four splits of 24 stages and the reduce beat 256 tiles of 64 x 64)
    const bool split128 = wg128 >= 32 && wg128 < 128 && nst >= 64;
    // 128 x 128 from 192 workgroups of it, else, when half-height or half-width tiles give 256 (wg128 >= 128), 64 x 128
    // (direct B: four waves of 64 x 32) or 128 x 64 (the others), else 64 x 64. Measured at M = 512, K = 2048, weights
    // cold, with the activation pass (us on 64 x 64 / 64 x 128 / 128 x 64 / 128 x 128): Q8_0 N = 4096 29.9 / 29.1 /
    // 29.1 / 32.8; N = 2048 21.4 / 24.0 / 27.1 / 29.2; N = 12288 73.8 / 57.5 / 64.1 / 49.1; the ASR q/k/v group 2048 +
    // 1024 + 1024 32.0 / 29.7 / 29.7 / 33.3 (a group's grid holds only its problems' own tiles, so it runs as a product
    // of its summed width); Q6_K N = 4096 39.2 / 33.7 / 39.4 / 39.8, N = 2048 28.2 / 31.4 / 31.6 / 38.2
    if (wg128 >= 192 || split128) pl.bm = pl.bn = 128;
    else if (wg128 >= 128 && M >= 128) {
        pl.bm = dirb ? 64 : 128;
        pl.bn = dirb ? 128 : 64;
    }
    if (dirb && M <= 32) {
        pl.bm = 32;
        pl.bn = 128;
    }
    if (o.tile_m || o.tile_n) {
        const int tm = o.tile_m, tn = o.tile_n;
        if (dirb && (tm == 32 || tm == 64) && tn == 128) {  // the direct-B types' 32 x 128 and 64 x 128
            pl.bm = tm;
            pl.bn = 128;
        } else if ((tm == 64 || tm == 128) && (tn == 64 || tn == 128) && !(tm == 64 && tn == 128)) {
            pl.bm = tm;
            pl.bn = tn;
        } else {
            pl.bm = pl.bn = 0;
            return pl;
        }
    }
    int64_t tiles = 0;
    for (int i = 0; i < nprob; i++) tiles += (N[i] + pl.bn - 1) / pl.bn;
    tiles *= (M + pl.bm - 1) / pl.bm;
    int64_t want = tiles < 256 && pl.bn == 64 ? (512 + tiles - 1) / tiles : 1;
    if (split128 && pl.bm == 128 && pl.bn == 128) want = (256 + tiles - 1) / tiles;
    if (pl.bm == 32) want = (MX_DQ_SKINNY_WG + tiles - 1) / tiles;
    const int forced = o.split;
    if (forced > 0) want = forced;
    want = std::min<int64_t>(want, std::max<int64_t>(1, forced > 0 ? nst : nst / 4));
    const int64_t per = (nst + want - 1) / want;  // stages per split; no split is left empty
    pl.nsplit = (int)((nst + per - 1) / per);
    return pl;
}

}  // namespace

// scratch: [xh: M K fp16][rs: M floats][partials: nsplit M ntot floats], each part 256-byte aligned
static size_t dq_rs_offset(int64_t M, int64_t K) { return (gemm_dq_act_bytes(M, K) + 255) / 256 * 256; }
static size_t dq_ws_offset(int64_t M, int64_t K) { return dq_rs_offset(M, K) + ((size_t)M * 4 + 255) / 256 * 256; }

size_t gemm_dq_scratch_bytes(int type, int nprob, const int64_t *N, int64_t M, int64_t K, const Options &o) {
    const DqPlan pl = dq_plan(type, nprob, N, M, K, o);
    size_t b = dq_ws_offset(M, K);
    if (pl.nsplit > 1) b += (size_t)pl.nsplit * (size_t)M * (size_t)pl.ntot * 4;
    return b;
}

hipError_t launch_gemm_dq_act(int type, int rounding, const float *x, int64_t x_stride, int64_t M, int64_t K,
                              void *xh, hipStream_t s) {
    float *rs = (float *)((uint8_t *)xh + dq_rs_offset(M, K));
    if (M == 0) return hipSuccess;
    if (type == MX_TYPE_Q8_0) {
        hipLaunchKernelGGL(k_dq_act_q8_0, dim3((unsigned)M), dim3(DQ_ACT_NT), 0, s, x, x_stride, (int)K, rounding,
                           (_Float16 *)xh, rs);
    } else if ((type == MX_TYPE_Q6_K || type == MX_TYPE_Q5_K) && K % 256 == 0) {  // Q8_K has one rounding form
        hipLaunchKernelGGL(k_dq_act_q8k, dim3((unsigned)M), dim3(DQ_ACT_NT), 0, s, x, x_stride, (int)K, (_Float16 *)xh,
                           rs);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// gy: the routed form's chunk slots (grid.y); the dense form covers M.
template <int WT, int BM, int BN, int WGM, int WGN, bool RT = false>
static hipError_t launch_dq(const DqArgs &a, int maxN, hipStream_t s, int gy = 0) {
    using L = DqLds<WT, BM, BN, WGM * WGN, RT>;
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_gemm_dq<WT, BM, BN, WGM, WGN, RT>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, L::SIZE);
        if (e != hipSuccess) return e;
        attr = true;
    }
    int64_t tiles = 0;  // dense: every split's tiles of every problem
    for (int i = 0; i < a.nprob; i++) tiles += (int64_t)((a.prob[i].N + BN - 1) / BN) * ((a.M + BM - 1) / BM);
    const dim3 grid = RT ? dim3((unsigned)((maxN + BN - 1) / BN), (unsigned)gy, (unsigned)a.nprob)
                         : dim3((unsigned)(tiles * a.nsplit));
    hipLaunchKernelGGL((k_gemm_dq<WT, BM, BN, WGM, WGN, RT>), grid, dim3(64 * WGM * WGN), L::SIZE, s, a);
    return hipGetLastError();
}

template <int WT>
static hipError_t launch_dq_type(const DqArgs &a, const DqPlan &pl, int maxN, hipStream_t s) {
    if constexpr ((WT == MX_TYPE_Q8_0 && MX_DQ_DIRECT_B && MX_DQ_Q8_WGM128 == 1) || (WT == MX_TYPE_Q6_K && MX_DQ_DIRECT_B6) ||
                  (WT == MX_TYPE_Q5_K && MX_DQ_DIRECT_B5)) {
        // direct B: four waves of 128 x 32, so every B fragment is converted by one wave only
        if (pl.bm == 128 && pl.bn == 128) return launch_dq<WT, 128, 128, 1, 4>(a, maxN, s);
        if (pl.bm == 64 && pl.bn == 128) return launch_dq<WT, 64, 128, 1, 4>(a, maxN, s);
        if (pl.bm == 32) return launch_dq<WT, 32, 128, 1, 4>(a, maxN, s);
    }
    if (pl.bm == 32 || (pl.bm == 64 && pl.bn == 128)) return hipErrorInvalidValue;
    if (pl.bm == 128 && pl.bn == 128) return launch_dq<WT, 128, 128, 2, MX_DQ_WGN128>(a, maxN, s);
    if (pl.bm == 128) return launch_dq<WT, 128, 64, 4, 2>(a, maxN, s);
    return launch_dq<WT, 64, 64, 2, 2>(a, maxN, s);
}

hipError_t launch_gemm_dq(int type, int nprob, const WPlanes *w, const int64_t *N, float *const *y,
                          const int64_t *ldy, int64_t M, int64_t K, void *scratch, const Options &o, hipStream_t s) {
    if (nprob < 1 || nprob > 4 || !gemm_dq_supported(type, M, K)) return hipErrorInvalidValue;
    const DqPlan pl = dq_plan(type, nprob, N, M, K, o);
    if (pl.bm == 0) return hipErrorInvalidValue;
    DqArgs a{};
    int64_t maxN = 0;
    for (int i = 0; i < nprob; i++) {
        if (N[i] * K >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
        a.prob[i] = DqProblem{w[i], (int)N[i], y[i], ldy[i]};
        a.col0[i] = i == 0 ? 0 : a.col0[i - 1] + (int)N[i - 1];
        maxN = N[i] > maxN ? N[i] : maxN;
    }
    if (maxN == 0 || M == 0) return hipSuccess;
    if (pl.nsplit > 1 && M * pl.ntot * pl.nsplit >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    a.M = (int)M;
    a.K = (int)K;
    a.xh = (const _Float16 *)scratch;
    a.rs = (const float *)((const uint8_t *)scratch + dq_rs_offset(M, K));
    a.nprob = nprob;
    a.nsplit = pl.nsplit;
    a.ntot = (int)pl.ntot;
    a.ws = (float *)((uint8_t *)scratch + dq_ws_offset(M, K));
    const hipError_t e = type == MX_TYPE_Q8_0   ? launch_dq_type<MX_TYPE_Q8_0>(a, pl, (int)maxN, s)
                         : type == MX_TYPE_Q6_K ? launch_dq_type<MX_TYPE_Q6_K>(a, pl, (int)maxN, s)
                                                : launch_dq_type<MX_TYPE_Q5_K>(a, pl, (int)maxN, s);
    if (e != hipSuccess || pl.nsplit == 1) return e;
    bool v4 = true;
    for (int i = 0; i < nprob; i++) v4 = v4 && N[i] % 4 == 0 && ldy[i] % 4 == 0 && (uintptr_t)y[i] % 16 == 0;
    if (v4) hipLaunchKernelGGL(k_dq_reduce<4>, dim3((unsigned)((pl.ntot / 4 + 255) / 256), (unsigned)M), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(k_dq_reduce<1>, dim3((unsigned)((pl.ntot + 255) / 256), (unsigned)M), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int WT>
static hipError_t dq_routed(const DqArgs &a, int tile, int maxN, int gy, hipStream_t s) {
    switch (tile) {
        case 32128: return launch_dq<WT, 32, 128, 1, 4, true>(a, maxN, s, gy);
        case 32064: return launch_dq<WT, 32, 64, 1, 2, true>(a, maxN, s, gy);
        case 64064: return launch_dq<WT, 64, 64, 2, 2, true>(a, maxN, s, gy);
        default: return hipErrorInvalidValue;
    }
}

// The routed form's tile: 32 x 128 for the direct-B types (Q8_0, Q6_K; measured for Q6_K at 256 tokens over 64 experts:
// 252 us per layer against 311 on 64 x 64), 64 x 64 for Q5_K, unless a backend's tile option forces one the form has
// (32 x 128, 32 x 64 or 64 x 64; 0 x 0 if it has not). Its rows are a chunk's.
static void dq_routed_tile(const MulMatIdArgs &m, int &bm, int &bn) {
    const bool dirb = (m.type == MX_TYPE_Q8_0 && MX_DQ_DIRECT_B) || (m.type == MX_TYPE_Q6_K && MX_DQ_DIRECT_B6) ||
                      (m.type == MX_TYPE_Q5_K && MX_DQ_DIRECT_B5);
    bm = dirb ? 32 : 64;
    bn = dirb ? 128 : 64;
    if (m.tile_m || m.tile_n) {
        const bool ok = (m.tile_m == 32 && (m.tile_n == 128 || m.tile_n == 64)) || (m.tile_m == 64 && m.tile_n == 64);
        bm = ok ? m.tile_m : 0;
        bn = ok ? m.tile_n : 0;
    }
}

int mmid_dq_chunk(const MulMatIdArgs &m) {
    int bm, bn;
    dq_routed_tile(m, bm, bn);
    return bm;
}

hipError_t launch_gemm_dq_routed(const MulMatIdArgs &m, hipStream_t s) {
    int bm, bn;
    dq_routed_tile(m, bm, bn);
    if (m.nprob < 1 || m.nprob > 4 || bm == 0 || m.chunk != bm || !gemm_dq_supported(m.type, MAX_COLS + 1, m.K))
        return hipErrorInvalidValue;
    if (m.N == 0) return hipSuccess;
    DqArgs a{};
    for (int i = 0; i < m.nprob; i++) a.prob[i] = DqProblem{m.wg[i], (int)m.N, m.dstg[i], 0};
    a.M = 0;  // rows come from the chunks
    a.K = (int)m.K;
    a.xh = m.xh;
    a.rs = m.rs;
    a.nprob = m.nprob;
    a.nsplit = 1;
    a.tiles = m.tiles;
    a.ntiles = m.ntiles;
    a.pairs = m.pairs;
    a.n_ids = (int)m.n_ids;
    a.b_ne1 = (int)m.b_ne1;
    a.y_nb1 = m.dst_nb1 / 4;
    a.y_nb2 = m.dst_nb2 / 4;
    const int gy = (int)m.max_tiles, maxN = (int)m.N;
    const int tile = bm * 1000 + bn;
    switch (m.type) {
        case MX_TYPE_Q8_0: return dq_routed<MX_TYPE_Q8_0>(a, tile, maxN, gy, s);
        case MX_TYPE_Q6_K: return dq_routed<MX_TYPE_Q6_K>(a, tile, maxN, gy, s);
        case MX_TYPE_Q5_K: return dq_routed<MX_TYPE_Q5_K>(a, tile, maxN, gy, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
