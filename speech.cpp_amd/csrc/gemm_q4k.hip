// Prefill products on Q4_K weights (M > 8) with Q8_K activations, on int8 MFMA with the sub-block scales folded into
// the operands.
//
// ggml-cpu's vec_dot_q4_K_q8_K per 256-element super-block of weight row n and activation row m:
//   y += dx * (d * sum_j sc_j * S_j  -  dmin * sum_j mn_j * bsum_j)        (eight sub-blocks j of 32)
// with S_j the exact int32 dot of sub-block j's 4-bit codes q with the activation quants, and sc_j, mn_j 6-bit.
//
// The scale is split, sc = 8 hi + lo with hi, lo in 0..7, so hi * q and lo * q (at most 105) are int8 operands: two
// v_mfma_i32_32x32x32_i8 per sub-block accumulate A_hi = sum_j hi_j S_j and A_lo = sum_j lo_j S_j over the whole
// super-block with no VALU work, and 8 A_hi + A_lo = sum_j sc_j S_j exactly (|.| < 2^25). The codes are scaled in
// registers with packed 16-bit multiplies (no byte overflows). The min term is one v_mfma_f32_32x32x16_f16 per
// super-block: bsum_j = 64 h_j + l_j (h in -64..63, l in 0..63) puts 64 h_j and l_j in fp16 exactly, and every product
// and partial sum is an integer below 2^24, so the fp32 result is exact. Float scales are applied once per
// super-block: acc += dx * (d * I - dmin * Mt).
//
// Work split: waves of 64 x 32 (two 32 x 32 MFMA tiles sharing every scaled weight fragment); eight of them (two along
// M, four along N, two to a SIMD) make a 128 x 128 workgroup tile, or four a 128 x 64 one for smaller products.
// Operands (quants, codes, scale splats) go through a two-stage LDS ring and the epilogue inputs (activation d and
// sums, weight d, dmin and mins) through a three-stage one. With eight waves, the two waves of a SIMD split into an
// early one (epilogue of super-block sb after sb's MFMAs) and a late one (epilogue of sb - 1 before them), so that one
// wave's MFMAs meet the other's float epilogue.
//
// The kernel is VALU-bound: per super-block a wave issues 34 MFMAs and about 340 VALU ops (80 per 32 x 32 tile for the
// float epilogue, 130 to unpack and scale the codes), and a VALU op costs about as much issue time as an eighth of an
// MFMA. The per-block float scales of the format are what cost: an int8 product with per-32 or per-256 fp scales needs
// a few VALU ops per output per block, whatever the MFMA shape.
#include "mx_common.h"
#include "mx_device.h"

#include <cstdlib>

namespace mx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// LDS rows are unpadded and 16-byte chunks are XOR-swizzled so that the MFMA fragment reads (32 rows, one chunk
// each) meet distinct banks whether the LDS serves 128 or 256 bytes a clock (8 or 16 lanes of a ds_read_b128):
//   activations, 256-byte rows: chunk c of row r at r * 256 + 16 (c ^ (r & 15));
//   weight codes, 128-byte rows: chunk c of row r at r * 128 + 16 (c ^ bswz(r)), where bswz gives the eight rows of
//   any aligned group of 8 distinct chunk slots, and rows r and r + 8 (same 128-byte half of a 256-byte line) too;
//   [64 h | l] halves, 32-byte rows: half h of row r at r * 32 + 16 (h ^ (((r >> 2) ^ (r >> 3)) & 1)).
// The global -> LDS copies (lane i of a wave writes 16 bytes at base + 16 i) pick each lane's source chunk to land in
// that order.
__device__ __forceinline__ int bswz(int r) { return ((r >> 1) & 3) | (((r & 1) ^ ((r >> 3) & 1)) << 2); }
__device__ __forceinline__ int hswz(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }
__device__ __forceinline__ int a_slot(int r, int c) { return r * 256 + 16 * (c ^ (r & 15)); }
__device__ __forceinline__ int b_slot(int r, int c) { return r * 128 + 16 * (c ^ bswz(r)); }
__device__ __forceinline__ int h_slot(int r, int h) { return r * 32 + 16 * (h ^ hswz(r)); }

// Activation rows -> Q8_K for this kernel: int8 quants [M][K], fp32 d [M][K/256], and per super-block 16 fp16 values
// [64 h_0 .. 64 h_7, l_0 .. l_7] with bsum32_j = 64 h_j + l_j (the sums of the eight sub-blocks' quants).
__global__ __launch_bounds__(256) void k_gemm_q4k_quant(const float *x, int64_t x_stride, int K, int8_t *xq,
                                                        float *xd, _Float16 *x16) {
    const int64_t m = blockIdx.x;  // rows on x: grid.y holds at most 65,535
    const int lane = threadIdx.x & 63;
    const int sb = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int nsb = K / 256;
    if (sb >= nsb) return;  // whole wave
    const float4 v = *(const float4 *)(x + m * x_stride + (int64_t)sb * 256 + 4 * lane);
    float d;
    int bs16;
    const int q = quant256_wave(v, lane, &d, &bs16);
    const int bs32 = bs16 + dpp_i<dpp::HALF_MIRROR>(0, bs16);  // lanes 8j..8j+7 hold sub-block j's sum
    *(int *)(xq + m * K + (int64_t)sb * 256 + 4 * lane) = q;
    if (lane == 0) xd[m * nsb + sb] = d;
    if ((lane & 7) == 0) {
        const int j = lane >> 3;
        const int h = bs32 >> 6;  // floor(bs32 / 64)
        _Float16 *o = x16 + (m * nsb + sb) * 16;
        o[j] = (_Float16)(64 * h);
        o[8 + j] = (_Float16)(bs32 - 64 * h);
    }
}

struct Q4gProblem {
    const uint8_t *qs, *sc, *dm;  // planes of the matrix: 128 code bytes, 12 scale bytes, fp16 d | fp16 dmin per block
    float *y;
    int64_t ldy;                  // floats between rows of y
    int N;
};
struct Q4gArgs {
    Q4gProblem prob[4];
    int nprob, M, nsb;
    int64_t K;
    const int8_t *xq;
    const float *xd;
    const _Float16 *x16;
};

// Workgroup tile (32 NMT WM) x (32 WN): WM x WN waves, each with NMT 32 x 32 MFMA tiles stacked along M.
template <int NMT_, int WM_, int WN_>
struct Q4gT {
    static constexpr int NMT = NMT_, WM = WM_, WN = WN_;
    static constexpr int BM = 32 * NMT * WM, BN = 32 * WN, NW = WM * WN, NT = 64 * NW;
    // operand rings: activation quants (two slots), weight codes (three: their copies run two super-blocks ahead,
    // the activations', from the L2 mostly, one), scale splats (two)
    static constexpr int A = 0;                     // in an A slot: int8 quants, BM rows of 256 (swizzled)
    static constexpr int B = 0;                     // in a B slot: packed codes, BN rows of 128 (swizzled)
    static constexpr int BSC = 0;                   // in a splat slot: [sub-block j][column]: (hi, hi), (lo, lo) u16
    static constexpr int SA = BM * 256, SB = BN * 128, SS = 8 * BN * 8;  // slot sizes
    static constexpr int RA = 0, RB = RA + 2 * SA, RS = RB + 3 * SB, RE = RS + 2 * SS;  // ring bases
    // epilogue stage
    static constexpr int A16 = 0;                   // fp16 [64 h | l], 32 B per row (swizzled halves)
    static constexpr int ADX = A16 + BM * 32;       // fp32 d per row
    static constexpr int BMN = ADX + BM * 4;        // per column 8 fp16 mins
    static constexpr int BD = BMN + BN * 16;        // per column fp32 d, dmin
    static constexpr int EP = BD + BN * 8;
    static constexpr int LDS = RE + 3 * EP;
    // global -> LDS copy instructions per stage (64 lanes each), and per wave
    static constexpr int NA = BM / 4, NB = BN / 8, NA16 = BM / 32, NDX = BM / 64;
    static constexpr int QA = NA / NW, QB = NB / NW;
    static_assert(NA % NW == 0 && NB % NW == 0 && NA16 <= NW && NDX <= NW && NDX >= 1, "copies split over waves");
    static constexpr int TPC = NT / BN;             // threads decoding each weight column's scales
    static_assert(TPC == 2 || TPC == 4, "two or four threads per weight column");
    static_assert(LDS <= 160 * 1024, "LDS of one workgroup");
};

// One workgroup's global -> LDS copies through buffer loads (buffer_load_dword* ... lds): a per-lane byte offset
// fixed for the whole K loop and a per-stage uniform offset (sb times the per-block stride of each source: 256 B of
// quants, 32 B of [64 h | l], 4 B of d per activation row; 128 code bytes per weight row). The waves share the
// activation instructions (4 rows each) and the weight ones (8 rows each) evenly; waves 0..3 copy the [64 h | l]
// rows (32 each) and waves 0..1 the d values (64 each). Buffer bounds (num_records) make any read past a buffer's end
// return zeros; rows past M or N are clamped to the last row anyway.
template <class Q>
struct Q4gDma {
    uint32_t a[Q::QA], b[Q::QB], a16, dx;
    v4u ra, rb, r16, rdx;

    __device__ __forceinline__ void init(int wave, const int8_t *xq, const _Float16 *x16, const float *xd,
                                         const uint8_t *qs, int m0, int n0, int M, int N, int K, int nsb) {
        const int lane = threadIdx.x & 63;
        ra = buf_rsrc(xq, (uint32_t)(M * K));
        rb = buf_rsrc(qs, (uint32_t)(N * nsb * 128));
        r16 = buf_rsrc(x16, (uint32_t)(M * nsb * 32));
        rdx = buf_rsrc(xd, (uint32_t)(M * nsb * 4));
#pragma unroll
        for (int q = 0; q < Q::QA; q++) {
            const int r = 4 * (wave * Q::QA + q) + (lane >> 4), cs = lane & 15;
            a[q] = (uint32_t)min(m0 + r, M - 1) * (uint32_t)K + 16u * (uint32_t)(cs ^ (r & 15));
        }
#pragma unroll
        for (int q = 0; q < Q::QB; q++) {
            const int r = 8 * (wave * Q::QB + q) + (lane >> 3), cs = lane & 7;
            b[q] = (uint32_t)min(n0 + r, N - 1) * (uint32_t)nsb * 128u + 16u * (uint32_t)(cs ^ bswz(r));
        }
        {
            const int r = 32 * min(wave, Q::NA16 - 1) + (lane >> 1);
            a16 = (uint32_t)min(m0 + r, M - 1) * (uint32_t)nsb * 32u + 16u * (uint32_t)((lane & 1) ^ hswz(r));
        }
        dx = (uint32_t)min(m0 + 64 * min(wave, Q::NDX - 1) + lane, M - 1) * (uint32_t)nsb * 4u;
    }

    // wave is uniform (readfirstlane), so every LDS destination is a scalar. The weight codes of a super-block (QB
    // instructions per wave) are issued on their own, last of a step's copies.
    __device__ __forceinline__ void issue_b(uint8_t *opb, int wave, int sb) const {
#pragma unroll
        for (int q = 0; q < Q::QB; q++) dma16_lds(rb, lds_addr(opb + Q::B + 1024 * (wave * Q::QB + q)), b[q], sb * 128);
    }
    __device__ __forceinline__ void issue_a(uint8_t *opa, uint8_t *ep, int wave, int sb) const {
#pragma unroll
        for (int q = 0; q < Q::QA; q++) dma16_lds(ra, lds_addr(opa + Q::A + 1024 * (wave * Q::QA + q)), a[q], sb * 256);
        if (wave < Q::NA16) dma16_lds(r16, lds_addr(ep + Q::A16 + 1024 * wave), a16, sb * 32);  // uniform
        if (wave < Q::NDX) dma4_lds(rdx, lds_addr(ep + Q::ADX + 256 * wave), dx, sb * 4);        // uniform
    }
};

// The raw scale bytes a thread decodes for a stage: thread t handles weight column t / TPC and 8 / TPC of its
// sub-blocks.
struct Q4gScales {
    uint32_t s0, s1, s2, dm;

    // Issued through asm, like the copies, so that the compiler inserts no wait for them: `landed` (after the
    // explicit vmcnt wait that covers them) is their first use.
    __device__ __forceinline__ void load(const uint8_t *scp, const uint8_t *dmp, uint32_t blk0, int sb) {
        const uint32_t blk = blk0 + (uint32_t)sb;  // scalar bases, 32-bit lane offsets
        asm volatile("global_load_dword %0, %4, %5\n\tglobal_load_dword %1, %4, %5 offset:4\n\t"
                     "global_load_dword %2, %4, %5 offset:8\n\tglobal_load_dword %3, %6, %7"
                     : "=&v"(s0), "=&v"(s1), "=&v"(s2), "=&v"(dm)
                     : "v"(blk * 12u), "s"(scp), "v"(blk * 4u), "s"(dmp)
                     : "memory");
    }
    __device__ __forceinline__ void landed() { asm volatile("" : "+v"(s0), "+v"(s1), "+v"(s2), "+v"(dm)); }

    __device__ static __forceinline__ uint32_t byte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
        const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
        return (w >> (8 * (i & 3))) & 0xFF;
    }

    // ggml-quants.c get_scale_min_k4: scale splats into the operand stage, mins, d and dmin into the epilogue stage.
    template <class Q>
    __device__ __forceinline__ void store(uint8_t *ops, uint8_t *ep) const {
        constexpr int PER = 8 / Q::TPC;
        const int t = threadIdx.x, n = t / Q::TPC, q = t % Q::TPC;
        uint32_t *bsc = (uint32_t *)(ops + Q::BSC + n * 8);
        _Float16 *bmn = (_Float16 *)(ep + Q::BMN + n * 16);
#pragma unroll
        for (int h = 0; h < PER; h++) {
            const int j = PER * q + h;
            uint32_t sc, mn;
            if (j < 4) {
                sc = byte(s0, s1, s2, j) & 63;
                mn = byte(s0, s1, s2, j + 4) & 63;
            } else {
                sc = (byte(s0, s1, s2, j + 4) & 0xF) | ((byte(s0, s1, s2, j - 4) >> 6) << 4);
                mn = (byte(s0, s1, s2, j + 4) >> 4) | ((byte(s0, s1, s2, j) >> 6) << 4);
            }
            const uint32_t hi = sc >> 3, lo = sc & 7;
            bsc[j * 2 * Q::BN] = hi | (hi << 16);
            bsc[j * 2 * Q::BN + 1] = lo | (lo << 16);
            bmn[j] = (_Float16)(float)mn;
        }
        if (q == 0) {
            float *bd = (float *)(ep + Q::BD + n * 8);
            bd[0] = h2f((uint16_t)(dm & 0xFFFF));
            bd[1] = h2f((uint16_t)(dm >> 16));
        }
    }
};

// Two u16 lanes of two codes each times (s, s): each byte's product stays below 256, so bytes do not interact.
__device__ __forceinline__ int pk_mul_u16(int codes, uint32_t s2) {
    int r;
    asm("v_pk_mul_lo_u16 %0, %1, %2" : "=v"(r) : "v"(codes), "v"(s2));
    return r;
}
__device__ __forceinline__ v4i scale_codes(v4i c, uint32_t s2) {
    return v4i{pk_mul_u16(c.x, s2), pk_mul_u16(c.y, s2), pk_mul_u16(c.z, s2), pk_mul_u16(c.w, s2)};
}

// One wave's view of the workgroup: its rows, its column, and the LDS base.
struct Q4gWave {
    uint8_t *smem;
    int wave, wm, br, fr, hf;
};

// acc += dx * (d * (8 A_hi + A_lo) - dmin * Mt) for rows 8g + 4hf + 0..3 of tile t (one quarter of the tile).
// Epilogue inputs of one super-block for this lane: the column's d, dmin and mins, and per tile the rows' [64 h | l]
// and d values. Loaded in one go, ahead of use.
template <class Q>
struct Q4gEpi {
    float2 dd;
    v8h b16;
    v8h a16[Q::NMT];
    float4 dx[Q::NMT][4];

    __device__ __forceinline__ void load(const Q4gWave &w, const uint8_t *ep) {
        dd = *(const float2 *)(ep + Q::BD + w.br * 8);
        b16 = *(const v8h *)(ep + Q::BMN + w.br * 16);
#pragma unroll
        for (int t = 0; t < Q::NMT; t++) {
            a16[t] = *(const v8h *)(ep + Q::A16 + h_slot(w.wm + 32 * t + w.fr, w.hf));
#pragma unroll
            for (int g = 0; g < 4; g++) dx[t][g] = *(const float4 *)(ep + Q::ADX + (w.wm + 32 * t + 8 * g + 4 * w.hf) * 4);
        }
    }

    // acc += dx * (d * (8 A_hi + A_lo) - dmin * Mt), with the min term Mt of each tile from one fp16 MFMA (exact).
    __device__ __forceinline__ void apply(const v16i (&I)[2 * Q::NMT], float (&acc)[Q::NMT][16]) const {
        const v16f zerof = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < Q::NMT; t++) {
            const v16f mt = __builtin_amdgcn_mfma_f32_32x32x16_f16(a16[t], b16, zerof, 0, 0, 0);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float dxs[4] = {dx[t][g].x, dx[t][g].y, dx[t][g].z, dx[t][g].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * g + i;
                    const int v = (I[2 * t][r] << 3) + I[2 * t + 1][r];
                    acc[t][r] = fmaf(dxs[i], fmaf(-dd.y, mt[r], dd.x * (float)v), acc[t][r]);
                }
            }
        }
    }
};

// LDS operands of sub-blocks 2 pr and 2 pr + 1: this lane's 16 packed code bytes and the two scale splat pairs
// (weights), and the activation fragments of every tile.
struct Q4gWFrag {
    v4i pk;
    uint2 hl[2];
};
template <class Q>
struct Q4gAFrag {
    v4i a[2][Q::NMT];
};
// The scaled weight fragments (hi and lo splits of each sub-block's scale) of a sub-block pair.
struct Q4gBFrag {
    v4i bh[2], bl[2];
};

template <class Q>
__device__ __forceinline__ Q4gWFrag q4g_load_w(const Q4gWave &w, const uint8_t *opb, const uint8_t *ops, int pr) {
    Q4gWFrag f;
    f.pk = *(const v4i *)(opb + Q::B + b_slot(w.br, 2 * pr + w.hf));
    const uint2 *bsc = (const uint2 *)(ops + Q::BSC + w.br * 8);
    f.hl[0] = bsc[(2 * pr) * Q::BN];
    f.hl[1] = bsc[(2 * pr + 1) * Q::BN];
    return f;
}

template <class Q>
__device__ __forceinline__ Q4gAFrag<Q> q4g_load_a(const Q4gWave &w, const uint8_t *opa, int pr) {
    Q4gAFrag<Q> f;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int t = 0; t < Q::NMT; t++)
            f.a[h][t] = *(const v4i *)(opa + Q::A + a_slot(w.wm + 32 * t + w.fr, 2 * (2 * pr + h) + w.hf));
    return f;
}

__device__ __forceinline__ Q4gBFrag q4g_scale(const Q4gWFrag &f) {
    const v4i m4 = {0x0F0F0F0F, 0x0F0F0F0F, 0x0F0F0F0F, 0x0F0F0F0F};
    const v4i codes[2] = {f.pk & m4, (f.pk >> 4) & m4};
    Q4gBFrag b;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        b.bh[h] = scale_codes(codes[h], f.hl[h].x);
        b.bl[h] = scale_codes(codes[h], f.hl[h].y);
    }
    return b;
}

template <class Q>
__device__ __forceinline__ void q4g_mfma(const Q4gAFrag<Q> &a, const Q4gBFrag &b, v16i (&I)[2 * Q::NMT]) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int t = 0; t < Q::NMT; t++) {
            I[2 * t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.a[h][t], b.bh[h], I[2 * t], 0, 0, 0);
            I[2 * t + 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a.a[h][t], b.bl[h], I[2 * t + 1], 0, 0, 0);
        }
}

template <class Q>
__device__ __forceinline__ void q4g_epilogue(const Q4gWave &w, const uint8_t *ep, const v16i (&I)[2 * Q::NMT],
                                             float (&acc)[Q::NMT][16]) {
    Q4gEpi<Q> e;
    e.load(w, ep);
    e.apply(I, acc);
}

// Iteration sb of one wave: start the copies of super-block sb + 1 (activations, epilogue inputs, scales) and of the
// weight codes of sb + 2, then sb's MFMAs into `I` ({A_hi, A_lo} per tile) and a float epilogue: an early wave (the
// first half of the workgroup) runs the epilogue of sb after its MFMAs, a late wave runs the epilogue of sb - 1 before
// them. The two waves sharing a SIMD are one early and one late, so that one's MFMAs meet the other's epilogue between
// any two barriers; the three-stage epilogue ring keeps sb - 1's inputs in LDS for the late wave. Then the scales of
// sb + 1 and the stage barrier, which waits for everything but the codes of sb + 2.
template <class Q>
__device__ __forceinline__ void q4g_step(const Q4gWave &w, bool late, const Q4gDma<Q> &dma, Q4gScales &sc,
                                         const uint8_t *scp, const uint8_t *dmp, uint32_t scblk, int sb, int nsb,
                                         v16i (&I)[2 * Q::NMT], float (&acc)[Q::NMT][16]) {
    const int e = sb % 3, en = e == 2 ? 0 : e + 1, ep2 = e == 0 ? 2 : e - 1;  // sb, sb + 1 and sb - 1 (= sb + 2) mod 3
    const uint8_t *opa = w.smem + Q::RA + (sb & 1) * Q::SA, *opb = w.smem + Q::RB + e * Q::SB;
    const uint8_t *ops = w.smem + Q::RS + (sb & 1) * Q::SS;
    uint8_t *opan = w.smem + Q::RA + ((sb + 1) & 1) * Q::SA, *opbn2 = w.smem + Q::RB + ep2 * Q::SB;
    uint8_t *opsn = w.smem + Q::RS + ((sb + 1) & 1) * Q::SS;
    uint8_t *epbase = w.smem + Q::RE;
    uint8_t *epn = epbase + en * Q::EP;
    const uint8_t *epc = epbase + e * Q::EP;
    const uint8_t *epp = epbase + ep2 * Q::EP;
    // past the end, copies repeat the last super-block into slots no later step reads
    dma.issue_a(opan, epn, w.wave, min(sb + 1, nsb - 1));
    sc.load(scp, dmp, scblk, min(sb + 1, nsb - 1));
    asm volatile("" ::: "memory");  // the codes go out last: the stage barrier leaves only them in flight
    dma.issue_b(opbn2, w.wave, min(sb + 2, nsb - 1));

    // Software pipeline over the four sub-block pairs: weight bytes read two pairs ahead, activation fragments and
    // the scaling one pair ahead, so no MFMA waits on LDS or on the VALU that prepares its operand.
    Q4gWFrag wf[3];
    Q4gAFrag<Q> af[2];
    Q4gBFrag bf[2];
    wf[0] = q4g_load_w<Q>(w, opb, ops, 0);
    wf[1] = q4g_load_w<Q>(w, opb, ops, 1);
    af[0] = q4g_load_a<Q>(w, opa, 0);
    Q4gEpi<Q> ep;
    ep.load(w, late ? epp : epc);
    bf[0] = q4g_scale(wf[0]);
    if (late) ep.apply(I, acc);
    const v16i zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 2 * Q::NMT; i++) I[i] = zero16;
#pragma unroll
    for (int pr = 0; pr < 4; pr++) {
        if (pr + 2 < 4) wf[(pr + 2) % 3] = q4g_load_w<Q>(w, opb, ops, pr + 2);
        if (pr + 1 < 4) {
            af[(pr + 1) & 1] = q4g_load_a<Q>(w, opa, pr + 1);
            bf[(pr + 1) & 1] = q4g_scale(wf[(pr + 1) % 3]);
        }
        q4g_mfma<Q>(af[pr & 1], bf[pr & 1], I);
    }
    if (!late) ep.apply(I, acc);

    // this wave's copies and scale loads of sb + 1 have landed (the codes of sb + 2, its last QB copies, may not)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Q::QB) : "memory");
    sc.landed();
    sc.store<Q>(opsn, epn);
    // and its LDS writes are done; then every wave's. The barrier is the bare instruction: __syncthreads' release fence
    // would wait for the codes of sb + 2 too.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <class Q>
__global__ __launch_bounds__(Q::NT) void k_gemm_q4k(Q4gArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    // The grid is one dimension of the problems' tiles, problem after problem, each (N_z / BN) x (M / BM) with n
    // fastest: no workgroup of a narrower problem's missing columns (a grid of the widest problem's width per problem
    // launched those, and the launch ran as if it had that many more workgroups). A column's M tiles stay a multiple
    // of the column count apart, which keeps them on one XCD when that count is a multiple of 8.
    const int MT = (a.M + Q::BM - 1) / Q::BM;
    int t = blockIdx.x, z = 0;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const int Ni = i == 0 ? a.prob[0].N : (i == 1 ? a.prob[1].N : a.prob[2].N);
        const int ti = (Ni + Q::BN - 1) / Q::BN * MT;
        if (z == i && i + 1 < a.nprob && t >= ti) {
            t -= ti;
            z = i + 1;
        }
    }
    const uint8_t *qs = z == 0 ? a.prob[0].qs : (z == 1 ? a.prob[1].qs : (z == 2 ? a.prob[2].qs : a.prob[3].qs));
    const uint8_t *scp = z == 0 ? a.prob[0].sc : (z == 1 ? a.prob[1].sc : (z == 2 ? a.prob[2].sc : a.prob[3].sc));
    const uint8_t *dmp = z == 0 ? a.prob[0].dm : (z == 1 ? a.prob[1].dm : (z == 2 ? a.prob[2].dm : a.prob[3].dm));
    float *y = z == 0 ? a.prob[0].y : (z == 1 ? a.prob[1].y : (z == 2 ? a.prob[2].y : a.prob[3].y));
    const int N = z == 0 ? a.prob[0].N : (z == 1 ? a.prob[1].N : (z == 2 ? a.prob[2].N : a.prob[3].N));
    const int64_t ldy = z == 0 ? a.prob[0].ldy : (z == 1 ? a.prob[1].ldy : (z == 2 ? a.prob[2].ldy : a.prob[3].ldy));
    const int ntz = (N + Q::BN - 1) / Q::BN;
    const int n0 = (t % ntz) * Q::BN, m0 = (t / ntz) * Q::BM;
    const int M = a.M, nsb = a.nsb;
    const int tid = threadIdx.x, lane = tid & 63;

    Q4gWave w;
    w.smem = smem;
    w.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    w.wm = (w.wave / Q::WN) * 32 * Q::NMT;
    w.fr = lane & 31;
    w.hf = lane >> 5;
    w.br = (w.wave % Q::WN) * 32 + w.fr;

    Q4gDma<Q> dma;
    dma.init(w.wave, a.xq, a.x16, a.xd, qs, m0, n0, M, N, (int)a.K, nsb);
    const uint32_t scblk = (uint32_t)min(n0 + tid / Q::TPC, N - 1) * (uint32_t)nsb;
    Q4gScales sc;
    uint8_t *ep0 = smem + Q::RE;
    dma.issue_a(smem + Q::RA, ep0, w.wave, 0);
    dma.issue_b(smem + Q::RB, w.wave, 0);
    sc.load(scp, dmp, scblk, 0);
    dma.issue_b(smem + Q::RB + Q::SB, w.wave, min(1, nsb - 1));
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Q::QB) : "memory");  // all but the codes of super-block 1
    sc.landed();
    sc.store<Q>(smem + Q::RS, ep0);
    {
        // Epilogue stage 2 (the "previous" one of iteration 0) starts as zeros: iteration 0 runs its epilogue with zero
        // accumulators, which adds exactly 0.
        uint8_t *ep2 = ep0 + 2 * Q::EP;
        const v4i z4 = {0, 0, 0, 0};
        for (int o = 16 * tid; o < Q::EP; o += 16 * Q::NT) *(v4i *)(ep2 + o) = z4;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    const v16i zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    v16i I[2 * Q::NMT];
#pragma unroll
    for (int i = 0; i < 2 * Q::NMT; i++) I[i] = zero16;
    float acc[Q::NMT][16];
#pragma unroll
    for (int t = 0; t < Q::NMT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;

    // With eight waves, waves w and w + 4 share a SIMD and the second half of the workgroup runs late; four waves have
    // a SIMD each and all run early.
    const bool late = Q::NW == 8 && w.wave >= 4;
#pragma unroll 1
    for (int sb = 0; sb < nsb; sb++) q4g_step<Q>(w, late, dma, sc, scp, dmp, scblk, sb, nsb, I, acc);
    if (late) q4g_epilogue<Q>(w, ep0 + ((nsb - 1) % 3) * Q::EP, I, acc);

    const int n = n0 + w.br;
    if (n < N) {
#pragma unroll
        for (int t = 0; t < Q::NMT; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + w.wm + 32 * t + 8 * (r >> 2) + 4 * w.hf + (r & 3);
                if (m < M) y[(int64_t)m * ldy + n] = acc[t][r];
            }
    }
}

size_t gemm_q4k_act_bytes(int64_t M, int64_t K) {
    return align_up((uint64_t)(M * K), 256) + align_up((uint64_t)M * (uint64_t)(K / 256) * 4, 256) +
           align_up((uint64_t)M * (uint64_t)(K / 256) * 32, 256);
}

struct Q4gScratch {
    int8_t *xq;
    float *xd;
    _Float16 *x16;
};

static Q4gScratch q4g_scratch(const void *scratch, int64_t M, int64_t K) {
    Q4gScratch p;
    p.xq = (int8_t *)scratch;
    p.xd = (float *)((uint8_t *)scratch + align_up((uint64_t)(M * K), 256));
    p.x16 = (_Float16 *)((uint8_t *)p.xd + align_up((uint64_t)M * (uint64_t)(K / 256) * 4, 256));
    return p;
}

hipError_t launch_gemm_q4k_quant(const float *x, int64_t x_stride, int64_t M, int64_t K, void *scratch,
                                 hipStream_t s) {
    if (K % 256 != 0 || M <= 0) return hipErrorInvalidValue;
    const Q4gScratch p = q4g_scratch(scratch, M, K);
    hipLaunchKernelGGL(k_gemm_q4k_quant, dim3((unsigned)M, (unsigned)((K / 256 + 3) / 4)), dim3(256), 0, s, x,
                       x_stride, (int)K, p.xq, p.xd, p.x16);
    return hipGetLastError();
}

template <class Q>
static hipError_t launch_q4g(const Q4gArgs &a, hipStream_t s) {
    static bool configured = false;
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_gemm_q4k<Q>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 Q::LDS);
        if (e != hipSuccess) return e;
        configured = true;
    }
    int64_t tiles = 0;
    for (int i = 0; i < a.nprob; i++)
        tiles += (int64_t)((a.prob[i].N + Q::BN - 1) / Q::BN) * ((a.M + Q::BM - 1) / Q::BM);
    hipLaunchKernelGGL(k_gemm_q4k<Q>, dim3((unsigned)tiles), dim3(Q::NT), Q::LDS, s, a);
    return hipGetLastError();
}

hipError_t launch_gemm_q4k(int nprob, const WPlanes *w, const int64_t *N, float *const *y, const int64_t *ldy,
                           int64_t M, int64_t K, const void *scratch, const Options &o, hipStream_t s) {
    if (nprob < 1 || nprob > 4 || K % 256 != 0 || M <= 0) return hipErrorInvalidValue;
    // 32-bit buffer offsets: activations M * K bytes, weight codes N * K / 2 bytes
    if ((uint64_t)M * (uint64_t)K >= (1ull << 31)) return hipErrorInvalidValue;
    const Q4gScratch sp = q4g_scratch(scratch, M, K);
    Q4gArgs a{};
    for (int i = 0; i < nprob; i++) {
        if (N[i] <= 0 || (uint64_t)N[i] * (uint64_t)K / 2 >= (1ull << 31)) return hipErrorInvalidValue;
        a.prob[i] = Q4gProblem{w[i].p0, w[i].p1, w[i].p2, y[i], ldy[i], (int)N[i]};
    }
    a.nprob = nprob;
    a.M = (int)M;
    a.nsb = (int)(K / 256);
    a.K = K;
    a.xq = sp.xq;
    a.xd = sp.xd;
    a.x16 = sp.x16;
    // Tile: 128 x 128 (eight waves, two per SIMD, each with two 32 x 32 tiles) when that gives a workgroup to every
    // CU, else 64 x 64 (four waves of one 32 x 32 tile; 75 KB of LDS, two workgroups per CU). Measured at M = 512, K =
    // 2048, weights cold, with the activation pass (us on 128 x 128 / 64 x 64 / 64 x 128 eight-wave / 128 x 64
    // four-wave): N = 4096 28.7 / 22.7 / 22.4-22.5 / 22.9; N = 2048 27.1 / 16.6 / 20.7 / 21.8; N = 12288 51.0-53.9 /
    // 51.9 / 52.9-53.8 / 55.1-55.4.
    // A backend's tile option forces 128 x 128, 64 x 64, 64 x 128 or 128 x 64; any other forced pair is refused.
    int64_t wg_big = 0;
    for (int i = 0; i < nprob; i++) wg_big += (N[i] + 127) / 128 * ((M + 127) / 128);
    int tile = wg_big >= 256 ? 0 : 3;  // 0: 128 x 128, 1: 64 x 128, 2: 128 x 64, 3: 64 x 64
    if (o.tile_m || o.tile_n) {
        if (o.tile_m == 128 && o.tile_n == 128) tile = 0;
        else if (o.tile_m == 64 && o.tile_n == 128) tile = 1;
        else if (o.tile_m == 128 && o.tile_n == 64) tile = 2;
        else if (o.tile_m == 64 && o.tile_n == 64) tile = 3;
        else return hipErrorInvalidValue;
    }
    if (tile == 0) return launch_q4g<Q4gT<2, 2, 4>>(a, s);
    if (tile == 1) return launch_q4g<Q4gT<1, 2, 4>>(a, s);
    if (tile == 3) return launch_q4g<Q4gT<1, 2, 2>>(a, s);
    return launch_q4g<Q4gT<2, 2, 2>>(a, s);
}

}  // namespace mx
