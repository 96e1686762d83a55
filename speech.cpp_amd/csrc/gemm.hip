// Prefill products (M > 8): Y[m, n] = sum_b dx[m, b] * dw[n, b] * S_b[m, n], where S_b is the exact int32 dot of
// block b's int8 quants -- the sum ggml-cpu's vec_dot_q8_0_q8_0 forms one block at a time, here formed by int8 MFMA.
//
// Activations are quantized once into scratch (k_gemm_quant), then each workgroup computes a BM x BN tile of Y:
// 4 waves in a 2 x 2 arrangement, each owning (BM/2) x (BN/2) of the tile as 32 x 32 MFMA tiles. K advances in
// stages of 128 through a ring of NS stages in LDS, filled by buffer-to-LDS copies (no registers between global
// memory and LDS): NS - 1 stages are in flight while one is computed, which a grid of one or two workgroups per CU
// needs to cover the memory latency (one stage ahead, each 128-wide stage cost a round trip). The 64 x 128 tile, picked
// only for grids of 512 workgroups or more, keeps two stages and covers the latency with three workgroups per CU.
//
// Per 32-element block and 32 x 32 tile: one v_mfma_i32_32x32x32_i8 (the integer sums, exact), one
// v_mfma_f32_32x32x8_f16 whose only non-zero k is dx (x) dw -- the outer product of the two fp16 scales, exact in
// fp32 -- and per element one int -> float conversion and one fma into the fp32 accumulator.
#include "mx_common.h"
#include "mx_device.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace mx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int KS = 128;       // K per LDS stage
// Per tile: ring stages, blocks whose MFMAs a wave has in flight at once, and the waves per SIMD its registers are
// allocated for. 64 x 64: four stages (70 KB, two workgroups per CU), block kb + 1's MFMAs issued before block kb's
// VALU. 64 x 128: two stages (52 KB) and one block at a time (162 VGPRs), so three workgroups share a CU; measured at
// M = 512 on the ASR gate/up group (768 workgroups) 50.7 -> 46.7 us against three stages and two blocks (212 VGPRs,
// two workgroups per CU), while the 64 x 64 tile measured slower that way (down, K = 6144: 37.3 -> 40.8 us).
template <int BM, int BN>
struct I8Cfg {
    static constexpr bool WIDE = BM == 64 && BN == 128;
    static constexpr int NS = BM == 64 && BN == 64 ? 4 : (WIDE ? 2 : 3);
    static constexpr int PD = BM == 64 && BN == 64 ? 2 : 1;
    static constexpr int WPE = WIDE ? 3 : 2;
};

// Activation rows -> int8 quants [M][K], fp16 block scales [M][K/32] (d rounded to fp16, as the Q8_0 the weights
// pair with stores it).
__global__ __launch_bounds__(256) void k_gemm_quant_q8(const float *x, int64_t x_stride, int64_t K, int rounding,
                                                       int8_t *xq, uint16_t *xd) {
    const int64_t m = blockIdx.x;  // rows on x: grid.y holds at most 65,535
    const int64_t e = (int64_t)blockIdx.y * 1024 + 4 * threadIdx.x;
    const bool valid = e < K;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) v = *(const float4 *)(x + m * x_stride + e);
    float d;
    int sum;
    const int q = quant32_lane(v, rounding, &d, &sum);
    if (valid) {
        *(int *)(xq + m * K + e) = q;
        if ((threadIdx.x & 7) == 0) xd[m * (K / 32) + e / 32] = f2h(d);
    }
}

struct GemmProblem {
    WPlanes w;
    int64_t N;
    float *y;
    int64_t ldy;     // floats between consecutive m rows of Y
};
// Up to four weights sharing the activations. The grid is one dimension: split after split, problem after problem,
// (N_p / BN) x (M / BM) tiles with n fastest. Split s covers the K stages [s per, (s + 1) per); with nsplit > 1 each
// split writes its partial sums to ws ([nsplit][M][ntot], problem p at columns col0[p] ..) and k_gemm_reduce adds
// them in split order.
struct GemmArgs {
    GemmProblem prob[4];
    int nprob, nsplit;
    int64_t M, K;
    const int8_t *xq;
    const uint16_t *xd;  // fp16 bits
    int64_t ntot, col0[4];
    float *ws;
};

template <class T>
__device__ __forceinline__ T pick4(int i, T v0, T v1, T v2, T v3) {
    return i == 0 ? v0 : (i == 1 ? v1 : (i == 2 ? v2 : v3));
}
// Problem pi's fields one by one (selecting the whole struct by a run-time index copies the arguments to scratch).
__device__ __forceinline__ GemmProblem problem(const GemmArgs &a, int pi) {
    GemmProblem p{};
    p.w.p0 = pick4(pi, a.prob[0].w.p0, a.prob[1].w.p0, a.prob[2].w.p0, a.prob[3].w.p0);
    p.w.p1 = pick4(pi, a.prob[0].w.p1, a.prob[1].w.p1, a.prob[2].w.p1, a.prob[3].w.p1);
    p.N = pick4(pi, a.prob[0].N, a.prob[1].N, a.prob[2].N, a.prob[3].N);
    p.y = pick4(pi, a.prob[0].y, a.prob[1].y, a.prob[2].y, a.prob[3].y);
    p.ldy = pick4(pi, a.prob[0].ldy, a.prob[1].ldy, a.prob[2].ldy, a.prob[3].ldy);
    return p;
}

__device__ __forceinline__ _Float16 as_half(uint16_t b) {
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return h;
}


// The LDS ring: NS stages, each of A (BM rows of 128 quants), B (BN rows), and the four fp16 block scales of each
// activation row (DX) and weight row (DW). Quant rows are stored as 8 chunks of 16 bytes, chunk c of row r at slot
// c ^ i8_swz(r): the 16 rows one fragment read visits at a time fall on 16 distinct 16-byte bank groups.
template <int BM, int BN>
struct I8Lds {
    static constexpr int NS = I8Cfg<BM, BN>::NS;
    static constexpr int SA = BM * KS, SB = BN * KS, SDX = BM * 8, SDW = BN * 8;  // slot sizes (bytes)
    static constexpr int A = 0, B = A + NS * SA, DX = B + NS * SB, DW = DX + NS * SDX, SIZE = DW + NS * SDW;
    // copies per stage and wave: 16-byte ones of 8 quant rows each; 4-byte ones of 32 scale rows each, shared by the
    // waves (a wave past the last scale copy repeats it: the same bytes to the same place)
    static constexpr int QA = BM / 32, QB = BN / 32, NDX = BM / 32, NSC = (BM + BN) / 32, QS = (NSC + 3) / 4;
    static constexpr int OPS = QA + QB + QS;
    static_assert(SIZE <= 80 * 1024 || (BM == 128 && BN == 128), "two workgroups per CU");
    static_assert(NS >= 2, "a ring of two stages or more");
};

__device__ __forceinline__ int i8_swz(int r) { return (r >> 1) & 7; }

// One wave's copies of a stage: per-lane byte offsets fixed for the whole K loop (rows past M or N clamped to the
// last row), a per-stage uniform offset (k0 bytes of quants, k0 / 16 bytes of scales per row).
template <int BM, int BN>
struct I8Dma {
    using L = I8Lds<BM, BN>;
    uint32_t a[L::QA], b[L::QB], s[L::QS], ls[L::QS];
    v4u ra, rb, rs[L::QS];
    uint32_t la, lb;  // LDS offsets of this wave's first A and B copy in a slot

    __device__ __forceinline__ void init(int wave, const GemmArgs &g, const GemmProblem &pb, int64_t m0, int64_t n0) {
        const int lane = threadIdx.x & 63;
        const uint32_t K = (uint32_t)g.K, nblk = K / 32, M = (uint32_t)g.M, N = (uint32_t)pb.N;
        ra = buf_rsrc(g.xq, M * K);
        rb = buf_rsrc(pb.w.p0, N * K);
        const v4u rdx = buf_rsrc(g.xd, M * nblk * 2), rdw = buf_rsrc(pb.w.p1, N * nblk * 2);
#pragma unroll
        for (int q = 0; q < L::QA; q++) {
            const int r = 8 * (wave * L::QA + q) + (lane >> 3);
            a[q] = (uint32_t)min<int64_t>(m0 + r, M - 1) * K + 16u * (uint32_t)((lane & 7) ^ i8_swz(r));
        }
#pragma unroll
        for (int q = 0; q < L::QB; q++) {
            const int r = 8 * (wave * L::QB + q) + (lane >> 3);
            b[q] = (uint32_t)min<int64_t>(n0 + r, N - 1) * K + 16u * (uint32_t)((lane & 7) ^ i8_swz(r));
        }
        la = (uint32_t)(wave * L::QA) * 1024u;
        lb = (uint32_t)(wave * L::QB) * 1024u;
#pragma unroll
        for (int u = 0; u < L::QS; u++) {
            const int j = min(wave * L::QS + u, L::NSC - 1);  // scale copy j: DX rows 32 j .., then DW rows
            const bool isx = j < L::NDX;
            const int r = 32 * (isx ? j : j - L::NDX) + (lane >> 1);
            const int64_t row = isx ? min<int64_t>(m0 + r, M - 1) : min<int64_t>(n0 + r, N - 1);
            s[u] = (uint32_t)row * nblk * 2u + 4u * (uint32_t)(lane & 1);
            rs[u] = isx ? rdx : rdw;
            ls[u] = isx ? (uint32_t)(L::DX + 256 * j) : (uint32_t)(L::DW + 256 * (j - L::NDX));
        }
    }

    // stage k0 into ring slot `slot` (lds: the ring's LDS address)
    __device__ __forceinline__ void issue(uint32_t lds, int slot, int k0) const {
        const uint32_t sa = lds + L::A + slot * L::SA + la, sb = lds + L::B + slot * L::SB + lb;
#pragma unroll
        for (int q = 0; q < L::QA; q++) dma16_lds(ra, sa + 1024u * q, a[q], (uint32_t)k0);
#pragma unroll
        for (int q = 0; q < L::QB; q++) dma16_lds(rb, sb + 1024u * q, b[q], (uint32_t)k0);
#pragma unroll
        for (int u = 0; u < L::QS; u++) {
            const uint32_t sl = ls[u] < (uint32_t)L::DW ? (uint32_t)(slot * L::SDX) : (uint32_t)(slot * L::SDW);
            dma4_lds(rs[u], lds + ls[u] + sl, s[u], (uint32_t)(k0 / 16));
        }
    }
};

// 32 x 32 accumulator layout of the 32x32 MFMAs: lane l, register r holds (row 8*(r/4) + 4*(l/32) + r%4, col l%32).
template <int BM, int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, I8Cfg<BM, BN>::WPE))) void k_gemm_q8_0_i8(
    GemmArgs a) {
    using L = I8Lds<BM, BN>;
    constexpr int WM = BM / 2, WN = BN / 2;   // wave tile
    constexpr int TM = WM / 32, TN = WN / 32; // MFMA tiles per wave
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_void *)smem;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t MT = (a.M + BM - 1) / BM;
    int64_t per = 0;  // tiles of one split
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (i < a.nprob) per += (a.prob[i].N + BN - 1) / BN * MT;
    int64_t t = blockIdx.x;
    const int split = (int)(t / per);
    t -= split * per;
    int pi = 0;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const int64_t ti = (a.prob[i].N + BN - 1) / BN * MT;
        if (pi == i && i + 1 < a.nprob && t >= ti) {
            t -= ti;
            pi = i + 1;
        }
    }
    const GemmProblem pb = problem(a, pi);
    const int64_t ntp = (pb.N + BN - 1) / BN;
    const int64_t m0 = (t / ntp) * BM, n0 = (t % ntp) * BN;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    const int nst = (int)(a.K / KS), sper = (nst + a.nsplit - 1) / a.nsplit;
    const int kb0 = split * sper * KS, nloc = min(nst - split * sper, sper);  // this split's stages (never none)

    I8Dma<BM, BN> dma;
    dma.init(wave, a, pb, m0, n0);
#pragma unroll
    for (int s = 0; s < L::NS - 1; s++)
        if (s < nloc) dma.issue(lds, s, kb0 + s * KS);

    float acc[TM][TN][16];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // this lane's fragment offsets in a slot: row wm + 32 i + fr (A) or wn + 32 j + fr (B), chunk 2 kb + fh
    const int fr = lane & 31, fh = lane >> 5;
    uint32_t aoff[TM][4], boff[TN][4], dxo[TM], dwo[TN];
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int r = wm + 32 * i + fr;
#pragma unroll
        for (int kb = 0; kb < 4; kb++) aoff[i][kb] = (uint32_t)(r * KS + 16 * ((2 * kb + fh) ^ i8_swz(r)));
        dxo[i] = (uint32_t)(r * 8);
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int r = wn + 32 * j + fr;
#pragma unroll
        for (int kb = 0; kb < 4; kb++) boff[j][kb] = (uint32_t)(r * KS + 16 * ((2 * kb + fh) ^ i8_swz(r)));
        dwo[j] = (uint32_t)(r * 8);
    }
    const _Float16 hz = (_Float16)0.0f;

    for (int s = 0; s < nloc; s++) {
        // this wave's copies of stage s have landed (those of the stages after it that were issued may not), then
        // every wave's, and every wave has read the slot the next copies overwrite. The barrier is the bare
        // instruction: __syncthreads' release fence would wait for the copies still in flight too.
        const int rem = nloc - 1 - s;  // stages issued after s: min(rem, NS - 2)
        if (rem >= L::NS - 2) wait_vm<(L::NS - 2) * L::OPS>();
        else if (L::NS > 3 && rem == 1) wait_vm<L::OPS>();
        else wait_vm<0>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (s + L::NS - 1 < nloc) dma.issue(lds, (s + L::NS - 1) % L::NS, kb0 + (s + L::NS - 1) * KS);
        const int slot = s % L::NS;
        const uint8_t *sa = smem + L::A + slot * L::SA, *sb = smem + L::B + slot * L::SB;
        const uint8_t *sdx = smem + L::DX + slot * L::SDX, *sdw = smem + L::DW + slot * L::SDW;
        // every fragment and scale of the stage first, so the reads overlap each other and the MFMAs that follow
        v4i af[4][TM], bf[4][TN];
        uint2 dx4[TM], dw4[TN];  // the row's (column's) four fp16 block scales
#pragma unroll
        for (int i = 0; i < TM; i++) {
            dx4[i] = *(const uint2 *)(sdx + dxo[i]);
#pragma unroll
            for (int kb = 0; kb < 4; kb++) af[kb][i] = *(const v4i *)(sa + aoff[i][kb]);
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            dw4[j] = *(const uint2 *)(sdw + dwo[j]);
#pragma unroll
            for (int kb = 0; kb < 4; kb++) bf[kb][j] = *(const v4i *)(sb + boff[j][kb]);
        }
        // block kb's integer sums and scale products; with PD = 2 block kb + 1's MFMAs are issued before block kb's
        // conversions and fmas, so the matrix cores and the VALU overlap within the wave
        constexpr int PD = I8Cfg<BM, BN>::PD;
        v16i S[PD][TM][TN];
        v16f C[PD][TM][TN];
        auto mfma = [&](int kb, int d) {
            v4h as[TM], bs[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t w = kb < 2 ? dx4[i].x : dx4[i].y;
                as[i] = v4h{fh ? hz : as_half((uint16_t)(kb & 1 ? w >> 16 : w & 0xFFFF)), hz, hz, hz};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t w = kb < 2 ? dw4[j].x : dw4[j].y;
                bs[j] = v4h{fh ? hz : as_half((uint16_t)(kb & 1 ? w >> 16 : w & 0xFFFF)), hz, hz, hz};
            }
            const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
            const v16f fz = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    S[d][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[kb][i], bf[kb][j], zero, 0, 0, 0);
                    C[d][i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(as[i], bs[j], fz, 0, 0, 0);
                }
        };
        auto fold = [&](int d) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = fmaf((float)S[d][i][j][r], C[d][i][j][r], acc[i][j][r]);
        };
        mfma(0, 0);
#pragma unroll
        for (int kb = 0; kb < KS / 32; kb++) {
            if (PD == 2 && kb + 1 < KS / 32) mfma(kb + 1, (kb + 1) % PD);
            fold(kb % PD);
            if (PD == 1 && kb + 1 < KS / 32) mfma(kb + 1, 0);
        }
    }

    float *y = pb.y;
    int64_t ldy = pb.ldy;
    if (a.nsplit > 1) {  // this split's partial sums
        y = a.ws + (int64_t)split * a.M * a.ntot + pick4(pi, a.col0[0], a.col0[1], a.col0[2], a.col0[3]);
        ldy = a.ntot;
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int64_t n = n0 + wn + 32 * j + fr;
            if (n >= pb.N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < a.M) y[m * ldy + n] = acc[i][j][r];
            }
        }
}

// y[m][col] = the nsplit partials of (m, col) added in split order (split 0 first); one thread per column.
__global__ __launch_bounds__(256) void k_gemm_reduce(GemmArgs a) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
    if (c >= a.ntot) return;
    const int64_t plane = a.M * a.ntot;
    const float *ws = a.ws + m * a.ntot + c;
    float v[8], sum = 0.0f;
    for (int s0 = 0; s0 < a.nsplit; s0 += 8) {  // eight partials' loads in flight at a time
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (s0 + u < a.nsplit) v[u] = ws[(s0 + u) * plane];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (s0 + u < a.nsplit) sum += v[u];
    }
    int pi = 0;
#pragma unroll
    for (int i = 1; i < 4; i++) pi += i < a.nprob && c >= a.col0[i];
    const GemmProblem p = problem(a, pi);
    p.y[m * p.ldy + (c - pick4(pi, a.col0[0], a.col0[1], a.col0[2], a.col0[3]))] = sum;
}

// ------------------------------------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------------------------------------
// scratch: [xq: M K int8][xd: M K/32 fp16][partials: nsplit M ntot floats], each part 256-byte aligned
static size_t gemm_xd_offset(int64_t M, int64_t K) { return ((size_t)M * (size_t)K + 255) / 256 * 256; }
static size_t gemm_ws_offset(int64_t M, int64_t K) {
    return gemm_xd_offset(M, K) + ((size_t)M * (size_t)(K / 32) * 2 + 255) / 256 * 256;
}

hipError_t launch_gemm_quant(int type, int rounding, const float *x, int64_t x_stride, int64_t M, int64_t K,
                             void *scratch, hipStream_t s) {
    if (type != MX_TYPE_Q8_0) return hipErrorInvalidValue;
    int8_t *xq = (int8_t *)scratch;
    uint16_t *xd = (uint16_t *)((uint8_t *)scratch + gemm_xd_offset(M, K));
    if (M == 0) return hipSuccess;
    const dim3 grid((unsigned)M, (unsigned)((K + 1023) / 1024));
    hipLaunchKernelGGL(k_gemm_quant_q8, grid, dim3(256), 0, s, x, x_stride, K, rounding, xq, xd);
    return hipGetLastError();
}

namespace {
struct GemmPlan {
    int bm = 64, bn = 64, nsplit = 1;
    int64_t ntot = 0;
};

// Tile: 64 x 128 when that tile gives 512 workgroups, else 64 x 64. A backend's tile option (tile_m x tile_n: 64 x 64,
// 64 x 128 or 128 x 128) overrides it; any other forced pair is refused (bm = 0). K is split, into as many splits as
// bring the grid to about 256 workgroups (each of at least four 128-wide stages), where the tiles are fewer than 256
// and either K is long (32 stages or more) or the tiles number at most 64: elsewhere the partial sums' traffic (8
// bytes per split, row and column) and the reduce cost more than the wider grid gains. A forced split count (1 ..
// 64, at most one per stage) overrides that. Measured at K = 2048 (q/k/v 2048 + 1024 + 1024, N = 2048, gate/up
// 2 x 6144) and K = 6144 (down, N = 2048), weights cold, best split (us): down M = 33 8 splits 14.3 (one: 32.9);
// M = 130 4 splits 24.2 (33.2); M = 256 2 splits 28.5 (35.5); M = 512 one 37.4 (2 splits 41.8); N = 2048 at M = 33
// 4 splits 11.1 (14.1), at M = 130 one 14.5 (2 splits 14.9), M = 256 one 15.0 (17.3); gate/up at M = 33 one 16.5
// (2 splits 21.8).
GemmPlan gemm_plan(int nprob, const int64_t *N, int64_t M, int64_t K, const Options &o) {
    GemmPlan pl;
    int64_t t128 = 0;
    for (int i = 0; i < nprob; i++) {
        t128 += (N[i] + 127) / 128;
        pl.ntot += N[i];
    }
    t128 *= (M + 63) / 64;
    if (t128 >= 512) pl.bn = 128;
    if (o.tile_m || o.tile_n) {
        if (!((o.tile_m == 64 && (o.tile_n == 64 || o.tile_n == 128)) || (o.tile_m == 128 && o.tile_n == 128))) {
            pl.bm = 0;
            return pl;
        }
        pl.bm = o.tile_m;
        pl.bn = o.tile_n;
    }
    int64_t tiles = 0;
    for (int i = 0; i < nprob; i++) tiles += (N[i] + pl.bn - 1) / pl.bn;
    tiles *= (M + pl.bm - 1) / pl.bm;
    const int64_t nst = K / KS;
    int64_t want = tiles > 0 && tiles < 256 && (nst >= 32 || tiles <= 64) ? (256 + tiles - 1) / tiles : 1;
    want = std::min<int64_t>(want, std::max<int64_t>(1, nst / 4));
    if (o.split > 0) want = std::min<int64_t>(o.split, nst);
    const int64_t per = (nst + want - 1) / want;  // stages per split; no split is left empty
    pl.nsplit = (int)((nst + per - 1) / per);
    return pl;
}
}  // namespace

template <int BM, int BN>
static hipError_t launch_i8(dim3 grid, const GemmArgs &a, hipStream_t s) {
    constexpr int bytes = I8Lds<BM, BN>::SIZE;
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_gemm_q8_0_i8<BM, BN>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((k_gemm_q8_0_i8<BM, BN>), grid, dim3(256), bytes, s, a);
    return hipGetLastError();
}

size_t gemm_scratch_bytes(int nprob, const int64_t *N, int64_t M, int64_t K, const Options &o) {
    const GemmPlan pl = gemm_plan(nprob, N, M, K, o);
    size_t b = gemm_ws_offset(M, K);
    if (pl.nsplit > 1) b += (size_t)pl.nsplit * (size_t)M * (size_t)pl.ntot * 4;
    return b;
}

hipError_t launch_gemm(int type, int nprob, const WPlanes *w, const int64_t *N, float *const *y, const int64_t *ldy,
                       int64_t M, int64_t K, void *scratch, const Options &o, hipStream_t s) {
    if (type != MX_TYPE_Q8_0 || K % KS != 0 || nprob < 1 || nprob > 4 || M * K >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;
    const GemmPlan pl = gemm_plan(nprob, N, M, K, o);
    if (pl.bm == 0) return hipErrorInvalidValue;
    GemmArgs a{};
    int64_t tiles = 0;
    for (int i = 0; i < nprob; i++) {
        if (N[i] * K >= ((int64_t)1 << 31)) return hipErrorInvalidValue;  // the copies' 32-bit byte offsets
        a.prob[i] = GemmProblem{w[i], N[i], y[i], ldy[i]};
        a.col0[i] = i == 0 ? 0 : a.col0[i - 1] + N[i - 1];
        tiles += (N[i] + pl.bn - 1) / pl.bn;
    }
    tiles *= (M + pl.bm - 1) / pl.bm;
    if (tiles == 0) return hipSuccess;
    a.nprob = nprob;
    a.nsplit = pl.nsplit;
    a.M = M;
    a.K = K;
    a.xq = (const int8_t *)scratch;
    a.xd = (const uint16_t *)((const uint8_t *)scratch + gemm_xd_offset(M, K));
    a.ntot = pl.ntot;
    a.ws = (float *)((uint8_t *)scratch + gemm_ws_offset(M, K));
    const dim3 grid((unsigned)(tiles * pl.nsplit));
    hipError_t e = pl.bm == 128  ? launch_i8<128, 128>(grid, a, s)
                   : pl.bn == 128 ? launch_i8<64, 128>(grid, a, s)
                                  : launch_i8<64, 64>(grid, a, s);
    if (e != hipSuccess || pl.nsplit == 1) return e;
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((pl.ntot + 255) / 256), (unsigned)M), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mx
