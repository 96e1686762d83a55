// Prefill products (M > 8): Y[m, n] = sum_b dx[m, b] * dw[n, b] * S_b[m, n], where S_b is the exact int32 dot of
// block b's int8 quants -- the sum ggml-cpu's vec_dot_q8_0_q8_0 forms one block at a time, here formed by int8 MFMA.
//
// Activations are quantized once into scratch (k_gemm_quant), then each workgroup computes a BM x BN tile of Y:
// 4 waves in a 2 x 2 arrangement, each owning (BM/2) x (BN/2) of the tile as 32 x 32 MFMA tiles. K advances in
// stages of 128 staged through LDS (rows padded so 16-byte fragment reads spread over the banks); the next stage's
// global loads are issued before the current stage's MFMAs run.
//
// Per 32-element block and 32 x 32 tile: one v_mfma_i32_32x32x32_i8 (the integer sums, exact), one
// v_mfma_f32_32x32x8_f16 whose only non-zero k is dx (x) dw -- the outer product of the two fp16 scales, exact in
// fp32 -- and per element one int -> float conversion and one fma into the fp32 accumulator.
#include "mx_common.h"
#include "mx_device.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace mx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int KS = 128;       // K per LDS stage
constexpr int LROW = KS + 16; // padded LDS row (bytes)

// Activation rows -> int8 quants [M][K], fp32 block scales [M][K/32] (the fp16-rounded d, for Q8_0 weights).
__global__ __launch_bounds__(256) void k_gemm_quant_q8(const float *x, int64_t x_stride, int64_t K, int rounding,
                                                       int8_t *xq, float *xd) {
    const int64_t m = blockIdx.y;
    const int64_t e = (int64_t)blockIdx.x * 1024 + 4 * threadIdx.x;
    const bool valid = e < K;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) v = *(const float4 *)(x + m * x_stride + e);
    float d;
    int sum;
    const int q = quant32_lane(v, rounding, &d, &sum);
    if (valid) {
        *(int *)(xq + m * K + e) = q;
        if ((threadIdx.x & 7) == 0) xd[m * (K / 32) + e / 32] = h2f(f2h(d));
    }
}

struct GemmArgs {
    WPlanes w;
    int64_t M, N, K;
    const int8_t *xq;
    const float *xd;
    float *y;
    int64_t ldy;     // floats between consecutive m rows of Y
    const _Float16 *xh;  // the same quants as fp16 values (fp16-MFMA kernel)
};

// One K stage of the workgroup's tiles in flight from global memory: 16 bytes of int8 quants per thread and pass
// (8 threads cover a 128-byte row), plus the four fp16 block scales of one activation row and one weight row.
template <int BM, int BN>
struct Stage {
    static constexpr int XP = BM * 8 / 256, WP = BN * 8 / 256;
    v4i xr[XP], wr[WP];  // native vectors: HIP's int4 is a union type whose copies defeat register promotion
    float dx[4];         // activation scales (fp16 values held in fp32), converted only when stored to LDS
    uint32_t dw01, dw23;
};

// Per-thread source rows of the staging loads, clamped to the matrix once; a stage adds its K offset.
template <int BM, int BN>
struct StageSrc {
    const int8_t *x[Stage<BM, BN>::XP];
    const int8_t *w[Stage<BM, BN>::WP];
    const float *dx;       // this thread's activation row of block scales
    const uint16_t *dw;    // this thread's weight row of block scales
};

template <int BM, int BN>
__device__ __forceinline__ StageSrc<BM, BN> stage_src(const GemmArgs &a, int64_t m0, int64_t n0, int tid) {
    StageSrc<BM, BN> src;
    const int64_t K = a.K, nblk = K / 32;
    const int srow = tid >> 3, scol = (tid & 7) * 16;
#pragma unroll
    for (int p = 0; p < Stage<BM, BN>::XP; p++) {
        int64_t m = m0 + srow + 32 * p;
        m = m < a.M ? m : a.M - 1;
        src.x[p] = a.xq + m * K + scol;
    }
#pragma unroll
    for (int p = 0; p < Stage<BM, BN>::WP; p++) {
        int64_t n = n0 + srow + 32 * p;
        n = n < a.N ? n : a.N - 1;
        src.w[p] = (const int8_t *)a.w.p0 + n * K + scol;
    }
    int64_t m = m0 + (tid & (BM - 1));
    m = m < a.M ? m : a.M - 1;
    src.dx = a.xd + m * nblk;
    int64_t n = n0 + (tid & (BN - 1));
    n = n < a.N ? n : a.N - 1;
    src.dw = (const uint16_t *)a.w.p1 + n * nblk;
    return src;
}

template <int BM, int BN>
__device__ __forceinline__ void load_stage(Stage<BM, BN> &st, const StageSrc<BM, BN> &src, int k0) {
#pragma unroll
    for (int p = 0; p < Stage<BM, BN>::XP; p++) st.xr[p] = *(const v4i *)(src.x[p] + k0);
#pragma unroll
    for (int p = 0; p < Stage<BM, BN>::WP; p++) st.wr[p] = *(const v4i *)(src.w[p] + k0);
    // Every thread loads (rows clamped): no branch around the loads, so none of them is waited for here.
    const float4 f = *(const float4 *)(src.dx + k0 / 32);
    st.dx[0] = f.x;
    st.dx[1] = f.y;
    st.dx[2] = f.z;
    st.dx[3] = f.w;
    const uint32_t *p = (const uint32_t *)(src.dw + k0 / 32);
    st.dw01 = p[0];
    st.dw23 = p[1];
}

template <int BM, int BN>
__device__ __forceinline__ void store_stage(const Stage<BM, BN> &st, int8_t *xs, int8_t *ws, uint16_t *dxs,
                                            uint16_t *dws, int tid) {
    const int srow = tid >> 3, scol = (tid & 7) * 16;
#pragma unroll
    for (int p = 0; p < Stage<BM, BN>::XP; p++) *(v4i *)(xs + (srow + 32 * p) * LROW + scol) = st.xr[p];
#pragma unroll
    for (int p = 0; p < Stage<BM, BN>::WP; p++) *(v4i *)(ws + (srow + 32 * p) * LROW + scol) = st.wr[p];
    if (tid < BM) {
        // the scales are fp16 values held in fp32: converting back is exact
#pragma unroll
        for (int b = 0; b < 4; b++) dxs[b * BM + tid] = f2h(st.dx[b]);
    }
    if (tid >= 128 && tid < 128 + BN) {
        const int n = tid - 128;
        dws[0 * BN + n] = (uint16_t)(st.dw01 & 0xFFFF);
        dws[1 * BN + n] = (uint16_t)(st.dw01 >> 16);
        dws[2 * BN + n] = (uint16_t)(st.dw23 & 0xFFFF);
        dws[3 * BN + n] = (uint16_t)(st.dw23 >> 16);
    }
}

__device__ __forceinline__ _Float16 as_half(uint16_t b) {
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return h;
}

// 32 x 32 accumulator layout of the 32x32 MFMAs: lane l, register r holds (row 8*(r/4) + 4*(l/32) + r%4, col l%32).
template <int BM, int BN>
__global__ __launch_bounds__(256) void k_gemm_q8_0_i8(GemmArgs a) {
    constexpr int WM = BM / 2, WN = BN / 2;   // wave tile
    constexpr int TM = WM / 32, TN = WN / 32; // MFMA tiles per wave
    __shared__ __align__(16) int8_t xs[BM * LROW];
    __shared__ __align__(16) int8_t ws[BN * LROW];
    __shared__ uint16_t dxs[KS / 32 * BM];   // fp16 bits, [block][m]
    __shared__ uint16_t dws[KS / 32 * BN];   // fp16 bits, [block][n]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    const int K = (int)a.K;
    Stage<BM, BN> st;
    const StageSrc<BM, BN> src = stage_src<BM, BN>(a, m0, n0, tid);

    float acc[TM][TN][16];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int fr = lane & 31, fk = (lane >> 5) * 16;  // fragment row and k offset of this lane
    load_stage<BM, BN>(st, src, 0);
    for (int k0 = 0; k0 < K; k0 += KS) {
        __syncthreads();  // the previous stage's fragments have been read
        store_stage<BM, BN>(st, xs, ws, dxs, dws, tid);
        __syncthreads();
        // the next stage's loads are in flight while this stage computes (the last stage reloads itself: no branch,
        // so the staging stays in registers)
        load_stage<BM, BN>(st, src, k0 + KS < K ? k0 + KS : k0);
#pragma unroll 1
        for (int kb = 0; kb < KS / 32; kb++) {
            v4i af[TM], bf[TN];
            v4h as[TM], bs[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                af[i] = *(const v4i *)(xs + (wm + 32 * i + fr) * LROW + kb * 32 + fk);
                const _Float16 s = lane < 32 ? as_half(dxs[kb * BM + wm + 32 * i + fr]) : (_Float16)0.0f;
                as[i] = v4h{s, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                bf[j] = *(const v4i *)(ws + (wn + 32 * j + fr) * LROW + kb * 32 + fk);
                const _Float16 s = lane < 32 ? as_half(dws[kb * BN + wn + 32 * j + fr]) : (_Float16)0.0f;
                bs[j] = v4h{s, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
                    v16f fz = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                    const v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], zero, 0, 0, 0);
                    const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(as[i], bs[j], fz, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = fmaf((float)S[r], sc[r], acc[i][j][r]);
                }
        }
    }

#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int64_t n = n0 + wn + 32 * j + fr;
            if (n >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < a.M) a.y[m * a.ldy + n] = acc[i][j][r];
            }
        }
}

// ------------------------------------------------------------------------------------------------------------------
// The same products on the fp16 matrix cores. int8 quants are exact fp16 values and a 32-element block sum
// (|S| <= 32 * 127 * 127 < 2^24) is exact in the fp32 accumulator, so two chained v_mfma_f32_32x32x16_f16 give
// float(S_b) exactly -- the block sums are identical to the int8 kernel's -- and the per-block epilogue is one fma.
// Activations are written as fp16 by k_gemm_quant_q8_f16; weights are converted from int8 once per workgroup while
// a stage is staged into LDS. Stage: 64 of K (two blocks).
// ------------------------------------------------------------------------------------------------------------------
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
constexpr int KSH = 64;             // K per stage
constexpr int LROWH = KSH * 2 + 16; // padded LDS row in bytes (64 fp16)

__global__ __launch_bounds__(256) void k_gemm_quant_q8_f16(const float *x, int64_t x_stride, int64_t K, int rounding,
                                                           _Float16 *xh, float *xd) {
    const int64_t m = blockIdx.y;
    const int64_t e = (int64_t)blockIdx.x * 1024 + 4 * threadIdx.x;
    const bool valid = e < K;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) v = *(const float4 *)(x + m * x_stride + e);
    float d;
    int sum;
    const int q = quant32_lane(v, rounding, &d, &sum);
    if (valid) {
        typedef _Float16 v4h_ __attribute__((ext_vector_type(4)));
        const v4h_ h = {(_Float16)(int8_t)(q & 0xFF), (_Float16)(int8_t)((q >> 8) & 0xFF),
                        (_Float16)(int8_t)((q >> 16) & 0xFF), (_Float16)(int8_t)((q >> 24) & 0xFF)};
        *(v4h_ *)(xh + m * K + e) = h;
        if ((threadIdx.x & 7) == 0) xd[m * (K / 32) + e / 32] = h2f(f2h(d));
    }
}

// Four signed bytes -> four exact fp16 values: (0x64 << 8 | (b ^ 0x80)) is the fp16 of 1152 + b, and 1152 is
// subtracted exactly.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, v2h &lo, v2h &hi) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const v2h off = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(v2h, p0) - off;
    hi = __builtin_bit_cast(v2h, p1) - off;
}

template <int BM, int BN>
struct StageH {
    static constexpr int XP = BM * 8 / 256;   // 16-byte fp16 loads (8 per 128-byte row)
    static constexpr int WP = BN * 4 / 256;   // 16-byte int8 loads (4 per 64-byte row)
    v4i xr[XP], wr[WP];
    float dx[2];
    uint32_t dw;
};

template <int BM, int BN>
__device__ __forceinline__ void load_stage_h(StageH<BM, BN> &st, const GemmArgs &a, int64_t m0, int64_t n0,
                                             int64_t k0, int tid) {
    const int64_t K = a.K, nblk = K / 32;
#pragma unroll
    for (int p = 0; p < StageH<BM, BN>::XP; p++) {
        int64_t m = m0 + (tid >> 3) + 32 * p;
        m = m < a.M ? m : a.M - 1;
        st.xr[p] = *(const v4i *)(a.xh + m * K + k0 + (tid & 7) * 8);
    }
#pragma unroll
    for (int p = 0; p < StageH<BM, BN>::WP; p++) {
        int64_t n = n0 + (tid >> 2) + 64 * p;
        n = n < a.N ? n : a.N - 1;
        st.wr[p] = *(const v4i *)(a.w.p0 + n * K + k0 + (tid & 3) * 16);
    }
    {
        int64_t m = m0 + (tid & (BM - 1));
        m = m < a.M ? m : a.M - 1;
        const float2 f = *(const float2 *)(a.xd + m * nblk + k0 / 32);
        st.dx[0] = f.x;
        st.dx[1] = f.y;
    }
    {
        int64_t n = n0 + (tid & (BN - 1));
        n = n < a.N ? n : a.N - 1;
        st.dw = *(const uint32_t *)(a.w.p1 + (n * nblk + k0 / 32) * 2);
    }
}

template <int BM, int BN>
__device__ __forceinline__ void store_stage_h(const StageH<BM, BN> &st, uint8_t *xs, uint8_t *ws, uint16_t *dxs,
                                              uint16_t *dws, int tid) {
#pragma unroll
    for (int p = 0; p < StageH<BM, BN>::XP; p++)
        *(v4i *)(xs + ((tid >> 3) + 32 * p) * LROWH + (tid & 7) * 16) = st.xr[p];
#pragma unroll
    for (int p = 0; p < StageH<BM, BN>::WP; p++) {
        v2h h[8];
        i8x4_to_f16((uint32_t)st.wr[p].x, h[0], h[1]);
        i8x4_to_f16((uint32_t)st.wr[p].y, h[2], h[3]);
        i8x4_to_f16((uint32_t)st.wr[p].z, h[4], h[5]);
        i8x4_to_f16((uint32_t)st.wr[p].w, h[6], h[7]);
        uint8_t *dst = ws + ((tid >> 2) + 64 * p) * LROWH + (tid & 3) * 32;
        *(v4i *)dst = v4i{__builtin_bit_cast(int, h[0]), __builtin_bit_cast(int, h[1]), __builtin_bit_cast(int, h[2]),
                          __builtin_bit_cast(int, h[3])};
        *(v4i *)(dst + 16) = v4i{__builtin_bit_cast(int, h[4]), __builtin_bit_cast(int, h[5]),
                                 __builtin_bit_cast(int, h[6]), __builtin_bit_cast(int, h[7])};
    }
    if (tid < BM) {
        dxs[0 * BM + tid] = f2h(st.dx[0]);
        dxs[1 * BM + tid] = f2h(st.dx[1]);
    }
    if (tid >= 128 && tid < 128 + BN) {
        dws[0 * BN + tid - 128] = (uint16_t)(st.dw & 0xFFFF);
        dws[1 * BN + tid - 128] = (uint16_t)(st.dw >> 16);
    }
}

template <int BM, int BN>
__global__ __launch_bounds__(256) void k_gemm_q8_0_f16(GemmArgs a) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    __shared__ __align__(16) uint8_t xs[BM * LROWH];
    __shared__ __align__(16) uint8_t ws[BN * LROWH];
    __shared__ uint16_t dxs[2 * BM];
    __shared__ uint16_t dws[2 * BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    const int64_t K = a.K;
    StageH<BM, BN> st;

    float acc[TM][TN][16];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int fr = lane & 31, fk = (lane >> 5) * 16;  // fragment row; byte offset of this lane's 8 fp16
    load_stage_h<BM, BN>(st, a, m0, n0, 0, tid);
    for (int64_t k0 = 0; k0 < K; k0 += KSH) {
        __syncthreads();
        store_stage_h<BM, BN>(st, xs, ws, dxs, dws, tid);
        __syncthreads();
        load_stage_h<BM, BN>(st, a, m0, n0, k0 + KSH < K ? k0 + KSH : k0, tid);
#pragma unroll 1
        for (int kb = 0; kb < 2; kb++) {
            v8h af[TM][2], bf[TN][2];
            v4h as[TM], bs[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint8_t *row = xs + (wm + 32 * i + fr) * LROWH + kb * 64 + fk;
                af[i][0] = *(const v8h *)row;
                af[i][1] = *(const v8h *)(row + 32);
                const _Float16 s = lane < 32 ? as_half(dxs[kb * BM + wm + 32 * i + fr]) : (_Float16)0.0f;
                as[i] = v4h{s, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint8_t *row = ws + (wn + 32 * j + fr) * LROWH + kb * 64 + fk;
                bf[j][0] = *(const v8h *)row;
                bf[j][1] = *(const v8h *)(row + 32);
                const _Float16 s = lane < 32 ? as_half(dws[kb * BN + wn + 32 * j + fr]) : (_Float16)0.0f;
                bs[j] = v4h{s, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    v16f fz = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                    v16f S = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][0], bf[j][0], fz, 0, 0, 0);
                    S = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][1], bf[j][1], S, 0, 0, 0);
                    const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(as[i], bs[j], fz, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = fmaf(S[r], sc[r], acc[i][j][r]);
                }
        }
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int64_t n = n0 + wn + 32 * j + fr;
            if (n >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < a.M) a.y[m * a.ldy + n] = acc[i][j][r];
            }
        }
}

// ------------------------------------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------------------------------------
// Which matrix cores the Q8_0 products run on: 0 = int8 (the default), 1 = fp16. MX_GEMM_MODE=i8|f16 overrides it.
int gemm_mode() {
    static const int mode = [] {
        const char *e = getenv("MX_GEMM_MODE");
        return (e && strcmp(e, "f16") == 0) ? 1 : 0;
    }();
    return mode;
}

size_t gemm_act_bytes(int64_t M, int64_t K) {
    return (size_t)M * (size_t)K * (gemm_mode() ? 2 : 1);
}

hipError_t launch_gemm_quant(int type, int rounding, const float *x, int64_t x_stride, int64_t M, int64_t K,
                             void *xq, float *xd, hipStream_t s) {
    if (type != MX_TYPE_Q8_0) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((K + 1023) / 1024), (unsigned)M);
    if (gemm_mode())
        hipLaunchKernelGGL(k_gemm_quant_q8_f16, grid, dim3(256), 0, s, x, x_stride, K, rounding, (_Float16 *)xq, xd);
    else
        hipLaunchKernelGGL(k_gemm_quant_q8, grid, dim3(256), 0, s, x, x_stride, K, rounding, (int8_t *)xq, xd);
    return hipGetLastError();
}

// Tile: 64 x 128 when the grid still gives about four workgroups per CU, else 64 x 64. MX_GEMM_TILE=BMxBN overrides.
static void pick_tile(int64_t M, int64_t N, int &bm, int &bn) {
    static const char *tile_env = getenv("MX_GEMM_TILE");
    bm = 64;
    bn = ((M + 63) / 64) * ((N + 127) / 128) >= 1024 ? 128 : 64;
    if (tile_env) {
        int tm = 0, tn = 0;
        if (sscanf(tile_env, "%dx%d", &tm, &tn) == 2 && (tm == 64 || tm == 128) && (tn == 64 || tn == 128)) {
            bm = tm;
            bn = tn;
        }
    }
}

hipError_t launch_gemm(int type, const WPlanes &w, int64_t M, int64_t N, int64_t K, const void *xq, const float *xd,
                       float *y, int64_t ldy, hipStream_t s) {
    if (type != MX_TYPE_Q8_0 || K % KS != 0) return hipErrorInvalidValue;
    int bm, bn;
    pick_tile(M, N, bm, bn);
    GemmArgs a{w, M, N, K, (const int8_t *)xq, xd, y, ldy, (const _Float16 *)xq};
    const dim3 grid((unsigned)((N + bn - 1) / bn), (unsigned)((M + bm - 1) / bm));
    if (gemm_mode()) {
        if (bm == 128 && bn == 128) hipLaunchKernelGGL((k_gemm_q8_0_f16<128, 128>), grid, dim3(256), 0, s, a);
        else if (bm == 64 && bn == 128) hipLaunchKernelGGL((k_gemm_q8_0_f16<64, 128>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_gemm_q8_0_f16<64, 64>), grid, dim3(256), 0, s, a);
    } else {
        if (bm == 128 && bn == 128) hipLaunchKernelGGL((k_gemm_q8_0_i8<128, 128>), grid, dim3(256), 0, s, a);
        else if (bm == 64 && bn == 128) hipLaunchKernelGGL((k_gemm_q8_0_i8<64, 128>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_gemm_q8_0_i8<64, 64>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace mx
