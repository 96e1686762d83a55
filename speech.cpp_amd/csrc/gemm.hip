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
// Host side.
// ------------------------------------------------------------------------------------------------------------------
size_t gemm_act_bytes(int64_t M, int64_t K) { return (size_t)M * (size_t)K; }

hipError_t launch_gemm_quant(int type, int rounding, const float *x, int64_t x_stride, int64_t M, int64_t K,
                             void *xq, float *xd, hipStream_t s) {
    if (type != MX_TYPE_Q8_0) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((K + 1023) / 1024), (unsigned)M);
    hipLaunchKernelGGL(k_gemm_quant_q8, grid, dim3(256), 0, s, x, x_stride, K, rounding, (int8_t *)xq, xd);
    return hipGetLastError();
}

// Tile: 64 x 128 when the grid still gives about four workgroups per CU, else 64 x 64. A backend's tile option
// (tile_m x tile_n: 64 x 64, 64 x 128 or 128 x 128) overrides it; any other forced pair is refused.
static bool pick_tile(int64_t M, int64_t N, const Options &o, int &bm, int &bn) {
    bm = 64;
    bn = ((M + 63) / 64) * ((N + 127) / 128) >= 1024 ? 128 : 64;
    if (o.tile_m || o.tile_n) {
        if (!((o.tile_m == 64 && (o.tile_n == 64 || o.tile_n == 128)) || (o.tile_m == 128 && o.tile_n == 128)))
            return false;
        bm = o.tile_m;
        bn = o.tile_n;
    }
    return true;
}

hipError_t launch_gemm(int type, const WPlanes &w, int64_t M, int64_t N, int64_t K, const void *xq, const float *xd,
                       float *y, int64_t ldy, const Options &o, hipStream_t s) {
    if (type != MX_TYPE_Q8_0 || K % KS != 0) return hipErrorInvalidValue;
    int bm, bn;
    if (!pick_tile(M, N, o, bm, bn)) return hipErrorInvalidValue;
    GemmArgs a{w, M, N, K, (const int8_t *)xq, xd, y, ldy};
    const dim3 grid((unsigned)((N + bn - 1) / bn), (unsigned)((M + bm - 1) / bm));
    if (bm == 128 && bn == 128) hipLaunchKernelGGL((k_gemm_q8_0_i8<128, 128>), grid, dim3(256), 0, s, a);
    else if (bm == 64 && bn == 128) hipLaunchKernelGGL((k_gemm_q8_0_i8<64, 128>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_gemm_q8_0_i8<64, 64>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mx
