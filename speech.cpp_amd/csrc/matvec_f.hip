// Small-M products on F16 / F32 weights: y[n, m] = W[n, :] . x[:, m], weights in ggml's own row-major layout.
//
// ggml-cpu pairs F16 weights with F16 activations (type_traits_cpu[F16].vec_dot_type; src1 rows go through
// ggml_cpu_fp32_to_fp16, round to nearest even) and sums the fp32 products of the fp16 values (ggml_vec_dot_f16);
// F32 weights take src1 as it is (ggml_vec_dot_f32). The products are the same here -- an fp16 x fp16 product is
// exact in fp32 -- and only the order of the fp32 sum differs.
//
// One launch: the workgroup stages its NC activation columns in LDS (rounded through fp16 for F16 weights), then each
// group of LPR lanes reduces one weight row from 16-byte loads (8 halves or 4 floats), its first chunks requested
// before the staging so that their HBM round trip overlaps it.
#include "mx_common.h"
#include "mx_device.h"

#include <cstdlib>

namespace mx {

template <int WT>
struct FChunk {
    static constexpr int elems = WT == MX_TYPE_F16 ? 8 : 4;  // elements per 16-byte load
};

constexpr int FPRE = 2;  // chunks per lane loaded before the activation staging

template <int WT>
__device__ __forceinline__ void fma_chunk(uint4 w, const float *xc, float &acc) {
    if constexpr (WT == MX_TYPE_F16) {
        const float4 x0 = *(const float4 *)xc, x1 = *(const float4 *)(xc + 4);
        acc = fmaf(h2f((uint16_t)(w.x & 0xFFFF)), x0.x, acc);
        acc = fmaf(h2f((uint16_t)(w.x >> 16)), x0.y, acc);
        acc = fmaf(h2f((uint16_t)(w.y & 0xFFFF)), x0.z, acc);
        acc = fmaf(h2f((uint16_t)(w.y >> 16)), x0.w, acc);
        acc = fmaf(h2f((uint16_t)(w.z & 0xFFFF)), x1.x, acc);
        acc = fmaf(h2f((uint16_t)(w.z >> 16)), x1.y, acc);
        acc = fmaf(h2f((uint16_t)(w.w & 0xFFFF)), x1.z, acc);
        acc = fmaf(h2f((uint16_t)(w.w >> 16)), x1.w, acc);
    } else {
        const float4 x0 = *(const float4 *)xc;
        acc = fmaf(__uint_as_float(w.x), x0.x, acc);
        acc = fmaf(__uint_as_float(w.y), x0.y, acc);
        acc = fmaf(__uint_as_float(w.z), x0.z, acc);
        acc = fmaf(__uint_as_float(w.w), x0.w, acc);
    }
}

template <int WT, int NC, int LPR>
__global__ __launch_bounds__(256) void k_matvec_f(MatvecArgs a) {
    extern __shared__ __align__(16) float xs[];  // [NC][K]
    constexpr int EL = FChunk<WT>::elems;
    constexpr int ES = WT == MX_TYPE_F16 ? 2 : 4;  // bytes per weight element
    const int K = (int)a.K;
    const int tid = threadIdx.x;
    int i12 = 0, i13 = 0, mat = 0;
    if (a.nbatch > 1) {
        const unsigned z = blockIdx.z;
        i12 = (int)(z % (unsigned)a.ne12);
        i13 = (int)(z / (unsigned)a.ne12);
        mat = (int)((unsigned)i12 / (unsigned)a.r2) + (int)((unsigned)i13 / (unsigned)a.r3) * a.ne02;
    }
    const float *x = a.x + i12 * a.x_b2 + i13 * a.x_b3;

    const MatvecProblem p = (int)blockIdx.y == 0 ? a.prob[0]
                            : ((int)blockIdx.y == 1 ? a.prob[1] : ((int)blockIdx.y == 2 ? a.prob[2] : a.prob[3]));
    constexpr int G = 64 / LPR;
    const int lane = tid & 63, wave = tid >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int64_t row = (int64_t)blockIdx.x * (4 * G) + wave * G + grp;
    const bool has_row = row < p.N;
    const int64_t grow = p.row0 + (int64_t)mat * p.N + (has_row ? row : p.N - 1);
    const uint8_t *wr = p.w.p0 + grow * (int64_t)K * ES;
    const int nchunks = K / EL;

    uint4 pre[FPRE];
#pragma unroll
    for (int i = 0; i < FPRE; i++) {
        const int c = sub + i * LPR;
        pre[i] = *(const uint4 *)(wr + (int64_t)(c < nchunks ? c : nchunks - 1) * 16);
    }

#pragma unroll
    for (int c = 0; c < NC; c++) {
        const float *xc = x + c * a.x_col_stride;
        for (int e = 4 * tid; e < K; e += 1024) {
            float4 v = *(const float4 *)(xc + e);
            if constexpr (WT == MX_TYPE_F16) {
                v.x = h2f(f2h(v.x));
                v.y = h2f(f2h(v.y));
                v.z = h2f(f2h(v.z));
                v.w = h2f(f2h(v.w));
            }
            *(float4 *)(xs + c * K + e) = v;
        }
    }
    __syncthreads();
    if (!has_row) return;  // whole LPR-lane groups leave together; no barrier follows

    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = 0.0f;
#pragma unroll
    for (int i = 0; i < FPRE; i++) {
        const int ch = sub + i * LPR;
        if (ch < nchunks)
#pragma unroll
            for (int c = 0; c < NC; c++) fma_chunk<WT>(pre[i], xs + c * K + ch * EL, acc[c]);
    }
#pragma unroll 4
    for (int ch = sub + FPRE * LPR; ch < nchunks; ch += LPR) {
        const uint4 w = *(const uint4 *)(wr + (int64_t)ch * 16);
#pragma unroll
        for (int c = 0; c < NC; c++) fma_chunk<WT>(w, xs + c * K + ch * EL, acc[c]);
    }
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = sum_lanes<LPR>(acc[c]);
    if (sub == LPR - 1) {
        float *y = p.y + i12 * a.y_b2 + i13 * a.y_b3 + row;
#pragma unroll
        for (int c = 0; c < NC; c++) y[c * p.y_col_stride] = acc[c];
    }
}

template <int WT, int NC, int LPR>
static hipError_t launch_f_one(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    constexpr int G = 64 / LPR;
    dim3 grid((unsigned)((maxN + 4 * G - 1) / (4 * G)), (unsigned)a.nprob, (unsigned)a.nbatch);
    hipLaunchKernelGGL((k_matvec_f<WT, NC, LPR>), grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int WT, int NC>
static hipError_t launch_f_nc(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    // lanes per row: the fewest (16, 32, 64) that cover the row in four 16-byte loads per lane; longer rows take 64
    const int64_t nchunks = a.K / FChunk<WT>::elems;
    if (nchunks <= 4 * 16) return launch_f_one<WT, NC, 16>(a, maxN, lds, s);
    if (nchunks <= 4 * 32) return launch_f_one<WT, NC, 32>(a, maxN, lds, s);
    return launch_f_one<WT, NC, 64>(a, maxN, lds, s);
}

template <int WT>
static hipError_t launch_f_type(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    switch (a.ncols) {
        case 1: return launch_f_nc<WT, 1>(a, maxN, lds, s);
        case 2: return launch_f_nc<WT, 2>(a, maxN, lds, s);
        case 3: return launch_f_nc<WT, 3>(a, maxN, lds, s);
        case 4: return launch_f_nc<WT, 4>(a, maxN, lds, s);
        case 5: return launch_f_nc<WT, 5>(a, maxN, lds, s);
        case 6: return launch_f_nc<WT, 6>(a, maxN, lds, s);
        case 7: return launch_f_nc<WT, 7>(a, maxN, lds, s);
        case 8: return launch_f_nc<WT, 8>(a, maxN, lds, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matvec_f(const MatvecArgs &a, hipStream_t s) {
    if (a.ids) return hipErrorInvalidValue;  // routed experts are quantized
    if (a.K % FChunk<MX_TYPE_F16>::elems != 0 && a.type == MX_TYPE_F16) return hipErrorInvalidValue;
    if (a.K % FChunk<MX_TYPE_F32>::elems != 0) return hipErrorInvalidValue;
    int64_t maxN = 0;
    for (int i = 0; i < a.nprob; i++) maxN = a.prob[i].N > maxN ? a.prob[i].N : maxN;
    if (maxN == 0) return hipSuccess;
    const size_t lds = (size_t)a.ncols * (size_t)a.K * 4;
    switch (a.type) {
        case MX_TYPE_F16: return launch_f_type<MX_TYPE_F16>(a, maxN, lds, s);
        case MX_TYPE_F32: return launch_f_type<MX_TYPE_F32>(a, maxN, lds, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
