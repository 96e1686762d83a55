// Small-M quantized products (decode M = 1, draft verification M <= 5): y[n, m] = W[n, :] . quant(x[:, m]).
//
// One launch does everything: the workgroup first quantizes its NC activation columns into LDS (the ggml CPU src1
// conversion, bit for bit), then streams weight rows with 16-byte loads from the planar layout and reduces each row
// over LPR lanes. HBM-bound by design: each weight byte is read once per launch.
#include "mx_common.h"
#include "mx_device.h"
#include "mx_dot.h"

#include <cstdlib>

namespace mx {

__device__ __forceinline__ MatvecProblem pick_problem(const MatvecArgs &a, int i) {
    // Uniform selection keeps the kernel-argument struct out of private memory.
    return i == 0 ? a.prob[0] : (i == 1 ? a.prob[1] : (i == 2 ? a.prob[2] : a.prob[3]));
}

// Chunks of weights each lane loads before the activation prologue, so the weight stream's first HBM round trip
// overlaps the load and quantization of x instead of following it.
constexpr int PRELOAD = 4;

template <int TYPE, int NC, int LPR>
__global__ __launch_bounds__(256) void k_matvec(MatvecArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int64_t K = a.K;
    const int64_t z = blockIdx.z;
    const int64_t i12 = z % a.ne12, i13 = z / a.ne12;
    const MatvecProblem p = pick_problem(a, (int)blockIdx.y);
    constexpr int G = 64 / LPR;  // rows in flight per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int64_t row = (int64_t)blockIdx.x * (4 * G) + wave * G + grp;
    const bool has_row = row < p.N;
    // Rows past the end load (and then ignore) the last row, chunks past the end the last chunk: the preloads carry no
    // branch, so they issue back to back.
    const int64_t grow = p.row0 + (i12 / a.r2 + (i13 / a.r3) * a.ne02) * p.N + (has_row ? row : p.N - 1);
    const int nchunks = (int)(K / chunk_elems<TYPE>());

    WChunk<TYPE> pre[PRELOAD];
#pragma unroll
    for (int i = 0; i < PRELOAD; i++) {
        const int c = sub + i * LPR;
        pre[i] = load_chunk<TYPE>(p.w, grow, K, c < nchunks ? c : nchunks - 1);
    }

    const float *x = a.x + i12 * a.x_b2 + i13 * a.x_b3;
    int8_t *xq = (int8_t *)smem;
    float *xd = (float *)(smem + (size_t)NC * K);
    int *xbs = (int *)(xd + NC * (TYPE == MX_TYPE_Q8_0 ? K / 32 : K / 256));
    quantize_cols_to_lds<TYPE, NC, false>(x, a.x_col_stride, K, NC, a.rounding, xq, xd, xbs);
    __syncthreads();
    if (!has_row) return;  // whole LPR-lane groups leave together; no barrier follows

    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = 0.0f;
#pragma unroll
    for (int i = 0; i < PRELOAD; i++) {
        const int c = sub + i * LPR;
        if (c < nchunks) dot_chunk<TYPE, NC, false>(pre[i], K, c, xq, xd, xbs, NC, acc);
    }
#pragma unroll 4
    for (int c = sub + PRELOAD * LPR; c < nchunks; c += LPR)
        chunk_dot<TYPE, NC, false>(p.w, grow, K, c, xq, xd, xbs, NC, acc);
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = sum_lanes<LPR>(acc[c]);
    if (sub == 0) {
        float *y = p.y + i12 * a.y_b2 + i13 * a.y_b3 + row;
#pragma unroll
        for (int c = 0; c < NC; c++) y[c * p.y_col_stride] = acc[c];
    }
}

template <int TYPE, int NC, int LPR>
static hipError_t launch_one(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    constexpr int G = 64 / LPR;
    dim3 grid((unsigned)((maxN + 4 * G - 1) / (4 * G)), (unsigned)a.nprob, (unsigned)(a.ne12 * a.ne13));
    hipLaunchKernelGGL((k_matvec<TYPE, NC, LPR>), grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

// Lanes per row: the fewest lanes (longest per-lane streams) that still give the launch enough workgroups to cover
// the chip twice; small matrices get more lanes per row and so more, shorter workgroups. MX_MATVEC_LPR overrides it.
static int pick_lpr(int64_t nchunks, int64_t maxN, int nprob, int64_t batches) {
    static const int forced = [] {
        const char *e = getenv("MX_MATVEC_LPR");
        return e ? atoi(e) : 0;
    }();
    if (forced == 16 || forced == 32 || forced == 64) return forced;
    const int64_t target = 512;
    for (int lpr = 16; lpr <= 64; lpr *= 2) {
        if (lpr > 16 && nchunks < lpr) return lpr / 2;
        const int64_t rows_per_wg = 4 * (64 / lpr);
        const int64_t wgs = (maxN + rows_per_wg - 1) / rows_per_wg * nprob * batches;
        if (wgs >= target) return lpr;
    }
    return nchunks >= 64 ? 64 : (nchunks >= 32 ? 32 : 16);
}

template <int TYPE, int NC>
static hipError_t launch_nc(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    const int64_t nchunks = a.K / chunk_elems<TYPE>();
    switch (pick_lpr(nchunks, maxN, a.nprob, a.ne12 * a.ne13)) {
        case 16: return launch_one<TYPE, NC, 16>(a, maxN, lds, s);
        case 32: return launch_one<TYPE, NC, 32>(a, maxN, lds, s);
        default: return launch_one<TYPE, NC, 64>(a, maxN, lds, s);
    }
}

template <int TYPE>
static hipError_t launch_type(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    switch (a.ncols) {
        case 1: return launch_nc<TYPE, 1>(a, maxN, lds, s);
        case 2: return launch_nc<TYPE, 2>(a, maxN, lds, s);
        case 3: return launch_nc<TYPE, 3>(a, maxN, lds, s);
        case 4: return launch_nc<TYPE, 4>(a, maxN, lds, s);
        case 5: return launch_nc<TYPE, 5>(a, maxN, lds, s);
        case 6: return launch_nc<TYPE, 6>(a, maxN, lds, s);
        case 7: return launch_nc<TYPE, 7>(a, maxN, lds, s);
        case 8: return launch_nc<TYPE, 8>(a, maxN, lds, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matvec(const MatvecArgs &a, hipStream_t s) {
    int64_t maxN = 0;
    for (int i = 0; i < a.nprob; i++) maxN = a.prob[i].N > maxN ? a.prob[i].N : maxN;
    if (maxN == 0) return hipSuccess;
    const size_t lds = act_lds_bytes(a.type, a.K, a.ncols);
    switch (a.type) {
        case MX_TYPE_Q8_0: return launch_type<MX_TYPE_Q8_0>(a, maxN, lds, s);
        case MX_TYPE_Q4_K: return launch_type<MX_TYPE_Q4_K>(a, maxN, lds, s);
        case MX_TYPE_Q6_K: return launch_type<MX_TYPE_Q6_K>(a, maxN, lds, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
