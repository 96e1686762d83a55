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

// float4s of each activation column every thread loads ahead of the weights (elements 1024 i + 4 tid, i < XPRE).
template <int NC>
__host__ __device__ constexpr int xpre() { return NC == 1 ? 4 : (NC == 2 ? 2 : 1); }

// Quantizes the 1024-element piece at `base` of one activation column (v = elements base + 4 tid .. + 3) into LDS:
// Q8_0 weights take 32-blocks (d rounded to fp16 and back, as the CPU dot reads it), K-quants Q8_K 256-blocks with
// their 16-element sums (Q4_K: quants in unit order and sums of 32, as its dot reads them). Every wave of the
// workgroup calls it with the same `base`.
template <int TYPE>
__device__ __forceinline__ void quantize_piece(float4 v, int base, int K, int rounding, int8_t *xq, float *xd,
                                               int *xbs) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int e = base + 4 * tid;
    if constexpr (TYPE == MX_TYPE_Q8_0) {
        float d;
        int sum;
        const int q = quant32_lane(v, rounding, &d, &sum);
        if (e < K) {  // K % 32 == 0: the eight lanes of a block agree
            *(int *)(xq + e) = q;
            if ((tid & 7) == 0) xd[e / 32] = h2f(f2h(d));
        }
    } else {
        if (base + 256 * (tid >> 6) < K) {  // a whole wave per super-block
            float d;
            int bs;
            const int q = quant256_wave(v, lane, &d, &bs);
            if (lane == 0) xd[e / 256] = d;
            if constexpr (TYPE == MX_TYPE_Q4_K) {  // unit order, and sums of 32
                *(int *)(xq + q4u_xq_offset(e, K)) = q;
                const int bs32 = bs + dpp_i<dpp::HALF_MIRROR>(0, bs);  // lanes 8j..8j+7: quants 32j..32j+31
                if ((lane & 7) == 0) xbs[e / 32] = bs32;
            } else {
                *(int *)(xq + e) = q;
                if ((lane & 3) == 0) xbs[e / 16] = bs;
            }
        }
    }
}

__device__ __forceinline__ float4 load_x4(const float *xc, int e, int K) {
    const float4 v = *(const float4 *)(xc + (e < K ? e : K - 4));
    return e < K ? v : make_float4(0.f, 0.f, 0.f, 0.f);
}

// The fused prologue: each column x becomes silu(x) * glu_b (ggml_vec_swiglu_f32's scalar form) when glu_b is set,
// then mul(rms_norm(x, eps), norm_w) when norm_w is set -- the squares (rounded to float) summed in double over the
// workgroup, the mean rounded to float, x * (1 / sqrtf(mean + eps)) then times the weight, as the separate ops round
// -- and is quantized. Pieces of 1024 elements past the preloaded ones are read again after the sum.
template <int TYPE, int NC>
__device__ __forceinline__ void fused_prologue(const MatvecArgs &a, const float *x, int xi12, int i13,
                                               float4 (&xr)[NC][xpre<NC>()], const float4 (&br)[NC][xpre<NC>()],
                                               const float4 (&wr)[xpre<NC>()], int8_t *xq, float *xd, int *xbs) {
    constexpr int XP = xpre<NC>();
    constexpr int XDB = TYPE == MX_TYPE_Q8_0 ? 32 : 256;
    const int K = (int)a.K;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ double red[NC][4];
    const float *gb = a.glu_b ? a.glu_b + xi12 * a.x_b2 + i13 * a.x_b3 : nullptr;
    // glu of one loaded piece; the preloaded pieces' second operands came in with x (br)
    auto piece_b = [&](float4 v, float4 b) -> float4 {
        v.x = v.x / (1.0f + expf(-v.x)) * b.x;
        v.y = v.y / (1.0f + expf(-v.y)) * b.y;
        v.z = v.z / (1.0f + expf(-v.z)) * b.z;
        v.w = v.w / (1.0f + expf(-v.w)) * b.w;
        return v;
    };
    auto piece = [&](int c, int base, float4 v) -> float4 {
        if (gb) {
            const float4 b = load_x4(gb + c * a.x_col_stride, base + 4 * tid, K);
            v.x = v.x / (1.0f + expf(-v.x)) * b.x;
            v.y = v.y / (1.0f + expf(-v.y)) * b.y;
            v.z = v.z / (1.0f + expf(-v.z)) * b.z;
            v.w = v.w / (1.0f + expf(-v.w)) * b.w;
        }
        return v;
    };
    if (gb) {
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int i = 0; i < XP; i++) xr[c][i] = piece_b(xr[c][i], br[c][i]);
    }
    float scale[NC];
    if (a.norm_w) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < XP; i++) {
                const float4 v = xr[c][i];  // zero past K
                ss += (double)(v.x * v.x) + (double)(v.y * v.y) + (double)(v.z * v.z) + (double)(v.w * v.w);
            }
            for (int base = 1024 * XP; base < K; base += 1024) {
                const float4 v = piece(c, base, load_x4(x + c * a.x_col_stride, base + 4 * tid, K));
                ss += (double)(v.x * v.x) + (double)(v.y * v.y) + (double)(v.z * v.z) + (double)(v.w * v.w);
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
            if (lane == 0) red[c][wave] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const double tot = red[c][0] + red[c][1] + red[c][2] + red[c][3];
            const float mean = (float)(tot / (double)K);
            scale[c] = 1.0f / sqrtf(mean + a.norm_eps);
        }
    }
    auto normed = [&](int c, int base, float4 v) -> float4 {
        if (a.norm_w) {
            const float4 w = base < 1024 * XP ? wr[base / 1024] : load_x4(a.norm_w, base + 4 * tid, K);
            v.x = (v.x * scale[c]) * w.x;
            v.y = (v.y * scale[c]) * w.y;
            v.z = (v.z * scale[c]) * w.z;
            v.w = (v.w * scale[c]) * w.w;
        }
        return v;
    };
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const float *xc = x + c * a.x_col_stride;
#pragma unroll
        for (int i = 0; i < XP; i++)
            if (1024 * i < K)
                quantize_piece<TYPE>(normed(c, 1024 * i, xr[c][i]), 1024 * i, K, a.rounding, xq + c * K,
                                     xd + c * (K / XDB), xbs + c * xbs_per_col<TYPE>(K));
        for (int base = 1024 * XP; base < K; base += 1024)
            quantize_piece<TYPE>(normed(c, base, piece(c, base, load_x4(xc, base + 4 * tid, K))), base, K, a.rounding,
                                 xq + c * K, xd + c * (K / XDB), xbs + c * xbs_per_col<TYPE>(K));
    }
}

// FUSED: the instantiation that reads the fused operands (norm weight, SwiGLU input, residual); the plain one is
// compiled without them, so products with no fusion keep their smaller register footprint.
template <int TYPE, int NC, int LPR, bool FUSED>
__global__ __launch_bounds__(256) void k_matvec(MatvecArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int K = (int)a.K;
    const int tid = threadIdx.x;
    // The argument block's fields on the way to the first weight load, requested together into scalar registers:
    // left to the compiler, the branches below would each wait on a scalar load of their own, several round trips in
    // a row before the weights could be requested.
    const MatvecProblem p = pick_problem(a, (int)blockIdx.y);
    {
        const int nbatch = a.nbatch, rounding = a.rounding;
        const int32_t *ids = a.ids;
        const float *xa = a.x;
        const int64_t xcs = a.x_col_stride;
        asm volatile("" ::"s"(nbatch), "s"(rounding), "s"(ids), "s"(xa), "s"(xcs), "s"(a.K), "s"(a.x_b2), "s"(a.x_b3),
                     "s"(p.w.p0), "s"(p.w.p1), "s"(p.N), "s"(p.row0));
        if constexpr (TYPE != MX_TYPE_Q8_0) asm volatile("" ::"s"(p.w.p2));
        if constexpr (TYPE == MX_TYPE_Q5_K || TYPE == MX_TYPE_Q6_K) asm volatile("" ::"s"(p.w.p3));
        if constexpr (FUSED) asm volatile("" ::"s"(a.glu_b), "s"(a.norm_w), "s"(p.res));
    }
    // Batch slice; a single slice (decode) takes no division.
    int i12 = 0, i13 = 0, mat = 0;
    if (a.nbatch > 1) {
        const unsigned z = blockIdx.z;
        i12 = (int)(z % (unsigned)a.ne12);
        i13 = (int)(z / (unsigned)a.ne12);
        mat = (int)((unsigned)i12 / (unsigned)a.r2) + (int)((unsigned)i13 / (unsigned)a.r3) * a.ne02;
    }
    int xi12 = i12;
    if (a.ids) {  // routed expert: the slice's matrix comes from ids (uniform over the workgroup)
        mat = *(const int32_t *)((const uint8_t *)a.ids + i12 * a.ids_nb0 + i13 * a.ids_nb1);
        if (mat < 0 || mat >= a.n_mats) {  // ggml-cpu asserts; this pair's output is left as it was and reported
            if (tid == 0) atomicOr(a.err, 2);
            return;
        }
        xi12 = (int)((unsigned)i12 % (unsigned)a.x_ne12);
    }
    const float *x = a.x + xi12 * a.x_b2 + i13 * a.x_b3;

    // The activation loads go first: x -> quantization -> LDS is the prologue's critical path, and the memory counter
    // retires loads in order, so waiting for x then does not wait for the weight loads issued after it.
    constexpr int XP = xpre<NC>();
    float4 xr[NC][XP];
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
        for (int i = 0; i < XP; i++) xr[c][i] = load_x4(x + c * a.x_col_stride, 1024 * i + 4 * tid, K);
    // the fused prologue's other operands come in with x: SwiGLU's second input and the norm weight
    float4 br[NC][XP], wr[XP];
    if (FUSED && a.glu_b) {
        const float *gb = a.glu_b + xi12 * a.x_b2 + i13 * a.x_b3;
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int i = 0; i < XP; i++) br[c][i] = load_x4(gb + c * a.x_col_stride, 1024 * i + 4 * tid, K);
    }
    if (FUSED && a.norm_w) {
#pragma unroll
        for (int i = 0; i < XP; i++) wr[i] = load_x4(a.norm_w, 1024 * i + 4 * tid, K);
    }

    constexpr int G = 64 / LPR;  // rows in flight per wave
    const int lane = tid & 63, wave = tid >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int64_t row = (int64_t)blockIdx.x * (4 * G) + wave * G + grp;
    const bool has_row = row < p.N;
    // Rows past the end load (and then ignore) the last row, chunks past the end the last chunk: the preloads carry no
    // lane-dependent branch, so they issue back to back.
    const int64_t grow = p.row0 + (int64_t)mat * p.N + (has_row ? row : p.N - 1);
    const int nchunks = K / chunk_elems<TYPE>();

    // the residual the epilogue adds, requested now rather than after the reduction
    const int64_t yoff = i12 * a.y_b2 + i13 * a.y_b3 + row;
    float rr[NC];
    if (FUSED && p.res && has_row && sub == LPR - 1) {
#pragma unroll
        for (int c = 0; c < NC; c++) rr[c] = p.res[yoff + c * p.y_col_stride];
    }

    // weight chunks requested before the activation prologue, so the weight stream's first HBM round trip overlaps
    // the load and quantization of x instead of following it
    constexpr int PRE = preload_of<TYPE>();
    WChunk<TYPE> pre[PRE];
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const int c = sub + i * LPR;
        pre[i] = load_chunk<TYPE>(p.w, grow, K, c < nchunks ? c : nchunks - 1);
    }

    int8_t *xq = (int8_t *)smem;
    float *xd = (float *)(smem + (size_t)NC * K);
    constexpr int XDB = TYPE == MX_TYPE_Q8_0 ? 32 : 256;
    int *xbs = (int *)(xd + NC * (K / XDB));
    if constexpr (FUSED) {
        if (a.glu_b || a.norm_w) {  // uniform: the fused prologue
            fused_prologue<TYPE, NC>(a, x, xi12, i13, xr, br, wr, xq, xd, xbs);
        } else {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const float *xc = x + c * a.x_col_stride;
#pragma unroll
                for (int i = 0; i < XP; i++)
                    if (1024 * i < K)
                        quantize_piece<TYPE>(xr[c][i], 1024 * i, K, a.rounding, xq + c * K, xd + c * (K / XDB),
                                             xbs + c * xbs_per_col<TYPE>(K));
                for (int base = 1024 * XP; base < K; base += 1024)
                    quantize_piece<TYPE>(load_x4(xc, base + 4 * tid, K), base, K, a.rounding, xq + c * K,
                                         xd + c * (K / XDB), xbs + c * xbs_per_col<TYPE>(K));
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const float *xc = x + c * a.x_col_stride;
#pragma unroll
            for (int i = 0; i < XP; i++)
                if (1024 * i < K) quantize_piece<TYPE>(xr[c][i], 1024 * i, K, a.rounding, xq + c * K, xd + c * (K / XDB),
                                                       xbs + c * xbs_per_col<TYPE>(K));
            for (int base = 1024 * XP; base < K; base += 1024)
                quantize_piece<TYPE>(load_x4(xc, base + 4 * tid, K), base, K, a.rounding, xq + c * K,
                                     xd + c * (K / XDB), xbs + c * xbs_per_col<TYPE>(K));
        }
    }
    __syncthreads();
    if (!has_row) return;  // whole LPR-lane groups leave together; no barrier follows

    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = 0.0f;
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const int c = sub + i * LPR;
        if (c < nchunks) dot_chunk<TYPE, NC, false>(pre[i], K, c, xq, xd, xbs, NC, acc);
    }
    if constexpr (TYPE == MX_TYPE_Q4_K) {  // a unit's registers are four chunks': one at a time
#pragma unroll 1
        for (int c = sub + PRE * LPR; c < nchunks; c += LPR)
            chunk_dot<TYPE, NC, false>(p.w, grow, K, c, xq, xd, xbs, NC, acc);
    } else {
#pragma unroll 4
        for (int c = sub + PRE * LPR; c < nchunks; c += LPR)
            chunk_dot<TYPE, NC, false>(p.w, grow, K, c, xq, xd, xbs, NC, acc);
    }
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = sum_lanes<LPR>(acc[c]);
    if (sub == LPR - 1) {  // the lane holding the group's sum
        float *y = p.y + yoff;
        if (FUSED && p.res) {  // the residual ADD that follows the product, fused
#pragma unroll
            for (int c = 0; c < NC; c++) y[c * p.y_col_stride] = rr[c] + acc[c];
        } else {
#pragma unroll
            for (int c = 0; c < NC; c++) y[c * p.y_col_stride] = acc[c];
        }
    }
}

// Lanes per row: the fewest (16, 32 or 64) whose chunks per lane all fit the preload, so every weight byte of a lane
// is requested before the activation prologue; rows longer than that take 64 lanes. Measured on the decode shapes
// (K 1024..3072): one full preload beats more workgroups with shorter streams. A backend's option forces it.
static int pick_lpr(int64_t nchunks, int preload, int forced) {
    if (forced == 16 || forced == 32 || forced == 64) return forced;
    int lpr = 16;
    while (lpr < 64 && nchunks > (int64_t)preload * lpr) lpr *= 2;
    return lpr;
}

template <int TYPE, int NC, int LPR>
static hipError_t launch_one(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    constexpr int G = 64 / LPR;
    dim3 grid((unsigned)((maxN + 4 * G - 1) / (4 * G)), (unsigned)a.nprob, (unsigned)a.nbatch);
    bool fused = a.glu_b || a.norm_w;
    for (int i = 0; i < a.nprob; i++) fused = fused || a.prob[i].res;
    if (fused) hipLaunchKernelGGL((k_matvec<TYPE, NC, LPR, true>), grid, dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_matvec<TYPE, NC, LPR, false>), grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int TYPE, int NC>
static hipError_t launch_nc(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    const int64_t nchunks = a.K / chunk_elems<TYPE>();
    switch (pick_lpr(nchunks, preload_of<TYPE>(), a.lpr)) {
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
    if (a.type == MX_TYPE_F16 || a.type == MX_TYPE_F32) return launch_matvec_f(a, s);
    const size_t lds = act_lds_bytes(a.type, a.K, a.ncols);
    switch (a.type) {
        case MX_TYPE_Q8_0: return launch_type<MX_TYPE_Q8_0>(a, maxN, lds, s);
        case MX_TYPE_Q4_K: return launch_type<MX_TYPE_Q4_K>(a, maxN, lds, s);
        case MX_TYPE_Q5_K: return launch_type<MX_TYPE_Q5_K>(a, maxN, lds, s);
        case MX_TYPE_Q6_K: return launch_type<MX_TYPE_Q6_K>(a, maxN, lds, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
