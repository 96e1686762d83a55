// MUL_MAT_ID for routed experts: dst[:, s, t] = as[ids[s, t]] . quant(b[:, s % b_ne1, t]).
//
// Three launches, no host round trip:
//   1. bucket: one workgroup counts (token, slot) pairs per expert, builds the list of experts that have any, and
//      groups the pairs by expert (the matrix_row_counts / matrix_rows of ggml-cpu.c ggml_compute_forward_mul_mat_id).
//   2. quant: every activation row is quantized once (ggml-cpu quantizes src1 once, before the experts run).
//   3. experts: grid.y walks the experts that were touched; each workgroup streams a tile of its expert's rows once
//      and applies it to up to 8 of the expert's pairs per pass, so an expert's weights are read once per 8 pairs and
//      untouched experts cost nothing.
#include "mx_common.h"
#include "mx_device.h"
#include "mx_dot.h"

namespace mx {

static inline size_t al256(size_t v) { return (v + 255) / 256 * 256; }

size_t mul_mat_id_scratch(MulMatIdArgs *a, void *base) {
    const int64_t npairs = a->n_ids * a->T;
    const int64_t nrows = a->T * a->b_ne1;
    const int64_t nsc = a->type == MX_TYPE_Q8_0 ? a->K / 32 : a->K / 256;
    size_t off = 0;
    uint8_t *b = (uint8_t *)base;
    a->counts = (int32_t *)(b + off);  off += al256((size_t)a->E * 4);
    a->offsets = (int32_t *)(b + off); off += al256((size_t)a->E * 4);
    a->active = (int32_t *)(b + off);  off += al256((size_t)(a->E + 1) * 4);
    a->pairs = (int32_t *)(b + off);   off += al256((size_t)npairs * 4);
    a->xq = (int8_t *)(b + off);       off += al256((size_t)nrows * (size_t)a->K);
    a->xd = (float *)(b + off);        off += al256((size_t)nrows * (size_t)nsc * 4);
    a->xbs = (int32_t *)(b + off);     off += al256(a->type == MX_TYPE_Q8_0 ? 0 : (size_t)nrows * (size_t)(a->K / 16) * 4);
    return off;
}

__global__ __launch_bounds__(1024) void k_mmid_bucket(MulMatIdArgs a) {
    extern __shared__ int cnt[];  // [E]
    const int64_t npairs = a.n_ids * a.T;
    for (int64_t e = threadIdx.x; e < a.E; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int64_t p = threadIdx.x; p < npairs; p += 1024) {
        const int64_t t = p / a.n_ids, s = p % a.n_ids;
        const int32_t e = *(const int32_t *)((const uint8_t *)a.ids + s * a.ids_nb0 + t * a.ids_nb1);
        if (e < 0 || e >= a.E) atomicOr(a.err, 2);  // ggml-cpu asserts; this pair is dropped and reported
        else atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0, nact = 0;
        for (int64_t e = 0; e < a.E; e++) {
            const int c = cnt[e];
            a.counts[e] = c;
            a.offsets[e] = run;
            if (c > 0) a.active[1 + nact++] = (int32_t)e;
            cnt[e] = run;  // becomes the fill cursor
            run += c;
        }
        a.active[0] = nact;
    }
    __syncthreads();
    for (int64_t p = threadIdx.x; p < npairs; p += 1024) {
        const int64_t t = p / a.n_ids, s = p % a.n_ids;
        const int32_t e = *(const int32_t *)((const uint8_t *)a.ids + s * a.ids_nb0 + t * a.ids_nb1);
        if (e < 0 || e >= a.E) continue;
        const int pos = atomicAdd(&cnt[e], 1);
        a.pairs[pos] = (int32_t)p;
    }
}

// Quantizes activation row r = t * b_ne1 + s' of b into the scratch rows (same arithmetic as the fused prologue).
template <int TYPE>
__global__ __launch_bounds__(256) void k_mmid_quant(MulMatIdArgs a) {
    const int64_t r = blockIdx.y;
    const int64_t t = r / a.b_ne1, s = r % a.b_ne1;
    const float *x = (const float *)((const uint8_t *)a.b + s * a.b_nb1 + t * a.b_nb2);
    const int64_t K = a.K;
    const int64_t e = (int64_t)blockIdx.x * 1024 + 4 * threadIdx.x;
    const int lane = threadIdx.x & 63;
    if (TYPE == MX_TYPE_Q8_0) {
        const bool valid = e < K;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (valid) v = *(const float4 *)(x + e);
        float d;
        int sum;
        const int q = quant32_lane(v, a.rounding, &d, &sum);
        if (valid) {
            *(int *)(a.xq + r * K + e) = q;
            if ((threadIdx.x & 7) == 0) a.xd[r * (K / 32) + e / 32] = h2f(f2h(d));
        }
    } else {
        if ((int64_t)blockIdx.x * 1024 + 256 * (threadIdx.x >> 6) >= K) return;  // whole wave
        const float4 v = *(const float4 *)(x + e);
        float d;
        int bs;
        const int q = quant256_wave(v, lane, &d, &bs);
        *(int *)(a.xq + r * K + e) = q;
        if (lane == 0) a.xd[r * (K / 256) + e / 256] = d;
        if ((lane & 3) == 0) a.xbs[r * (K / 16) + e / 16] = bs;
    }
}

template <int TYPE, int LPR>
__global__ __launch_bounds__(256) void k_mmid_experts(MulMatIdArgs a) {
    constexpr int NC = MAX_COLS;
    extern __shared__ __align__(16) uint8_t smem[];
    const int j = blockIdx.y;
    const int nact = a.active[0];
    if (j >= nact) return;  // uniform: the whole workgroup leaves
    const int e = a.active[1 + j];
    const int cnt = a.counts[e], off = a.offsets[e];
    const int64_t K = a.K;
    const int64_t nsc = TYPE == MX_TYPE_Q8_0 ? K / 32 : K / 256;
    int8_t *xq = (int8_t *)smem;
    float *xd = (float *)(smem + (size_t)NC * K);
    int *xbs = (int *)(xd + NC * nsc);

    constexpr int G = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int64_t row = (int64_t)blockIdx.x * (4 * G) + wave * G + grp;
    const bool has_row = row < a.N;
    const int64_t grow = (int64_t)e * a.N + row;
    const int nchunks = (int)(K / chunk_elems<TYPE>());

    for (int g0 = 0; g0 < cnt; g0 += NC) {
        const int ng = cnt - g0 < NC ? cnt - g0 : NC;
        __syncthreads();  // the previous pass is done with LDS
        for (int col = 0; col < ng; col++) {
            const int p = a.pairs[off + g0 + col];
            const int64_t t = p / a.n_ids, s = p % a.n_ids;
            const int64_t r = t * a.b_ne1 + (s % a.b_ne1);
            for (int64_t k = 16 * threadIdx.x; k < K; k += 16 * 256)
                *(int4 *)(xq + col * K + k) = *(const int4 *)(a.xq + r * K + k);
            for (int64_t k = threadIdx.x; k < nsc; k += 256) xd[col * nsc + k] = a.xd[r * nsc + k];
            if (TYPE != MX_TYPE_Q8_0)
                for (int64_t k = threadIdx.x; k < K / 16; k += 256) xbs[col * (K / 16) + k] = a.xbs[r * (K / 16) + k];
        }
        __syncthreads();
        if (has_row) {
            float acc[NC];
#pragma unroll
            for (int c = 0; c < NC; c++) acc[c] = 0.0f;
#pragma unroll 2
            for (int c = sub; c < nchunks; c += LPR) chunk_dot<TYPE, NC, true>(a.w, grow, K, c, xq, xd, xbs, ng, acc);
#pragma unroll
            for (int c = 0; c < NC; c++) acc[c] = sum_lanes<LPR>(acc[c]);
            if (sub == LPR - 1) {  // the lane holding the group's sum
#pragma unroll
                for (int col = 0; col < NC; col++) {
                    if (col < ng) {
                        const int p = a.pairs[off + g0 + col];
                        const int64_t t = p / a.n_ids, s = p % a.n_ids;
                        float *y = (float *)((uint8_t *)a.dst + s * a.dst_nb1 + t * a.dst_nb2);
                        y[row] = acc[col];
                    }
                }
            }
        }
    }
}

template <int TYPE>
static hipError_t launch_typed(const MulMatIdArgs &a, hipStream_t s) {
    const int64_t nrows = a.T * a.b_ne1;
    hipLaunchKernelGGL(k_mmid_bucket, dim3(1), dim3(1024), (size_t)a.E * 4, s, a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_mmid_quant<TYPE>, dim3((unsigned)((a.K + 1023) / 1024), (unsigned)nrows), dim3(256), 0, s, a);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int64_t npairs = a.n_ids * a.T;
    const unsigned gy = (unsigned)(npairs < a.E ? npairs : a.E);
    const size_t lds = act_lds_bytes(TYPE, a.K, MAX_COLS);
    const int64_t nchunks = a.K / chunk_elems<TYPE>();
    if (nchunks <= 128) {
        hipLaunchKernelGGL((k_mmid_experts<TYPE, 16>), dim3((unsigned)((a.N + 15) / 16), gy), dim3(256), lds, s, a);
    } else if (nchunks <= 256) {
        hipLaunchKernelGGL((k_mmid_experts<TYPE, 32>), dim3((unsigned)((a.N + 7) / 8), gy), dim3(256), lds, s, a);
    } else {
        hipLaunchKernelGGL((k_mmid_experts<TYPE, 64>), dim3((unsigned)((a.N + 3) / 4), gy), dim3(256), lds, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_mul_mat_id(const MulMatIdArgs &a, hipStream_t s) {
    if (a.n_ids * a.T == 0 || a.N == 0) return hipSuccess;
    switch (a.type) {
        case MX_TYPE_Q8_0: return launch_typed<MX_TYPE_Q8_0>(a, s);
        case MX_TYPE_Q4_K: return launch_typed<MX_TYPE_Q4_K>(a, s);
        case MX_TYPE_Q6_K: return launch_typed<MX_TYPE_Q6_K>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
