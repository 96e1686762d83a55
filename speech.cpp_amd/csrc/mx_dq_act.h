// The activation rows of the fp16 dequantizing GEMM (gemm_dq.hip), one row per workgroup of NT threads: the row
// quantized exactly as ggml-cpu quantizes src1 for the weight's vec_dot (Q8_0 blocks with the fp16-rounded d for Q8_0
// weights, Q8_K blocks with their fp32 d for the K-quants), written as fp16(2^e d q) with the row's 2^-e beside it.
// Shared by the dense GEMM's activation pass and the MUL_MAT_ID prep that feeds the GEMM's routed-expert form.
#pragma once

#include "mx_device.h"

namespace mx {

typedef _Float16 dq_v4h __attribute__((ext_vector_type(4)));

// The fp16 activation values of a row carry a power-of-two scale 2^e, e chosen so that the row's largest |d q| lands
// in [2^14, 2^15): clear of fp16's overflow (65504) and of its subnormals, where ggml's fp32 sums lose nothing. The
// GEMM multiplies its sums by rs[m] = 2^-e. Both scalings are exact, so a row that fp16 already holds in its normal
// range gives the same bits as unscaled values would. e is at most 126, so rs stays a normal float: a row whose
// largest |d q| is below 2^-112 (possible with Q8_K's fp32 d) lands lower than 2^14 but still in fp16's normal range
// down to 2^-140.
__device__ __forceinline__ int dq_row_exp(float amax) {
    if (amax == 0.0f) return 0;
    int E = (int)((__float_as_uint(amax) >> 23) & 0xFF);  // amax in [2^(E-127), 2^(E-126))
    if (E == 0) E = 1;
    const int e = 141 - E;
    return e < -126 ? -126 : (e > 126 ? 126 : e);  // 2^-e stays a normal float (2^-127 would be subnormal)
}
__device__ __forceinline__ float dq_pow2(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

template <int NT>
__device__ __forceinline__ float dq_block_max(float v, float *red) {  // over an NT-thread workgroup; red: NT / 64
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) r = fmaxf(r, red[w]);
    return r;
}

constexpr int DQ_ACT_REG = 4;  // 4-element pieces per thread a row keeps in registers

__device__ __forceinline__ float4 dq_ld4(const float *xr, int e, int K) {
    return e < K ? *(const float4 *)(xr + e) : make_float4(0.f, 0.f, 0.f, 0.f);
}

// d q of four packed codes, each exact in fp32 for Q8_0's fp16 d (11 + 7 bits); for Q8_K's fp32 d the product ggml's
// dequantize_row_q8_K forms
__device__ __forceinline__ float4 dq_vals(int q, float d) {
    return make_float4(d * (float)(int8_t)(q & 0xFF), d * (float)(int8_t)((q >> 8) & 0xFF),
                       d * (float)(int8_t)((q >> 16) & 0xFF), d * (float)(int8_t)((q >> 24) & 0xFF));
}
__device__ __forceinline__ float dq_amax4(float4 p) { return fmaxf(fmaxf(fabsf(p.x), fabsf(p.y)), fmaxf(fabsf(p.z), fabsf(p.w))); }
__device__ __forceinline__ dq_v4h dq_h4(float4 p, float sc) {
    return dq_v4h{(_Float16)(p.x * sc), (_Float16)(p.y * sc), (_Float16)(p.z * sc), (_Float16)(p.w * sc)};
}

// Row xr (K floats) -> Q8_0 blocks (ggml's quantize_row_q8_0, d rounded to fp16 as the dot reads it) ->
// fp16(2^e d q) at out, 2^-e at *rs: d q is exact in fp32 and so is its scaling; one rounding to fp16. The row is
// quantized once, its codes kept in registers while the workgroup finds the row's largest |d q| (rows longer than
// DQ_ACT_REG * 4 NT are quantized twice). red: NT / 64 floats of LDS.
template <int NT>
__device__ __forceinline__ void dq_act_row_q8_0(const float *xr, int K, int rounding, _Float16 *out, float *rs,
                                                float *red) {
    constexpr int CH = 4 * NT;  // elements per pass of the workgroup
    const int t4 = 4 * threadIdx.x;
    float amax = 0.0f;
    if (K <= DQ_ACT_REG * CH) {
        float4 v[DQ_ACT_REG];
        int q[DQ_ACT_REG];
        float dh[DQ_ACT_REG];
#pragma unroll
        for (int c = 0; c < DQ_ACT_REG; c++) v[c] = dq_ld4(xr, CH * c + t4, K);
#pragma unroll
        for (int c = 0; c < DQ_ACT_REG; c++)
            if (CH * c < K) {  // uniform: every lane joins the 8-lane block reductions
                float d;
                int sum;
                q[c] = quant32_lane(v[c], rounding, &d, &sum);
                dh[c] = h2f(f2h(d));
                amax = fmaxf(amax, dq_amax4(dq_vals(q[c], dh[c])));
            }
        const int ex = dq_row_exp(dq_block_max<NT>(amax, red));
        if (threadIdx.x == 0) *rs = dq_pow2(-ex);
        const float sc = dq_pow2(ex);
#pragma unroll
        for (int c = 0; c < DQ_ACT_REG; c++)
            if (CH * c + t4 < K) *(dq_v4h *)(out + CH * c + t4) = dq_h4(dq_vals(q[c], dh[c]), sc);
        return;
    }
    for (int c = 0; c < K; c += CH) {
        float d;
        int sum;
        const int q = quant32_lane(dq_ld4(xr, c + t4, K), rounding, &d, &sum);
        amax = fmaxf(amax, dq_amax4(dq_vals(q, h2f(f2h(d)))));
    }
    const int ex = dq_row_exp(dq_block_max<NT>(amax, red));
    if (threadIdx.x == 0) *rs = dq_pow2(-ex);
    for (int c = 0; c < K; c += CH) {
        float d;
        int sum;
        const int q = quant32_lane(dq_ld4(xr, c + t4, K), rounding, &d, &sum);
        if (c + t4 < K) *(dq_v4h *)(out + c + t4) = dq_h4(dq_vals(q, h2f(f2h(d))), dq_pow2(ex));
    }
}

// Row xr (K floats, K % 256 == 0) -> Q8_K blocks (ggml's quantize_row_q8_K_ref, the pairing of Q5_K / Q6_K weights)
// -> fp16(2^e fp32(d q)), the product ggml's dequantize_row_q8_K forms, scaled and rounded once more. Wave w takes
// blocks w, w + NT / 64, ...
template <int NT>
__device__ __forceinline__ void dq_act_row_q8k(const float *xr, int K, _Float16 *out, float *rs, float *red) {
    constexpr int NWV = NT / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nsb = K / 256;
    float amax = 0.0f;
    if (nsb <= NWV * DQ_ACT_REG) {
        float4 v[DQ_ACT_REG];
        int q[DQ_ACT_REG];
        float dq[DQ_ACT_REG];
#pragma unroll
        for (int i = 0; i < DQ_ACT_REG; i++) {
            const int sb = wave + NWV * i;
            v[i] = sb < nsb ? *(const float4 *)(xr + sb * 256 + 4 * lane) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < DQ_ACT_REG; i++)
            if (wave + NWV * i < nsb) {  // wave-uniform
                int bs16;
                q[i] = quant256_wave(v[i], lane, &dq[i], &bs16);
                amax = fmaxf(amax, dq_amax4(dq_vals(q[i], dq[i])));
            }
        const int ex = dq_row_exp(dq_block_max<NT>(amax, red));
        if (threadIdx.x == 0) *rs = dq_pow2(-ex);
        const float sc = dq_pow2(ex);
#pragma unroll
        for (int i = 0; i < DQ_ACT_REG; i++) {
            const int sb = wave + NWV * i;
            if (sb < nsb) *(dq_v4h *)(out + sb * 256 + 4 * lane) = dq_h4(dq_vals(q[i], dq[i]), sc);
        }
        return;
    }
    for (int sb = wave; sb < nsb; sb += NWV) {
        float d;
        int bs16;
        const int q = quant256_wave(*(const float4 *)(xr + sb * 256 + 4 * lane), lane, &d, &bs16);
        amax = fmaxf(amax, dq_amax4(dq_vals(q, d)));
    }
    const int ex = dq_row_exp(dq_block_max<NT>(amax, red));
    if (threadIdx.x == 0) *rs = dq_pow2(-ex);
    for (int sb = wave; sb < nsb; sb += NWV) {
        float d;
        int bs16;
        const int q = quant256_wave(*(const float4 *)(xr + sb * 256 + 4 * lane), lane, &d, &bs16);
        *(dq_v4h *)(out + sb * 256 + 4 * lane) = dq_h4(dq_vals(q, d), dq_pow2(ex));
    }
}

}  // namespace mx
