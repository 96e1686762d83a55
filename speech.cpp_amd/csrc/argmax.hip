// ARGMAX over rows of f32 logits: dst[r] = the index of the largest value of row r, the first of equal ones, as
// speech.cpp's ggml fork picks it (fastconformer/decoder.cpp:56-62 first_argmax; qwen3-decoder.cpp:428,501 pick the
// next token on the device this way and read back four bytes). A NaN never compares greater: NaNs past index 0 are
// passed over, and a NaN at index 0 keeps index 0 (nothing is greater than it).
//
// One workgroup per row: 1024 threads read the row with 16-byte loads (one pass over HBM), keep the best (value,
// index) of their elements, and the pairs meet across lanes (DPP-free xor shuffles) and then across the 16 waves in
// LDS. "Better" is: not NaN, and greater, or equal with a smaller index -- the order first_argmax's scan induces.
#include "mx_common.h"
#include "mx_device.h"

namespace mx {

__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
    return !__builtin_isnan(v) && (__builtin_isnan(bv) || v > bv || (v == bv && i < bi));
}

constexpr int AM_THREADS = 1024;

__global__ __launch_bounds__(AM_THREADS) void k_argmax(const float *src, int64_t ne0, int64_t nb1, int32_t *dst,
                                                        int64_t dst_nb0) {
    __shared__ float sv[AM_THREADS / 64];
    __shared__ int si[AM_THREADS / 64];
    const int64_t r = blockIdx.x;
    const float *x = (const float *)((const uint8_t *)src + r * nb1);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = __builtin_nanf("");
    int bi = 0x7FFFFFFF;
    const int64_t n4 = ne0 / 4;
    for (int64_t j = tid; j < n4; j += AM_THREADS) {
        const float4 v = *(const float4 *)(x + 4 * j);
        const int i = (int)(4 * j);
        if (am_better(v.x, i, bv, bi)) { bv = v.x; bi = i; }
        if (am_better(v.y, i + 1, bv, bi)) { bv = v.y; bi = i + 1; }
        if (am_better(v.z, i + 2, bv, bi)) { bv = v.z; bi = i + 2; }
        if (am_better(v.w, i + 3, bv, bi)) { bv = v.w; bi = i + 3; }
    }
    for (int64_t i = 4 * n4 + tid; i < ne0; i += AM_THREADS) {
        if (am_better(x[i], (int)i, bv, bi)) { bv = x[i]; bi = (int)i; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        float v = sv[0];
        int i = si[0];
        for (int w = 1; w < AM_THREADS / 64; w++)
            if (am_better(sv[w], si[w], v, i)) { v = sv[w]; i = si[w]; }
        // nothing beats a NaN at index 0; a row without any non-NaN value also ends at 0
        if (__builtin_isnan(x[0]) || i == 0x7FFFFFFF) i = 0;
        *(int32_t *)((uint8_t *)dst + r * dst_nb0) = i;
    }
}

// Long rows split over `nparts` workgroups (a 151936-entry vocabulary row in one workgroup reads at ~35 GB/s): each
// writes its part's best (value, index) to `part`, and one wave per row picks the best of the parts with the same
// order -- the first of equal values, NaN never greater.
__global__ __launch_bounds__(AM_THREADS) void k_argmax_part(const float *src, int64_t ne0, int64_t nb1, int64_t per,
                                                             int nparts, float2 *part) {
    __shared__ float sv[AM_THREADS / 64];
    __shared__ int si[AM_THREADS / 64];
    const int64_t r = blockIdx.y, b = blockIdx.x;
    const float *x = (const float *)((const uint8_t *)src + r * nb1);
    const int64_t lo = b * per, hi = min(ne0, lo + per);  // per is a multiple of 4
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = __builtin_nanf("");
    int bi = 0x7FFFFFFF;
    for (int64_t j = lo + 4 * tid; j < hi; j += 4 * AM_THREADS) {
        if (j + 4 <= hi) {
            const float4 v = *(const float4 *)(x + j);
            const int i = (int)j;
            if (am_better(v.x, i, bv, bi)) { bv = v.x; bi = i; }
            if (am_better(v.y, i + 1, bv, bi)) { bv = v.y; bi = i + 1; }
            if (am_better(v.z, i + 2, bv, bi)) { bv = v.z; bi = i + 2; }
            if (am_better(v.w, i + 3, bv, bi)) { bv = v.w; bi = i + 3; }
        } else {
            for (int64_t k = j; k < hi; k++)
                if (am_better(x[k], (int)k, bv, bi)) { bv = x[k]; bi = (int)k; }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        float v = sv[0];
        int i = si[0];
        for (int w = 1; w < AM_THREADS / 64; w++)
            if (am_better(sv[w], si[w], v, i)) { v = sv[w]; i = si[w]; }
        part[r * nparts + b] = make_float2(v, __int_as_float(i));
    }
}

__global__ __launch_bounds__(64) void k_argmax_final(const float *src, int64_t nb1, int nparts, const float2 *part,
                                                      int32_t *dst, int64_t dst_nb0) {
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x;
    float bv = __builtin_nanf("");
    int bi = 0x7FFFFFFF;
    if (lane < nparts) {
        const float2 p = part[r * nparts + lane];
        bv = p.x;
        bi = __float_as_int(p.y);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) {
        const float *x = (const float *)((const uint8_t *)src + r * nb1);
        if (__builtin_isnan(x[0]) || bi == 0x7FFFFFFF) bi = 0;
        *(int32_t *)((uint8_t *)dst + r * dst_nb0) = bi;
    }
}

int argmax_parts(int64_t ne0, int64_t nrows) {
    int64_t n = ne0 / 4096;  // about 4 floats per thread and part
    if (nrows > 1) n = n / nrows;
    return (int)(n < 1 ? 1 : (n > 64 ? 64 : n));
}

hipError_t launch_argmax(const float *src, int64_t ne0, int64_t nrows, int64_t nb1, int32_t *dst, int64_t dst_nb0,
                         void *scratch, hipStream_t s) {
    if (nrows == 0) return hipSuccess;
    const int nparts = argmax_parts(ne0, nrows);
    if (nparts == 1) {
        hipLaunchKernelGGL(k_argmax, dim3((unsigned)nrows), dim3(AM_THREADS), 0, s, src, ne0, nb1, dst, dst_nb0);
        return hipGetLastError();
    }
    const int64_t per = ((ne0 + nparts - 1) / nparts + 3) / 4 * 4;
    hipLaunchKernelGGL(k_argmax_part, dim3((unsigned)nparts, (unsigned)nrows), dim3(AM_THREADS), 0, s, src, ne0, nb1,
                       per, nparts, (float2 *)scratch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)nrows), dim3(64), 0, s, src, nb1, nparts,
                       (const float2 *)scratch, dst, dst_nb0);
    return hipGetLastError();
}

}  // namespace mx
