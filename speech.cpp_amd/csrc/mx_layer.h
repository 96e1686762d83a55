// Device helpers of the decoder-layer kernels (layer.hip): wave64 reductions and the per-head q / k norm + NEOX RoPE
// of head size 128. Include after `#pragma clang fp contract(off)`:
// these expressions must round exactly as ggml-cpu forms them (no fused multiply-adds unless written as fmaf).
#pragma once

#include "mx_device.h"

namespace mx {

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// One head of 128 (lane l holds channels l and l + 64, the NEOX pair l): rms_norm then mul by w, then RoPE at position
// p; the arithmetic of k_rms_norm and k_rope_neox.
__device__ __forceinline__ void qk_norm_rope(float x0, float x1, float w0, float w1, int64_t p, float eps,
                                             float theta_scale, float freq_scale, int lane, float &o0, float &o1) {
    double ss = (double)(x0 * x0) + (double)(x1 * x1);
    ss = wave_sum_d(ss);
    const float mean = (float)(ss / 128.0);
    const float scale = 1.0f / sqrtf(mean + eps);
    const float y0 = (x0 * scale) * w0, y1 = (x1 * scale) * w1;
    float theta = (float)p;  // the chain p * theta_scale ... (lane factors), unrolled and branch-free
#pragma unroll
    for (int j = 0; j < 63; j++) {
        const float next = theta * theta_scale;
        theta = j < lane ? next : theta;
    }
    const float t = freq_scale * theta;
    const float c = cosf(t), s = sinf(t);
    o0 = y0 * c - y1 * s;
    o1 = y0 * s + y1 * c;
}

}  // namespace mx
