// Activation quantization to ggml blocks in global memory: the src1 conversion of ggml-cpu's mul_mat
// (type_traits_cpu[vec_dot_type].from_float), with the same device functions the fused product kernels use.
#include "mx_common.h"
#include "mx_device.h"

namespace mx {

// Q8_0 (34 B: d, qs[32]) or Q8_1 (36 B: d, s, qs[32]). 256 threads cover 32 blocks (1024 elements) of one row.
template <bool Q8_1>
__global__ __launch_bounds__(256) void k_quant32(const float *x, int64_t k, int64_t x_stride, uint8_t *out,
                                                 int rounding) {
    const int64_t row = blockIdx.y;
    const int64_t e = (int64_t)blockIdx.x * 1024 + 4 * threadIdx.x;
    const bool valid = e < k;  // k % 32 == 0, so a block's eight lanes are all valid or all not
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) v = *(const float4 *)(x + row * x_stride + e);
    float d;
    int sum;
    const int q = quant32_lane(v, rounding, &d, &sum);
    if (!valid) return;
    constexpr int BB = Q8_1 ? 36 : 34;
    uint8_t *blk = out + (row * (k / 32) + e / 32) * BB;
    const int j = (int)(threadIdx.x & 7);
    uint8_t *qs = blk + (Q8_1 ? 4 : 2) + 4 * j;
    qs[0] = (uint8_t)(q & 0xFF);
    qs[1] = (uint8_t)((q >> 8) & 0xFF);
    qs[2] = (uint8_t)((q >> 16) & 0xFF);
    qs[3] = (uint8_t)((q >> 24) & 0xFF);
    if (j == 0) {
        const uint16_t hd = f2h(d);
        blk[0] = (uint8_t)(hd & 0xFF);
        blk[1] = (uint8_t)(hd >> 8);
        if (Q8_1) {
            const uint16_t hs = f2h((float)sum * d);  // quantize_row_q8_1_ref: s = sum * d, rounded to fp16
            blk[2] = (uint8_t)(hs & 0xFF);
            blk[3] = (uint8_t)(hs >> 8);
        }
    }
}

// Q8_K (292 B: float d, qs[256], int16 bsums[16]). One wave per block, four waves per workgroup.
__global__ __launch_bounds__(256) void k_quant256(const float *x, int64_t k, int64_t x_stride, uint8_t *out) {
    const int64_t row = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int64_t sb = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (sb * 256 >= k) return;  // whole wave leaves together
    const float4 v = *(const float4 *)(x + row * x_stride + sb * 256 + 4 * lane);
    float d;
    int bs;
    const int q = quant256_wave(v, lane, &d, &bs);
    uint8_t *blk = out + (row * (k / 256) + sb) * 292;
    *(int *)(blk + 4 + 4 * lane) = q;
    if (lane == 0) *(float *)blk = d;
    if ((lane & 3) == 0) *(int16_t *)(blk + 260 + 2 * (lane >> 2)) = (int16_t)bs;
}

hipError_t launch_quantize_act(int type, int rounding, const float *x, int64_t k, int64_t nrows, int64_t x_stride,
                               void *out, hipStream_t s) {
    if (nrows == 0 || k == 0) return hipSuccess;
    if (type == MX_TYPE_Q8_K) {
        dim3 grid((unsigned)((k / 256 + 3) / 4), (unsigned)nrows);
        hipLaunchKernelGGL(k_quant256, grid, dim3(256), 0, s, x, k, x_stride, (uint8_t *)out);
    } else if (type == MX_TYPE_Q8_1) {
        dim3 grid((unsigned)((k + 1023) / 1024), (unsigned)nrows);
        hipLaunchKernelGGL(k_quant32<true>, grid, dim3(256), 0, s, x, k, x_stride, (uint8_t *)out, rounding);
    } else {
        dim3 grid((unsigned)((k + 1023) / 1024), (unsigned)nrows);
        hipLaunchKernelGGL(k_quant32<false>, grid, dim3(256), 0, s, x, k, x_stride, (uint8_t *)out, rounding);
    }
    return hipGetLastError();
}

}  // namespace mx
