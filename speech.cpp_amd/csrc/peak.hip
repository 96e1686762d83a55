// Peak micro-benchmarks: what one MI355X streams from HBM and issues on its matrix cores, measured with the same
// launch machinery as the product kernels. They give the practical ceilings beside the published ones (8 TB/s HBM,
// 5.0 POP/s dense int8, 2.5 PFLOP/s dense fp16) that the products' roofline fractions are quoted against.
#include "mx_common.h"

namespace mx {

typedef int pk_v4i __attribute__((ext_vector_type(4)));
typedef int pk_v16i __attribute__((ext_vector_type(16)));
typedef float pk_v16f __attribute__((ext_vector_type(16)));
typedef _Float16 pk_v8h __attribute__((ext_vector_type(8)));

// Every 16-byte chunk of src read once: thread t of the grid reads chunks t, t + T, t + 2T, ... (T threads in the
// grid), U loads in flight per thread, plain or nontemporal. The XOR of what a thread read is stored only if it equals
// a value the data never gives, so the loads cannot be dropped and nothing is written.
template <int U, bool NT>
__global__ __launch_bounds__(256) void k_peak_read(const pk_v4i *src, int64_t n, int *sink) {
    const int64_t T = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    int acc = 0;
    for (; i + (int64_t)(U - 1) * T < n; i += (int64_t)U * T) {
        pk_v4i v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = NT ? __builtin_nontemporal_load(src + i + u * T) : src[i + u * T];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n; i += T) {
        const pk_v4i v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x1F2E3D4C) sink[blockIdx.x] = acc;
}

// Each wave issues `iters` rounds of eight independent MFMAs on register operands (eight accumulators cover the
// matrix core's dependent-issue latency); the accumulators' sum is stored only if it equals a value no run gives.
__global__ __launch_bounds__(256) void k_peak_mfma_i8(int iters, int seed, int *sink) {
    const pk_v4i a = {seed, seed + 1, seed + 2, seed + 3}, b = {seed ^ 5, seed ^ 6, seed ^ 7, seed ^ 8};
    pk_v16i acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
        for (int e = 0; e < 16; e++) acc[j][e] = 0;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[j], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; j++)
        for (int e = 0; e < 16; e++) s += acc[j][e];
    if (s == 0x1F2E3D4C) sink[blockIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_peak_mfma_f16(int iters, int seed, int *sink) {
    const _Float16 h = (_Float16)(1.0f / (float)(seed | 1));
    const pk_v8h a = {h, h, h, h, h, h, h, h}, b = {h, h, h, h, h, h, h, h};
    pk_v16f acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
        for (int e = 0; e < 16; e++) acc[j][e] = 0.0f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++)
        for (int e = 0; e < 16; e++) s += acc[j][e];
    if (s == -1.0f) sink[blockIdx.x] = 1;
}

hipError_t launch_peak_read(const void *src, int64_t bytes, int workgroups, int loads, bool nontemporal, int *sink,
                            hipStream_t s) {
    const int64_t n = bytes / 16;
    const dim3 g((unsigned)workgroups), b(256);
    const pk_v4i *p = (const pk_v4i *)src;
#define MX_PEAK_READ(U)                                                                                  \
    if (loads == U) {                                                                                    \
        if (nontemporal) hipLaunchKernelGGL((k_peak_read<U, true>), g, b, 0, s, p, n, sink);            \
        else hipLaunchKernelGGL((k_peak_read<U, false>), g, b, 0, s, p, n, sink);                        \
        return hipGetLastError();                                                                        \
    }
    MX_PEAK_READ(1)
    MX_PEAK_READ(2)
    MX_PEAK_READ(4)
    MX_PEAK_READ(8)
    MX_PEAK_READ(16)
#undef MX_PEAK_READ
    return hipErrorInvalidValue;
}

hipError_t launch_peak_mfma(int kind, int workgroups, int iters, int *sink, hipStream_t s) {
    if (kind == 0) hipLaunchKernelGGL(k_peak_mfma_i8, dim3((unsigned)workgroups), dim3(256), 0, s, iters, 3, sink);
    else hipLaunchKernelGGL(k_peak_mfma_f16, dim3((unsigned)workgroups), dim3(256), 0, s, iters, 3, sink);
    return hipGetLastError();
}

}  // namespace mx
