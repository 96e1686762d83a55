// GET_ROWS: dst[:, i10, i11, i12] = dequantize(src0[:, ids[i10, i11, i12], i11, i12]) from the planar layout, the
// arithmetic of ggml-quants.c dequantize_row_{q8_0,q4_K,q5_K,q6_K} (bit-exact: the same fp32 products in the same
// order, with no product fused into a subtraction); F16 rows are widened (ggml_fp16_to_fp32_row), F32 rows copied.
#include "mx_common.h"
#include "mx_device.h"

namespace mx {

// Output row (i10, i11, i12): one workgroup, four consecutive elements per thread and step.
template <int TYPE>
__device__ __forceinline__ void get_row(const GetRowsArgs &a, const int64_t i10, const int64_t i11, const int64_t i12) {
    const int32_t r = *(const int32_t *)((const uint8_t *)a.ids + i10 * a.ids_nb0 + i11 * a.ids_nb1 + i12 * a.ids_nb2);
    float *y = (float *)((uint8_t *)a.dst + i10 * a.dst_nb1 + i11 * a.dst_nb2 + i12 * a.dst_nb3);
    if (r < 0 || r >= a.R) {
        // ggml's CPU backend asserts here; this device records the error for mx_backend_synchronize and writes zeros.
        if (threadIdx.x == 0) atomicOr(a.err, 1);
        for (int64_t e = 4 * threadIdx.x; e < a.K; e += 1024) *(float4 *)(y + e) = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const int64_t row = (int64_t)r + i11 * a.src_mat_rows1 + i12 * a.src_mat_rows2;
    const int64_t K = a.K;
    for (int64_t e = 4 * threadIdx.x; e < K; e += 1024) {
        float o[4];
        if (TYPE == MX_TYPE_F32) {
            const float4 v = *(const float4 *)((const float *)a.w.p0 + row * K + e);
            o[0] = v.x, o[1] = v.y, o[2] = v.z, o[3] = v.w;
        } else if (TYPE == MX_TYPE_F16) {
            const uint2 h = *(const uint2 *)((const uint16_t *)a.w.p0 + row * K + e);
            o[0] = h2f((uint16_t)(h.x & 0xFFFF)), o[1] = h2f((uint16_t)(h.x >> 16));
            o[2] = h2f((uint16_t)(h.y & 0xFFFF)), o[3] = h2f((uint16_t)(h.y >> 16));
        } else if (TYPE == MX_TYPE_Q8_0) {
            const int q4 = *(const int *)(a.w.p0 + row * K + e);
            const float d = h2f(*(const uint16_t *)(a.w.p1 + (row * (K / 32) + e / 32) * 2));
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = (float)(int8_t)(q4 >> (8 * j)) * d;
        } else if (TYPE == MX_TYPE_Q4_K || TYPE == MX_TYPE_Q5_K) {
            const int64_t sb = row * (K / 256) + e / 256;
            const int ie = (int)(e % 256);          // element within the super-block
            const int sub = ie / 32;                // sub-block 0..7
            const int byte = (ie / 64) * 32 + ie % 32;
            const uint32_t q4 = *(const uint32_t *)(a.w.p0 + sb * 128 + byte);
            // Q5_K: bit 4 of element l of sub-block j is bit j of qh[l]; its scales and d|dmin sit one plane later
            const uint32_t qh = TYPE == MX_TYPE_Q5_K ? *(const uint32_t *)(a.w.p1 + sb * 32 + ie % 32) : 0u;
            const uint8_t *s = (TYPE == MX_TYPE_Q5_K ? a.w.p2 : a.w.p1) + sb * 12;
            uint8_t sc, m;
            if (sub < 4) {
                sc = s[sub] & 63;
                m = s[sub + 4] & 63;
            } else {
                sc = (uint8_t)((s[sub + 4] & 0xF) | ((s[sub - 4] >> 6) << 4));
                m = (uint8_t)((s[sub + 4] >> 4) | ((s[sub] >> 6) << 4));
            }
            const uint32_t dm = *(const uint32_t *)((TYPE == MX_TYPE_Q5_K ? a.w.p3 : a.w.p2) + sb * 4);
            const float d1 = h2f((uint16_t)(dm & 0xFFFF)) * sc;
            const float m1 = h2f((uint16_t)(dm >> 16)) * m;
            const int shift = (ie % 64) < 32 ? 0 : 4;
            {
#pragma clang fp contract(off)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t q = ((q4 >> (8 * j + shift)) & 0xF) + (((qh >> (8 * j + sub)) & 1) << 4);
                    o[j] = d1 * (float)q - m1;
                }
            }
        } else {
            const int64_t sb = row * (K / 256) + e / 256;
            const int ie = (int)(e % 256);
            const int half = ie / 128, quarter = (ie % 128) / 32, l = ie % 32;
            const uint32_t ql = *(const uint32_t *)(a.w.p0 + sb * 128 + half * 64 + (quarter & 1) * 32 + l);
            const uint32_t qh = *(const uint32_t *)(a.w.p1 + sb * 64 + half * 32 + l);
            const float d = h2f(*(const uint16_t *)(a.w.p3 + sb * 2));
            const float dsc = d * (float)(int8_t)a.w.p2[sb * 16 + ie / 16];
            const int lshift = quarter < 2 ? 0 : 4;
            const int hshift = 2 * quarter;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int q = (int)(((ql >> (8 * j + lshift)) & 0xF) | (((qh >> (8 * j + hshift)) & 3) << 4)) - 32;
                o[j] = dsc * (float)q;
            }
        }
        *(float4 *)(y + e) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

// Workgroups stride over the output rows (one row at a time), four consecutive elements per thread and step. Row
// indices are 32-bit: the number of rows is below 2^31 (checked by the caller).
template <int TYPE>
__global__ __launch_bounds__(256) void k_get_rows(GetRowsArgs a) {
    // The fields on the way to the row index and the first row load, requested together into scalar registers (left to
    // the compiler, they came in over several round trips in a row).
    asm volatile("" ::"s"(a.n_ids0), "s"(a.n_ids1), "s"(a.n_ids2), "s"(a.ids), "s"(a.ids_nb0), "s"(a.ids_nb1),
                 "s"(a.ids_nb2), "s"(a.R), "s"(a.K), "s"(a.src_mat_rows1), "s"(a.src_mat_rows2), "s"(a.w.p0),
                 "s"(a.w.p1));
    asm volatile("" ::"s"(a.dst), "s"(a.dst_nb1), "s"(a.dst_nb2), "s"(a.dst_nb3));
    const uint32_t n0 = (uint32_t)a.n_ids0, n1 = (uint32_t)a.n_ids1;
    const uint32_t nrows = n0 * n1 * (uint32_t)a.n_ids2;
    for (uint32_t i = blockIdx.x; i < nrows; i += gridDim.x) get_row<TYPE>(a, i % n0, (i / n0) % n1, i / (n0 * n1));
}

hipError_t launch_get_rows(const GetRowsArgs &a, hipStream_t s) {
    const int64_t n = a.n_ids0 * a.n_ids1 * a.n_ids2;
    if (n == 0) return hipSuccess;
    dim3 grid((unsigned)std::min<int64_t>(n, 65536));
    switch (a.type) {
        case MX_TYPE_Q8_0: hipLaunchKernelGGL(k_get_rows<MX_TYPE_Q8_0>, grid, dim3(256), 0, s, a); break;
        case MX_TYPE_Q4_K: hipLaunchKernelGGL(k_get_rows<MX_TYPE_Q4_K>, grid, dim3(256), 0, s, a); break;
        case MX_TYPE_Q5_K: hipLaunchKernelGGL(k_get_rows<MX_TYPE_Q5_K>, grid, dim3(256), 0, s, a); break;
        case MX_TYPE_F16: hipLaunchKernelGGL(k_get_rows<MX_TYPE_F16>, grid, dim3(256), 0, s, a); break;
        case MX_TYPE_F32: hipLaunchKernelGGL(k_get_rows<MX_TYPE_F32>, grid, dim3(256), 0, s, a); break;
        case MX_TYPE_Q6_K: hipLaunchKernelGGL(k_get_rows<MX_TYPE_Q6_K>, grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mx
