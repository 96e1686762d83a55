// Device-side helpers for libmx's gfx950 kernels: fp16 conversion, wave64 reductions and the activation quantizers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mx.h"

namespace mx {

// fp16 bits <-> fp32. v_cvt_f16_f32 rounds to nearest even and keeps binary16 subnormals (the default FP mode of a
// HIP kernel), which is IEEE conversion as ggml_compute_fp32_to_fp16 performs it.
__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}
__device__ __forceinline__ uint16_t f2h(float f) {
    _Float16 v = (_Float16)f;
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// Cross-lane exchanges on DPP (a modifier of the consuming VALU op: no LDS round trip). Each control reads, for lane
// i: XOR1 / XOR2 lane i^1 / i^2 of its quad; HALF_MIRROR lane 7-i of its eight; MIRROR lane 15-i of its row of 16;
// BCAST15 lane 15 of the row below (written into rows 1 and 3 with row mask 0xA); BCAST31 lane 31 (rows 2 and 3, row
// mask 0xC). Lanes of rows outside the row mask get `old`.
namespace dpp {
constexpr int XOR1 = 0xB1, XOR2 = 0x4E, HALF_MIRROR = 0x141, MIRROR = 0x140, BCAST15 = 0x142, BCAST31 = 0x143;
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_i(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xF,
                                                      false));
}

// Sum over aligned groups of WIDTH lanes (16, 32 or 64). Exact in the group's last lane (lane % WIDTH == WIDTH - 1);
// for WIDTH 16 in every lane.
template <int WIDTH>
__device__ __forceinline__ float sum_lanes(float v) {
    static_assert(WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "group of 16, 32 or 64 lanes");
    v += dpp_f<dpp::XOR1>(0.0f, v);
    v += dpp_f<dpp::XOR2>(0.0f, v);
    v += dpp_f<dpp::HALF_MIRROR>(0.0f, v);
    v += dpp_f<dpp::MIRROR>(0.0f, v);
    if (WIDTH >= 32) v += dpp_f<dpp::BCAST15, 0xA>(0.0f, v);
    if (WIDTH >= 64) v += dpp_f<dpp::BCAST31, 0xC>(0.0f, v);
    return v;
}

// ------------------------------------------------------------------------------------------------------------------
// Buffer-to-LDS copies and their waits (the prefill GEMMs' and the MoE product's operand rings).
// ------------------------------------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// The LDS address of a pointer into the workgroup's shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)(const lds_void *)p; }

// A buffer descriptor for raw dword loads: base, no stride, `bytes` records (reads past them return zeros), format
// word as the buffer-resource builtin makes it for these loads.
__device__ __forceinline__ v4u buf_rsrc(const void *base, uint32_t bytes) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    return v4u{(uint32_t)b, (uint32_t)(b >> 32), bytes, 0x00020000u};
}

// Buffer-to-LDS copies (each lane's 16 or 4 bytes land at m0 + 16 or 4 x lane), issued through asm: issued as the
// builtin, the compiler counts them as LDS stores that every later LDS read may alias, and waits for all of them
// (the next stages' too) before the first fragment read of a stage. Their waits are counted by the caller (wait_vm).
__device__ __forceinline__ void dma16_lds(v4u r, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(r), "s"(soff)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4_lds(v4u r, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(r), "s"(soff)
                 : "memory", "m0");
}

// Waits until at most n vector memory ops of this wave are outstanding. The memory clobber keeps the compiler from
// moving loads and stores across it, so the LDS reads that follow see the copies it waited for.
template <int n>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
    return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((int)((unsigned)d << 24));
}

// ------------------------------------------------------------------------------------------------------------------
// 32-block quantizer (Q8_0 / Q8_1 activations). Eight consecutive lanes hold one block, four floats each (lane j of
// the eight holds elements 4j..4j+3).
//   REF (ggml-quants.c quantize_row_q8_{0,1}_ref): d = amax/127, id = d ? 1/d : 0, q = roundf(x*id).
//   X86 (ggml-cpu x86 quantize_row_q8_{0,1}):       d = amax/127, id = amax ? 127/amax : 0, q = rint(x*id).
// The divisions are IEEE (HIP's default correctly rounded fp32 division), the products single roundings.
// Returns the four quants packed in an int; *d gets fp32 d (unrounded), *sum the block's quant sum (all 8 lanes).
// ------------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ int quant32_lane(float4 v, int rounding, float *d_out, int *sum_out) {
    float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    a = fmaxf(a, dpp_f<dpp::XOR1>(0.0f, a));
    a = fmaxf(a, dpp_f<dpp::XOR2>(0.0f, a));
    a = fmaxf(a, dpp_f<dpp::HALF_MIRROR>(0.0f, a));  // every lane of the eight now holds the block's amax
    const float d = a / 127.0f;
    int q0, q1, q2, q3;
    if (rounding == MX_ROUND_X86) {
        const float id = a != 0.0f ? 127.0f / a : 0.0f;
        q0 = (int)rintf(v.x * id);
        q1 = (int)rintf(v.y * id);
        q2 = (int)rintf(v.z * id);
        q3 = (int)rintf(v.w * id);
    } else {
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        q0 = (int)roundf(v.x * id);
        q1 = (int)roundf(v.y * id);
        q2 = (int)roundf(v.z * id);
        q3 = (int)roundf(v.w * id);
    }
    int s = q0 + q1 + q2 + q3;
    s += dpp_i<dpp::XOR1>(0, s);
    s += dpp_i<dpp::XOR2>(0, s);
    s += dpp_i<dpp::HALF_MIRROR>(0, s);
    *d_out = d;
    *sum_out = s;
    return pack4(q0, q1, q2, q3);
}

// ------------------------------------------------------------------------------------------------------------------
// 256-block quantizer (Q8_K activations of Q4_K / Q6_K weights), ggml-quants.c quantize_row_q8_K_ref. One wave holds
// one block, four floats per lane (lane l holds elements 4l..4l+3).
//   max = the element of largest |x|, the first one on ties; iscale = -127/max; q = min(127, rint(iscale*x));
//   d = 1/iscale; bsums[j] = sum of q[16j..16j+15]. An all-zero block gives d = 0, q = 0 and bsums 0.
// Returns packed quants; *d the block's d; *bsum the sum over this lane's group of four lanes (16 elements).
// ------------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ int quant256_wave(float4 v, int lane, float *d_out, int *bsum_out) {
    const float e[4] = {v.x, v.y, v.z, v.w};
    const float ax = fabsf(v.x), ay = fabsf(v.y), az = fabsf(v.z), aw = fabsf(v.w);
    // amax: the largest |x| (fmaxf passes NaNs over, as ggml's strict '>' scan does), reduced within rows of 16, then
    // across rows into lane 63
    float a = fmaxf(fmaxf(ax, ay), fmaxf(az, aw));
    a = fmaxf(a, dpp_f<dpp::XOR1>(0.0f, a));
    a = fmaxf(a, dpp_f<dpp::XOR2>(0.0f, a));
    a = fmaxf(a, dpp_f<dpp::HALF_MIRROR>(0.0f, a));
    a = fmaxf(a, dpp_f<dpp::MIRROR>(0.0f, a));
    a = fmaxf(a, dpp_f<dpp::BCAST15, 0xA>(0.0f, a));
    a = fmaxf(a, dpp_f<dpp::BCAST31, 0xC>(0.0f, a));
    const float amax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 63));
    if (amax == 0.0f) {
        *d_out = 0.0f;
        *bsum_out = 0;
        return 0;
    }
    // max: the element of the first index (4 lane + j) whose |x| is amax -- the lowest lane holding one, its lowest j
    const uint64_t m0 = __ballot(ax == amax), m1 = __ballot(ay == amax), m2 = __ballot(az == amax),
                   m3 = __ballot(aw == amax);
    const int L = __builtin_ctzll(m0 | m1 | m2 | m3);
    const int c = ((m0 >> L) & 1) ? 0 : (((m1 >> L) & 1) ? 1 : (((m2 >> L) & 1) ? 2 : 3));
    const float mine = c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
    const float maxv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), L));
    const float iscale = -127.0f / maxv;
    int q[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int t = (int)rintf(iscale * e[j]);
        q[j] = t < 127 ? t : 127;
    }
    int s = q[0] + q[1] + q[2] + q[3];
    s += dpp_i<dpp::XOR1>(0, s);
    s += dpp_i<dpp::XOR2>(0, s);
    *d_out = 1.0f / iscale;
    *bsum_out = s;
    return pack4(q[0], q[1], q[2], q[3]);
}

}  // namespace mx
