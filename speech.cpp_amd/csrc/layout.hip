// Scatter / gather between ggml's array-of-blocks bytes and this device's planar layout (see mx_common.h).
#include "mx_common.h"

namespace mx {

SegMap segmap_of(int type, const Planes &pl) {
    SegMap m{};
    const TypeInfo *ti = type_info(type);
    m.blk_bytes = ti->blk_bytes;
    m.nseg = ti->nseg;
    for (int s = 0; s < ti->nseg; s++) m.seg[s] = ti->seg[s];
    for (int i = 0; i < 4; i++) m.plane_off[i] = pl.off[i];
    return m;
}

// Byte `pos` of ggml block `blk` -> its byte offset from the tensor's base in the planar layout.
__device__ __forceinline__ uint64_t planar_offset(const SegMap &m, uint64_t blk, uint32_t pos) {
    int s = 0;
#pragma unroll
    for (int k = 1; k < 4; k++)
        if (k < m.nseg && pos >= m.seg[k].begin) s = k;
    return m.plane_off[m.seg[s].plane] + blk * m.seg[s].len + (pos - m.seg[s].begin);
}

// MODE 0: scatter (planes <- src), 1: gather (dst <- planes), 2: fill (planes <- value).
template <int MODE>
__global__ __launch_bounds__(256) void k_permute(SegMap m, uint8_t *planes, const uint8_t *src, uint8_t *dst,
                                                 uint8_t value, uint64_t blk0, uint32_t pos0, uint32_t n) {
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) {
        const uint32_t t = pos0 + i;
        const uint64_t blk = blk0 + t / (uint32_t)m.blk_bytes;
        const uint32_t pos = t % (uint32_t)m.blk_bytes;
        const uint64_t o = planar_offset(m, blk, pos);
        if (MODE == 0) planes[o] = src[i];
        else if (MODE == 1) dst[i] = planes[o];
        else planes[o] = value;
    }
}

template <int MODE>
static hipError_t launch_permute(const SegMap &m, uint8_t *planes, const uint8_t *src, uint8_t *dst, uint8_t value,
                                 uint64_t offset, uint64_t n, hipStream_t s) {
    // Pieces are cut by the host to at most 1 GiB, so every index below fits 32 bits.
    if (n == 0) return hipSuccess;
    const uint64_t blk0 = offset / m.blk_bytes;
    const uint32_t pos0 = (uint32_t)(offset % m.blk_bytes);
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_permute<MODE>, dim3((unsigned)blocks), dim3(256), 0, s, m, planes, src, dst, value, blk0, pos0,
                       (uint32_t)n);
    return hipGetLastError();
}

hipError_t launch_scatter(const SegMap &m, uint8_t *base, const uint8_t *src, uint64_t offset, uint64_t n,
                          hipStream_t s) {
    return launch_permute<0>(m, base, src, nullptr, 0, offset, n, s);
}
hipError_t launch_gather(const SegMap &m, const uint8_t *base, uint8_t *dst, uint64_t offset, uint64_t n,
                         hipStream_t s) {
    return launch_permute<1>(m, const_cast<uint8_t *>(base), nullptr, dst, 0, offset, n, s);
}
hipError_t launch_fill(const SegMap &m, uint8_t *base, uint8_t value, uint64_t offset, uint64_t n, hipStream_t s) {
    return launch_permute<2>(m, base, nullptr, nullptr, value, offset, n, s);
}

}  // namespace mx
