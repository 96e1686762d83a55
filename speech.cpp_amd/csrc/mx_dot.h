// Per-chunk dot products of one weight row (planar layout) with up to NC quantized activation columns held in LDS.
//
// The integer part of every product is exact (v_dot4 over int8, int32 sums); scales are applied in fp32 as ggml's
// CPU dots apply them (ggml-cpu/quants.c ggml_vec_dot_q8_0_q8_0 / _q4_K_q8_K / _q5_K_q8_K / _q6_K_q8_K): d_w * d_x formed in fp32,
// then times the exact integer sum. Only the order of the fp32 cross-block sum differs from the CPU.
//
// Activations in LDS, column c:
//   xq[c*K + k]     int8 quants (Q4_K weights: in unit order, below)
//   xd[c*nsc + b]   fp32 scale of block b (the fp16-rounded d of Q8_0/Q8_1 for Q8_0 weights; Q8_K's fp32 d otherwise)
//   xbs[c*K/16 + j] sum of quants 16j..16j+15 (Q5_K / Q6_K: Q8_K's bsums); Q4_K: xbs[c*K/32 + j], the sums of
//                   quants 32j..32j+31 (a sub-block's, two bsums added)
//
// Q4_K is taken a unit of 128 elements at a time -- half a super-block: 64 bytes of qs, four sub-blocks and their
// scales / mins -- so one lane unpacks the 6-bit scales of four sub-blocks at once. Its activation quants sit in LDS
// as 16-byte pieces, piece i of unit u at byte 16 (i * K/128 + u): the lanes of a row read piece i of consecutive
// units from consecutive 16-byte words (no bank conflicts), where units in place would be 128 bytes apart.
#pragma once

#include "mx_common.h"
#include "mx_device.h"

namespace mx {

__device__ __forceinline__ int dot16(int4 a, int4 b, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// Chunks per row: a Q8_0 chunk is 16 quants (half a block); a Q5_K / Q6_K chunk is 32 elements (16 bytes of qs /
// ql); a Q4_K chunk is a unit of 128 elements (64 bytes of qs).
template <int TYPE>
__host__ __device__ constexpr int chunk_elems() { return TYPE == MX_TYPE_Q8_0 ? 16 : (TYPE == MX_TYPE_Q4_K ? 128 : 32); }
// Chunks a lane loads ahead of the activation prologue (the same bytes in flight: 64 per lane).
template <int TYPE>
__host__ __device__ constexpr int preload_of() { return TYPE == MX_TYPE_Q4_K ? 1 : 4; }
// ints of xbs per activation column.
template <int TYPE>
__host__ __device__ constexpr int64_t xbs_per_col(int64_t K) { return TYPE == MX_TYPE_Q4_K ? K / 32 : K / 16; }
// Byte of Q4_K activation element e in its column's xq (unit order).
__device__ __forceinline__ int q4u_xq_offset(int e, int K) {
    return ((((e >> 4) & 7) * (K >> 7) + (e >> 7)) << 4) + (e & 15);
}

// Unpack the 6-bit scale and min of sub-blocks j and j+1 (j even) from Q4_K's 12 packed bytes held in three words
// (ggml-quants.c get_scale_min_k4).
__device__ __forceinline__ uint32_t byte_of(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (w >> (8 * (i & 3))) & 0xFFu;
}
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int &sc, int &m) {
    if (j < 4) {
        sc = (int)(byte_of(s0, s1, s2, j) & 63);
        m = (int)(byte_of(s0, s1, s2, j + 4) & 63);
    } else {
        sc = (int)((byte_of(s0, s1, s2, j + 4) & 0xF) | ((byte_of(s0, s1, s2, j - 4) >> 6) << 4));
        m = (int)((byte_of(s0, s1, s2, j + 4) >> 4) | ((byte_of(s0, s1, s2, j) >> 6) << 4));
    }
}

// The weight bytes of one chunk, loaded ahead of the arithmetic so the loads of several chunks (and of the activation
// prologue) are in flight together.
template <int TYPE>
struct WChunk;
template <>
struct WChunk<MX_TYPE_Q8_0> {
    int4 q;        // 16 quants
    uint32_t d;    // fp16 scale of their block (low half)
};
template <>
struct WChunk<MX_TYPE_Q4_K> {
    int4 q[4];     // 64 qs bytes of half h of a super-block: q[0..1] sub-blocks 4h (low nibbles), 4h + 1 (high);
                   // q[2..3] sub-blocks 4h + 2 (low), 4h + 3 (high)
    uint32_t s0, s1, s2;  // the 12 packed scale / min bytes
    uint32_t dm;   // fp16 d | fp16 dmin << 16
};
template <>
struct WChunk<MX_TYPE_Q5_K> {
    int4 q;        // low 4 bits of 32 codes: 16 of sub-block j, 16 of sub-block j + 1
    int4 qh;       // the 16 qh bytes of the same positions (bit j: bit 4 of sub-block j's code)
    uint32_t s0, s1, s2;  // the 12 packed scale / min bytes
    uint32_t dm;   // fp16 d | fp16 dmin << 16
};
template <>
struct WChunk<MX_TYPE_Q6_K> {
    int4 ql, qh;
    uint32_t sc;   // the two int8 sub-block scales in bytes 0 and 1
    uint32_t d;    // fp16 d (low half)
};

// Weight bytes are read once per launch: they are loaded nontemporal (the streaming hint), which measured 10-40 %
// faster than plain loads for reads that miss the caches (the peak read micro-benchmark).
typedef int wl_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld_w16(const uint8_t *p) {
    const wl_v4i v = __builtin_nontemporal_load((const wl_v4i *)p);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ld_w32(const uint8_t *p) { return __builtin_nontemporal_load((const uint32_t *)p); }
__device__ __forceinline__ uint32_t ld_w16b(const uint8_t *p) { return __builtin_nontemporal_load((const uint16_t *)p); }
__device__ __forceinline__ uint32_t ld_w8(const uint8_t *p) { return __builtin_nontemporal_load(p); }

template <int TYPE>
__device__ __forceinline__ WChunk<TYPE> load_chunk(const WPlanes &w, int64_t grow, int64_t K, int c) {
    WChunk<TYPE> r;
    if constexpr (TYPE == MX_TYPE_Q8_0) {
        r.q = ld_w16(w.p0 + grow * K + 16 * c);
        r.d = ld_w16b(w.p1 + (grow * (K / 32) + (c >> 1)) * 2);
    } else if constexpr (TYPE == MX_TYPE_Q4_K) {  // unit c: half c & 1 of super-block c >> 1
        // Plain loads: a lane reads its 64 bytes in four 16-byte loads, so each 128-byte line is met by four load
        // instructions, and with the streaming hint a dense 61440 x 2048 product took 22.0 us against 15.4 us with
        // plain loads (its arithmetic switched off in both).
        const int64_t blk = grow * (K / 256) + (c >> 1);
        const uint8_t *qp = w.p0 + blk * 128 + 64 * (c & 1);
#pragma unroll
        for (int i = 0; i < 4; i++) r.q[i] = *(const int4 *)(qp + 16 * i);
        const uint32_t *sp = (const uint32_t *)(w.p1 + blk * 12);
        r.s0 = sp[0];
        r.s1 = sp[1];
        r.s2 = sp[2];
        r.dm = *(const uint32_t *)(w.p2 + blk * 4);
    } else if constexpr (TYPE == MX_TYPE_Q5_K) {
        const int64_t blk = grow * (K / 256) + (c >> 3);
        r.q = ld_w16(w.p0 + blk * 128 + 16 * (c & 7));
        r.qh = ld_w16(w.p1 + blk * 32 + 16 * (c & 1));
        const uint8_t *sp = w.p2 + blk * 12;
        r.s0 = ld_w32(sp);
        r.s1 = ld_w32(sp + 4);
        r.s2 = ld_w32(sp + 8);
        r.dm = ld_w32(w.p3 + blk * 4);
    } else {
        const int64_t blk = grow * (K / 256) + (c >> 3);
        const int t = c & 7, h = t >> 2, u = t & 3;
        r.ql = ld_w16(w.p0 + blk * 128 + 64 * h + 16 * u);
        r.qh = ld_w16(w.p1 + blk * 64 + 32 * h + 16 * (u & 1));
        const int lo_sc = 8 * h + 2 * (u >> 1) + (u & 1);  // (128h + 32(u>>1) + 16(u&1)) / 16
        const uint8_t *sp = w.p2 + blk * 16;
        r.sc = ld_w8(sp + lo_sc) | (ld_w8(sp + lo_sc + 4) << 8);
        r.d = ld_w16b(w.p3 + blk * 2);
    }
    return r;
}

// acc[col] += contribution of chunk c (whose bytes are in `wc`) against the activation columns in LDS.
template <int TYPE, int NC, bool GUARD>
__device__ __forceinline__ void dot_chunk(const WChunk<TYPE> &wc, int64_t K, int c, const int8_t *xq,
                                          const float *xd, const int *xbs, int ncols, float *acc) {
    if constexpr (TYPE == MX_TYPE_Q8_0) {
        const int64_t nblk = K / 32;
        const float dw = h2f((uint16_t)wc.d);
#pragma unroll
        for (int col = 0; col < NC; col++) {
            if (GUARD && col >= ncols) break;
            const int4 xv = *(const int4 *)(xq + col * K + 16 * c);
            const int s = dot16(wc.q, xv, 0);
            acc[col] += (float)s * (dw * xd[col * nblk + (c >> 1)]);
        }
    } else if constexpr (TYPE == MX_TYPE_Q4_K) {
        // unit c: half h of super-block sb, sub-blocks 4h .. 4h + 3 (get_scale_min_k4 of ggml-quants.c for all four:
        // h = 0 takes the low six bits of bytes 0..3 / 4..7, h = 1 the nibbles of bytes 8..11 with the top two bits
        // of bytes 0..3 / 4..7)
        const int64_t nsb = K / 256, nu = K / 128;
        const int sb = c >> 1;
        const bool h = (c & 1) != 0;
        const uint32_t SC = h ? ((wc.s2 & 0x0F0F0F0Fu) | ((wc.s0 >> 2) & 0x30303030u)) : (wc.s0 & 0x3F3F3F3Fu);
        const uint32_t MN = h ? (((wc.s2 >> 4) & 0x0F0F0F0Fu) | ((wc.s1 >> 2) & 0x30303030u)) : (wc.s1 & 0x3F3F3F3Fu);
        const float d = h2f((uint16_t)(wc.dm & 0xFFFF)), dmin = h2f((uint16_t)(wc.dm >> 16));
        int4 lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int4 q = wc.q[i];
            lo[i] = make_int4(q.x & 0x0F0F0F0F, q.y & 0x0F0F0F0F, q.z & 0x0F0F0F0F, q.w & 0x0F0F0F0F);
            hi[i] = make_int4((q.x >> 4) & 0x0F0F0F0F, (q.y >> 4) & 0x0F0F0F0F, (q.z >> 4) & 0x0F0F0F0F,
                              (q.w >> 4) & 0x0F0F0F0F);
        }
#pragma unroll
        for (int col = 0; col < NC; col++) {
            if (GUARD && col >= ncols) break;
            // pieces 0..7 of the unit's 128 quants (16 each): sub-block k covers pieces 2k, 2k + 1
            const int8_t *xc = xq + col * K + 16 * c;
            const int4 *xp = (const int4 *)xc;
            const int64_t pstride = nu;  // int4s between pieces i and i + 1 of a unit
            const int d0 = dot16(lo[1], xp[1 * pstride], dot16(lo[0], xp[0], 0));
            const int d1 = dot16(hi[1], xp[3 * pstride], dot16(hi[0], xp[2 * pstride], 0));
            const int d2 = dot16(lo[3], xp[5 * pstride], dot16(lo[2], xp[4 * pstride], 0));
            const int d3 = dot16(hi[3], xp[7 * pstride], dot16(hi[2], xp[6 * pstride], 0));
            const int4 b = *(const int4 *)(xbs + col * (K / 32) + 4 * c);
            const int isum = (int)(SC & 0xFF) * d0 + (int)((SC >> 8) & 0xFF) * d1 + (int)((SC >> 16) & 0xFF) * d2 +
                             (int)(SC >> 24) * d3;
            const int msum = (int)(MN & 0xFF) * b.x + (int)((MN >> 8) & 0xFF) * b.y + (int)((MN >> 16) & 0xFF) * b.z +
                             (int)(MN >> 24) * b.w;
            const float dx = xd[col * nsb + sb];
            acc[col] += (d * dx) * (float)isum - (dmin * dx) * (float)msum;
        }
    } else if constexpr (TYPE == MX_TYPE_Q5_K) {
        const int64_t nsb = K / 256;
        const int sb = c >> 3, t = c & 7;
        const float d = h2f((uint16_t)(wc.dm & 0xFFFF)), dmin = h2f((uint16_t)(wc.dm >> 16));
        const int jlo = 2 * (t >> 1);
        int sc_lo, m_lo, sc_hi, m_hi;
        q4k_scale_min(wc.s0, wc.s1, wc.s2, jlo, sc_lo, m_lo);
        q4k_scale_min(wc.s0, wc.s1, wc.s2, jlo + 1, sc_hi, m_hi);
        const int4 q = wc.q;
        int4 qlo = make_int4(q.x & 0x0F0F0F0F, q.y & 0x0F0F0F0F, q.z & 0x0F0F0F0F, q.w & 0x0F0F0F0F);
        int4 qhi = make_int4((q.x >> 4) & 0x0F0F0F0F, (q.y >> 4) & 0x0F0F0F0F, (q.z >> 4) & 0x0F0F0F0F,
                             (q.w >> 4) & 0x0F0F0F0F);
        {  // codes 0..31: bit 4 of sub-block j sits in bit j of each qh byte
            const int4 h = wc.qh;
            qlo.x |= ((h.x >> jlo) & 0x01010101) << 4;
            qlo.y |= ((h.y >> jlo) & 0x01010101) << 4;
            qlo.z |= ((h.z >> jlo) & 0x01010101) << 4;
            qlo.w |= ((h.w >> jlo) & 0x01010101) << 4;
            qhi.x |= ((h.x >> (jlo + 1)) & 0x01010101) << 4;
            qhi.y |= ((h.y >> (jlo + 1)) & 0x01010101) << 4;
            qhi.z |= ((h.z >> (jlo + 1)) & 0x01010101) << 4;
            qhi.w |= ((h.w >> (jlo + 1)) & 0x01010101) << 4;
        }
        const int lo_off = sb * 256 + 64 * (t >> 1) + 16 * (t & 1);
#pragma unroll
        for (int col = 0; col < NC; col++) {
            if (GUARD && col >= ncols) break;
            const int8_t *xc = xq + col * K;
            const int dlo = dot16(qlo, *(const int4 *)(xc + lo_off), 0);
            const int dhi = dot16(qhi, *(const int4 *)(xc + lo_off + 32), 0);
            const int *bs = xbs + col * (K / 16);
            const int isum = sc_lo * dlo + sc_hi * dhi;
            const int msum = m_lo * bs[lo_off >> 4] + m_hi * bs[(lo_off >> 4) + 2];
            const float dx = xd[col * nsb + sb];
            acc[col] += (d * dx) * (float)isum - (dmin * dx) * (float)msum;
        }
    } else {  // Q6_K
        const int64_t nsb = K / 256;
        const int sb = c >> 3, t = c & 7;
        const int h = t >> 2, u = t & 3;
        const int sh = 2 * (u >> 1);
        const int4 ql = wc.ql, qh = wc.qh;
        const int4 qlo = make_int4((ql.x & 0x0F0F0F0F) | (((qh.x >> sh) & 0x03030303) << 4),
                                   (ql.y & 0x0F0F0F0F) | (((qh.y >> sh) & 0x03030303) << 4),
                                   (ql.z & 0x0F0F0F0F) | (((qh.z >> sh) & 0x03030303) << 4),
                                   (ql.w & 0x0F0F0F0F) | (((qh.w >> sh) & 0x03030303) << 4));
        const int4 qhi = make_int4(((ql.x >> 4) & 0x0F0F0F0F) | (((qh.x >> (sh + 4)) & 0x03030303) << 4),
                                   ((ql.y >> 4) & 0x0F0F0F0F) | (((qh.y >> (sh + 4)) & 0x03030303) << 4),
                                   ((ql.z >> 4) & 0x0F0F0F0F) | (((qh.z >> (sh + 4)) & 0x03030303) << 4),
                                   ((ql.w >> 4) & 0x0F0F0F0F) | (((qh.w >> (sh + 4)) & 0x03030303) << 4));
        const int sc_lo = (int)(int8_t)(wc.sc & 0xFF);
        const int sc_hi = (int)(int8_t)((wc.sc >> 8) & 0xFF);
        const float d = h2f((uint16_t)wc.d);
        const int lo_off = sb * 256 + 128 * h + 32 * (u >> 1) + 16 * (u & 1);
#pragma unroll
        for (int col = 0; col < NC; col++) {
            if (GUARD && col >= ncols) break;
            const int8_t *xc = xq + col * K;
            const int *bs = xbs + col * (K / 16);
            // The codes are 0..63; (q - 32) . x = q . x - 32 * sum(x), and sum(x) over 16 elements is a Q8_K bsum.
            const int dlo = dot16(qlo, *(const int4 *)(xc + lo_off), 0) - 32 * bs[lo_off >> 4];
            const int dhi = dot16(qhi, *(const int4 *)(xc + lo_off + 64), 0) - 32 * bs[(lo_off >> 4) + 4];
            const int isum = sc_lo * dlo + sc_hi * dhi;
            acc[col] += (d * xd[col * nsb + sb]) * (float)isum;
        }
    }
}

// acc[col] += contribution of chunk c of weight row `grow` (global row index within the tensor's planes).
template <int TYPE, int NC, bool GUARD>
__device__ __forceinline__ void chunk_dot(const WPlanes &w, int64_t grow, int64_t K, int c, const int8_t *xq,
                                          const float *xd, const int *xbs, int ncols, float *acc) {
    dot_chunk<TYPE, NC, GUARD>(load_chunk<TYPE>(w, grow, K, c), K, c, xq, xd, xbs, ncols, acc);
}

// LDS bytes the activations of `ncols` columns take.
__host__ __device__ inline size_t act_lds_bytes(int type, int64_t K, int ncols) {
    if (type == MX_TYPE_F16 || type == MX_TYPE_F32) return (size_t)ncols * (size_t)K * 4;  // fp32 (or fp16-rounded)
    if (type == MX_TYPE_Q8_0) return (size_t)ncols * (size_t)K + (size_t)ncols * (size_t)(K / 32) * 4;
    if (type == MX_TYPE_Q4_K)
        return (size_t)ncols * (size_t)K + (size_t)ncols * (size_t)(K / 256) * 4 + (size_t)ncols * (size_t)(K / 32) * 4;
    return (size_t)ncols * (size_t)K + (size_t)ncols * (size_t)(K / 256) * 4 + (size_t)ncols * (size_t)(K / 16) * 4;
}

}  // namespace mx
