// The decoder layer's other ops on the device (src/common/qwen3-decoder.cpp:350-410): RMS_NORM (with the norm weight's
// MUL fused when the graph has it next), ADD / MUL with broadcast, GLU SWIGLU, ROPE in NEOX mode, SET_ROWS into the
// f16 KV cache, and FLASH_ATTN_EXT over that cache. Each restates ggml-cpu's arithmetic for f32 rows:
//   RMS_NORM: squares rounded to float, summed in double, mean rounded to float, y = x * (1 / sqrtf(mean + eps));
//   ROPE NEOX: angles p * theta_scale^k formed by the same chain of float products as ggml_rope_cache_init;
//   SET_ROWS: fp16 of each value, round to nearest even (bit-exact);
//   FLASH_ATTN_EXT: q rounded to fp16, k.q as an fp32 sum of exact products, online softmax; the V accumulator is
//                   fp32, as the graph requests with ggml_prec_set_acc(GGML_PREC_F32) (ggml-cpu's own loop keeps it
//                   in fp16).
#include "mx_common.h"

#ifndef MX_FA_GROUP_WGS
#define MX_FA_GROUP_WGS 256  // k_fa_gqa workgroups a launch aims for (at most one 64-position chunk each, if so many)
#endif
#include "mx_device.h"

// No contraction of a * b + c into an fma unless written as fmaf: ggml-cpu forms RoPE's x0 cos - x1 sin (and the other
// expressions here) with separate roundings, and the same expression inlined into two kernels must round alike (the
// fused q / k post and attention kernels give the bits of the separate ones).
#pragma clang fp contract(off)

#include "mx_layer.h"

namespace mx {

// ---------------------------------------------------------------------------------------------------------- RMS_NORM
// One wave per row; rows (i1, i2, i3) of src and dst at their byte strides; w (ne0 floats) multiplies the normalized
// row when given (the MUL by the norm weight that follows ggml_rms_norm in the graph, with its own rounding).
__global__ __launch_bounds__(256) void k_rms_norm(RowsArgs a, float eps, const float *w) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.nrows) return;  // whole wave
    const int lane = threadIdx.x & 63;
    const int64_t i1 = row % a.ne1, i2 = (row / a.ne1) % a.ne2, i3 = row / (a.ne1 * a.ne2);
    const float *x = (const float *)((const uint8_t *)a.src + i1 * a.s_nb1 + i2 * a.s_nb2 + i3 * a.s_nb3);
    float *y = (float *)((uint8_t *)a.dst + i1 * a.d_nb1 + i2 * a.d_nb2 + i3 * a.d_nb3);
    // eight loads per lane in flight at a time; each lane still adds its elements in index order
    const int64_t n = a.ne0, full = n - n % 512;
    double sum = 0.0;
    for (int64_t i0 = 0; i0 < full; i0 += 512) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = x[i0 + 64 * u + lane];
#pragma unroll
        for (int u = 0; u < 8; u++) sum += (double)(v[u] * v[u]);
    }
    for (int64_t i = full + lane; i < n; i += 64) {
        const float v = x[i];
        sum += (double)(v * v);
    }
    sum = wave_sum_d(sum);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i0 = 0; i0 < full; i0 += 512) {
        float v[8], g[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            v[u] = x[i0 + 64 * u + lane];
            g[u] = w ? w[i0 + 64 * u + lane] : 1.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float t = v[u] * scale;
            y[i0 + 64 * u + lane] = w ? t * g[u] : t;
        }
    }
    for (int64_t i = full + lane; i < n; i += 64) {
        const float t = x[i] * scale;
        y[i] = w ? t * w[i] : t;
    }
}

// ------------------------------------------------------------------------------------------------------ ADD / MUL
// dst[i] = a[i] op b[i mod b's shape] (ggml's repeat broadcast), dst contiguous in a's shape.
__global__ __launch_bounds__(256) void k_binary(BinaryArgs a) {
    const int64_t n = a.ne[0] * a.ne[1] * a.ne[2] * a.ne[3];
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
        const int64_t i0 = e % a.ne[0], i1 = (e / a.ne[0]) % a.ne[1], i2 = (e / (a.ne[0] * a.ne[1])) % a.ne[2];
        const int64_t i3 = e / (a.ne[0] * a.ne[1] * a.ne[2]);
        const float u = *(const float *)((const uint8_t *)a.a + i0 * 4 + i1 * a.a_nb[1] + i2 * a.a_nb[2] +
                                         i3 * a.a_nb[3]);
        const float v = *(const float *)((const uint8_t *)a.b + (i0 % a.b_ne[0]) * 4 + (i1 % a.b_ne[1]) * a.b_nb[1] +
                                         (i2 % a.b_ne[2]) * a.b_nb[2] + (i3 % a.b_ne[3]) * a.b_nb[3]);
        float *y = (float *)((uint8_t *)a.dst + i0 * 4 + i1 * a.d_nb[1] + i2 * a.d_nb[2] + i3 * a.d_nb[3]);
        *y = a.op == 0 ? u + v : u * v;
    }
}

// ---------------------------------------------------------------------------------------------------------- SWIGLU
// dst = silu(a) * b, silu(x) = x / (1 + expf(-x)) (ggml_vec_swiglu_f32's scalar form); rows at byte strides.
__global__ __launch_bounds__(256) void k_swiglu(RowsArgs a, const float *b, int64_t b_nb1) {
    const int64_t n = a.ne0 * a.nrows;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
        const int64_t i0 = e % a.ne0, r = e / a.ne0;
        const float u = ((const float *)((const uint8_t *)a.src + r * a.s_nb1))[i0];
        const float v = ((const float *)((const uint8_t *)b + r * b_nb1))[i0];
        ((float *)((uint8_t *)a.dst + r * a.d_nb1))[i0] = u / (1.0f + expf(-u)) * v;
    }
}

// ------------------------------------------------------------------------------------------------------ ROPE NEOX
// x [ne0, ne1 = heads, ne2 = rows] at byte strides, one position per row. Thread per (pair k, head, row): the angle is
// p * theta_scale^k by the float chain theta = p; theta *= theta_scale (k times), then times freq_scale.
__global__ __launch_bounds__(256) void k_rope_neox(RowsArgs a, const int32_t *pos, int n_dims, float theta_scale,
                                                   float freq_scale) {
    const int64_t half = n_dims / 2;
    const int64_t n = half * a.ne1 * a.ne2;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
        const int64_t k = e % half, h = (e / half) % a.ne1, r = e / (half * a.ne1);
        const float *x = (const float *)((const uint8_t *)a.src + h * a.s_nb1 + r * a.s_nb2);
        float *y = (float *)((uint8_t *)a.dst + h * a.d_nb1 + r * a.d_nb2);
        float theta = (float)pos[r];
        for (int64_t j = 0; j < k; j++) theta *= theta_scale;
        const float t = freq_scale * theta;
        const float c = cosf(t), s = sinf(t);
        const float x0 = x[k], x1 = x[k + half];
        y[k] = x0 * c - x1 * s;
        y[k + half] = x0 * s + x1 * c;
    }
    // channels past n_dims are copied
    const int64_t rest = a.ne0 - n_dims;
    if (rest > 0) {
        const int64_t m = rest * a.ne1 * a.ne2;
        for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < m; e += (int64_t)gridDim.x * 256) {
            const int64_t i = n_dims + e % rest, h = (e / rest) % a.ne1, r = e / (rest * a.ne1);
            ((float *)((uint8_t *)a.dst + h * a.d_nb1 + r * a.d_nb2))[i] =
                ((const float *)((const uint8_t *)a.src + h * a.s_nb1 + r * a.s_nb2))[i];
        }
    }
}

// -------------------------------------------------------------------------------------------------------- SET_ROWS
// dst row idx[i] (f16, byte stride d_nb1) = fp16(src row i); an index outside [0, dst_rows) sets error bit 2 and
// leaves the cache as it was.
__global__ __launch_bounds__(256) void k_set_rows_f16(RowsArgs a, const void *idx, int idx_i64, int64_t dst_rows,
                                                      int *err) {
    const int64_t n = a.ne0 * a.nrows;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
        const int64_t i0 = e % a.ne0, r = e / a.ne0;
        const int64_t d = idx_i64 ? ((const int64_t *)idx)[r] : (int64_t)((const int32_t *)idx)[r];
        if (d < 0 || d >= dst_rows) {
            if (i0 == 0) atomicOr(err, 4);
            continue;
        }
        const float v = ((const float *)((const uint8_t *)a.src + r * a.s_nb1))[i0];
        ((uint16_t *)((uint8_t *)a.dst + d * a.d_nb1))[i0] = f2h(v);
    }
}

// ------------------------------------------------------------------------------------- q / k norm, RoPE, KV stores
// The attention block's per-head work between the q/k/v products and attention (qwen3-decoder.cpp:366-378) in one
// launch, head size 128 with RoPE over all of it: one wave per (head item, row); lane l holds channels l and l + 64,
// which are the NEOX pair l. Items 0 .. nq-1: q heads, normed (rms_norm then mul by q_norm), turned, written to
// q_out; nq .. nq+nkv-1: k heads, normed with k_norm, turned, written to the f16 K cache at row pos; then the v heads
// written to the V cache at row pos. Arithmetic as k_rms_norm, k_rope_neox and k_set_rows_f16 perform it.
__global__ __launch_bounds__(256) void k_qkv_post(QkvPostArgs a) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6), r = blockIdx.y;
    const int lane = threadIdx.x & 63;
    if (item >= a.nq + 2 * a.nkv) return;  // whole wave
    const bool isq = item < a.nq, isv = item >= a.nq + a.nkv;
    const int64_t h = isq ? item : (isv ? item - a.nq - a.nkv : item - a.nq);
    const float *x = isq ? (const float *)((const uint8_t *)a.q + h * a.q_nb1 + r * a.q_nb2)
                         : isv ? (const float *)((const uint8_t *)a.v + h * a.v_nb1 + r * a.v_nb2)
                               : (const float *)((const uint8_t *)a.k + h * a.k_nb1 + r * a.k_nb2);
    const float x0 = x[lane], x1 = x[lane + 64];  // the head's loads go out with the position's
    float w0 = 0.0f, w1 = 0.0f;
    if (!isv) {
        const float *w = isq ? a.qw : a.kw;
        w0 = w[lane];
        w1 = w[lane + 64];
    }
    const int64_t p = a.pos[r];
    const bool bad = p < 0 || p >= a.cache_rows;  // nothing is stored at a bad row; q is still written
    if (bad && lane == 0 && item == 0) atomicOr(a.err, 4);
    if (isv) {
        if (bad) return;
        uint16_t *dst = (uint16_t *)((uint8_t *)a.vc + p * a.vc_nb1) + h * 128;
        dst[lane] = f2h(x0);
        dst[lane + 64] = f2h(x1);
        return;
    }
    float o0, o1;
    qk_norm_rope(x0, x1, w0, w1, p, a.eps, a.theta_scale, a.freq_scale, lane, o0, o1);
    if (isq) {
        float *o = (float *)((uint8_t *)a.q_out + h * a.qo_nb1 + r * a.qo_nb2);
        o[lane] = o0;
        o[lane + 64] = o1;
    } else if (!bad) {
        uint16_t *dst = (uint16_t *)((uint8_t *)a.kc + p * a.kc_nb1) + h * 128;
        dst[lane] = f2h(o0);
        dst[lane + 64] = f2h(o1);
    }
}

hipError_t launch_qkv_post(const QkvPostArgs &a, int64_t rows, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const dim3 grid((unsigned)((a.nq + 2 * a.nkv + 3) / 4), (unsigned)rows);
    hipLaunchKernelGGL(k_qkv_post, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

// -------------------------------------------------------------------------------------------------- FLASH_ATTN_EXT
// Pass 1 splits the positions into whole 64-position blocks and writes (max, sum, D accumulated channels) per (split,
// head, row) to the partials -- or, when there is one split, the normalized row to dst. Head size 128 with 1, 2 or 4
// q heads per kv head takes k_fa_gqa (one workgroup per kv head's group); other shapes take k_fa_split, one wave per
// (kv split, head, query row): lane j scores position j of each 64-position chunk, then each lane accumulates D/64
// adjacent channels of V over the chunk, all of the chunk's V loads in flight before the first product.
// Pass 2 (k_fa_merge) merges the splits of each (head, row).
// The loads of one 64-position chunk, issued together ahead of their use: lane j's key row (position base + j),
// every lane's DL channels of the 64 value rows, and lane j's mask value. Positions past the split repeat its last
// one; their score is -inf, so neither their key nor their value counts.
template <int D>
struct FaChunk {
    uint4 k[D / 8];
    uint32_t v[64];  // D = 128: channels 2l, 2l + 1 of row t; D = 64: channel l (low half)
    float mv;
};

template <int D>
__device__ __forceinline__ void fa_load_k(FaChunk<D> &c, const FaArgs &a, const uint8_t *kb, const uint16_t *mrow,
                                          int64_t base, int64_t j1) {
    const int lane = threadIdx.x;
    const int64_t j = base + lane, jj = min(j, j1 - 1);
    const uint4 *kr = (const uint4 *)(kb + jj * a.k_nb1);
#pragma unroll
    for (int t = 0; t < D / 8; t++) c.k[t] = kr[t];
    c.mv = j < j1 ? (mrow ? h2f(mrow[j]) : 0.0f) : -INFINITY;
}
template <int D>
__device__ __forceinline__ void fa_load_v(FaChunk<D> &c, const FaArgs &a, const uint8_t *vb, int64_t base,
                                          int64_t j1) {
    const int lane = threadIdx.x;
#pragma unroll
    for (int t = 0; t < 64; t++) {
        const uint8_t *row = vb + min(base + t, j1 - 1) * a.v_nb1;
        c.v[t] = D == 128 ? *(const uint32_t *)(row + 4 * lane) : (uint32_t)*(const uint16_t *)(row + 2 * lane);
    }
}

template <int D>
__global__ __launch_bounds__(64) void k_fa_split(FaArgs a) {
    static_assert(D == 64 || D == 128, "head size 64 or 128");
    constexpr int DL = D / 64;  // channels per lane
    __shared__ float qs[D];
    __shared__ float ps[64];
    const int lane = threadIdx.x;
    const int64_t split = blockIdx.x, h = blockIdx.y, i = blockIdx.z;
    const int64_t hk = h / a.gqa;
    const uint8_t *kb = (const uint8_t *)a.k + hk * a.k_nb2;
    const uint8_t *vb = (const uint8_t *)a.v + hk * a.v_nb2;
    const uint16_t *mrow = a.mask ? (const uint16_t *)((const uint8_t *)a.mask + i * a.m_nb1) : nullptr;
    const int64_t j0 = split * a.split_len, j1 = min(a.n_kv, j0 + a.split_len);
    FaChunk<D> ch;
    if (j0 < j1) {  // the first chunk's loads go out before q's
        fa_load_k<D>(ch, a, kb, mrow, j0, j1);
        fa_load_v<D>(ch, a, vb, j0, j1);
    }
    const float *q = (const float *)((const uint8_t *)a.q + i * a.q_nb1 + h * a.q_nb2);
    for (int d = lane; d < D; d += 64) qs[d] = h2f(f2h(q[d]));  // ggml converts q to K's f16 first
    __syncthreads();

    float M = -INFINITY, S = 0.0f;
    float acc[DL];
#pragma unroll
    for (int c = 0; c < DL; c++) acc[c] = 0.0f;
    for (int64_t base = j0; base < j1; base += 64) {
        const bool more = base + 64 < j1;  // uniform
        float s = -INFINITY;
        if (ch.mv != -INFINITY) {
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < D / 8; c++) {
                const uint32_t wv[4] = {ch.k[c].x, ch.k[c].y, ch.k[c].z, ch.k[c].w};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    dot = fmaf(h2f((uint16_t)(wv[t] & 0xFFFF)), qs[8 * c + 2 * t], dot);
                    dot = fmaf(h2f((uint16_t)(wv[t] >> 16)), qs[8 * c + 2 * t + 1], dot);
                }
            }
            s = dot * a.scale + ch.mv;
        }
        if (more) fa_load_k<D>(ch, a, kb, mrow, base + 64, j1);  // the key registers are free again
        const float mc = wave_max_f(s);
        if (mc != -INFINITY) {  // uniform: a chunk with every position masked adds nothing
            const float Mn = fmaxf(M, mc);
            const float r = expf(M - Mn);  // 0 while M is -inf
            const float p = s == -INFINITY ? 0.0f : expf(s - Mn);
            S = S * r + wave_sum_f(p);
#pragma unroll
            for (int c = 0; c < DL; c++) acc[c] *= r;
            M = Mn;
            ps[lane] = p;
            __syncthreads();
#pragma unroll
            for (int t = 0; t < 64; t++) {
                const float pt = ps[t];
                if constexpr (D == 128) {
                    acc[0] = fmaf(pt, h2f((uint16_t)(ch.v[t] & 0xFFFF)), acc[0]);
                    acc[1] = fmaf(pt, h2f((uint16_t)(ch.v[t] >> 16)), acc[1]);
                } else {
                    acc[0] = fmaf(pt, h2f((uint16_t)ch.v[t]), acc[0]);
                }
            }
            __syncthreads();
        }
        if (more) fa_load_v<D>(ch, a, vb, base + 64, j1);
    }
    // lane l holds channels DL l .. DL l + DL - 1
    if (a.nsplit == 1) {
        float *o = a.dst + (i * a.n_head + h) * D;
        const float inv = S == 0.0f ? 0.0f : 1.0f / S;
#pragma unroll
        for (int c = 0; c < DL; c++) o[DL * lane + c] = acc[c] * inv;
        return;
    }
    float *part = a.part + ((i * a.n_head + h) * a.nsplit + split) * (D + 2);
#pragma unroll
    for (int c = 0; c < DL; c++) part[2 + DL * lane + c] = acc[c];
    if (lane == 0) {
        part[0] = M;
        part[1] = S;
    }
}

// Pass 2: one wave per (head, row). Lane s holds split s's max and sum (nsplit <= 64), so the splits' weights
// exp(m_s - M) and the total come from one round of loads and two wave reductions; the channels are gathered 64 / DL
// splits at a time, their loads in flight together (the first round's with the maxima's).
template <int D>
__device__ __forceinline__ void fa_merge_head(const FaArgs &a, int64_t h, int64_t i, int lane) {
    constexpr int DL = D / 64, NB = 64 / DL;  // NB splits' channels per round of loads (64 registers)
    const int ns = a.nsplit;
    const float *part = a.part + (i * a.n_head + h) * ns * (D + 2);
    // every lane loads (lanes past the splits read the last one's and then drop it): a load under a branch is waited
    // for at the branch's join, before the first round's loads below would be issued
    float ms = part[min(lane, ns - 1) * (D + 2)], ss = part[min(lane, ns - 1) * (D + 2) + 1];
    float v[NB][DL];
    auto gather = [&](int s0) {
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int sp = min(s0 + u, ns - 1);
#pragma unroll
            for (int c = 0; c < DL; c++) v[u][c] = part[sp * (D + 2) + 2 + DL * lane + c];
        }
    };
    gather(0);  // the first round's loads travel with the maxima's: the asm, after them, is the maxima's first use
    asm volatile("" : "+v"(ms), "+v"(ss)::"memory");
    if (lane >= ns) {
        ms = -INFINITY;
        ss = 0.0f;
    }
    const float M = wave_max_f(ms);
    const float w = (ms == -INFINITY) ? 0.0f : expf(ms - M);  // a split with nothing visible weighs 0
    const float S = wave_sum_f(ss * w);
    float acc[DL];
#pragma unroll
    for (int c = 0; c < DL; c++) acc[c] = 0.0f;
    for (int s0 = 0; s0 < ns; s0 += NB) {
        if (s0 > 0) gather(s0);
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const float wu = s0 + u < ns ? __shfl(w, min(s0 + u, ns - 1), 64) : 0.0f;
#pragma unroll
            for (int c = 0; c < DL; c++) acc[c] = fmaf(v[u][c], wu, acc[c]);
        }
    }
    float *o = a.dst + (i * a.n_head + h) * D;
    const float inv = S == 0.0f ? 0.0f : 1.0f / S;
#pragma unroll
    for (int c = 0; c < DL; c++) o[DL * lane + c] = acc[c] * inv;
}

template <int D>
__global__ __launch_bounds__(64) void k_fa_merge(FaArgs a) {
    fa_merge_head<D>(a, blockIdx.x, blockIdx.y, threadIdx.x);
}

// One 64-position chunk of 256-byte K and V rows for 256 threads: thread t copies 16 bytes of rows t / 16 + 16 u,
// threads 0..63 the mask of position t, kept as its f16 bits until the chunk is staged (converted at the load, its
// wait would hold the thread until every load of the chunk had landed). Rows past j1 repeat row j1 - 1 and are
// masked (-inf).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));  // (HIP's uint4 class here is kept in scratch)
struct FaStage {
    u32x4 k[4], v[4];
    uint32_t mh;
};

// NT: nontemporal loads, for a decode row, whose workgroups each read their cache chunk once (several query rows
// read each chunk once per row, and keep the plain loads that leave it in the cache for the next).
template <bool NT>
__device__ __forceinline__ void fa_stage_rows(FaStage &st, const FaArgs &a, const uint8_t *kb, const uint8_t *vb,
                                              int64_t base, int64_t j1, int tid) {
    const int lr = tid >> 4, seg = tid & 15;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int64_t jr = min(base + lr + 16 * u, j1 - 1);
        const u32x4 *kp = (const u32x4 *)(kb + jr * a.k_nb1 + 16 * seg);
        const u32x4 *vp = (const u32x4 *)(vb + jr * a.v_nb1 + 16 * seg);
        st.k[u] = NT ? __builtin_nontemporal_load(kp) : *kp;
        st.v[u] = NT ? __builtin_nontemporal_load(vp) : *vp;
    }
}
// Every thread loads, with no branch (a branch's join would wait for the load at once): position base + (tid & 63)
// clamped into the split, or with no mask the first bytes of the head's K rows; fa_mask_value picks the value.
__device__ __forceinline__ void fa_stage_mask(FaStage &st, const uint16_t *mrow, const uint8_t *kb, int64_t base,
                                              int64_t j1, int tid) {
    st.mh = *(mrow ? mrow + min(base + (tid & 63), j1 - 1) : (const uint16_t *)kb);
}
__device__ __forceinline__ float fa_mask_value(const FaStage &st, const uint16_t *mrow, int64_t base, int64_t j1,
                                               int tid) {
    return base + tid < j1 ? (mrow ? h2f((uint16_t)st.mh) : 0.0f) : -INFINITY;
}

// Pass 1 for head size 128 and GQA groups of G = 1, 2 or 4 q heads per kv head: one 256-thread workgroup per (split,
// kv head, query row) serves the group's G heads, so a group reads K and V once. Per 64-position chunk the keys and
// values are copied to LDS with coalesced 16-byte loads (sixteen threads per 256-byte row), the next chunk's loads
// issued before this chunk's arithmetic; T = 256 / (64 G) threads share each score (CPT channels each, then a shuffle
// sum); one wave per head runs the online softmax over the chunk; and for P.V each thread owns a channel pair of one
// head over PLEN positions, the position parts added at the end. The split count aims at MX_FA_GROUP_WGS workgroups:
// at decode that is one chunk per workgroup, the fastest form measured (fewer, longer splits serialize their chunks).
//
// POST (one query row): the q / k norms, RoPE and KV-cache stores of k_qkv_post run in the prologue, from the raw
// q / k / v of pa (heads at pa.*_nb1): wave g turns q head hk G + g into qs; the workgroup whose split holds the new
// position p (the last split when p lies past the positions read) turns kv head hk's key, stores key and value into
// the caches at row p and stages them from LDS in place of that row's (not yet written) cache bytes. No other
// workgroup reads row p, so the stores race with nothing.
template <int G, bool POST>
__global__ __launch_bounds__(256) void k_fa_gqa(FaArgs a, QkvPostArgs pa) {
    constexpr int D = 128, T = 256 / (G * 64), CPT = D / T, PP = 256 / G / 64, PLEN = 64 / PP;
    constexpr int KS = D * 2 + 16;  // bytes per K row in LDS: padded so 16 rows read at one offset miss each other
    __shared__ __align__(16) uint8_t Ks[64 * KS];
    __shared__ __align__(16) uint32_t Vs[64 * 64];  // [position][channel pair]
    __shared__ __align__(16) float qs[G][D];
    __shared__ float ps[G][64], mvs[64], hm[G], hs[G], hr[G];
    __shared__ __align__(16) float accs[PP * G * D];
    // The fields on the way to the first loads, requested together into scalar registers (left to the compiler, they
    // came in over several round trips in a row).
    asm volatile("" ::"s"(a.k), "s"(a.v), "s"(a.k_nb2), "s"(a.v_nb2), "s"(a.mask), "s"(a.m_nb1), "s"(a.split_len),
                 "s"(a.n_kv), "s"(a.k_nb1), "s"(a.v_nb1));
    if constexpr (POST)
        asm volatile("" ::"s"(pa.pos), "s"(pa.cache_rows), "s"(pa.q), "s"(pa.q_nb1), "s"(pa.qw), "s"(pa.k), "s"(pa.v),
                     "s"(pa.k_nb1), "s"(pa.v_nb1), "s"(pa.kw), "s"(a.nsplit));
    else
        asm volatile("" ::"s"(a.q), "s"(a.q_nb1), "s"(a.q_nb2));
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t split = blockIdx.x, hk = blockIdx.y, i = blockIdx.z;
    const uint8_t *kb = (const uint8_t *)a.k + hk * a.k_nb2;
    const uint8_t *vb = (const uint8_t *)a.v + hk * a.v_nb2;
    const uint16_t *mrow = a.mask ? (const uint16_t *)((const uint8_t *)a.mask + i * a.m_nb1) : nullptr;
    const int64_t j0 = split * a.split_len, j1 = min(a.n_kv, j0 + a.split_len);
    const int lr = tid >> 4, seg = tid & 15;  // copy role: 16 threads per row, rows lr + 16 t, 16 bytes each
    __shared__ __align__(16) uint16_t knew[POST ? D : 1], vnew[POST ? D : 1];
    bool mine = false;  // POST: this workgroup stores (and reads from LDS) the new row p
    int64_t p = -1;
    float hx0 = 0.f, hx1 = 0.f, hw0 = 0.f, hw1 = 0.f, kx0 = 0.f, kx1 = 0.f, kw0 = 0.f, kw1 = 0.f, v0f = 0.f, v1f = 0.f;
    // POST: the position, the raw heads and the first chunk go out together, before anything waits on the position.
    // Every workgroup loads its kv head's raw key and value (768 bytes): only the one holding the new row uses them,
    // and loading them after the position had arrived would add a dependent round trip to that workgroup.
    // The waits for these loads are counted in loads issued after them, and where the paths into a wait issued
    // different numbers of loads the count falls to the smallest. So every wave issues the same loads, with no branch,
    // after its head loads: the mask (its branches) goes first, each wave loads a q head (waves past the group's heads
    // repeat its last) and the kv head's key and value, then the chunk (a decode row's splits all hold positions).
    FaStage st;
    if constexpr (POST) {
        // A scalar load (nothing writes the positions while the kernel runs), first used by the empty asm after the
        // chunk's loads: its wait is then on the scalar counter, behind every load of the prologue.
        int32_t p32 = *(const __attribute__((address_space(4))) int32_t *)pa.pos;
        fa_stage_mask(st, mrow, kb, j0, j1, tid);
        const float *x = (const float *)((const uint8_t *)pa.q + (hk * G + min(wave, G - 1)) * pa.q_nb1);
        hx0 = x[lane];
        hx1 = x[lane + 64];
        hw0 = pa.qw[lane];
        hw1 = pa.qw[lane + 64];
        const float *xk = (const float *)((const uint8_t *)pa.k + hk * pa.k_nb1);
        const float *xv = (const float *)((const uint8_t *)pa.v + hk * pa.v_nb1);
        kx0 = xk[lane];
        kx1 = xk[lane + 64];
        kw0 = pa.kw[lane];
        kw1 = pa.kw[lane + 64];
        v0f = xv[lane];
        v1f = xv[lane + 64];
        fa_stage_rows<true>(st, a, kb, vb, j0, j1, tid);
        asm volatile("" : "+s"(p32));
        p = p32;
    } else if (j0 < j1) {  // the first chunk's loads go out before q's
        fa_stage_rows<false>(st, a, kb, vb, j0, j1, tid);
        fa_stage_mask(st, mrow, kb, j0, j1, tid);
    }
    if constexpr (POST) {
        const bool bad = p < 0 || p >= pa.cache_rows;
        mine = !bad && ((p >= j0 && p < j1) || (split == a.nsplit - 1 && p >= j1));
        if (bad && split == 0 && hk == 0 && tid == 0) atomicOr(pa.err, 4);
    }
    if constexpr (!POST) {
        for (int e = tid; e < G * D; e += 256) {
            const int g = e / D, d = e % D;
            const float *q = (const float *)((const uint8_t *)a.q + i * a.q_nb1 + (hk * G + g) * a.q_nb2);
            qs[g][d] = h2f(f2h(q[d]));  // ggml converts q to K's f16 first
        }
    } else {  // nothing is stored at a bad row; q is still turned
        if (wave < G) {
            float o0, o1;
            qk_norm_rope(hx0, hx1, hw0, hw1, p, pa.eps, pa.theta_scale, pa.freq_scale, lane, o0, o1);
            qs[wave][lane] = h2f(f2h(o0));  // ggml converts q to K's f16 first
            qs[wave][lane + 64] = h2f(f2h(o1));
        }
        if (mine && wave == (G & 3)) {  // a wave with no q head (wave 0 after its head when G = 4)
            // v's conversion stays here: moved up to its loads, its wait would come before the chunk loads
            asm volatile("" : "+v"(v0f), "+v"(v1f));
            float o0, o1;
            qk_norm_rope(kx0, kx1, kw0, kw1, p, pa.eps, pa.theta_scale, pa.freq_scale, lane, o0, o1);
            const uint16_t k0 = f2h(o0), k1 = f2h(o1), v0 = f2h(v0f), v1 = f2h(v1f);
            uint16_t *kc = (uint16_t *)((uint8_t *)pa.kc + p * pa.kc_nb1) + hk * D;
            uint16_t *vc = (uint16_t *)((uint8_t *)pa.vc + p * pa.vc_nb1) + hk * D;
            kc[lane] = k0;
            kc[lane + 64] = k1;
            vc[lane] = v0;
            vc[lane + 64] = v1;
            knew[lane] = k0;
            knew[lane + 64] = k1;
            vnew[lane] = v0;
            vnew[lane + 64] = v1;
        }
    }
    if (tid < G) {
        hm[tid] = -INFINITY;
        hs[tid] = 0.0f;
    }
    // roles: score (g_s, pos_s, part_s); P.V (g_v, channel pair cp, positions part_v)
    const int dot = tid / T, g_s = dot / 64, pos_s = dot % 64, part_s = tid % T;
    const int wv = tid % (256 / G), g_v = tid / (256 / G), cp = wv % 64, part_v = wv / 64;
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int64_t base = j0; base < j1; base += 64) {
        __syncthreads();  // the previous chunk is done with Ks, Vs, ps
#pragma unroll
        for (int t = 0; t < 4; t++) {
            u32x4 kk = st.k[t], vv = st.v[t];
            if (POST && mine && base + lr + 16 * t == p) {  // the new row, from the prologue
                kk = *(const u32x4 *)(knew + 8 * seg);
                vv = *(const u32x4 *)(vnew + 8 * seg);
            }
            *(u32x4 *)(Ks + (lr + 16 * t) * KS + 16 * seg) = kk;
            *(u32x4 *)(Vs + (lr + 16 * t) * 64 + 4 * seg) = vv;
        }
        if (tid < 64) mvs[tid] = fa_mask_value(st, mrow, base, j1, tid);
        __syncthreads();
        if (base + 64 < j1) {  // overlaps this chunk's work
            fa_stage_rows<POST>(st, a, kb, vb, base + 64, j1, tid);
            fa_stage_mask(st, mrow, kb, base + 64, j1, tid);
        }
        // scores
        {
            const uint8_t *kr = Ks + pos_s * KS + part_s * CPT * 2;
            const float *qv = qs[g_s] + part_s * CPT;
            float d0 = 0.0f;
#pragma unroll
            for (int c = 0; c < CPT / 8; c++) {
                const uint4 w = *(const uint4 *)(kr + 16 * c);
                const float4 qa = *(const float4 *)(qv + 8 * c), qb = *(const float4 *)(qv + 8 * c + 4);
                d0 = fmaf(h2f((uint16_t)(w.x & 0xFFFF)), qa.x, d0);
                d0 = fmaf(h2f((uint16_t)(w.x >> 16)), qa.y, d0);
                d0 = fmaf(h2f((uint16_t)(w.y & 0xFFFF)), qa.z, d0);
                d0 = fmaf(h2f((uint16_t)(w.y >> 16)), qa.w, d0);
                d0 = fmaf(h2f((uint16_t)(w.z & 0xFFFF)), qb.x, d0);
                d0 = fmaf(h2f((uint16_t)(w.z >> 16)), qb.y, d0);
                d0 = fmaf(h2f((uint16_t)(w.w & 0xFFFF)), qb.z, d0);
                d0 = fmaf(h2f((uint16_t)(w.w >> 16)), qb.w, d0);
            }
            if constexpr (T >= 2) d0 += __shfl_xor(d0, 1, 64);
            if constexpr (T >= 4) d0 += __shfl_xor(d0, 2, 64);
            const float m = mvs[pos_s];
            if (part_s == 0) ps[g_s][pos_s] = m == -INFINITY ? -INFINITY : d0 * a.scale + m;
        }
        __syncthreads();
        // online softmax, one wave per head
        if (wave < G) {
            const float sv = ps[wave][lane];
            const float mc = wave_max_f(sv);
            const float Mold = hm[wave];
            float r = 1.0f, p = 0.0f, Mn = Mold;
            if (mc != -INFINITY) {
                Mn = fmaxf(Mold, mc);
                r = expf(Mold - Mn);
                p = sv == -INFINITY ? 0.0f : expf(sv - Mn);
            }
            const float sum = wave_sum_f(p);
            ps[wave][lane] = p;
            if (lane == 0) {
                hr[wave] = r;
                hm[wave] = Mn;
                hs[wave] = hs[wave] * r + sum;
            }
        }
        __syncthreads();
        // P.V
        {
            const float r = hr[g_v];
            acc0 *= r;
            acc1 *= r;
#pragma unroll
            for (int t = 0; t < PLEN; t++) {
                const int j = part_v * PLEN + t;
                const float pj = ps[g_v][j];
                const uint32_t v2 = Vs[j * 64 + cp];
                acc0 = fmaf(pj, h2f((uint16_t)(v2 & 0xFFFF)), acc0);
                acc1 = fmaf(pj, h2f((uint16_t)(v2 >> 16)), acc1);
            }
        }
    }
    __syncthreads();
    accs[(part_v * G + g_v) * D + 2 * cp] = acc0;
    accs[(part_v * G + g_v) * D + 2 * cp + 1] = acc1;
    __syncthreads();
    for (int e = tid; e < G * D; e += 256) {
        const int g = e / D, c = e % D;
        float tot = 0.0f;
#pragma unroll
        for (int pp = 0; pp < PP; pp++) tot += accs[(pp * G + g) * D + c];
        const int64_t h = hk * G + g;
        if (a.nsplit == 1) {
            const float S = hs[g];
            a.dst[(i * a.n_head + h) * D + c] = tot * (S == 0.0f ? 0.0f : 1.0f / S);
        } else {
            float *part = a.part + ((i * a.n_head + h) * a.nsplit + split) * (D + 2);
            part[2 + c] = tot;
            if (c == 0) {
                part[0] = hm[g];
                part[1] = hs[g];
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------- launches
static unsigned grid_for(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return (unsigned)(g < 1 ? 1 : (g > 65535 ? 65535 : g));
}

hipError_t launch_rms_norm(const RowsArgs &a, float eps, const float *w, hipStream_t s) {
    if (a.nrows == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)((a.nrows + 3) / 4)), dim3(256), 0, s, a, eps, w);
    return hipGetLastError();
}

hipError_t launch_binary(const BinaryArgs &a, hipStream_t s) {
    const int64_t n = a.ne[0] * a.ne[1] * a.ne[2] * a.ne[3];
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_binary, dim3(grid_for(n)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_swiglu(const RowsArgs &a, const float *b, int64_t b_nb1, hipStream_t s) {
    const int64_t n = a.ne0 * a.nrows;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_swiglu, dim3(grid_for(n)), dim3(256), 0, s, a, b, b_nb1);
    return hipGetLastError();
}

hipError_t launch_rope_neox(const RowsArgs &a, const int32_t *pos, int n_dims, float theta_scale, float freq_scale,
                            hipStream_t s) {
    const int64_t n = (int64_t)(n_dims / 2) * a.ne1 * a.ne2;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_neox, dim3(grid_for(n)), dim3(256), 0, s, a, pos, n_dims, theta_scale, freq_scale);
    return hipGetLastError();
}

hipError_t launch_set_rows_f16(const RowsArgs &a, const void *idx, bool idx_i64, int64_t dst_rows, int *err,
                               hipStream_t s) {
    const int64_t n = a.ne0 * a.nrows;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_set_rows_f16, dim3(grid_for(n)), dim3(256), 0, s, a, idx, (int)idx_i64, dst_rows, err);
    return hipGetLastError();
}

static bool fa_grouped(int D, int64_t gqa) { return D == 128 && (gqa == 1 || gqa == 2 || gqa == 4); }

int fa_splits(int64_t n_q, int64_t n_head, int64_t n_kv, int64_t gqa, int D) {
    // each split a whole number of 64-position blocks: about MX_FA_GROUP_WGS (split, kv head, row) workgroups for
    // k_fa_gqa, about 512 (split, head, row) waves for k_fa_split
    const int64_t blocks = (n_kv + 63) / 64;
    const bool grouped = fa_grouped(D, gqa);
    const int64_t units = grouped ? n_q * (n_head / gqa) : n_q * n_head;
    if (blocks == 0 || units == 0) return 1;  // nothing to split: no positions (the rows come out zero) or no rows
    const int64_t target = grouped ? MX_FA_GROUP_WGS : 512;
    int64_t want = (target + units - 1) / units;
    want = want < 1 ? 1 : (want > blocks ? blocks : want);
    want = want > 64 ? 64 : want;  // the merge holds one split per lane
    const int64_t per = (blocks + want - 1) / want;  // blocks per split
    return (int)((blocks + per - 1) / per);
}

hipError_t launch_flash_attn(const FaArgs &a, hipStream_t s) {
    if (a.n_q == 0 || a.n_head == 0) return hipSuccess;
    const dim3 g1((unsigned)a.nsplit, (unsigned)a.n_head, (unsigned)a.n_q);
    const dim3 gk((unsigned)a.nsplit, (unsigned)(a.n_head / a.gqa), (unsigned)a.n_q);
    const QkvPostArgs none{};
    if (fa_grouped(a.D, a.gqa) && a.gqa == 2) hipLaunchKernelGGL((k_fa_gqa<2, false>), gk, dim3(256), 0, s, a, none);
    else if (fa_grouped(a.D, a.gqa) && a.gqa == 1) hipLaunchKernelGGL((k_fa_gqa<1, false>), gk, dim3(256), 0, s, a, none);
    else if (fa_grouped(a.D, a.gqa)) hipLaunchKernelGGL((k_fa_gqa<4, false>), gk, dim3(256), 0, s, a, none);
    else if (a.D == 128) hipLaunchKernelGGL(k_fa_split<128>, g1, dim3(64), 0, s, a);
    else if (a.D == 64) hipLaunchKernelGGL(k_fa_split<64>, g1, dim3(64), 0, s, a);
    else return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    const dim3 g2((unsigned)a.n_head, (unsigned)a.n_q);
    if (a.D == 128) hipLaunchKernelGGL(k_fa_merge<128>, g2, dim3(64), 0, s, a);
    else hipLaunchKernelGGL(k_fa_merge<64>, g2, dim3(64), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_attn_decode(const FaArgs &a, const QkvPostArgs &pa, hipStream_t s) {
    if (a.n_q != 1 || !fa_grouped(a.D, a.gqa)) return hipErrorInvalidValue;
    const dim3 gk((unsigned)a.nsplit, (unsigned)(a.n_head / a.gqa), 1);
    if (a.gqa == 2) hipLaunchKernelGGL((k_fa_gqa<2, true>), gk, dim3(256), 0, s, a, pa);
    else if (a.gqa == 1) hipLaunchKernelGGL((k_fa_gqa<1, true>), gk, dim3(256), 0, s, a, pa);
    else hipLaunchKernelGGL((k_fa_gqa<4, true>), gk, dim3(256), 0, s, a, pa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    hipLaunchKernelGGL(k_fa_merge<128>, dim3((unsigned)a.n_head, 1), dim3(64), 0, s, a);
    return hipGetLastError();
}

}  // namespace mx
