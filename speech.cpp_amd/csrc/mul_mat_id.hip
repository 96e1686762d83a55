// MUL_MAT_ID for routed experts: dst[:, s, t] = as[ids[s, t]] . quant(b[:, s % b_ne1, t]).
//
// A few (token, slot) pairs (a decode step) take one mat-vec launch: each pair streams its expert's rows with the
// activation quantized in the prologue. More pairs take two launches, no host round trip:
//   1. prep: workgroup 0 counts (token, slot) pairs per expert, lists the experts that have any, groups the pairs by
//      expert (the matrix_row_counts / matrix_rows of ggml-cpu.c ggml_compute_forward_mul_mat_id) and cuts each
//      expert's pairs into chunks; the other workgroups quantize every activation row once (ggml-cpu quantizes src1
//      once, before the experts run).
//   2. experts: Q4_K experts run as a grouped MFMA product over the chunks (mmid_q4k.hip); Q8_0, Q5_K and Q6_K experts
//      on the fp16 dequantizing GEMM's routed form, a chunk per row tile (gemm_dq.hip), or, when an option asks for it,
//      stream each touched expert's weights once per 8 pairs on dot4 (k_mmid_experts below). Untouched experts cost
//      nothing.
#include "mx_common.h"
#include "mx_device.h"
#include "mx_dot.h"
#include "mx_dq_act.h"

#include <cstdlib>

namespace mx {

static inline size_t al256(size_t v) { return (v + 255) / 256 * 256; }

// Few pairs per expert (at most four on average: a decode-sized batch) take one-tile chunks of 16 and the kernel form
// without a second tile (16 tokens x top-4 of 64 experts: 78.9 against 81.6 us per layer); larger batches share each
// expert's weights between 32 pairs.
int mmid_chunk_for(int64_t npairs, int64_t E, int forced) {
    if (forced == MMID_CHUNK_SMALL || forced == MMID_CHUNK) return forced;
    return npairs <= 4 * E ? MMID_CHUNK_SMALL : MMID_CHUNK;
}

size_t mul_mat_id_scratch(MulMatIdArgs *a, void *base) {
    const int64_t npairs = a->n_ids * a->T;
    const int64_t nrows = a->T * a->b_ne1;
    const int64_t nsc = a->type == MX_TYPE_Q8_0 ? a->K / 32 : a->K / 256;
    size_t off = 0;
    uint8_t *b = (uint8_t *)base;
    a->counts = (int32_t *)(b + off);  off += al256((size_t)a->E * 4);
    a->offsets = (int32_t *)(b + off); off += al256((size_t)a->E * 4);
    a->active = (int32_t *)(b + off);  off += al256((size_t)(a->E + 1) * 4);
    a->pairs = (int32_t *)(b + off);   off += al256((size_t)npairs * 4);
    // the activation rows: quantized blocks for the int8 kernels, or the fp16 GEMM's rows, in the same space (sized
    // for the larger, whichever kernel runs)
    const size_t rows0 = off;
    a->xq = (int8_t *)(b + off);       off += al256((size_t)nrows * (size_t)a->K);
    a->xd = (float *)(b + off);        off += al256((size_t)nrows * (size_t)nsc * 4);
    a->xbs = (int32_t *)(b + off);     off += al256(a->type == MX_TYPE_Q8_0 ? 0 : (size_t)nrows * (size_t)(a->K / 16) * 4);
    a->x16 = (_Float16 *)(b + off);    off += al256(a->type == MX_TYPE_Q4_K ? (size_t)nrows * (size_t)(a->K / 256) * 32 : 0);
    size_t dq = rows0;
    a->xh = (_Float16 *)(b + dq);      dq += al256((size_t)nrows * (size_t)a->K * 2);
    a->rs = (float *)(b + dq);         dq += al256((size_t)nrows * 4);
    off = off > dq ? off : dq;
    // chunks: sum over experts of ceil(count / chunk) <= npairs / chunk + (experts with pairs), sized for the
    // smaller chunk whichever the launch takes
    a->max_tiles = npairs / MMID_CHUNK_SMALL + (npairs < a->E ? npairs : a->E) + 1;
    a->tiles = (int32_t *)(b + off);   off += al256((size_t)a->max_tiles * 12);
    a->ntiles = (int32_t *)(b + off);  off += 256;
    return off;
}

// Exclusive prefix sums of three counters over the 256 threads of a workgroup (tmp: 4 waves' totals in LDS).
__device__ __forceinline__ int3 scan3_256(int3 v, int3 *tmp, int3 *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int3 inc = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int x = __shfl_up(inc.x, off, 64), y = __shfl_up(inc.y, off, 64), z = __shfl_up(inc.z, off, 64);
        if (lane >= off) inc = make_int3(inc.x + x, inc.y + y, inc.z + z);
    }
    if (lane == 63) tmp[wave] = inc;
    __syncthreads();
    int3 base = make_int3(0, 0, 0), all = make_int3(0, 0, 0);
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const int3 t = tmp[w];
        if (w < wave) base = make_int3(base.x + t.x, base.y + t.y, base.z + t.z);
        all = make_int3(all.x + t.x, all.y + t.y, all.z + t.z);
    }
    *total = all;
    return make_int3(base.x + inc.x - v.x, base.y + inc.y - v.y, base.z + inc.z - v.z);
}

// Workgroup 0 of the prep launch: counts (token, slot) pairs per expert, lists the experts that have any, groups the
// pairs by expert (the matrix_row_counts / matrix_rows of ggml-cpu.c ggml_compute_forward_mul_mat_id) and cuts each
// expert's pairs into chunks of up to a.chunk. The order of pairs within an expert does not matter: every pair's
// output is computed on its own.
__device__ void mmid_bucket(const MulMatIdArgs &a) {
    extern __shared__ int cnt[];  // [E]
    __shared__ int3 tmp[4];
    const int tid = threadIdx.x;
    const int E = (int)a.E;
    const int npairs = (int)(a.n_ids * a.T), chunk = a.chunk;
    // a thread's first HELD pairs' experts stay in registers for the second pass (no second round trip for them)
    constexpr int HELD = 8;
    int held[HELD];
    auto expert_of = [&](int p) {
        const int t = p / (int)a.n_ids, s = p - t * (int)a.n_ids;
        return *(const int32_t *)((const uint8_t *)a.ids + s * a.ids_nb0 + t * a.ids_nb1);
    };
#pragma unroll
    for (int k = 0; k < HELD; k++) held[k] = tid + 256 * k < npairs ? expert_of(tid + 256 * k) : -1;
    for (int e = tid; e < E; e += 256) cnt[e] = 0;
    __syncthreads();
    for (int p = tid, k = 0; p < npairs; p += 256, k++) {
        const int32_t e = k < HELD ? held[k] : expert_of(p);
        if (e < 0 || e >= E) atomicOr(a.err, 2);  // ggml-cpu asserts; this pair is dropped and reported
        else atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // each thread owns a run of consecutive experts
    const int ept = (E + 255) / 256, e0 = tid * ept, e1 = min(E, e0 + ept);
    int3 mine = make_int3(0, 0, 0);  // pairs, chunks, experts with pairs
    for (int e = e0; e < e1; e++) {
        const int c = cnt[e];
        mine = make_int3(mine.x + c, mine.y + (c + chunk - 1) / chunk, mine.z + (c > 0));
    }
    int3 total;
    int3 at = scan3_256(mine, tmp, &total);
    for (int e = e0; e < e1; e++) {
        const int c = cnt[e];
        a.counts[e] = c;
        a.offsets[e] = at.x;
        if (c > 0) a.active[1 + at.z++] = e;
        for (int i = 0; i < c; i += chunk, at.y++) {
            a.tiles[3 * at.y] = at.x + i;
            a.tiles[3 * at.y + 1] = min(chunk, c - i);
            a.tiles[3 * at.y + 2] = e;
        }
        cnt[e] = at.x;  // becomes the fill cursor
        at.x += c;
    }
    if (tid == 0) {
        a.active[0] = total.z;
        a.ntiles[0] = total.y;
    }
    __syncthreads();
    for (int p = tid, k = 0; p < npairs; p += 256, k++) {
        const int32_t e = k < HELD ? held[k] : expert_of(p);
        if (e < 0 || e >= E) continue;
        a.pairs[atomicAdd(&cnt[e], 1)] = p;
    }
}

// Quantizes activation row r = t * b_ne1 + s' of b into the scratch rows, 1024 elements per pass (the arithmetic of
// the mat-vec prologue). Q4_K also gets each super-block's sub-block sums split as [64 h_j | l_j] in fp16.
template <int TYPE>
__device__ void mmid_quant_row(const MulMatIdArgs &a, int64_t r) {
    const int64_t t = r / a.b_ne1, s = r % a.b_ne1;
    const float *x = (const float *)((const uint8_t *)a.b + s * a.b_nb1 + t * a.b_nb2);
    const int K = (int)a.K;
    const int lane = threadIdx.x & 63;
    constexpr int PRE = 4;
    float4 v[PRE];
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const int e = 1024 * i + 4 * threadIdx.x;
        v[i] = e < K ? *(const float4 *)(x + e) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int base = 0; base < K; base += 1024) {
        const int i = base / 1024;
        const int e = base + 4 * threadIdx.x;
        float4 xv;
        if (i < PRE) {
            xv = i == 0 ? v[0] : (i == 1 ? v[1] : (i == 2 ? v[2] : v[3]));
        } else {
            xv = e < K ? *(const float4 *)(x + e) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (TYPE == MX_TYPE_Q8_0) {
            float d;
            int sum;
            const int q = quant32_lane(xv, a.rounding, &d, &sum);
            if (e < K) {  // K % 32 == 0: the eight lanes of a block agree
                *(int *)(a.xq + r * K + e) = q;
                if ((threadIdx.x & 7) == 0) a.xd[r * (K / 32) + e / 32] = h2f(f2h(d));
            }
        } else {
            if (base + 256 * (threadIdx.x >> 6) >= K) continue;  // whole wave
            float d;
            int bs;
            const int q = quant256_wave(xv, lane, &d, &bs);
            *(int *)(a.xq + r * K + e) = q;
            if (lane == 0) a.xd[r * (K / 256) + e / 256] = d;
            if ((lane & 3) == 0) a.xbs[r * (K / 16) + e / 16] = bs;
            if (TYPE == MX_TYPE_Q4_K) {
                const int bs32 = bs + dpp_i<dpp::HALF_MIRROR>(0, bs);  // lanes 8j..8j+7: sub-block j's sum
                if ((lane & 7) == 0) {
                    const int j = lane >> 3, h = bs32 >> 6;  // floor(bs32 / 64)
                    _Float16 *o = a.x16 + (r * (K / 256) + e / 256) * 16;
                    o[j] = (_Float16)(64 * h);
                    o[8 + j] = (_Float16)(bs32 - 64 * h);
                }
            }
        }
    }
}

// One launch for both: workgroup 0 buckets the pairs, workgroup 1 + r quantizes activation row r.
template <int TYPE>
__global__ __launch_bounds__(256) void k_mmid_prep(MulMatIdArgs a) {
    // the fields both roles start from, requested together into scalar registers
    asm volatile("" ::"s"(a.n_ids), "s"(a.T), "s"(a.E), "s"(a.ids), "s"(a.ids_nb0), "s"(a.ids_nb1), "s"(a.chunk),
                 "s"(a.b), "s"(a.b_ne1), "s"(a.b_nb1), "s"(a.b_nb2), "s"(a.K));
    if (blockIdx.x == 0) mmid_bucket(a);
    else mmid_quant_row<TYPE>(a, (int64_t)blockIdx.x - 1);
}

// The same for the fp16 GEMM's routed form: workgroup 0 buckets the pairs into chunks of one row tile, workgroup
// 1 + r writes activation row r as that GEMM's own rows (fp16(2^e d q) of the ggml blocks the weight's dot pairs
// with, and 2^-e), the arithmetic of its dense activation pass.
template <int TYPE>
__global__ __launch_bounds__(256) void k_mmid_prep_dq(MulMatIdArgs a) {
    asm volatile("" ::"s"(a.n_ids), "s"(a.T), "s"(a.E), "s"(a.ids), "s"(a.ids_nb0), "s"(a.ids_nb1), "s"(a.chunk),
                 "s"(a.b), "s"(a.b_ne1), "s"(a.b_nb1), "s"(a.b_nb2), "s"(a.K));
    __shared__ float red[4];
    if (blockIdx.x == 0) {
        mmid_bucket(a);
        return;
    }
    const int64_t r = (int64_t)blockIdx.x - 1, t = r / a.b_ne1, s = r % a.b_ne1;
    const float *x = (const float *)((const uint8_t *)a.b + s * a.b_nb1 + t * a.b_nb2);
    if constexpr (TYPE == MX_TYPE_Q8_0) dq_act_row_q8_0<256>(x, (int)a.K, a.rounding, a.xh + r * a.K, a.rs + r, red);
    else dq_act_row_q8k<256>(x, (int)a.K, a.xh + r * a.K, a.rs + r, red);
}

// Q8_0 / Q5_K / Q6_K experts go to the fp16 dequantizing GEMM over the chunks once their pairs share each expert's
// weights enough: measured over 64 experts of 2048 x 1536 (top-4, us per layer, the GEMM against the experts kernel),
// Q8_0 from one pair per expert on average (16 tokens: 130 against 130; 32: 171 against 203; 256: 200 against
// 1,235), the K-quants from three (Q6_K at 32 tokens, two per expert: 221 against 182; 64 tokens: 243 against 280;
// 256: 252 against 983; Q5_K 278 / 233 and 308 / 373). An option forces the experts kernel (1) or the GEMM (2,
// wherever it takes the rows' K).
bool mmid_dq_route(const MulMatIdArgs &a) {
    if (a.type != MX_TYPE_Q8_0 && a.type != MX_TYPE_Q5_K && a.type != MX_TYPE_Q6_K) return false;
    if (a.generic == 1 || !gemm_dq_supported(a.type, a.T * a.b_ne1, a.K)) return false;
    if (a.generic == 2) return true;
    const int64_t npairs = a.n_ids * a.T;
    return npairs >= (a.type == MX_TYPE_Q8_0 ? 1 : 3) * a.E;
}


// Quantized activation row r of the scratch into LDS column col, in the layout the dots read (Q4_K: unit order, and
// the sums of 32 from pairs of bsums).
template <int TYPE>
__device__ __forceinline__ void copy_act_row(const MulMatIdArgs &a, int64_t r, int col, int8_t *xq, float *xd,
                                             int *xbs) {
    const int K = (int)a.K;
    const int nsc = TYPE == MX_TYPE_Q8_0 ? K / 32 : K / 256;
    for (int k = 16 * threadIdx.x; k < K; k += 16 * 256) {
        const int dst = TYPE == MX_TYPE_Q4_K ? q4u_xq_offset(k, K) : k;
        *(int4 *)(xq + col * K + dst) = *(const int4 *)(a.xq + r * K + k);
    }
    for (int k = threadIdx.x; k < nsc; k += 256) xd[col * nsc + k] = a.xd[r * nsc + k];
    if constexpr (TYPE == MX_TYPE_Q4_K) {
        for (int k = threadIdx.x; k < K / 32; k += 256)
            xbs[col * (K / 32) + k] = a.xbs[r * (K / 16) + 2 * k] + a.xbs[r * (K / 16) + 2 * k + 1];
    } else if constexpr (TYPE != MX_TYPE_Q8_0) {
        for (int k = threadIdx.x; k < K / 16; k += 256) xbs[col * (K / 16) + k] = a.xbs[r * (K / 16) + k];
    }
}

// Q4_K rows against the pass's activation columns one column at a time (a runtime loop: the unit's decoded codes are
// shared, and the registers stay those of one column whatever the pass holds), each column's units summed in the
// order the many-column dot sums them. `pre` holds the lane's first unit when `held`.
template <int LPR>
__device__ __forceinline__ void experts_q4k_columns(const MulMatIdArgs &a, const WChunk<MX_TYPE_Q4_K> &pre, bool held,
                                                    int64_t grow, int64_t row, int sub, int nchunks, int first, int ng,
                                                    const int8_t *xq, const float *xd, const int *xbs) {
    const int64_t K = a.K;
#pragma unroll 1
    for (int col = 0; col < ng; col++) {
        const int8_t *cq = xq + col * K;
        const float *cd = xd + col * (K / 256);
        const int *cb = xbs + col * (K / 32);
        float acc = 0.0f;
        int c = sub;
        if (held) {
            if (c < nchunks) dot_chunk<MX_TYPE_Q4_K, 1, false>(pre, K, c, cq, cd, cb, 1, &acc);
            c += LPR;
        }
#pragma unroll 1
        for (; c < nchunks; c += LPR)
            dot_chunk<MX_TYPE_Q4_K, 1, false>(load_chunk<MX_TYPE_Q4_K>(a.w, grow, K, c), K, c, cq, cd, cb, 1, &acc);
        acc = sum_lanes<LPR>(acc);
        if (sub == LPR - 1) {
            const int p = a.pairs[first + col];
            const int64_t t = p / a.n_ids, s = p % a.n_ids;
            float *y = (float *)((uint8_t *)a.dst + s * a.dst_nb1 + t * a.dst_nb2);
            y[row] = acc;
        }
    }
}

// One workgroup per (block of 4 G weight rows, active expert): the expert's pairs in passes of up to NC columns, each
// pass copying their quantized rows to LDS and streaming the rows' weights against them. An expert with at most NC
// pairs (every one at small batches) runs in one pass whose weight loads go out first.
template <int TYPE, int LPR>
__global__ __launch_bounds__(256) void k_mmid_experts(MulMatIdArgs a) {
    constexpr int NC = MAX_COLS;
    extern __shared__ __align__(16) uint8_t smem[];
    const int j = blockIdx.y;
    const int nact = a.active[0];
    if (j >= nact) return;  // uniform: the whole workgroup leaves
    const int e = a.active[1 + j];
    const int cnt = a.counts[e], off = a.offsets[e];
    const int64_t K = a.K;
    const int64_t nsc = TYPE == MX_TYPE_Q8_0 ? K / 32 : K / 256;
    int8_t *xq = (int8_t *)smem;
    float *xd = (float *)(smem + (size_t)NC * K);
    int *xbs = (int *)(xd + NC * nsc);

    constexpr int G = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int64_t row = (int64_t)blockIdx.x * (4 * G) + wave * G + grp;
    const bool has_row = row < a.N;
    const int64_t grow = (int64_t)e * a.N + row;
    const int nchunks = (int)(K / chunk_elems<TYPE>());

    if (cnt <= NC) {  // uniform: one pass, whose weight chunks go out before the activation copies
        constexpr int PRE = preload_of<TYPE>();  // requested before the activation rows are copied to LDS
        const int64_t prow = (int64_t)e * a.N + (has_row ? row : a.N - 1);  // rows past the end load the last row
        WChunk<TYPE> pre[PRE];
#pragma unroll
        for (int i = 0; i < PRE; i++) {
            const int c = sub + i * LPR;
            pre[i] = load_chunk<TYPE>(a.w, prow, K, c < nchunks ? c : nchunks - 1);
        }
        for (int col = 0; col < cnt; col++) {
            const int p = a.pairs[off + col];
            const int64_t t = p / a.n_ids, s = p % a.n_ids;
            const int64_t r = t * a.b_ne1 + (s % a.b_ne1);
            copy_act_row<TYPE>(a, r, col, xq, xd, xbs);
        }
        __syncthreads();
        if (!has_row) return;  // whole LPR-lane groups leave together; no barrier follows
        if constexpr (TYPE == MX_TYPE_Q4_K) {
            static_assert(PRE == 1, "one held Q4_K unit");
            experts_q4k_columns<LPR>(a, pre[0], true, grow, row, sub, nchunks, off, cnt, xq, xd, xbs);
        } else {
            float acc[NC];
#pragma unroll
            for (int c = 0; c < NC; c++) acc[c] = 0.0f;
#pragma unroll
            for (int i = 0; i < PRE; i++) {
                const int c = sub + i * LPR;
                if (c < nchunks) dot_chunk<TYPE, NC, true>(pre[i], K, c, xq, xd, xbs, cnt, acc);
            }
#pragma unroll 1
            for (int c = sub + PRE * LPR; c < nchunks; c += LPR) chunk_dot<TYPE, NC, true>(a.w, grow, K, c, xq, xd, xbs, cnt, acc);
#pragma unroll
            for (int c = 0; c < NC; c++) acc[c] = sum_lanes<LPR>(acc[c]);
            if (sub == LPR - 1) {
#pragma unroll
                for (int col = 0; col < NC; col++) {
                    if (col < cnt) {
                        const int p = a.pairs[off + col];
                        const int64_t t = p / a.n_ids, s = p % a.n_ids;
                        float *y = (float *)((uint8_t *)a.dst + s * a.dst_nb1 + t * a.dst_nb2);
                        y[row] = acc[col];
                    }
                }
            }
        }
        return;
    }
    for (int g0 = 0; g0 < cnt; g0 += NC) {
        const int ng = cnt - g0 < NC ? cnt - g0 : NC;
        __syncthreads();  // the previous pass is done with LDS
        for (int col = 0; col < ng; col++) {
            const int p = a.pairs[off + g0 + col];
            const int64_t t = p / a.n_ids, s = p % a.n_ids;
            const int64_t r = t * a.b_ne1 + (s % a.b_ne1);
            copy_act_row<TYPE>(a, r, col, xq, xd, xbs);
        }
        __syncthreads();
        if constexpr (TYPE == MX_TYPE_Q4_K) {
            if (has_row)
                experts_q4k_columns<LPR>(a, WChunk<MX_TYPE_Q4_K>{}, false, grow, row, sub, nchunks, off + g0, ng, xq, xd,
                                         xbs);
        } else if (has_row) {
            float acc[NC];
#pragma unroll
            for (int c = 0; c < NC; c++) acc[c] = 0.0f;
#pragma unroll 1
            for (int c = sub; c < nchunks; c += LPR) chunk_dot<TYPE, NC, true>(a.w, grow, K, c, xq, xd, xbs, ng, acc);
#pragma unroll
            for (int c = 0; c < NC; c++) acc[c] = sum_lanes<LPR>(acc[c]);
            if (sub == LPR - 1) {  // the lane holding the group's sum
#pragma unroll
                for (int col = 0; col < NC; col++) {
                    if (col < ng) {
                        const int p = a.pairs[off + g0 + col];
                        const int64_t t = p / a.n_ids, s = p % a.n_ids;
                        float *y = (float *)((uint8_t *)a.dst + s * a.dst_nb1 + t * a.dst_nb2);
                        y[row] = acc[col];
                    }
                }
            }
        }
    }
}

template <int TYPE>
static hipError_t launch_typed(const MulMatIdArgs &a, hipStream_t s) {
    const int64_t nrows = a.T * a.b_ne1;
    if constexpr (TYPE != MX_TYPE_Q4_K) {
        if (mmid_dq_route(a)) {
            MulMatIdArgs b = a;
            b.chunk = mmid_dq_chunk(a);  // one row tile per chunk
            hipLaunchKernelGGL(k_mmid_prep_dq<TYPE>, dim3((unsigned)(nrows + 1)), dim3(256), (size_t)a.E * 4, s, b);
            const hipError_t err = hipGetLastError();
            if (err != hipSuccess) return err;
            return launch_gemm_dq_routed(b, s);
        }
    }
    hipLaunchKernelGGL(k_mmid_prep<TYPE>, dim3((unsigned)(nrows + 1)), dim3(256), (size_t)a.E * 4, s, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int64_t npairs = a.n_ids * a.T;
    // Q4_K: the grouped MFMA product unless an option asks for the experts kernel (measured at 16 tokens x top-4 of
    // 64 experts, 64 pairs: 86 us per layer grouped against 114 us on the one-pass experts kernel)
    const bool grouped = a.generic != 1;
    if (TYPE == MX_TYPE_Q4_K && grouped && mmid_q4k_supported(a)) return launch_mmid_q4k(a, s);
    const unsigned gy = (unsigned)(npairs < a.E ? npairs : a.E);
    const size_t lds = act_lds_bytes(TYPE, a.K, MAX_COLS);
    // lanes per row: the fewest whose chunks per lane fit the preload (as the mat-vec picks them); one launch per
    // product, all reading the one prep's tables and rows
    const int64_t nchunks = a.K / chunk_elems<TYPE>();
    MulMatIdArgs b = a;
    for (int p = 0; p < a.nprob; p++) {
        b.w = a.wg[p];
        b.dst = a.dstg[p];
        if (nchunks <= 16 * preload_of<TYPE>()) {
            hipLaunchKernelGGL((k_mmid_experts<TYPE, 16>), dim3((unsigned)((a.N + 15) / 16), gy), dim3(256), lds, s, b);
        } else if (nchunks <= 32 * preload_of<TYPE>()) {
            hipLaunchKernelGGL((k_mmid_experts<TYPE, 32>), dim3((unsigned)((a.N + 7) / 8), gy), dim3(256), lds, s, b);
        } else {
            hipLaunchKernelGGL((k_mmid_experts<TYPE, 64>), dim3((unsigned)((a.N + 3) / 4), gy), dim3(256), lds, s, b);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Up to a.matvec_pairs (token, slot) pairs (16 unless a backend's option says otherwise) run as one mat-vec launch
// per pair: each pair streams its expert's rows with the activation quantized in the prologue, so a decode step's
// MUL_MAT_ID is a single launch. More pairs go through the bucket and share each expert's weights between them.
static hipError_t launch_matvec_ids(const MulMatIdArgs &a, hipStream_t s) {
    MatvecArgs m{};
    m.type = a.type;
    m.ncols = 1;
    m.rounding = a.rounding;
    m.K = a.K;
    m.x = a.b;
    m.x_col_stride = 0;
    m.nbatch = (int)(a.n_ids * a.T);
    m.ne12 = (int)a.n_ids;
    m.ne02 = 1;
    m.r2 = 1;
    m.r3 = 1;
    m.x_b2 = a.b_nb1 / 4;
    m.x_b3 = a.b_nb2 / 4;
    m.y_b2 = a.dst_nb1 / 4;
    m.y_b3 = a.dst_nb2 / 4;
    m.nprob = a.nprob;  // the products share x and ids: one launch
    for (int p = 0; p < a.nprob; p++) {
        m.prob[p].w = a.wg[p];
        m.prob[p].N = a.N;
        m.prob[p].row0 = 0;
        m.prob[p].y = a.dstg[p];
        m.prob[p].y_col_stride = 0;
    }
    m.ids = a.ids;
    m.ids_nb0 = a.ids_nb0;
    m.ids_nb1 = a.ids_nb1;
    m.n_mats = (int)a.E;
    m.x_ne12 = (int)a.b_ne1;
    m.err = a.err;
    m.lpr = a.lpr;
    return launch_matvec(m, s);
}

hipError_t launch_mul_mat_id(const MulMatIdArgs &a, hipStream_t s) {
    if (a.n_ids * a.T == 0 || a.N == 0) return hipSuccess;
    if (a.n_ids * a.T <= a.matvec_pairs) return launch_matvec_ids(a, s);
    switch (a.type) {
        case MX_TYPE_Q8_0: return launch_typed<MX_TYPE_Q8_0>(a, s);
        case MX_TYPE_Q4_K: return launch_typed<MX_TYPE_Q4_K>(a, s);
        case MX_TYPE_Q5_K: return launch_typed<MX_TYPE_Q5_K>(a, s);
        case MX_TYPE_Q6_K: return launch_typed<MX_TYPE_Q6_K>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
