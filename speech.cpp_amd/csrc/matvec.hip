// Small-M quantized products (decode M = 1, draft verification M <= 5): y[n, m] = W[n, :] . quant(x[:, m]).
//
// One launch does everything: the workgroup first quantizes its NC activation columns into LDS (the ggml CPU src1
// conversion, bit for bit), then streams weight rows with 16-byte loads from the planar layout and reduces each row
// over LPR lanes. HBM-bound by design: each weight byte is read once per launch.
#include "mx_common.h"
#include "mx_device.h"
#include "mx_dot.h"

#include <cstdlib>

namespace mx {

__device__ __forceinline__ MatvecProblem pick_problem(const MatvecArgs &a, int i) {
    // Uniform selection keeps the kernel-argument struct out of private memory.
    return i == 0 ? a.prob[0] : (i == 1 ? a.prob[1] : (i == 2 ? a.prob[2] : a.prob[3]));
}

// Chunks of weights each lane loads before the activation prologue (preload_of: four 16-byte chunks, or one 64-byte
// Q4_K unit), so the weight stream's first HBM round trip overlaps the load and quantization of x instead of
// following it.

// float4s of each activation column every thread loads ahead of the weights (elements 1024 i + 4 tid, i < XPRE).
template <int NC>
__host__ __device__ constexpr int xpre() { return NC == 1 ? 4 : (NC == 2 ? 2 : 1); }

// Quantizes the 1024-element piece at `base` of one activation column (v = elements base + 4 tid .. + 3) into LDS:
// Q8_0 weights take 32-blocks (d rounded to fp16 and back, as the CPU dot reads it), K-quants Q8_K 256-blocks with
// their 16-element sums. Every wave of the workgroup calls it with the same `base`.
template <int TYPE>
__device__ __forceinline__ void quantize_piece(float4 v, int base, int K, int rounding, int8_t *xq, float *xd,
                                               int *xbs) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int e = base + 4 * tid;
    if constexpr (TYPE == MX_TYPE_Q8_0) {
        float d;
        int sum;
        const int q = quant32_lane(v, rounding, &d, &sum);
        if (e < K) {  // K % 32 == 0: the eight lanes of a block agree
            *(int *)(xq + e) = q;
            if ((tid & 7) == 0) xd[e / 32] = h2f(f2h(d));
        }
    } else {
        if (base + 256 * (tid >> 6) < K) {  // a whole wave per super-block
            float d;
            int bs;
            const int q = quant256_wave(v, lane, &d, &bs);
            if (lane == 0) xd[e / 256] = d;
            if constexpr (TYPE == MX_TYPE_Q4_K) {  // unit order, and sums of 32
                *(int *)(xq + q4u_xq_offset(e, K)) = q;
                const int bs32 = bs + dpp_i<dpp::HALF_MIRROR>(0, bs);  // lanes 8j..8j+7: quants 32j..32j+31
                if ((lane & 7) == 0) xbs[e / 32] = bs32;
            } else {
                *(int *)(xq + e) = q;
                if ((lane & 3) == 0) xbs[e / 16] = bs;
            }
        }
    }
}

__device__ __forceinline__ float4 load_x4(const float *xc, int e, int K) {
    const float4 v = *(const float4 *)(xc + (e < K ? e : K - 4));
    return e < K ? v : make_float4(0.f, 0.f, 0.f, 0.f);
}

// The fused prologue: each column x becomes silu(x) * glu_b (ggml_vec_swiglu_f32's scalar form) when glu_b is set,
// then mul(rms_norm(x, eps), norm_w) when norm_w is set -- the squares (rounded to float) summed in double over the
// workgroup, the mean rounded to float, x * (1 / sqrtf(mean + eps)) then times the weight, as the separate ops round
// -- and is quantized. Pieces of 1024 elements past the preloaded ones are read again after the sum.
template <int TYPE, int NC>
__device__ __forceinline__ void fused_prologue(const MatvecArgs &a, const float *x, int xi12, int i13,
                                               float4 (&xr)[NC][xpre<NC>()], const float4 (&br)[NC][xpre<NC>()],
                                               const float4 (&wr)[xpre<NC>()], int8_t *xq, float *xd, int *xbs) {
    constexpr int XP = xpre<NC>();
    constexpr int XDB = TYPE == MX_TYPE_Q8_0 ? 32 : 256;
    const int K = (int)a.K;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ double red[NC][4];
    const float *gb = a.glu_b ? a.glu_b + xi12 * a.x_b2 + i13 * a.x_b3 : nullptr;
    // glu of one loaded piece; the preloaded pieces' second operands came in with x (br)
    auto piece_b = [&](float4 v, float4 b) -> float4 {
        v.x = v.x / (1.0f + expf(-v.x)) * b.x;
        v.y = v.y / (1.0f + expf(-v.y)) * b.y;
        v.z = v.z / (1.0f + expf(-v.z)) * b.z;
        v.w = v.w / (1.0f + expf(-v.w)) * b.w;
        return v;
    };
    auto piece = [&](int c, int base, float4 v) -> float4 {
        if (gb) {
            const float4 b = load_x4(gb + c * a.x_col_stride, base + 4 * tid, K);
            v.x = v.x / (1.0f + expf(-v.x)) * b.x;
            v.y = v.y / (1.0f + expf(-v.y)) * b.y;
            v.z = v.z / (1.0f + expf(-v.z)) * b.z;
            v.w = v.w / (1.0f + expf(-v.w)) * b.w;
        }
        return v;
    };
    if (gb) {
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int i = 0; i < XP; i++) xr[c][i] = piece_b(xr[c][i], br[c][i]);
    }
    float scale[NC];
    if (a.norm_w) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < XP; i++) {
                const float4 v = xr[c][i];  // zero past K
                ss += (double)(v.x * v.x) + (double)(v.y * v.y) + (double)(v.z * v.z) + (double)(v.w * v.w);
            }
            for (int base = 1024 * XP; base < K; base += 1024) {
                const float4 v = piece(c, base, load_x4(x + c * a.x_col_stride, base + 4 * tid, K));
                ss += (double)(v.x * v.x) + (double)(v.y * v.y) + (double)(v.z * v.z) + (double)(v.w * v.w);
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
            if (lane == 0) red[c][wave] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const double tot = red[c][0] + red[c][1] + red[c][2] + red[c][3];
            const float mean = (float)(tot / (double)K);
            scale[c] = 1.0f / sqrtf(mean + a.norm_eps);
        }
    }
    auto normed = [&](int c, int base, float4 v) -> float4 {
        if (a.norm_w) {
            const float4 w = base < 1024 * XP ? wr[base / 1024] : load_x4(a.norm_w, base + 4 * tid, K);
            v.x = (v.x * scale[c]) * w.x;
            v.y = (v.y * scale[c]) * w.y;
            v.z = (v.z * scale[c]) * w.z;
            v.w = (v.w * scale[c]) * w.w;
        }
        return v;
    };
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const float *xc = x + c * a.x_col_stride;
#pragma unroll
        for (int i = 0; i < XP; i++)
            if (1024 * i < K)
                quantize_piece<TYPE>(normed(c, 1024 * i, xr[c][i]), 1024 * i, K, a.rounding, xq + c * K,
                                     xd + c * (K / XDB), xbs + c * xbs_per_col<TYPE>(K));
        for (int base = 1024 * XP; base < K; base += 1024)
            quantize_piece<TYPE>(normed(c, base, piece(c, base, load_x4(xc, base + 4 * tid, K))), base, K, a.rounding,
                                 xq + c * K, xd + c * (K / XDB), xbs + c * xbs_per_col<TYPE>(K));
    }
}

// FUSED: the instantiation that reads the fused operands (norm weight, SwiGLU input, residual); the plain one is
// compiled without them, so products with no fusion keep their smaller register footprint.
template <int TYPE, int NC, int LPR, bool FUSED>
__global__ __launch_bounds__(256) void k_matvec(MatvecArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int K = (int)a.K;
    const int tid = threadIdx.x;
    // Batch slice; a single slice (decode) takes no division.
    int i12 = 0, i13 = 0, mat = 0;
    if (a.nbatch > 1) {
        const unsigned z = blockIdx.z;
        i12 = (int)(z % (unsigned)a.ne12);
        i13 = (int)(z / (unsigned)a.ne12);
        mat = (int)((unsigned)i12 / (unsigned)a.r2) + (int)((unsigned)i13 / (unsigned)a.r3) * a.ne02;
    }
    int xi12 = i12;
    if (a.ids) {  // routed expert: the slice's matrix comes from ids (uniform over the workgroup)
        mat = *(const int32_t *)((const uint8_t *)a.ids + i12 * a.ids_nb0 + i13 * a.ids_nb1);
        if (mat < 0 || mat >= a.n_mats) {  // ggml-cpu asserts; this pair's output is left as it was and reported
            if (tid == 0) atomicOr(a.err, 2);
            return;
        }
        xi12 = (int)((unsigned)i12 % (unsigned)a.x_ne12);
    }
    const float *x = a.x + xi12 * a.x_b2 + i13 * a.x_b3;

    // The activation loads go first: x -> quantization -> LDS is the prologue's critical path, and the memory counter
    // retires loads in order, so waiting for x then does not wait for the weight loads issued after it.
    constexpr int XP = xpre<NC>();
    float4 xr[NC][XP];
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
        for (int i = 0; i < XP; i++) xr[c][i] = load_x4(x + c * a.x_col_stride, 1024 * i + 4 * tid, K);
    // the fused prologue's other operands come in with x: SwiGLU's second input and the norm weight
    float4 br[NC][XP], wr[XP];
    if (FUSED && a.glu_b) {
        const float *gb = a.glu_b + xi12 * a.x_b2 + i13 * a.x_b3;
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int i = 0; i < XP; i++) br[c][i] = load_x4(gb + c * a.x_col_stride, 1024 * i + 4 * tid, K);
    }
    if (FUSED && a.norm_w) {
#pragma unroll
        for (int i = 0; i < XP; i++) wr[i] = load_x4(a.norm_w, 1024 * i + 4 * tid, K);
    }

    const MatvecProblem p = pick_problem(a, (int)blockIdx.y);
    constexpr int G = 64 / LPR;  // rows in flight per wave
    const int lane = tid & 63, wave = tid >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int64_t row = (int64_t)blockIdx.x * (4 * G) + wave * G + grp;
    const bool has_row = row < p.N;
    // Rows past the end load (and then ignore) the last row, chunks past the end the last chunk: the preloads carry no
    // lane-dependent branch, so they issue back to back.
    const int64_t grow = p.row0 + (int64_t)mat * p.N + (has_row ? row : p.N - 1);
    const int nchunks = K / chunk_elems<TYPE>();

    // the residual the epilogue adds, requested now rather than after the reduction
    const int64_t yoff = i12 * a.y_b2 + i13 * a.y_b3 + row;
    float rr[NC];
    if (FUSED && p.res && has_row && sub == LPR - 1) {
#pragma unroll
        for (int c = 0; c < NC; c++) rr[c] = p.res[yoff + c * p.y_col_stride];
    }

    constexpr int PRE = preload_of<TYPE>();
    WChunk<TYPE> pre[PRE];
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const int c = sub + i * LPR;
        pre[i] = load_chunk<TYPE>(p.w, grow, K, c < nchunks ? c : nchunks - 1);
    }

    int8_t *xq = (int8_t *)smem;
    float *xd = (float *)(smem + (size_t)NC * K);
    constexpr int XDB = TYPE == MX_TYPE_Q8_0 ? 32 : 256;
    int *xbs = (int *)(xd + NC * (K / XDB));
    if constexpr (FUSED) {
        if (a.glu_b || a.norm_w) {  // uniform: the fused prologue
            fused_prologue<TYPE, NC>(a, x, xi12, i13, xr, br, wr, xq, xd, xbs);
        } else {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const float *xc = x + c * a.x_col_stride;
#pragma unroll
                for (int i = 0; i < XP; i++)
                    if (1024 * i < K)
                        quantize_piece<TYPE>(xr[c][i], 1024 * i, K, a.rounding, xq + c * K, xd + c * (K / XDB),
                                             xbs + c * xbs_per_col<TYPE>(K));
                for (int base = 1024 * XP; base < K; base += 1024)
                    quantize_piece<TYPE>(load_x4(xc, base + 4 * tid, K), base, K, a.rounding, xq + c * K,
                                         xd + c * (K / XDB), xbs + c * xbs_per_col<TYPE>(K));
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const float *xc = x + c * a.x_col_stride;
#pragma unroll
            for (int i = 0; i < XP; i++)
                if (1024 * i < K) quantize_piece<TYPE>(xr[c][i], 1024 * i, K, a.rounding, xq + c * K, xd + c * (K / XDB),
                                                       xbs + c * xbs_per_col<TYPE>(K));
            for (int base = 1024 * XP; base < K; base += 1024)
                quantize_piece<TYPE>(load_x4(xc, base + 4 * tid, K), base, K, a.rounding, xq + c * K,
                                     xd + c * (K / XDB), xbs + c * xbs_per_col<TYPE>(K));
        }
    }
    __syncthreads();
    if (!has_row) return;  // whole LPR-lane groups leave together; no barrier follows

    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = 0.0f;
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const int c = sub + i * LPR;
        if (c < nchunks) dot_chunk<TYPE, NC, false>(pre[i], K, c, xq, xd, xbs, NC, acc);
    }
    if constexpr (TYPE == MX_TYPE_Q4_K) {  // a unit's registers are four chunks': one at a time
#pragma unroll 1
        for (int c = sub + PRE * LPR; c < nchunks; c += LPR)
            chunk_dot<TYPE, NC, false>(p.w, grow, K, c, xq, xd, xbs, NC, acc);
    } else {
#pragma unroll 4
        for (int c = sub + PRE * LPR; c < nchunks; c += LPR)
            chunk_dot<TYPE, NC, false>(p.w, grow, K, c, xq, xd, xbs, NC, acc);
    }
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = sum_lanes<LPR>(acc[c]);
    if (sub == LPR - 1) {  // the lane holding the group's sum
        float *y = p.y + yoff;
        if (FUSED && p.res) {  // the residual ADD that follows the product, fused
#pragma unroll
            for (int c = 0; c < NC; c++) y[c * p.y_col_stride] = rr[c] + acc[c];
        } else {
#pragma unroll
            for (int c = 0; c < NC; c++) y[c * p.y_col_stride] = acc[c];
        }
    }
}

// Lanes per row: the fewest (16, 32 or 64) whose chunks per lane all fit the preload, so every weight byte of a lane
// is requested before the activation prologue; rows longer than that take 64 lanes. Measured on the decode shapes
// (K 1024..3072): one full preload beats more workgroups with shorter streams. A backend's option forces it.
static int pick_lpr(int64_t nchunks, int preload, int forced) {
    if (forced == 16 || forced == 32 || forced == 64) return forced;
    int lpr = 16;
    while (lpr < 64 && nchunks > (int64_t)preload * lpr) lpr *= 2;
    return lpr;
}

// ------------------------------------------------------------------------------------------ routed experts, small T
// MUL_MAT_ID at small batches (src/families/drama3/text-model.cpp:208-210: gate / up / down over the routed experts)
// in one launch with no scratch and no bucketing pass. Workgroup (row block, slot j, product z) reads every (token,
// slot) pair's expert id, takes the j-th distinct expert (ascending ids; slots past the number of distinct experts
// leave), quantizes the activation rows of that expert's pairs into LDS itself, MMID_SMALL_COLS at a time, and streams
// the expert's rows against them -- each weight row is read once per launch whatever the number of pairs sharing the
// expert, and the weight loads go out before the activation rows are quantized. Every pair's output is computed on
// its own, so the order of an expert's pairs does not matter. Ids outside [0, E) are left out and reported (bit 2),
// as the bucketing pass does.
// Expert planes: the planar layout's planes advanced by `first_row` rows of K elements (the bytes one row holds in each
// plane), so that a row and chunk within the expert take 32-bit offsets.
template <int TYPE>
__device__ __forceinline__ WPlanes expert_planes(const WPlanes &w, int64_t first_row, int64_t K) {
    WPlanes r = w;
    if constexpr (TYPE == MX_TYPE_Q8_0) {
        r.p0 += first_row * K;
        r.p1 += first_row * (K / 16);
    } else if constexpr (TYPE == MX_TYPE_Q4_K) {
        r.p0 += first_row * (K / 2);
        r.p1 += first_row * (K / 256 * 12);
        r.p2 += first_row * (K / 256 * 4);
    } else if constexpr (TYPE == MX_TYPE_Q5_K) {
        r.p0 += first_row * (K / 2);
        r.p1 += first_row * (K / 8);
        r.p2 += first_row * (K / 256 * 12);
        r.p3 += first_row * (K / 256 * 4);
    } else {
        r.p0 += first_row * (K / 2);
        r.p1 += first_row * (K / 4);
        r.p2 += first_row * (K / 16);
        r.p3 += first_row * (K / 128);
    }
    return r;
}

// load_chunk with 32-bit offsets from the planes' bases (rows of one expert).
template <int TYPE>
__device__ __forceinline__ WChunk<TYPE> load_chunk32(const WPlanes &w, uint32_t row, uint32_t K, int c) {
    WChunk<TYPE> r;
    const uint32_t cc = (uint32_t)c;
    if constexpr (TYPE == MX_TYPE_Q8_0) {
        r.q = ld_w16(w.p0 + (row * K + 16u * cc));
        r.d = ld_w16b(w.p1 + (row * (K / 32u) + (cc >> 1)) * 2u);
    } else if constexpr (TYPE == MX_TYPE_Q4_K) {  // unit c: half c & 1 of super-block c >> 1
        const uint32_t blk = row * (K / 256u) + (cc >> 1);
        const uint8_t *qp = w.p0 + (blk * 128u + 64u * (cc & 1u));
#pragma unroll
        for (int i = 0; i < 4; i++) r.q[i] = ld_w16(qp + 16 * i);
        const uint8_t *sp = w.p1 + blk * 12u;
        r.s0 = ld_w32(sp);
        r.s1 = ld_w32(sp + 4);
        r.s2 = ld_w32(sp + 8);
        r.dm = ld_w32(w.p2 + blk * 4u);
    } else if constexpr (TYPE == MX_TYPE_Q5_K) {
        const uint32_t blk = row * (K / 256u) + (cc >> 3);
        r.q = ld_w16(w.p0 + (blk * 128u + 16u * (cc & 7u)));
        r.qh = ld_w16(w.p1 + (blk * 32u + 16u * (cc & 1u)));
        const uint8_t *sp = w.p2 + blk * 12u;
        r.s0 = ld_w32(sp);
        r.s1 = ld_w32(sp + 4);
        r.s2 = ld_w32(sp + 8);
        r.dm = ld_w32(w.p3 + blk * 4u);
    } else {
        const uint32_t blk = row * (K / 256u) + (cc >> 3);
        const uint32_t t = cc & 7u, h = t >> 2, u = t & 3u;
        r.ql = ld_w16(w.p0 + (blk * 128u + 64u * h + 16u * u));
        r.qh = ld_w16(w.p1 + (blk * 64u + 32u * h + 16u * (u & 1u)));
        const uint32_t lo_sc = 8u * h + 2u * (u >> 1) + (u & 1u);
        const uint8_t *sp = w.p2 + blk * 16u;
        r.sc = ld_w8(sp + lo_sc) | (ld_w8(sp + lo_sc + 4) << 8);
        r.d = ld_w16b(w.p3 + blk * 2u);
    }
    return r;
}

// Chunks each lane holds per row block of the small-batch kernel: one Q4_K unit, else MMID_SMALL_PRE chunks.
template <int TYPE>
constexpr int small_pre() { return TYPE == MX_TYPE_Q4_K ? 1 : MMID_SMALL_PRE; }

template <int TYPE, int LPR>
__global__ __launch_bounds__(256) void k_mmid_small(MulMatIdArgs a) {
    constexpr int NC = MMID_SMALL_COLS, SP = small_pre<TYPE>();
    constexpr int XDB = TYPE == MX_TYPE_Q8_0 ? 32 : 256;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ __align__(16) uint8_t s_flag[MMID_SMALL_MAX_E];
    __shared__ int16_t s_list[MMID_SMALL_MAX_PAIRS];
    __shared__ int s_wsum[4];
    __shared__ int s_e, s_cnt;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = (int)a.E, nid = (int)a.n_ids, npairs = (int)(a.n_ids * a.T);
    const int K = (int)a.K;

    // every pair's expert: pair p = tid + 256 i, token p / n_ids, slot p % n_ids; -1 past the pairs, -2 out of range
    int ex[MMID_SMALL_MAX_PAIRS / 256];
#pragma unroll
    for (int i = 0; i < MMID_SMALL_MAX_PAIRS / 256; i++) {
        const int p = tid + 256 * i;
        ex[i] = -1;
        if (p < npairs) {
            const int t = p / nid, s = p - t * nid;
            const int32_t e = *(const int32_t *)((const uint8_t *)a.ids + s * a.ids_nb0 + t * a.ids_nb1);
            ex[i] = (e >= 0 && e < E) ? e : -2;
        }
    }
    for (int e = 4 * tid; e < E; e += 4 * 256) *(uint32_t *)(s_flag + e) = 0u;
    if (tid == 0) {
        s_e = -1;
        s_cnt = 0;
    }
    __syncthreads();
    bool bad = false;
#pragma unroll
    for (int i = 0; i < MMID_SMALL_MAX_PAIRS / 256; i++) {
        if (ex[i] >= 0) s_flag[ex[i]] = 1;
        bad = bad || ex[i] == -2;
    }
    if (bad && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) atomicOr(a.err, 2);
    __syncthreads();
    // the j-th distinct expert: thread tid counts the flags of experts 4 tid .. 4 tid + 3 (E <= 1024), and an exclusive
    // scan of the counts over the workgroup places it
    const uint32_t f4 = 4 * tid < E ? *(const uint32_t *)(s_flag + 4 * tid) : 0u;
    const int c = (int)(f4 & 1u) + (int)((f4 >> 8) & 1u) + (int)((f4 >> 16) & 1u) + (int)(f4 >> 24);
    int inc = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(inc, off, 64);
        if (lane >= off) inc += v;
    }
    if (lane == 63) s_wsum[wave] = inc;
    __syncthreads();
    int base = inc - c;
#pragma unroll
    for (int w = 0; w < 4; w++)
        if (w < wave) base += s_wsum[w];
    const int j = (int)blockIdx.y;
    if (j >= base && j < base + c) {
        int k = j - base;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            if ((f4 >> (8 * b)) & 1u) {
                if (k == 0) s_e = 4 * tid + b;
                k--;
            }
        }
    }
    __syncthreads();
    const int e = s_e;
    if (e < 0) return;  // uniform: fewer distinct experts than slots
#pragma unroll
    for (int i = 0; i < MMID_SMALL_MAX_PAIRS / 256; i++)
        if (ex[i] == e) s_list[atomicAdd(&s_cnt, 1)] = (int16_t)(tid + 256 * i);

    __syncthreads();
    const int cnt = s_cnt;

    // product z, expert e's planes (uniform bases: the loads take 32-bit offsets); this workgroup's run of row blocks
    // of 4 G rows
    const int z = (int)blockIdx.z;
    const WPlanes wz = z == 0 ? a.wg[0] : (z == 1 ? a.wg[1] : (z == 2 ? a.wg[2] : a.wg[3]));
    float *const dst = z == 0 ? a.dstg[0] : (z == 1 ? a.dstg[1] : (z == 2 ? a.dstg[2] : a.dstg[3]));
    const WPlanes w = expert_planes<TYPE>(wz, (int64_t)__builtin_amdgcn_readfirstlane(e) * a.N, a.K);
    constexpr int G = 64 / LPR;
    const int sub = lane % LPR, grp = lane / LPR;
    const int nblocks = (int)((a.N + 4 * G - 1) / (4 * G));
    const int per = (nblocks + (int)gridDim.x - 1) / (int)gridDim.x;
    const int rb0 = (int)blockIdx.x * per, nb = min(per, nblocks - rb0);
    const int nchunks = K / chunk_elems<TYPE>();
    auto row_of = [&](int rb) { return rb * (4 * G) + wave * G + grp; };
    auto load_block = [&](int rb, WChunk<TYPE> (&c)[SP]) {
        const int row = row_of(rb);
        const uint32_t r = (uint32_t)(row < a.N ? row : a.N - 1);  // rows past the end load the last row
#pragma unroll
        for (int i = 0; i < SP; i++) {
            const int ch = sub + i * LPR;
            c[i] = load_chunk32<TYPE>(w, r, (uint32_t)K, ch < nchunks ? ch : nchunks - 1);
        }
    };

    int8_t *xq = (int8_t *)smem;
    float *xd = (float *)(smem + (size_t)NC * K);
    int *xbs = (int *)(xd + NC * (K / XDB));
    const int KP = (K + 1023) / 1024;  // 1024-element pieces per activation row
    // pieces q0 .. q0 + 3 of the pass's rows (piece q: row q / KP, elements 1024 (q % KP) ..)
    auto load_pieces = [&](int g0, int nq, int q0, float4 (&v)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int q = q0 + u;
            if (q < nq) {
                const int col = q / KP, piece = q - col * KP;
                const int p = s_list[g0 + col];
                const int t = p / nid, s = p - t * nid;
                const float *xr = (const float *)((const uint8_t *)a.b + (s % (int)a.b_ne1) * a.b_nb1 + t * a.b_nb2);
                v[u] = load_x4(xr, 1024 * piece + 4 * tid, K);
            }
        }
    };
    auto quantize_pieces = [&](int nq, int q0, const float4 (&v)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int q = q0 + u;
            if (q < nq) {
                const int col = q / KP, piece = q - col * KP;
                quantize_piece<TYPE>(v[u], 1024 * piece, K, a.rounding, xq + col * K, xd + col * (K / XDB),
                                     xbs + col * xbs_per_col<TYPE>(K));
            }
        }
    };
    // Passes of up to NC of the expert's pairs: the pass's activation rows into LDS, then the run of row blocks against
    // them. The pass's first pieces are requested before the first block's weight chunks (the memory counter retires
    // loads in order, so the quantization waits for the pieces alone); later passes (experts with more pairs) read the
    // blocks again, from the caches.
    WChunk<TYPE> cur[SP];
#pragma unroll 1
    for (int g0 = 0; g0 < cnt; g0 += NC) {
        const int ng = cnt - g0 < NC ? cnt - g0 : NC, nq = ng * KP;
        if (g0 > 0) __syncthreads();  // the previous pass is done with the rows in LDS
        {
            float4 v[4];
            load_pieces(g0, nq, 0, v);
            load_block(rb0, cur);
            quantize_pieces(nq, 0, v);
        }
#pragma unroll 1
        for (int q0 = 4; q0 < nq; q0 += 4) {
            float4 v[4];
            load_pieces(g0, nq, q0, v);
            quantize_pieces(nq, q0, v);
        }
        __syncthreads();
#pragma unroll 1
        for (int r = 0; r < nb; r++) {
            if (r > 0) load_block(rb0 + r, cur);
            const int row = row_of(rb0 + r);
            if (row < a.N) {
                // one column at a time, each a one-column dot over the held chunks: the registers stay those of one
                // column, whatever the pass holds
#pragma unroll 1
                for (int col = 0; col < ng; col++) {
                    const int8_t *cq = xq + col * K;
                    const float *cd = xd + col * (K / XDB);
                    const int *cb = xbs + col * xbs_per_col<TYPE>(K);
                    float acc = 0.0f;
#pragma unroll
                    for (int i = 0; i < SP; i++) {
                        const int ch = sub + i * LPR;
                        if (ch < nchunks) dot_chunk<TYPE, 1, false>(cur[i], K, ch, cq, cd, cb, 1, &acc);
                    }
#pragma unroll 1
                    for (int ch = sub + SP * LPR; ch < nchunks; ch += LPR)
                        dot_chunk<TYPE, 1, false>(load_chunk32<TYPE>(w, (uint32_t)row, (uint32_t)K, ch), K, ch, cq, cd,
                                                  cb, 1, &acc);
                    acc = sum_lanes<LPR>(acc);
                    if (sub == LPR - 1) {  // the lane holding the group's sum
                        const int p = s_list[g0 + col];
                        const int t = p / nid, s = p - t * nid;
                        float *y = (float *)((uint8_t *)dst + s * a.dst_nb1 + t * a.dst_nb2);
                        y[row] = acc;
                    }
                }
            }
        }
    }
}

bool mmid_small_supported(const MulMatIdArgs &a) {
    const bool typed = a.type == MX_TYPE_Q8_0 || a.type == MX_TYPE_Q4_K || a.type == MX_TYPE_Q5_K ||
                       a.type == MX_TYPE_Q6_K;
    return typed && a.n_ids * a.T <= MMID_SMALL_MAX_PAIRS && a.E <= MMID_SMALL_MAX_E && a.nprob >= 1 && a.nprob <= 4 &&
           act_lds_bytes(a.type, a.K, MMID_SMALL_COLS) <= MMID_SMALL_MAX_LDS;
}

template <int TYPE, int LPR>
static hipError_t launch_small_lpr(const MulMatIdArgs &a, hipStream_t s) {
    constexpr int G = 64 / LPR;
    const int64_t npairs = a.n_ids * a.T, slots = npairs < a.E ? npairs : a.E;
    // row blocks per workgroup: about MMID_SMALL_WGS workgroups over the slots and products, at most 8 blocks each
    const int64_t nblocks = (a.N + 4 * G - 1) / (4 * G), all = nblocks * slots * a.nprob;
    int64_t per = (all + MMID_SMALL_WGS - 1) / MMID_SMALL_WGS;
    per = per < 1 ? 1 : (per > 8 ? 8 : per);
    const dim3 grid((unsigned)((nblocks + per - 1) / per), (unsigned)slots, (unsigned)a.nprob);
    hipLaunchKernelGGL((k_mmid_small<TYPE, LPR>), grid, dim3(256), act_lds_bytes(TYPE, a.K, MMID_SMALL_COLS), s, a);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_small_type(const MulMatIdArgs &a, hipStream_t s) {
    // lanes per row: the fewest whose chunks per lane fit the held ones (else 64), or as forced
    switch (pick_lpr(a.K / chunk_elems<TYPE>(), small_pre<TYPE>(), a.lpr)) {
        case 16: return launch_small_lpr<TYPE, 16>(a, s);
        case 32: return launch_small_lpr<TYPE, 32>(a, s);
        default: return launch_small_lpr<TYPE, 64>(a, s);
    }
}

hipError_t launch_mmid_small(const MulMatIdArgs &a, hipStream_t s) {
    if (!mmid_small_supported(a)) return hipErrorInvalidValue;
    switch (a.type) {
        case MX_TYPE_Q8_0: return launch_small_type<MX_TYPE_Q8_0>(a, s);
        case MX_TYPE_Q4_K: return launch_small_type<MX_TYPE_Q4_K>(a, s);
        case MX_TYPE_Q5_K: return launch_small_type<MX_TYPE_Q5_K>(a, s);
        default: return launch_small_type<MX_TYPE_Q6_K>(a, s);
    }
}

template <int TYPE, int NC, int LPR>
static hipError_t launch_one(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    constexpr int G = 64 / LPR;
    dim3 grid((unsigned)((maxN + 4 * G - 1) / (4 * G)), (unsigned)a.nprob, (unsigned)a.nbatch);
    bool fused = a.glu_b || a.norm_w;
    for (int i = 0; i < a.nprob; i++) fused = fused || a.prob[i].res;
    if (fused) hipLaunchKernelGGL((k_matvec<TYPE, NC, LPR, true>), grid, dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_matvec<TYPE, NC, LPR, false>), grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int TYPE, int NC>
static hipError_t launch_nc(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    const int64_t nchunks = a.K / chunk_elems<TYPE>();
    switch (pick_lpr(nchunks, preload_of<TYPE>(), a.lpr)) {
        case 16: return launch_one<TYPE, NC, 16>(a, maxN, lds, s);
        case 32: return launch_one<TYPE, NC, 32>(a, maxN, lds, s);
        default: return launch_one<TYPE, NC, 64>(a, maxN, lds, s);
    }
}

template <int TYPE>
static hipError_t launch_type(const MatvecArgs &a, int64_t maxN, size_t lds, hipStream_t s) {
    switch (a.ncols) {
        case 1: return launch_nc<TYPE, 1>(a, maxN, lds, s);
        case 2: return launch_nc<TYPE, 2>(a, maxN, lds, s);
        case 3: return launch_nc<TYPE, 3>(a, maxN, lds, s);
        case 4: return launch_nc<TYPE, 4>(a, maxN, lds, s);
        case 5: return launch_nc<TYPE, 5>(a, maxN, lds, s);
        case 6: return launch_nc<TYPE, 6>(a, maxN, lds, s);
        case 7: return launch_nc<TYPE, 7>(a, maxN, lds, s);
        case 8: return launch_nc<TYPE, 8>(a, maxN, lds, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matvec(const MatvecArgs &a, hipStream_t s) {
    int64_t maxN = 0;
    for (int i = 0; i < a.nprob; i++) maxN = a.prob[i].N > maxN ? a.prob[i].N : maxN;
    if (maxN == 0) return hipSuccess;
    if (a.type == MX_TYPE_F16 || a.type == MX_TYPE_F32) return launch_matvec_f(a, s);
    const size_t lds = act_lds_bytes(a.type, a.K, a.ncols);
    switch (a.type) {
        case MX_TYPE_Q8_0: return launch_type<MX_TYPE_Q8_0>(a, maxN, lds, s);
        case MX_TYPE_Q4_K: return launch_type<MX_TYPE_Q4_K>(a, maxN, lds, s);
        case MX_TYPE_Q5_K: return launch_type<MX_TYPE_Q5_K>(a, maxN, lds, s);
        case MX_TYPE_Q6_K: return launch_type<MX_TYPE_Q6_K>(a, maxN, lds, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mx
