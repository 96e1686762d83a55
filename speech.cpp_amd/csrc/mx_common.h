// Internal declarations shared by libmx's host code and its HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/mx.h"

namespace mx {

constexpr int QK8 = 32;    // elements of a Q8_0 / Q8_1 block
constexpr int QKK = 256;   // elements of a K-quant super-block
constexpr size_t PLANE_ALIGN = 256;

// ------------------------------------------------------------------------------------------------------------------
// Device layout of a quantized tensor.
//
// ggml stores a tensor as an array of blocks (ggml-common.h): block_q8_0 {d, qs[32]} (34 B), block_q4_K {d, dmin,
// scales[12], qs[128]} (144 B), block_q5_K {d, dmin, scales[12], qh[32], qs[128]} (176 B), block_q6_K {ql[128],
// qh[64], scales[16], d} (210 B). On this device each field becomes a
// plane of its own: plane p holds that field of block 0, block 1, ... back to back, and each plane starts on a
// 256-byte boundary. Blocks are numbered in ggml order (row-major over all rows of all matrices), so a row's quants
// are contiguous and 16-byte aligned, which is what wide coalesced loads and MFMA tiles want.
//
//   Q8_0: plane 0 qs (32 B/block), plane 1 d (2 B/block)
//   Q4_K: plane 0 qs (128 B/block), plane 1 scales (12 B/block), plane 2 d,dmin (4 B/block)
//   Q5_K: plane 0 qs (128 B/block), plane 1 qh (32 B/block), plane 2 scales (12 B/block), plane 3 d,dmin (4 B/block)
//   Q6_K: plane 0 ql (128 B/block), plane 1 qh (64 B/block), plane 2 scales (16 B/block), plane 3 d (2 B/block)
//
// The map from a byte of ggml's block to (plane, byte in plane) is a permutation, so a partial upload of ggml bytes at
// any offset scatters into every plane without reading anything else.
// ------------------------------------------------------------------------------------------------------------------
struct Segment {
    uint16_t begin;  // first byte of the field in ggml's block
    uint16_t len;    // bytes of the field
    uint8_t plane;   // plane it goes to
};

struct TypeInfo {
    int type;
    int blk_elems;   // elements per block
    int blk_bytes;   // bytes per ggml block
    int nseg;
    Segment seg[4];  // ggml block fields in byte order
};

inline const TypeInfo *type_info(int type) {
    // Field order within ggml's structs: block_q8_0 {d, qs}; block_q4_K {d, dmin, scales, qs}; block_q5_K {d, dmin,
    // scales, qh, qs}; block_q6_K {ql, qh, scales, d}.
    static const TypeInfo q8_0 = {MX_TYPE_Q8_0, 32, 34, 2, {{0, 2, 1}, {2, 32, 0}, {0, 0, 0}, {0, 0, 0}}};
    static const TypeInfo q4_k = {MX_TYPE_Q4_K, 256, 144, 3, {{0, 4, 2}, {4, 12, 1}, {16, 128, 0}, {0, 0, 0}}};
    static const TypeInfo q5_k = {MX_TYPE_Q5_K, 256, 176, 4, {{0, 4, 3}, {4, 12, 2}, {16, 32, 1}, {48, 128, 0}}};
    static const TypeInfo q6_k = {MX_TYPE_Q6_K, 256, 210, 4, {{0, 128, 0}, {128, 64, 1}, {192, 16, 2}, {208, 2, 3}}};
    switch (type) {
        case MX_TYPE_Q8_0: return &q8_0;
        case MX_TYPE_Q4_K: return &q4_k;
        case MX_TYPE_Q5_K: return &q5_k;
        case MX_TYPE_Q6_K: return &q6_k;
        default: return nullptr;
    }
}

inline bool is_quantized(int type) {
    return type == MX_TYPE_Q8_0 || type == MX_TYPE_Q4_K || type == MX_TYPE_Q5_K || type == MX_TYPE_Q6_K;
}

struct Planes {
    int n = 0;
    uint64_t off[4] = {0, 0, 0, 0};      // byte offset of each plane from the tensor's base
    uint32_t per_blk[4] = {0, 0, 0, 0};  // bytes per block in each plane
    int64_t nblocks = 0;
    uint64_t total = 0;                   // allocation size
};

inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

inline Planes planes_of(int type, int64_t nelements) {
    Planes p;
    const TypeInfo *ti = type_info(type);
    if (!ti) return p;
    p.nblocks = nelements / ti->blk_elems;
    p.n = ti->nseg;
    for (int s = 0; s < ti->nseg; s++) p.per_blk[ti->seg[s].plane] = ti->seg[s].len;
    uint64_t off = 0;
    for (int i = 0; i < p.n; i++) {
        p.off[i] = off;
        off = align_up(off + (uint64_t)p.nblocks * p.per_blk[i], PLANE_ALIGN);
    }
    p.total = off;
    return p;
}

// The planes of a quantized weight, as kernels take them.
struct WPlanes {
    const uint8_t *p0, *p1, *p2, *p3;
};

inline WPlanes wplanes(const void *base, const Planes &pl) {
    const uint8_t *b = (const uint8_t *)base;
    return {b + pl.off[0], b + pl.off[1], pl.n > 2 ? b + pl.off[2] : nullptr, pl.n > 3 ? b + pl.off[3] : nullptr};
}

// ------------------------------------------------------------------------------------------------------------------
// Kernel choices of one backend (mx_backend_set_option). Zero everywhere is the dispatcher's own pick; a forced
// choice reaches one kernel so that every kernel the dispatcher can pick is testable in one process.
// ------------------------------------------------------------------------------------------------------------------
struct Options {
    int gemm_q8_0 = 0;              // Q8_0 at M > 8: 0 picked (int8 MFMA), 1 int8 MFMA, 2 fp16 dequantizing
    int gemm_kquant = 0;            // Q4_K / Q6_K at M > 8: 0 as picked, 1 the VALU-scaled int8 GEMM (k_gemm_kq)
    int tile_m = 0, tile_n = 0;     // GEMM tile (0: picked per product)
    int split = 0;                  // K splits of the prefill GEMMs that split K (0: picked)
    int matvec_lpr = 0;             // lanes per row of the mat-vec: 16, 32 or 64 (0: picked)
    int mmid_kernel = 0;            // MUL_MAT_ID with many pairs: 0 as picked, 1 the experts kernel, 2 the grouped
                                    // product (Q4_K: int8 MFMA; Q8_0, Q5_K, Q6_K: the fp16 GEMM over expert chunks)
    int64_t mmid_matvec_pairs = 16; // MUL_MAT_ID runs as one mat-vec launch up to this many (token, slot) pairs
    int mmid_chunk = 0;             // pairs per chunk of the grouped Q4_K product: 16 or 32 (0: picked)
};

// ------------------------------------------------------------------------------------------------------------------
// Kernel launchers (defined in the .hip files). All run on `s`. Return hipError_t of the launch.
// ------------------------------------------------------------------------------------------------------------------
// Scatter `n` ggml-layout bytes (from device staging `src`), which are bytes [offset, offset + n) of a tensor of
// `type`, into the planes at `base`; gather is the inverse.
// A tensor's byte permutation, passed to kernels by value.
struct SegMap {
    int blk_bytes;
    int nseg;
    Segment seg[4];
    uint64_t plane_off[4];
};
SegMap segmap_of(int type, const Planes &pl);
hipError_t launch_scatter(const SegMap &m, uint8_t *base, const uint8_t *src, uint64_t offset, uint64_t n,
                          hipStream_t s);
hipError_t launch_gather(const SegMap &m, const uint8_t *base, uint8_t *dst, uint64_t offset, uint64_t n,
                         hipStream_t s);
hipError_t launch_fill(const SegMap &m, uint8_t *base, uint8_t value, uint64_t offset, uint64_t n, hipStream_t s);

// Activation quantization to ggml blocks (Q8_0, Q8_1 or Q8_K) in global memory.
hipError_t launch_quantize_act(int type, int rounding, const float *x, int64_t k, int64_t nrows, int64_t x_stride,
                               void *out, hipStream_t s);

// GET_ROWS for one 2-D slice batch.
struct GetRowsArgs {
    int type;
    WPlanes w;
    int64_t K;            // elements per row
    int64_t R;            // rows per matrix of src0 (bound for ids)
    int64_t n_ids0, n_ids1, n_ids2;  // ids ne[0..2]
    int64_t src_mat_rows1, src_mat_rows2;  // row offset of matrix (i11, i12): i11 * rows1 + i12 * rows2
    const int32_t *ids;
    int64_t ids_nb0, ids_nb1, ids_nb2;     // strides in bytes
    float *dst;
    int64_t dst_nb1, dst_nb2, dst_nb3;     // bytes
    int *err;
};
hipError_t launch_get_rows(const GetRowsArgs &a, hipStream_t s);

// Mat-vec / small-M products: up to MAX_COLS columns of src1 per launch, all batch slices in grid.z.
constexpr int MAX_COLS = 8;
constexpr int64_t MAX_BATCH = 65535;  // batch slices of one mat-vec launch (grid.z)
struct MatvecProblem {
    WPlanes w;
    int64_t N;             // rows of the matrix (outputs)
    int64_t row0;          // first row of the matrix within the tensor's planes
    float *y;              // dst column 0 of this problem
    int64_t y_col_stride;  // floats between its dst columns
    const float *res;      // residual added to the product (same layout as y; may be y), or null
};
struct MatvecArgs {
    int type;
    int ncols;             // columns of src1 in this launch (1..MAX_COLS)
    int rounding;
    int64_t K;
    const float *x;        // src1 column 0 of batch slice (0, 0)
    int64_t x_col_stride;  // floats between columns
    // batch slices (grid.z = nbatch = ne12 * ne13 <= MAX_BATCH): matrix (i12 / r2, i13 / r3) of src0 meets slice
    // (i12, i13) of src1
    int nbatch, ne12, ne02, r2, r3;
    int64_t x_b2, x_b3, y_b2, y_b3;  // float strides of src1 / dst slices
    // problems sharing x (grid.y picks the problem)
    int nprob;
    MatvecProblem prob[4];
    // MUL_MAT_ID with few (token, slot) pairs: when ids is set, slice (i12, i13) is slot i12 of token i13, its matrix
    // is ids[i12, i13] (of n_mats), and it reads src1 slice (i12 % x_ne12, i13). Out-of-range ids set bit 2 of *err.
    const int32_t *ids;
    int64_t ids_nb0, ids_nb1;  // bytes
    int n_mats, x_ne12;
    int *err;
    // Fusions of the neighbouring decoder ops into the prologue (no ids mode): each src1 column becomes
    // silu(x) * glu_b (glu_b: same layout as x) and then mul(rms_norm(., norm_eps), norm_w) before it is quantized.
    const float *glu_b;
    const float *norm_w;
    float norm_eps;
    int lpr;               // lanes per row forced (16, 32, 64), or 0 to pick by K
};
hipError_t launch_matvec(const MatvecArgs &a, hipStream_t s);
// The same products on F16 / F32 weights in ggml's row-major layout (prob[i].w.p0 = the weight's data; K % 8 == 0 for
// F16, K % 4 == 0 for F32; no ids mode).
hipError_t launch_matvec_f(const MatvecArgs &a, hipStream_t s);

// Prefill GEMM on int8 MFMA (Q8_0, M > 8): launch_gemm_quant writes the activations as Q8_0 (int8 quants and fp32
// block scales) at the start of `scratch`, launch_gemm runs up to four weights sharing them in one launch (plus a
// reduce launch when K is split; the partial sums follow the activations in scratch). gemm_scratch_bytes is the
// scratch both need (for the tile and split `o` forces, or those picked). A forced tile the kernel lacks is refused
// (hipErrorInvalidValue).
size_t gemm_scratch_bytes(int nprob, const int64_t *N, int64_t M, int64_t K, const Options &o);
hipError_t launch_gemm_quant(int type, int rounding, const float *x, int64_t x_stride, int64_t M, int64_t K,
                             void *scratch, hipStream_t s);
hipError_t launch_gemm(int type, int nprob, const WPlanes *w, const int64_t *N, float *const *y, const int64_t *ldy,
                       int64_t M, int64_t K, void *scratch, const Options &o, hipStream_t s);
inline bool gemm_supported(int type, int64_t M, int64_t K) {
    return type == MX_TYPE_Q8_0 && K % 128 == 0 && M * K < ((int64_t)1 << 31);
}

// Prefill GEMM on the fp16 matrix cores over dequantized tiles (Q8_0 weights): launch_gemm_dq_act writes the
// activations' quantized values as fp16 at the start of `scratch`, launch_gemm_dq runs up to four weights sharing
// them in one launch (plus a reduce launch when K is split; the partial sums follow the activations in scratch).
// gemm_dq_scratch_bytes is the scratch both need (for the tile and split `o` forces, or those picked).
bool gemm_dq_supported(int type, int64_t M, int64_t K);
size_t gemm_dq_act_bytes(int64_t M, int64_t K);
size_t gemm_dq_scratch_bytes(int type, int nprob, const int64_t *N, int64_t M, int64_t K, const Options &o);
hipError_t launch_gemm_dq_act(int type, int rounding, const float *x, int64_t x_stride, int64_t M, int64_t K,
                              void *scratch, hipStream_t s);
hipError_t launch_gemm_dq(int type, int nprob, const WPlanes *w, const int64_t *N, float *const *y,
                          const int64_t *ldy, int64_t M, int64_t K, void *scratch, const Options &o, hipStream_t s);

// Prefill GEMM on Q4_K / Q6_K weights: launch_gemm_kq_quant writes x (M rows of K floats, row stride x_stride) as
// Q8_K into `scratch` (gemm_kq_act_bytes), launch_gemm_kq multiplies it into y (row stride ldy).
size_t gemm_kq_act_bytes(int64_t M, int64_t K);
hipError_t launch_gemm_kq_quant(const float *x, int64_t x_stride, int64_t M, int64_t K, void *scratch, hipStream_t s);
hipError_t launch_gemm_kq(int type, const WPlanes &w, int64_t M, int64_t N, int64_t K, const void *scratch, float *y,
                          int64_t ldy, hipStream_t s);
// Q4_K prefill GEMM with the sub-block scales folded into the MFMA operands: launch_gemm_q4k_quant writes x as Q8_K
// plus split sub-block sums into `scratch` (gemm_q4k_act_bytes); launch_gemm_q4k then runs up to four weights
// (w[i], N[i] rows, into y[i] with row stride ldy[i]) sharing those activations in one launch.
size_t gemm_q4k_act_bytes(int64_t M, int64_t K);
hipError_t launch_gemm_q4k_quant(const float *x, int64_t x_stride, int64_t M, int64_t K, void *scratch, hipStream_t s);
hipError_t launch_gemm_q4k(int nprob, const WPlanes *w, const int64_t *N, float *const *y, const int64_t *ldy,
                           int64_t M, int64_t K, const void *scratch, const Options &o, hipStream_t s);
inline bool gemm_kq_supported(int type, int64_t K) {
    return (type == MX_TYPE_Q4_K || type == MX_TYPE_Q6_K) && K % 256 == 0;
}

// MUL_MAT_ID.
struct MulMatIdArgs {
    int type;
    int rounding;
    WPlanes w;
    int64_t K, N, E;
    int64_t n_ids, T;
    const float *b;
    int64_t b_ne1;         // 1 (one row per token, broadcast to every slot) or n_ids
    int64_t b_nb1, b_nb2;  // bytes
    const int32_t *ids;
    int64_t ids_nb0, ids_nb1;  // bytes
    float *dst;
    int64_t dst_nb1, dst_nb2;  // bytes
    // scratch (mul_mat_id_scratch carves it)
    int32_t *counts;       // [E] pairs per expert
    int32_t *offsets;      // [E] first pair of each expert in `pairs`
    int32_t *active;       // [E + 1]: active[0] = number of experts with pairs, then their ids
    int32_t *pairs;        // [n_ids * T] flat pair index t * n_ids + s, grouped by expert
    int8_t *xq;            // [T * b_ne1][K] quantized activation rows
    float *xd;             // [T * b_ne1][K / blk] their scales
    int32_t *xbs;          // [T * b_ne1][K / 16] their 16-element sums (K-quants)
    _Float16 *x16;         // [T * b_ne1][K / 256][16] Q4_K: per super-block [64 h_j | l_j], bsum32_j = 64 h_j + l_j
    _Float16 *xh;          // the fp16 GEMM's routed form: [T * b_ne1][K] rows fp16(2^e d q) (sharing xq's space)
    float *rs;             // the fp16 GEMM's routed form: [T * b_ne1] their 2^-e
    int32_t *tiles;        // [max_tiles][3]: chunks of an expert's pairs: first (index into `pairs`), count, expert
    int32_t *ntiles;       // [1] tiles written by the bucket kernel
    int64_t max_tiles;
    int *err;
    int generic;               // 0 as picked, 1: the experts kernel, 2: the grouped MFMA product (Q4_K)
    int chunk;                 // pairs per chunk of an expert's pairs: MMID_CHUNK_SMALL or MMID_CHUNK
    // products sharing b and ids (1..4): product p reads expert weights wg[p] into dstg[p] (dst's strides); the
    // kernels that take one product at a time read w / dst, which the launcher points at each in turn
    int nprob;
    WPlanes wg[4];
    float *dstg[4];
    int64_t matvec_pairs;      // up to this many pairs: one mat-vec launch, no bucketing
    int lpr;                   // mat-vec lanes per row forced, or 0
    int tile_m, tile_n;        // the fp16 GEMM's routed tile forced, or 0
};
// Row-wise ops on f32 rows (layer.hip): src / dst rows (i1, i2, i3) at byte strides, ne0 contiguous floats.
struct RowsArgs {
    const void *src;
    void *dst;
    int64_t ne0, ne1, ne2, nrows;         // nrows = ne1 * ne2 * ne3
    int64_t s_nb1, s_nb2, s_nb3, d_nb1, d_nb2, d_nb3;
};
hipError_t launch_rms_norm(const RowsArgs &a, float eps, const float *w, hipStream_t s);
hipError_t launch_swiglu(const RowsArgs &a, const float *b, int64_t b_nb1, hipStream_t s);
// x [ne0, ne1 heads, ne2 rows] (s_nb1: head stride, s_nb2: row stride) rotated pairwise, NEOX layout.
hipError_t launch_rope_neox(const RowsArgs &a, const int32_t *pos, int n_dims, float theta_scale, float freq_scale,
                            hipStream_t s);
// f32 rows into f16 rows idx[r] of dst (d_nb1 bytes apart, dst_rows rows); a bad index sets *err |= 4.
hipError_t launch_set_rows_f16(const RowsArgs &a, const void *idx, bool idx_i64, int64_t dst_rows, int *err,
                               hipStream_t s);
// dst = a op b (op 0 add, 1 mul), b repeated over a's shape; byte strides, ne0 contiguous.
struct BinaryArgs {
    int op;
    const float *a, *b;
    float *dst;
    int64_t ne[4], a_nb[4], b_ne[4], b_nb[4], d_nb[4];
};
hipError_t launch_binary(const BinaryArgs &a, hipStream_t s);
// Flash attention over f16 K / V: q rows (i, h) at q + i q_nb1 + h q_nb2 (f32), K / V position j of kv head hk at
// k + j k_nb1 + hk k_nb2 (f16), mask row i at mask + i m_nb1 (f16, may be null); dst [D, n_head, n_q] contiguous.
// nsplit > 1 needs part: n_q * n_head * nsplit * (D + 2) floats.
struct FaArgs {
    const float *q;
    const void *k, *v, *mask;
    float *dst, *part;
    int D, nsplit;
    int64_t n_q, n_head, n_kv, gqa, split_len;
    int64_t q_nb1, q_nb2, k_nb1, k_nb2, v_nb1, v_nb2, m_nb1;
    float scale;
};
int fa_splits(int64_t n_q, int64_t n_head, int64_t n_kv, int64_t gqa, int D);
// q / k norm + NEOX RoPE + KV-cache stores for head size 128 (k_qkv_post): q, k, v heads h of row r at
// base + h nb1 + r nb2 (F32); q_out likewise; the caches' row p at kc / vc + p kc_nb1 / vc_nb1 (F16, head h at
// channel 128 h); pos[r] outside [0, cache_rows) sets *err |= 4 and stores nothing for that row.
struct QkvPostArgs {
    const float *q, *k, *v, *qw, *kw;
    const int32_t *pos;
    float *q_out;
    void *kc, *vc;
    int64_t nq, nkv, cache_rows;
    int64_t q_nb1, q_nb2, k_nb1, k_nb2, v_nb1, v_nb2, qo_nb1, qo_nb2, kc_nb1, vc_nb1;
    float eps, theta_scale, freq_scale;
    int *err;
};
hipError_t launch_qkv_post(const QkvPostArgs &a, int64_t rows, hipStream_t s);
hipError_t launch_flash_attn(const FaArgs &a, hipStream_t s);
// One decode row: launch_qkv_post and launch_flash_attn in one attention launch (head size 128, gqa 1, 2 or 4; the
// attention reads the caches pa stores into).
hipError_t launch_attn_decode(const FaArgs &a, const QkvPostArgs &pa, hipStream_t s);

// ARGMAX (first of equal values) over nrows rows of ne0 floats (row stride nb1 bytes) into dst (stride dst_nb0 bytes).
// Rows of more than 8192 floats split into argmax_parts(ne0, nrows) parts, whose (value, index) pairs go to scratch
// (nrows * parts float2).
int argmax_parts(int64_t ne0, int64_t nrows);
// Peak micro-benchmarks (peak.hip): a streaming read of `bytes` (a multiple of 16, 16-byte aligned) by `workgroups`
// of 256 threads with `loads` (1, 2, 4, 8, 16) 16-byte loads in flight per thread; `iters` rounds of eight independent
// MFMAs per wave (kind 0: v_mfma_i32_32x32x32_i8, 1: v_mfma_f32_32x32x16_f16). sink: workgroups ints, never written
// in practice.
hipError_t launch_peak_read(const void *src, int64_t bytes, int workgroups, int loads, bool nontemporal, int *sink,
                            hipStream_t s);
hipError_t launch_peak_mfma(int kind, int workgroups, int iters, int *sink, hipStream_t s);
hipError_t launch_argmax(const float *src, int64_t ne0, int64_t nrows, int64_t nb1, int32_t *dst, int64_t dst_nb0,
                         void *scratch, hipStream_t s);

// Pairs per chunk of one expert's (token, slot) pairs: two 16-row MFMA tiles that share each expanded weight fragment,
// or one tile (few pairs per expert: no second tile's operands to stage, and a lighter kernel form).
constexpr int MMID_CHUNK = 32, MMID_CHUNK_SMALL = 16;
// The chunk size a MUL_MAT_ID of npairs pairs over E experts takes (forced: a backend's option, 16 or 32; else 0).
int mmid_chunk_for(int64_t npairs, int64_t E, int forced);
// Scratch bytes MUL_MAT_ID needs and the carving of `base` into the fields above.
size_t mul_mat_id_scratch(MulMatIdArgs *a, void *base);
hipError_t launch_mul_mat_id(const MulMatIdArgs &a, hipStream_t s);
// Q4_K experts as a grouped product over chunks of up to a.chunk of an expert's pairs (16 x 16 x 64 int8 MFMA).
bool mmid_q4k_supported(const MulMatIdArgs &a);  // Q4_K, K <= 2048
hipError_t launch_mmid_q4k(const MulMatIdArgs &a, hipStream_t s);
// Q8_0 / Q5_K / Q6_K experts on the fp16 dequantizing GEMM (gemm_dq.hip): each chunk of up to mmid_dq_chunk(type) of
// an expert's pairs is one row tile (Q8_0: 32 x 128 tiles; Q5_K, Q6_K: 64 x 64), its rows the prep's (xh, rs) rows of
// the pairs, gathered, its outputs scattered to dst; the chunks past a.ntiles[0] of the a.max_tiles slots leave at
// once. mmid_dq_route is the dispatch rule that sends a MUL_MAT_ID there.
int mmid_dq_chunk(const MulMatIdArgs &a);
bool mmid_dq_route(const MulMatIdArgs &a);
hipError_t launch_gemm_dq_routed(const MulMatIdArgs &a, hipStream_t s);

}  // namespace mx
