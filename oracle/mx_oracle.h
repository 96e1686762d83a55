/*
 * CPU oracle for the MUL_MAT / MUL_MAT_ID / GET_ROWS path (Q8_0, Q4_K, Q5_K, Q6_K, F16, F32 weights).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests, the smoke check and the CPU-baseline leg of the
 * benchmark may call it; the product (libmx) never links or calls it.
 *
 * It restates, in plain C, the arithmetic of ggml's CPU backend that speech.cpp routes these ops to. ggml itself is an
 * un-vendored submodule of the reference (`.gitmodules:1-4`, fork nyosegawa/ggml branch `speech.cpp` on upstream
 * v0.27.0 per `docs/adr/ggml-comes-from-a-fork-...-speed-ups.md:5-7`), absent from the reference tree, so each function
 * names the ggml source it restates (ggml/src/ggml-quants.c, ggml/src/ggml-cpu/quants.c, ggml/src/ggml-cpu/ggml-cpu.c,
 * ggml/src/ggml-common.h) and the reference call site that reaches it.
 *
 * Data is in ggml's own block layout (array-of-blocks, little endian), exactly as GGUF stores it.
 */
#ifndef MX_ORACLE_H
#define MX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type numbering (ggml.h enum ggml_type). */
enum {
    ORC_TYPE_F32 = 0,
    ORC_TYPE_F16 = 1,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q8_1 = 9,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q5_K = 13,
    ORC_TYPE_Q6_K = 14,
    ORC_TYPE_Q8_K = 15,
    ORC_TYPE_I32 = 26,
};

/* Rounding variant of the 32-block activation quantizers:
 * ORC_ROUND_REF: quantize_row_q8_{0,1}_ref  -- id = 1/(amax/127), roundf (half away from zero).
 * ORC_ROUND_X86: ggml-cpu x86 AVX2 quantize_row_q8_{0,1} -- id = 127/amax, round half to even. */
enum { ORC_ROUND_REF = 0, ORC_ROUND_X86 = 1 };

/* fp16 <-> fp32, IEEE binary16 round-to-nearest-even with subnormals (ggml_compute_fp32_to_fp16 semantics). */
uint16_t orc_fp32_to_fp16(float f);
float orc_fp16_to_fp32(uint16_t h);

/* Block geometry: elements per block and bytes per block (ggml-common.h). */
int64_t orc_blck_size(int type);
size_t orc_type_size(int type);
size_t orc_row_size(int type, int64_t ne);
/* The activation type the CPU backend pairs with a weight type (type_traits_cpu[].vec_dot_type). */
int orc_vec_dot_type(int type);

/* Quantizers. */
void orc_quantize_row_q8_0(const float *x, void *y, int64_t k, int rounding);
void orc_quantize_row_q8_1(const float *x, void *y, int64_t k, int rounding);
void orc_quantize_row_q8_K(const float *x, void *y, int64_t k);
void orc_quantize_row_q4_K(const float *x, void *y, int64_t k);
void orc_quantize_row_q5_K(const float *x, void *y, int64_t k);
void orc_quantize_row_q6_K(const float *x, void *y, int64_t k);
/* The two candidate searches of the K-quant weight quantizers on one sub-block, exposed for the tests that pin them:
 * make_qkx2_quants (Q4_K / Q5_K: returns the scale, *neg_min = -min) and make_qx_quants with rmse_type 1 (Q6_K:
 * returns the scale; L holds code + nmax). n <= 256. */
float orc_make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L, float *neg_min,
                           float rmin, float rdelta, int nstep, int use_mad);
float orc_make_qx_quants(int n, int nmax, const float *x, int8_t *L);
/* ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, imatrix = NULL); returns bytes written. */
size_t orc_quantize_chunk(int type, const float *src, void *dst, int64_t start, int64_t nrows, int64_t n_per_row);

/* Dequantizers (ggml type_traits[type].to_float). */
int orc_dequantize_row(int type, const void *x, float *y, int64_t k);

/* vec_dot of one weight row (type) with one activation row in orc_vec_dot_type(type); ggml generic C order. */
float orc_vec_dot(int type, int64_t n, const void *x, const void *y);
/* The same dot with every per-block integer sum exact and the cross-block sum taken in double. */
double orc_vec_dot_exact(int type, int64_t n, const void *x, const void *y);

/* A ggml-shaped tensor in host memory. */
typedef struct orc_tensor {
    int32_t type;
    int64_t ne[4];
    size_t nb[4];
    void *data;
} orc_tensor;

/* ggml_compute_forward_mul_mat: dst[i0,i1,i2,i3] = vec_dot(src0 row i0 of matrix (i2/r2, i3/r3), quant(src1 row)). */
int orc_mul_mat(const orc_tensor *src0, const orc_tensor *src1, orc_tensor *dst, int rounding, int exact);
/* ggml_compute_forward_mul_mat_id: dst[:, s, t] = as[ids[s,t]] . quant(b[:, s % ne11, t]). */
int orc_mul_mat_id(const orc_tensor *as, const orc_tensor *b, const orc_tensor *ids, orc_tensor *dst, int rounding,
                   int exact);
/* ggml_compute_forward_get_rows: dst[:, i10, i11, i12] = dequant(src0[:, ids[i10,i11,i12], i11, i12]). */
int orc_get_rows(const orc_tensor *src0, const orc_tensor *ids, orc_tensor *dst);

/* ggml_argmax as speech.cpp's ggml fork computes it: dst[i1] = the index of the largest of row i1's ne0 values, the
 * first of equal ones (fastconformer/decoder.cpp:56-62 first_argmax, the rule of the fork's argmax). A NaN never
 * compares greater, so a NaN at index 0 keeps index 0 and NaNs elsewhere are passed over. src0 F32 [ne0, ne1],
 * dst I32 [ne1]. */
int orc_argmax(const orc_tensor *src0, orc_tensor *dst);

/* The decoder layer's other ops (src/common/qwen3-decoder.cpp:350-410) on contiguous f32 rows, as ggml-cpu computes
 * them: RMS_NORM, ADD / MUL with src1 rows repeated (op 0 add, 1 mul), GLU SWIGLU (split form), ROPE in NEOX mode,
 * SET_ROWS into an f16 cache, FLASH_ATTN_EXT over f16 K / V with an f16 mask (exact = 0: ggml-cpu's arithmetic with
 * its fp16 V accumulator; exact = 1: the same attention in double). Shapes are given with each function. */
void orc_rms_norm(const float *x, float *y, int64_t ne0, int64_t nrows, float eps);
void orc_binary(int op, const float *a, const float *b, float *y, int64_t ne0, int64_t nrows, int64_t nb_rows);
void orc_swiglu(const float *a, const float *b, float *y, int64_t n);
void orc_rope_neox(const float *x, const int32_t *pos, float *y, int64_t ne0, int64_t n_head, int64_t nrows,
                   int n_dims, float freq_base, float freq_scale);
int orc_set_rows_f16(const float *src, const int32_t *idx, uint16_t *dst, int64_t ne0, int64_t nrows,
                     int64_t dst_rows);
int orc_flash_attn_ext(const float *q, const uint16_t *k, const uint16_t *v, const uint16_t *mask, float *dst, int D,
                       int64_t n_q, int64_t n_head, int64_t n_kv, int64_t n_kv_head, float scale, int exact);

/* Seeded synthetic data: splitmix64 -> xoshiro256** -> Box-Muller in double -> float. Row r of a tensor draws from
 * its own stream seeded by (seed, r), so rows can be generated in any order or in parallel. */
void orc_fill_normal_rows(uint64_t seed, int64_t row0, int64_t nrows, int64_t n_per_row, float mean, float stddev,
                          float *out);

#ifdef __cplusplus
}
#endif
#endif
