/*
 * CPU oracle: a plain-C restatement of ggml's CPU arithmetic for Q8_0 / Q4_K / Q5_K / Q6_K / F16 / F32 MUL_MAT,
 * MUL_MAT_ID and GET_ROWS.
 *
 * TEST INFRASTRUCTURE ONLY -- the checker, never the thing measured or shipped.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no -march: the x86-64 baseline that ggml-base is compiled for,
 * which has no FMA, so no product is fused into a sum).
 *
 * The reference reaches this arithmetic through ggml (an empty submodule in the reference tree, `.gitmodules:1-4`):
 *   weights:      src/common/quantize.cpp:164-182  ggml_quantize_chunk(type, ..., imatrix = nullptr)
 *   decode/prefill: src/common/qwen3-decoder.cpp:362-364,403,406-407,410,426  ggml_mul_mat
 *   MoE:          src/families/drama3/text-model.cpp:198-221  ggml_mul_mat_id (via src/common/graph.h:21-26)
 *   embeddings:   src/common/qwen3-decoder.cpp:464,483,499  ggml_get_rows
 * Each function below names the ggml function it restates.
 */
#include "mx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define QK8_0 32
#define QK8_1 32
#define QK_K 256
#define K_SCALE_SIZE 12
#define GROUP_MAX_EPS 1e-15f

/* ggml-common.h block structs (sizes 34, 36, 292, 144, 176, 210 bytes; the reference confirms 34/144/210 in
 * checks/compare/quantize_compare.py:27). */
typedef struct { uint16_t d; int8_t qs[QK8_0]; } blk_q8_0;
typedef struct { uint16_t d; uint16_t s; int8_t qs[QK8_1]; } blk_q8_1;
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; } blk_q8_K;
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[K_SCALE_SIZE]; uint8_t qs[QK_K / 2]; } blk_q4_K;
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[K_SCALE_SIZE];
    uint8_t qh[QK_K / 8];
    uint8_t qs[QK_K / 2];
} blk_q5_K;
typedef struct { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; } blk_q6_K;

_Static_assert(sizeof(blk_q8_0) == 34, "q8_0 block");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1 block");
_Static_assert(sizeof(blk_q8_K) == 292, "q8_K block");
_Static_assert(sizeof(blk_q4_K) == 144, "q4_K block");
_Static_assert(sizeof(blk_q5_K) == 176, "q5_K block");
_Static_assert(sizeof(blk_q6_K) == 210, "q6_K block");

/* ------------------------------------------------------------------------------------------------------------------
 * fp16. IEEE binary16, round to nearest even, subnormals kept; NaN becomes the quiet NaN 0x7E00 with the sign kept
 * (the result ggml_compute_fp32_to_fp16 gives, ggml-impl.h). Written from the IEEE 754 definition.
 * ---------------------------------------------------------------------------------------------------------------- */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e32 = (x >> 23) & 0xFFu;
    const uint32_t m32 = x & 0x7FFFFFu;
    if (e32 == 0xFFu) return (uint16_t)(sign | (m32 ? 0x7E00u : 0x7C00u));
    if (e32 == 0) return (uint16_t)sign; /* fp32 subnormals are far below half of the least fp16 subnormal */
    const uint32_t sig = m32 | 0x800000u;       /* 24-bit significand, value = sig * 2^(e32-150) */
    int e16 = (int)e32 - 127 + 15;              /* biased binary16 exponent if the result is normal */
    int shift = 13;                             /* bits dropped going from 24 to 11 significant bits */
    if (e16 < 1) shift += 1 - e16;              /* subnormal result: drop more bits */
    if (shift > 25) return (uint16_t)sign;      /* below half of the least subnormal: rounds to zero */
    uint32_t q = sig >> shift;
    const uint32_t rem = sig & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    if (e16 < 1) return (uint16_t)(sign | q);   /* q may reach 0x400, the least normal, which encodes itself */
    if (q == 0x800u) { q >>= 1; e16++; }        /* rounding carried into the next binade */
    if (e16 >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | (q & 0x3FFu));
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t x;
    if (e == 0x1Fu) {
        x = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: value = m * 2^-24, exact in fp32 */
            float v = (float)m * 0x1p-24f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

#define FP16_TO_FP32(h) orc_fp16_to_fp32(h)
#define FP32_TO_FP16(f) orc_fp32_to_fp16(f)

int64_t orc_blck_size(int type) {
    switch (type) {
        case ORC_TYPE_F32: case ORC_TYPE_F16: case ORC_TYPE_I32: return 1;
        case ORC_TYPE_Q8_0: return QK8_0;
        case ORC_TYPE_Q8_1: return QK8_1;
        case ORC_TYPE_Q4_K: case ORC_TYPE_Q5_K: case ORC_TYPE_Q6_K: case ORC_TYPE_Q8_K: return QK_K;
        default: return 0;
    }
}

size_t orc_type_size(int type) {
    switch (type) {
        case ORC_TYPE_F32: case ORC_TYPE_I32: return 4;
        case ORC_TYPE_F16: return 2;
        case ORC_TYPE_Q8_0: return sizeof(blk_q8_0);
        case ORC_TYPE_Q8_1: return sizeof(blk_q8_1);
        case ORC_TYPE_Q4_K: return sizeof(blk_q4_K);
        case ORC_TYPE_Q5_K: return sizeof(blk_q5_K);
        case ORC_TYPE_Q6_K: return sizeof(blk_q6_K);
        case ORC_TYPE_Q8_K: return sizeof(blk_q8_K);
        default: return 0;
    }
}

size_t orc_row_size(int type, int64_t ne) {
    const int64_t b = orc_blck_size(type);
    return b ? (size_t)(ne / b) * orc_type_size(type) : 0;
}

/* ggml-cpu.c type_traits_cpu[...].vec_dot_type */
int orc_vec_dot_type(int type) {
    switch (type) {
        case ORC_TYPE_Q8_0: return ORC_TYPE_Q8_0;
        case ORC_TYPE_Q4_K: case ORC_TYPE_Q5_K: case ORC_TYPE_Q6_K: return ORC_TYPE_Q8_K;
        case ORC_TYPE_F16: return ORC_TYPE_F16;
        case ORC_TYPE_F32: return ORC_TYPE_F32;
        default: return -1;
    }
}

/* ggml-quants.c nearest_int: round to nearest, ties to even, for |v| <= 2^22 (the magic-constant float add). */
static inline int nearest_int(float v) { return (int)rintf(v); }

/* ------------------------------------------------------------------------------------------------------------------
 * 32-block activation quantizers.
 * REF: ggml-quants.c quantize_row_q8_0_ref / quantize_row_q8_1_ref.
 * X86: ggml-cpu/arch/x86/quants.c quantize_row_q8_0 / quantize_row_q8_1 (AVX2 branch): id = 127/amax, _MM_ROUND_NEAREST.
 * ---------------------------------------------------------------------------------------------------------------- */
static void quant32(const float *x, int8_t *qs, float *d_out, int *sum_out, int rounding) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    float id;
    if (rounding == ORC_ROUND_X86) id = amax != 0.0f ? 127.0f / amax : 0.0f;
    else id = d != 0.0f ? 1.0f / d : 0.0f;
    int sum = 0;
    for (int j = 0; j < 32; j++) {
        const float v = x[j] * id;
        const int q = rounding == ORC_ROUND_X86 ? (int)rintf(v) : (int)roundf(v);
        qs[j] = (int8_t)q;
        sum += q;
    }
    *d_out = d;
    *sum_out = sum;
}

void orc_quantize_row_q8_0(const float *x, void *vy, int64_t k, int rounding) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    for (int64_t i = 0; i < k / QK8_0; i++) {
        float d;
        int sum;
        quant32(x + i * QK8_0, y[i].qs, &d, &sum, rounding);
        y[i].d = FP32_TO_FP16(d);
    }
}

void orc_quantize_row_q8_1(const float *x, void *vy, int64_t k, int rounding) {
    blk_q8_1 *y = (blk_q8_1 *)vy;
    for (int64_t i = 0; i < k / QK8_1; i++) {
        float d;
        int sum;
        quant32(x + i * QK8_1, y[i].qs, &d, &sum, rounding);
        y[i].d = FP32_TO_FP16(d);
        y[i].s = FP32_TO_FP16((float)sum * d);
    }
}

/* ggml-quants.c quantize_row_q8_K_ref (the x86 CPU backend has no SIMD variant and calls it). ggml leaves bsums
 * unwritten for an all-zero block; this writes zeros there (every product that reads them is scaled by d = 0). */
void orc_quantize_row_q8_K(const float *x, void *vy, int64_t k) {
    blk_q8_K *y = (blk_q8_K *)vy;
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float *xb = x + i * QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < QK_K; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; max = xb[j]; }
        }
        if (amax == 0.0f) {
            y[i].d = 0.0f;
            memset(y[i].qs, 0, QK_K);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < QK_K; j++) {
            const int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int sum = 0;
            for (int l = 0; l < 16; l++) sum += y[i].qs[j * 16 + l];
            y[i].bsums[j] = (int16_t)sum;
        }
        y[i].d = 1.0f / iscale;
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * K-quant weight quantizers (imatrix = NULL), the fixture path of `speech quantize` (src/common/quantize.cpp:164-182).
 * ---------------------------------------------------------------------------------------------------------------- */

/* ggml-quants.c make_qkx2_quants: asymmetric n-value quantization with a search over 1 + nstep scale candidates. */
static float make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L, float *the_min,
                              uint8_t *Laux, float rmin, float rdelta, int nstep, int use_mad) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.0f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t)l;
        float diff = scale * L[i] + min - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        best_error += weights[i] * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = use_mad ? fabsf(diff) : diff * diff;
                mad += weights[i] * diff;
            }
            if (mad < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* ggml-quants.c get_scale_min_k4: the 6-bit scale and min of sub-block j from the 12 packed bytes. */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

/* ggml-quants.c quantize_row_q4_K_ref */
void orc_quantize_row_q4_K(const float *x, void *vy, int64_t k) {
    blk_q4_K *y = (blk_q4_K *)vy;
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    for (int64_t i = 0; i < k / QK_K; i++) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20, 0);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
            ls = ls < 63 ? ls : 63;
            lm = lm < 63 ? lm : 63;
            if (j < 4) {
                y[i].scales[j] = ls;
                y[i].scales[j + 4] = lm;
            } else {
                y[i].scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                y[i].scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                y[i].scales[j - 0] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        y[i].d = FP32_TO_FP16(max_scale / 63.f);
        y[i].dmin = FP32_TO_FP16(max_min / 63.f);
        uint8_t sc, m;
        for (int j = 0; j < QK_K / 32; ++j) {
            get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = FP16_TO_FP32(y[i].d) * sc;
            if (!d) continue;
            const float dm = FP16_TO_FP32(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((x[32 * j + ii] + dm) / d);
                l = l < 0 ? 0 : (l > 15 ? 15 : l);
                L[32 * j + ii] = (uint8_t)l;
            }
        }
        uint8_t *q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
        x += QK_K;
    }
}

/* ggml-quants.c quantize_row_q5_K_ref: the Q4_K search with 5-bit codes (nmax 31, rmin -0.5, 15 steps); code bit 4
 * of element l of sub-block j goes to bit j of qh[l]. */
void orc_quantize_row_q5_K(const float *x, void *vy, int64_t k) {
    blk_q5_K *y = (blk_q5_K *)vy;
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    for (int64_t i = 0; i < k / QK_K; i++) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 31, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15, 0);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
            ls = ls < 63 ? ls : 63;
            lm = lm < 63 ? lm : 63;
            if (j < 4) {
                y[i].scales[j] = ls;
                y[i].scales[j + 4] = lm;
            } else {
                y[i].scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                y[i].scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                y[i].scales[j - 0] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        y[i].d = FP32_TO_FP16(max_scale / 63.f);
        y[i].dmin = FP32_TO_FP16(max_min / 63.f);
        uint8_t sc, m;
        for (int j = 0; j < QK_K / 32; ++j) {
            get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = FP16_TO_FP32(y[i].d) * sc;
            if (!d) continue;
            const float dm = FP16_TO_FP32(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((x[32 * j + ii] + dm) / d);
                l = l < 0 ? 0 : (l > 31 ? 31 : l);
                L[32 * j + ii] = (uint8_t)l;
            }
        }
        uint8_t *qh = y[i].qh;
        uint8_t *ql = y[i].qs;
        memset(qh, 0, QK_K / 8);
        uint8_t m1 = 1, m2 = 2;
        for (int n = 0; n < QK_K; n += 64) {
            for (int j = 0; j < 32; ++j) {
                int l1 = L[n + j];
                if (l1 > 15) {
                    l1 -= 16;
                    qh[j] |= m1;
                }
                int l2 = L[n + j + 32];
                if (l2 > 15) {
                    l2 -= 16;
                    qh[j] |= m2;
                }
                ql[j] = (uint8_t)(l1 | (l2 << 4));
            }
            m1 <<= 2;
            m2 <<= 2;
            ql += 32;
        }
        x += QK_K;
    }
}

/* ggml-quants.c make_qx_quants with rmse_type = 1 and no importance weights (the only form quantize_row_q6_K_ref uses). */
static float make_qx_quants_rmse1(int n, int nmax, const float *x, int8_t *L) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t)(nmax + (l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

float orc_make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L, float *neg_min,
                           float rmin, float rdelta, int nstep, int use_mad) {
    uint8_t Laux[256];
    if (n < 1 || n > 256) return NAN;
    return make_qkx2_quants(n, nmax, x, weights, L, neg_min, Laux, rmin, rdelta, nstep, use_mad);
}

float orc_make_qx_quants(int n, int nmax, const float *x, int8_t *L) {
    if (n < 1 || n > 256) return NAN;
    return make_qx_quants_rmse1(n, nmax, x, L);
}

/* ggml-quants.c quantize_row_q6_K_ref */
void orc_quantize_row_q6_K(const float *x, void *vy, int64_t k) {
    blk_q6_K *y = (blk_q6_K *)vy;
    int8_t L[QK_K];
    float scales[QK_K / 16];
    for (int64_t i = 0; i < k / QK_K; i++) {
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            const float scale = make_qx_quants_rmse1(16, 32, x + 16 * ib, L + 16 * ib);
            scales[ib] = scale;
            const float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) {
                max_abs_scale = abs_scale;
                max_scale = scale;
            }
        }
        if (max_abs_scale < GROUP_MAX_EPS) {
            memset(&y[i], 0, sizeof(blk_q6_K));
            y[i].d = FP32_TO_FP16(0.f);
            x += QK_K;
            continue;
        }
        const float iscale = -128.f / max_scale;
        y[i].d = FP32_TO_FP16(1 / iscale);
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            const int v = nearest_int(iscale * scales[ib]);
            y[i].scales[ib] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            const float d = FP16_TO_FP32(y[i].d) * y[i].scales[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(x[16 * j + ii] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        uint8_t *ql = y[i].ql;
        uint8_t *qh = y[i].qh;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l + 0] & 0xF;
                const uint8_t q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF;
                const uint8_t q4 = L[j + l + 96] & 0xF;
                ql[l + 0] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                                  ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
        x += QK_K;
    }
}

/* ggml-quants.c ggml_quantize_chunk with imatrix = NULL: quantize_q8_0 / quantize_q4_K / quantize_q5_K /
 * quantize_q6_K, each of which quantizes the rows with the _ref quantizer; F16 rows are converted with
 * ggml_fp32_to_fp16_row and F32 rows copied. */
size_t orc_quantize_chunk(int type, const float *src, void *dst, int64_t start, int64_t nrows, int64_t n_per_row) {
    const int64_t b = orc_blck_size(type);
    if (b == 0 || n_per_row % b != 0 || start % n_per_row != 0) return 0;
    const size_t row_size = orc_row_size(type, n_per_row);
    uint8_t *out = (uint8_t *)dst + (size_t)(start / n_per_row) * row_size;
    const float *in = src + start;
    const int64_t n = nrows * n_per_row;
    switch (type) {
        case ORC_TYPE_Q8_0: orc_quantize_row_q8_0(in, out, n, ORC_ROUND_REF); break;
        case ORC_TYPE_Q4_K: orc_quantize_row_q4_K(in, out, n); break;
        case ORC_TYPE_Q5_K: orc_quantize_row_q5_K(in, out, n); break;
        case ORC_TYPE_Q6_K: orc_quantize_row_q6_K(in, out, n); break;
        case ORC_TYPE_F16:
            for (int64_t j = 0; j < n; j++) ((uint16_t *)out)[j] = FP32_TO_FP16(in[j]);
            break;
        case ORC_TYPE_F32: memcpy(out, in, (size_t)n * 4); break;
        default: return 0;
    }
    return (size_t)nrows * row_size;
}

/* ------------------------------------------------------------------------------------------------------------------
 * Dequantizers: ggml-quants.c dequantize_row_q8_0 / dequantize_row_q4_K / dequantize_row_q5_K /
 * dequantize_row_q6_K / dequantize_row_q8_K (fp32 d times each quant); ggml_fp16_to_fp32_row for F16.
 * ---------------------------------------------------------------------------------------------------------------- */
int orc_dequantize_row(int type, const void *vx, float *y, int64_t k) {
    switch (type) {
        case ORC_TYPE_Q8_0: {
            const blk_q8_0 *x = (const blk_q8_0 *)vx;
            for (int64_t i = 0; i < k / QK8_0; i++) {
                const float d = FP16_TO_FP32(x[i].d);
                for (int j = 0; j < QK8_0; ++j) y[i * QK8_0 + j] = x[i].qs[j] * d;
            }
            return 0;
        }
        case ORC_TYPE_Q4_K: {
            const blk_q4_K *x = (const blk_q4_K *)vx;
            for (int64_t i = 0; i < k / QK_K; i++) {
                const uint8_t *q = x[i].qs;
                const float d = FP16_TO_FP32(x[i].d);
                const float min = FP16_TO_FP32(x[i].dmin);
                int is = 0;
                uint8_t sc, m;
                for (int j = 0; j < QK_K; j += 64) {
                    get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
                    const float d1 = d * sc, m1 = min * m;
                    get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
                    const float d2 = d * sc, m2 = min * m;
                    for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
                    for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
                    q += 32;
                    is += 2;
                }
            }
            return 0;
        }
        case ORC_TYPE_Q5_K: {
            const blk_q5_K *x = (const blk_q5_K *)vx;
            for (int64_t i = 0; i < k / QK_K; i++) {
                const uint8_t *ql = x[i].qs;
                const uint8_t *qh = x[i].qh;
                const float d = FP16_TO_FP32(x[i].d);
                const float min = FP16_TO_FP32(x[i].dmin);
                int is = 0;
                uint8_t sc, m;
                uint8_t u1 = 1, u2 = 2;
                for (int j = 0; j < QK_K; j += 64) {
                    get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
                    const float d1 = d * sc, m1 = min * m;
                    get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
                    const float d2 = d * sc, m2 = min * m;
                    for (int l = 0; l < 32; ++l) *y++ = d1 * ((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)) - m1;
                    for (int l = 0; l < 32; ++l) *y++ = d2 * ((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)) - m2;
                    ql += 32;
                    is += 2;
                    u1 <<= 2;
                    u2 <<= 2;
                }
            }
            return 0;
        }
        case ORC_TYPE_Q6_K: {
            const blk_q6_K *x = (const blk_q6_K *)vx;
            for (int64_t i = 0; i < k / QK_K; i++) {
                const float d = FP16_TO_FP32(x[i].d);
                const uint8_t *ql = x[i].ql;
                const uint8_t *qh = x[i].qh;
                const int8_t *sc = x[i].scales;
                for (int n = 0; n < QK_K; n += 128) {
                    for (int l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l + 0] = d * sc[is + 0] * q1;
                        y[l + 32] = d * sc[is + 2] * q2;
                        y[l + 64] = d * sc[is + 4] * q3;
                        y[l + 96] = d * sc[is + 6] * q4;
                    }
                    y += 128;
                    ql += 64;
                    qh += 32;
                    sc += 8;
                }
            }
            return 0;
        }
        case ORC_TYPE_Q8_K: {
            const blk_q8_K *x = (const blk_q8_K *)vx;
            for (int64_t i = 0; i < k / QK_K; i++)
                for (int j = 0; j < QK_K; ++j) y[i * QK_K + j] = x[i].d * x[i].qs[j];
            return 0;
        }
        case ORC_TYPE_F16:
            for (int64_t i = 0; i < k; i++) y[i] = FP16_TO_FP32(((const uint16_t *)vx)[i]);
            return 0;
        case ORC_TYPE_F32:
            memcpy(y, vx, (size_t)k * 4);
            return 0;
        default: return -1;
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * Dot products (ggml-cpu/quants.c generic C: ggml_vec_dot_q8_0_q8_0_generic, ggml_vec_dot_q4_K_q8_K_generic,
 * ggml_vec_dot_q5_K_q8_K_generic, ggml_vec_dot_q6_K_q8_K_generic; ggml-cpu/vec.c ggml_vec_dot_f16 / ggml_vec_dot_f32
 * without SIMD: fp32 products summed in double). The x86 SIMD variants sum the same exact per-block integers (or the
 * same fp32 products) in another order.
 * ---------------------------------------------------------------------------------------------------------------- */

/* Q4_K: the 8 six-bit scales and mins of a super-block, unpacked (the utmp / kmask shuffle of the generic dot). */
static void q4k_scales_mins(const uint8_t *s, uint8_t *scales, uint8_t *mins) {
    for (int j = 0; j < 8; j++) get_scale_min_k4(j, s, &scales[j], &mins[j]);
}

float orc_vec_dot(int type, int64_t n, const void *vx, const void *vy) {
    if (type == ORC_TYPE_Q8_0) {
        const blk_q8_0 *x = (const blk_q8_0 *)vx;
        const blk_q8_0 *y = (const blk_q8_0 *)vy;
        float sumf = 0;
        for (int64_t ib = 0; ib < n / QK8_0; ++ib) {
            int sumi = 0;
            for (int j = 0; j < QK8_0; j++) sumi += x[ib].qs[j] * y[ib].qs[j];
            sumf += sumi * (FP16_TO_FP32(x[ib].d) * FP16_TO_FP32(y[ib].d));
        }
        return sumf;
    }
    if (type == ORC_TYPE_Q4_K) {
        const blk_q4_K *x = (const blk_q4_K *)vx;
        const blk_q8_K *y = (const blk_q8_K *)vy;
        int8_t aux8[QK_K];
        int16_t aux16[8];
        float sums[8];
        int32_t aux32[8];
        memset(sums, 0, sizeof(sums));
        float sumf = 0;
        for (int64_t i = 0; i < n / QK_K; ++i) {
            const uint8_t *q4 = x[i].qs;
            const int8_t *q8 = y[i].qs;
            memset(aux32, 0, sizeof(aux32));
            int8_t *a = aux8;
            for (int j = 0; j < QK_K / 64; ++j) {
                for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] & 0xF);
                a += 32;
                for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] >> 4);
                a += 32;
                q4 += 32;
            }
            uint8_t scales[8], mins[8];
            q4k_scales_mins(x[i].scales, scales, mins);
            int sumi = 0;
            for (int j = 0; j < QK_K / 16; ++j) sumi += y[i].bsums[j] * mins[j / 2];
            a = aux8;
            for (int j = 0; j < QK_K / 32; ++j) {
                const int32_t scale = scales[j];
                for (int r = 0; r < 4; r++) {
                    for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                    for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
                    q8 += 8;
                    a += 8;
                }
            }
            const float d = FP16_TO_FP32(x[i].d) * y[i].d;
            for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
            const float dmin = FP16_TO_FP32(x[i].dmin) * y[i].d;
            sumf -= dmin * sumi;
        }
        for (int l = 0; l < 8; ++l) sumf += sums[l];
        return sumf;
    }
    if (type == ORC_TYPE_Q5_K) {
        const blk_q5_K *x = (const blk_q5_K *)vx;
        const blk_q8_K *y = (const blk_q8_K *)vy;
        int8_t aux8[QK_K];
        int16_t aux16[8];
        float sums[8];
        int32_t aux32[8];
        memset(sums, 0, sizeof(sums));
        float sumf = 0;
        for (int64_t i = 0; i < n / QK_K; ++i) {
            const uint8_t *q4 = x[i].qs;
            const uint8_t *hm = x[i].qh;
            const int8_t *q8 = y[i].qs;
            memset(aux32, 0, sizeof(aux32));
            int8_t *a = aux8;
            uint8_t m = 1;
            for (int j = 0; j < QK_K / 64; ++j) {
                for (int l = 0; l < 32; ++l) a[l] = (int8_t)((q4[l] & 0xF) + (hm[l] & m ? 16 : 0));
                a += 32;
                m <<= 1;
                for (int l = 0; l < 32; ++l) a[l] = (int8_t)((q4[l] >> 4) + (hm[l] & m ? 16 : 0));
                a += 32;
                m <<= 1;
                q4 += 32;
            }
            uint8_t scales[8], mins[8];
            q4k_scales_mins(x[i].scales, scales, mins);
            int sumi = 0;
            for (int j = 0; j < QK_K / 16; ++j) sumi += y[i].bsums[j] * mins[j / 2];
            a = aux8;
            for (int j = 0; j < QK_K / 32; ++j) {
                const int32_t scale = scales[j];
                for (int r = 0; r < 4; r++) {
                    for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                    for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
                    q8 += 8;
                    a += 8;
                }
            }
            const float d = FP16_TO_FP32(x[i].d) * y[i].d;
            for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
            const float dmin = FP16_TO_FP32(x[i].dmin) * y[i].d;
            sumf -= dmin * sumi;
        }
        for (int l = 0; l < 8; ++l) sumf += sums[l];
        return sumf;
    }
    if (type == ORC_TYPE_F16) {
        const uint16_t *x = (const uint16_t *)vx, *y = (const uint16_t *)vy;
        double sumf = 0.0;
        for (int64_t i = 0; i < n; ++i) sumf += (double)(FP16_TO_FP32(x[i]) * FP16_TO_FP32(y[i]));
        return (float)sumf;
    }
    if (type == ORC_TYPE_F32) {
        const float *x = (const float *)vx, *y = (const float *)vy;
        double sumf = 0.0;
        for (int64_t i = 0; i < n; ++i) sumf += (double)(x[i] * y[i]);
        return (float)sumf;
    }
    if (type == ORC_TYPE_Q6_K) {
        const blk_q6_K *x = (const blk_q6_K *)vx;
        const blk_q8_K *y = (const blk_q8_K *)vy;
        int8_t aux8[QK_K];
        int16_t aux16[8];
        float sums[8];
        int32_t aux32[8];
        memset(sums, 0, sizeof(sums));
        for (int64_t i = 0; i < n / QK_K; ++i) {
            const uint8_t *q4 = x[i].ql;
            const uint8_t *qh = x[i].qh;
            const int8_t *q8 = y[i].qs;
            memset(aux32, 0, sizeof(aux32));
            int8_t *a = aux8;
            for (int j = 0; j < QK_K; j += 128) {
                for (int l = 0; l < 32; ++l) {
                    a[l + 0] = (int8_t)((q4[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    a[l + 32] = (int8_t)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    a[l + 64] = (int8_t)((q4[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    a[l + 96] = (int8_t)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                }
                a += 128;
                q4 += 64;
                qh += 32;
            }
            a = aux8;
            int is = 0;
            for (int j = 0; j < QK_K / 16; ++j) {
                const int scale = x[i].scales[is++];
                for (int r = 0; r < 2; r++) {
                    for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                    for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
                    q8 += 8;
                    a += 8;
                }
            }
            const float d = FP16_TO_FP32(x[i].d) * y[i].d;
            for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        }
        float sumf = 0;
        for (int l = 0; l < 8; ++l) sumf += sums[l];
        return sumf;
    }
    return NAN;
}

/* Exact per-block integer sums, scale products formed in fp32 as ggml forms them, cross-block sum in double. */
double orc_vec_dot_exact(int type, int64_t n, const void *vx, const void *vy) {
    double acc = 0.0;
    if (type == ORC_TYPE_Q8_0) {
        const blk_q8_0 *x = (const blk_q8_0 *)vx;
        const blk_q8_0 *y = (const blk_q8_0 *)vy;
        for (int64_t ib = 0; ib < n / QK8_0; ++ib) {
            int64_t s = 0;
            for (int j = 0; j < QK8_0; j++) s += (int64_t)x[ib].qs[j] * y[ib].qs[j];
            acc += (double)s * (double)(FP16_TO_FP32(x[ib].d) * FP16_TO_FP32(y[ib].d));
        }
        return acc;
    }
    if (type == ORC_TYPE_F16 || type == ORC_TYPE_F32) {
        for (int64_t i = 0; i < n; ++i)
            acc += type == ORC_TYPE_F16
                       ? (double)FP16_TO_FP32(((const uint16_t *)vx)[i]) * (double)FP16_TO_FP32(((const uint16_t *)vy)[i])
                       : (double)((const float *)vx)[i] * (double)((const float *)vy)[i];
        return acc;
    }
    if (type == ORC_TYPE_Q4_K || type == ORC_TYPE_Q5_K || type == ORC_TYPE_Q6_K) {
        const blk_q8_K *y = (const blk_q8_K *)vy;
        for (int64_t i = 0; i < n / QK_K; ++i) {
            int64_t isum = 0, msum = 0;
            if (type == ORC_TYPE_Q4_K || type == ORC_TYPE_Q5_K) {
                /* the two types share d, dmin and the packed scales at the start of the block; Q5_K adds bit 4 of
                 * element l of sub-block j as bit j of qh[l] */
                const blk_q4_K *x4 = (const blk_q4_K *)vx + i;
                const blk_q5_K *x5 = (const blk_q5_K *)vx + i;
                const uint8_t *sc_bytes = type == ORC_TYPE_Q4_K ? x4->scales : x5->scales;
                const uint8_t *qs = type == ORC_TYPE_Q4_K ? x4->qs : x5->qs;
                const uint16_t d16 = type == ORC_TYPE_Q4_K ? x4->d : x5->d;
                const uint16_t dmin16 = type == ORC_TYPE_Q4_K ? x4->dmin : x5->dmin;
                uint8_t scales[8], mins[8];
                q4k_scales_mins(sc_bytes, scales, mins);
                for (int j = 0; j < QK_K; j++) {
                    const int sub = j / 32, chunk = j / 64, pos = j % 32, hi = (j / 32) & 1;
                    const uint8_t byte = qs[chunk * 32 + pos];
                    int q = hi ? (byte >> 4) : (byte & 0xF);
                    if (type == ORC_TYPE_Q5_K) q += ((x5->qh[pos] >> sub) & 1) << 4;
                    isum += (int64_t)scales[sub] * q * y[i].qs[j];
                    msum += (int64_t)mins[sub] * y[i].qs[j];
                }
                acc += (double)(FP16_TO_FP32(d16) * y[i].d) * (double)isum -
                       (double)(FP16_TO_FP32(dmin16) * y[i].d) * (double)msum;
            } else {
                const blk_q6_K *x = (const blk_q6_K *)vx + i;
                for (int j = 0; j < QK_K; j++) {
                    const int half = j / 128, r = j % 128, quarter = r / 32, l = r % 32;
                    const uint8_t lbyte = x->ql[half * 64 + l + (quarter & 1) * 32];
                    const int lo = (quarter < 2) ? (lbyte & 0xF) : (lbyte >> 4);
                    const int hbits = (x->qh[half * 32 + l] >> (2 * quarter)) & 3;
                    const int q = (lo | (hbits << 4)) - 32;
                    isum += (int64_t)x->scales[j / 16] * q * y[i].qs[j];
                }
                acc += (double)(FP16_TO_FP32(x->d) * y[i].d) * (double)isum;
            }
        }
        return acc;
    }
    return NAN;
}

/* ------------------------------------------------------------------------------------------------------------------
 * Ops. ggml-cpu/ggml-cpu.c ggml_compute_forward_mul_mat / _mul_mat_id / _get_rows, single-threaded.
 * ---------------------------------------------------------------------------------------------------------------- */
/* src1 rows converted to the weight's vec_dot_type (ggml-cpu.c: type_traits_cpu[vec_dot_type].from_float). */
static void quantize_act_row(int vdt, const float *x, void *y, int64_t k, int rounding) {
    if (vdt == ORC_TYPE_Q8_0) orc_quantize_row_q8_0(x, y, k, rounding);
    else if (vdt == ORC_TYPE_Q8_K) orc_quantize_row_q8_K(x, y, k);
    else if (vdt == ORC_TYPE_F16) for (int64_t i = 0; i < k; i++) ((uint16_t *)y)[i] = FP32_TO_FP16(x[i]);
    else memcpy(y, x, (size_t)k * 4);
}

int orc_mul_mat(const orc_tensor *src0, const orc_tensor *src1, orc_tensor *dst, int rounding, int exact) {
    const int vdt = orc_vec_dot_type(src0->type);
    if (vdt < 0 || src1->type != ORC_TYPE_F32 || dst->type != ORC_TYPE_F32) return -1;
    const int64_t K = src0->ne[0];
    if (src1->ne[0] != K || K % orc_blck_size(src0->type) != 0) return -1;
    if (src1->ne[2] % src0->ne[2] != 0 || src1->ne[3] % src0->ne[3] != 0) return -1;
    if (src1->nb[0] != 4 || dst->nb[0] != 4) return -1;
    const int64_t r2 = src1->ne[2] / src0->ne[2], r3 = src1->ne[3] / src0->ne[3];
    const size_t qrow = orc_row_size(vdt, K);
    uint8_t *wq = (uint8_t *)malloc(qrow);
    if (!wq) return -1;
    for (int64_t i13 = 0; i13 < src1->ne[3]; i13++)
        for (int64_t i12 = 0; i12 < src1->ne[2]; i12++)
            for (int64_t i11 = 0; i11 < src1->ne[1]; i11++) {
                const float *x = (const float *)((const char *)src1->data + i11 * src1->nb[1] + i12 * src1->nb[2] +
                                                 i13 * src1->nb[3]);
                quantize_act_row(vdt, x, wq, K, rounding);
                const char *w = (const char *)src0->data + (i12 / r2) * src0->nb[2] + (i13 / r3) * src0->nb[3];
                float *y = (float *)((char *)dst->data + i11 * dst->nb[1] + i12 * dst->nb[2] + i13 * dst->nb[3]);
                for (int64_t i01 = 0; i01 < src0->ne[1]; i01++) {
                    const void *row = w + i01 * src0->nb[1];
                    y[i01] = exact ? (float)orc_vec_dot_exact(src0->type, K, row, wq)
                                   : orc_vec_dot(src0->type, K, row, wq);
                }
            }
    free(wq);
    return 0;
}

int orc_mul_mat_id(const orc_tensor *as, const orc_tensor *b, const orc_tensor *ids, orc_tensor *dst, int rounding,
                   int exact) {
    const int vdt = orc_vec_dot_type(as->type);
    if (vdt < 0 || b->type != ORC_TYPE_F32 || ids->type != ORC_TYPE_I32 || dst->type != ORC_TYPE_F32) return -1;
    const int64_t K = as->ne[0], N = as->ne[1], E = as->ne[2];
    const int64_t n_ids = ids->ne[0], T = ids->ne[1];
    if (b->ne[0] != K || b->ne[2] != T || (b->ne[1] != 1 && b->ne[1] != n_ids)) return -1;
    if (dst->ne[0] != N || dst->ne[1] != n_ids || dst->ne[2] != T) return -1;
    const size_t qrow = orc_row_size(vdt, K);
    uint8_t *wq = (uint8_t *)malloc(qrow);
    if (!wq) return -1;
    int rc = 0;
    for (int64_t t = 0; t < T && rc == 0; t++)
        for (int64_t s = 0; s < n_ids; s++) {
            const int32_t e = *(const int32_t *)((const char *)ids->data + s * ids->nb[0] + t * ids->nb[1]);
            if (e < 0 || e >= E) { rc = -2; break; }
            const float *x = (const float *)((const char *)b->data + (s % b->ne[1]) * b->nb[1] + t * b->nb[2]);
            quantize_act_row(vdt, x, wq, K, rounding);
            const char *w = (const char *)as->data + e * as->nb[2];
            float *y = (float *)((char *)dst->data + s * dst->nb[1] + t * dst->nb[2]);
            for (int64_t n = 0; n < N; n++) {
                const void *row = w + n * as->nb[1];
                y[n] = exact ? (float)orc_vec_dot_exact(as->type, K, row, wq) : orc_vec_dot(as->type, K, row, wq);
            }
        }
    free(wq);
    return rc;
}

int orc_get_rows(const orc_tensor *src0, const orc_tensor *ids, orc_tensor *dst) {
    if (ids->type != ORC_TYPE_I32 || dst->type != ORC_TYPE_F32) return -1;
    const int64_t nc = src0->ne[0];
    for (int64_t i12 = 0; i12 < ids->ne[2]; i12++)
        for (int64_t i11 = 0; i11 < ids->ne[1]; i11++)
            for (int64_t i10 = 0; i10 < ids->ne[0]; i10++) {
                const int32_t r = *(const int32_t *)((const char *)ids->data + i10 * ids->nb[0] + i11 * ids->nb[1] +
                                                     i12 * ids->nb[2]);
                if (r < 0 || r >= src0->ne[1]) return -2;
                const void *row = (const char *)src0->data + r * src0->nb[1] + i11 * src0->nb[2] + i12 * src0->nb[3];
                float *y = (float *)((char *)dst->data + i10 * dst->nb[1] + i11 * dst->nb[2] + i12 * dst->nb[3]);
                if (orc_dequantize_row(src0->type, row, y, nc) != 0) return -1;
            }
    return 0;
}

/* ggml_argmax with the first of equal values (speech.cpp fastconformer/decoder.cpp:56-62; the fork's argmax). */
int orc_argmax(const orc_tensor *src0, orc_tensor *dst) {
    if (src0->type != ORC_TYPE_F32 || dst->type != ORC_TYPE_I32 || dst->ne[0] != src0->ne[1]) return -1;
    for (int64_t r = 0; r < src0->ne[1]; r++) {
        const float *v = (const float *)((const char *)src0->data + r * src0->nb[1]);
        int64_t best = 0;
        for (int64_t i = 1; i < src0->ne[0]; i++)
            if (v[i] > v[best]) best = i;
        *(int32_t *)((char *)dst->data + r * dst->nb[0]) = (int32_t)best;
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------------------------
 * The decoder layer's other ops (qwen3-decoder.cpp:350-410), as ggml-cpu computes them on f32 rows.
 * ---------------------------------------------------------------------------------------------------------------- */
/* ggml-cpu ops.cpp ggml_compute_forward_rms_norm_f32: the sum of squares (each square rounded to float) in double,
 * mean = sum / ne0 rounded to float, y = x * (1 / sqrtf(mean + eps)). */
void orc_rms_norm(const float *x, float *y, int64_t ne0, int64_t nrows, float eps) {
    for (int64_t r = 0; r < nrows; r++) {
        const float *xr = x + r * ne0;
        double sum = 0.0;
        for (int64_t i = 0; i < ne0; i++) sum += (double)(xr[i] * xr[i]);
        const float mean = (float)(sum / (double)ne0);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < ne0; i++) y[r * ne0 + i] = xr[i] * scale;
    }
}

/* ggml-cpu binary ops (ggml_compute_forward_add / _mul on f32): dst = a op b with b's rows repeated over a's
 * (b has ne0 elements per row and nb_rows rows; a's row r meets b's row r % nb_rows). op 0 add, 1 mul. */
void orc_binary(int op, const float *a, const float *b, float *y, int64_t ne0, int64_t nrows, int64_t nb_rows) {
    for (int64_t r = 0; r < nrows; r++)
        for (int64_t i = 0; i < ne0; i++) {
            const float u = a[r * ne0 + i], v = b[(r % nb_rows) * ne0 + i];
            y[r * ne0 + i] = op == 0 ? u + v : u * v;
        }
}

/* ggml-cpu ggml_vec_swiglu_f32 in its scalar form: y = silu(a) * b, silu(x) = x / (1 + expf(-x)). */
void orc_swiglu(const float *a, const float *b, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = a[i] / (1.0f + expf(-a[i])) * b[i];
}

/* ggml-cpu ggml_compute_forward_rope_f32, GGML_ROPE_TYPE_NEOX, no frequency factors, ext_factor 0, attn_factor 1:
 * for position p the angles are theta_k = p * theta_scale^k (k = 0 .. n_dims/2 - 1), formed as ggml_rope_cache_init
 * forms them (theta = p; theta *= theta_scale after each pair, theta_scale = powf(freq_base, -2 / n_dims), all
 * float), and the pair (x[k], x[k + n_dims/2]) turns by theta_k. Channels past n_dims are copied. x: [ne0, n_head,
 * nrows] with one position per row (pos[r]). */
void orc_rope_neox(const float *x, const int32_t *pos, float *y, int64_t ne0, int64_t n_head, int64_t nrows,
                   int n_dims, float freq_base, float freq_scale) {
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    float *cache = (float *)malloc(sizeof(float) * (size_t)n_dims);
    for (int64_t r = 0; r < nrows; r++) {
        float theta = (float)pos[r];
        for (int i0 = 0; i0 < n_dims; i0 += 2) {
            const float t = freq_scale * theta;
            cache[i0] = cosf(t);
            cache[i0 + 1] = sinf(t);
            theta *= theta_scale;
        }
        for (int64_t h = 0; h < n_head; h++) {
            const float *xr = x + (r * n_head + h) * ne0;
            float *yr = y + (r * n_head + h) * ne0;
            for (int i0 = 0; i0 < n_dims; i0 += 2) {
                const int ic = i0 / 2;
                const float c = cache[i0], sn = cache[i0 + 1];
                const float x0 = xr[ic], x1 = xr[ic + n_dims / 2];
                yr[ic] = x0 * c - x1 * sn;
                yr[ic + n_dims / 2] = x0 * sn + x1 * c;
            }
            for (int64_t i = n_dims; i < ne0; i++) yr[i] = xr[i];
        }
    }
    free(cache);
}

/* ggml-cpu ggml_compute_forward_set_rows with an f16 destination: dst row idx[i] = fp16(src row i) (from_float,
 * round to nearest even). dst holds dst_rows rows of ne0 halves; returns -2 for an index out of range. */
int orc_set_rows_f16(const float *src, const int32_t *idx, uint16_t *dst, int64_t ne0, int64_t nrows,
                     int64_t dst_rows) {
    for (int64_t i = 0; i < nrows; i++) {
        if (idx[i] < 0 || idx[i] >= dst_rows) return -2;
        for (int64_t j = 0; j < ne0; j++) dst[idx[i] * ne0 + j] = FP32_TO_FP16(src[i * ne0 + j]);
    }
    return 0;
}

/* ggml-cpu ggml_compute_forward_flash_attn_ext_f16 (one chunk, F16 K and V, an f16 mask, no ALiBi, no softcap).
 * Shapes as the decoder builds them: q [D, n_q, n_head] f32 (rows of one head contiguous: q[(h * n_q + i) * D]),
 * K, V [D, n_kv, n_kv_head] f16 (k[(hk * n_kv + j) * D]), mask [n_kv, n_q] f16, dst [D, n_head, n_q] f32
 * (dst[(i * n_head + h) * D], the permuted output). Head h reads K/V head h / (n_head / n_kv_head).
 * exact = 0: the CPU's arithmetic -- q rounded to fp16, each k.q an fp32 sum of exact products, online softmax with
 *            the V accumulator held in fp16 (ggml_vec_scale_f16 / ggml_vec_mad_f16 round after every step);
 * exact = 1: the same attention with q rounded to fp16, every score and the softmax in double. */
int orc_flash_attn_ext(const float *q, const uint16_t *k, const uint16_t *v, const uint16_t *mask, float *dst, int D,
                       int64_t n_q, int64_t n_head, int64_t n_kv, int64_t n_kv_head, float scale, int exact) {
    if (n_head % n_kv_head != 0) return -1;
    const int64_t g = n_head / n_kv_head;
    uint16_t *qh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)D);
    uint16_t *acc16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)D);
    double *accd = (double *)malloc(sizeof(double) * (size_t)D);
    double *sc = (double *)malloc(sizeof(double) * (size_t)(n_kv > 0 ? n_kv : 1));
    for (int64_t h = 0; h < n_head; h++) {
        const int64_t hk = h / g;
        for (int64_t i = 0; i < n_q; i++) {
            const float *qr = q + (h * n_q + i) * D;
            for (int d = 0; d < D; d++) qh[d] = FP32_TO_FP16(qr[d]);
            float *out = dst + (i * n_head + h) * D;
            const uint16_t *mr = mask ? mask + i * n_kv : NULL;
            if (!exact) {
                float S = 0.0f, M = -INFINITY;
                for (int d = 0; d < D; d++) acc16[d] = 0;
                for (int64_t j = 0; j < n_kv; j++) {
                    const float mv = mr ? FP16_TO_FP32(mr[j]) : 0.0f;
                    if (mv == -INFINITY) continue;
                    const uint16_t *kr = k + (hk * n_kv + j) * D;
                    float s = 0.0f;
                    for (int d = 0; d < D; d++) s += FP16_TO_FP32(kr[d]) * FP16_TO_FP32(qh[d]);
                    s = s * scale;
                    s += mv;
                    const float Mold = M;
                    float ms = 1.0f, vs = 1.0f;
                    const uint16_t *vr = v + (hk * n_kv + j) * D;
                    if (s > M) {
                        M = s;
                        ms = expf(Mold - M);
                        for (int d = 0; d < D; d++) acc16[d] = FP32_TO_FP16(FP16_TO_FP32(acc16[d]) * ms);
                    } else {
                        vs = expf(s - M);
                    }
                    for (int d = 0; d < D; d++)
                        acc16[d] = FP32_TO_FP16(FP16_TO_FP32(acc16[d]) + FP16_TO_FP32(vr[d]) * vs);
                    S = S * ms + vs;
                }
                const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
                for (int d = 0; d < D; d++) out[d] = FP16_TO_FP32(acc16[d]) * S_inv;
            } else {
                double M = -INFINITY;
                for (int64_t j = 0; j < n_kv; j++) {
                    const double mv = mr ? (double)FP16_TO_FP32(mr[j]) : 0.0;
                    if (mv == -INFINITY) { sc[j] = -INFINITY; continue; }
                    const uint16_t *kr = k + (hk * n_kv + j) * D;
                    double s = 0.0;
                    for (int d = 0; d < D; d++) s += (double)FP16_TO_FP32(kr[d]) * (double)FP16_TO_FP32(qh[d]);
                    sc[j] = s * (double)scale + mv;
                    if (sc[j] > M) M = sc[j];
                }
                double S = 0.0;
                for (int d = 0; d < D; d++) accd[d] = 0.0;
                for (int64_t j = 0; j < n_kv; j++) {
                    if (sc[j] == -INFINITY) continue;
                    const double p = exp(sc[j] - M);
                    S += p;
                    const uint16_t *vr = v + (hk * n_kv + j) * D;
                    for (int d = 0; d < D; d++) accd[d] += p * (double)FP16_TO_FP32(vr[d]);
                }
                for (int d = 0; d < D; d++) out[d] = S == 0.0 ? 0.0f : (float)(accd[d] / S);
            }
        }
    }
    free(qh);
    free(acc16);
    free(accd);
    free(sc);
    return 0;
}

/* ------------------------------------------------------------------------------------------------------------------
 * Seeded synthetic data.
 * ---------------------------------------------------------------------------------------------------------------- */
static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static uint64_t xoshiro256ss(uint64_t s[4]) {
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

void orc_fill_normal_rows(uint64_t seed, int64_t row0, int64_t nrows, int64_t n_per_row, float mean, float stddev,
                          float *out) {
    for (int64_t r = 0; r < nrows; r++) {
        uint64_t sm = seed ^ ((uint64_t)(row0 + r) * 0xD1B54A32D192ED03ull);
        uint64_t s[4];
        for (int i = 0; i < 4; i++) s[i] = splitmix64(&sm);
        float *o = out + r * n_per_row;
        for (int64_t j = 0; j < n_per_row; j += 2) {
            const double u1 = ((xoshiro256ss(s) >> 11) + 1) * 0x1.0p-53; /* (0, 1] */
            const double u2 = (xoshiro256ss(s) >> 11) * 0x1.0p-53;       /* [0, 1) */
            const double rad = sqrt(-2.0 * log(u1));
            const double th = 6.283185307179586476925286766559 * u2;
            o[j] = (float)(mean + stddev * rad * cos(th));
            if (j + 1 < n_per_row) o[j + 1] = (float)(mean + stddev * rad * sin(th));
        }
    }
}
