/*
 * Multi-threaded AVX2 / AVX-512-VNNI restatement of ggml's CPU MUL_MAT for Q8_0 / Q4_K / Q6_K weights.
 *
 * TEST INFRASTRUCTURE ONLY: the timed CPU baseline beside the GPU figures (kind "port": ggml itself is absent from the
 * reference tree, see `.gitmodules:1-4`). It follows ggml_compute_forward_mul_mat (ggml-cpu/ggml-cpu.c): src1 is
 * quantized once to the weight type's vec_dot_type (x86 quantize_row_q8_0 for Q8_0, quantize_row_q8_K for K-quants),
 * then src0 rows are split into chunks across threads, and each output is an AVX2 int8 dot
 * (ggml-cpu/arch/x86/quants.c ggml_vec_dot_{q8_0_q8_0,q4_K_q8_K,q6_K_q8_K}) with fp32 cross-block sums.
 * The thread count mirrors speech.cpp's default of one thread per physical core (src/common/backend.cpp:122-167);
 * callers pass it explicitly.
 */
#include "mx_oracle.c"

#include <immintrin.h>
#include <omp.h>

#define AVX2 __attribute__((target("avx2,fma,f16c")))

AVX2 static inline float hsum8(__m256 v) {
    __m128 r = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    return _mm_cvtss_f32(r);
}

/* signed x signed int8 products summed in pairs then in fours: |x| * sign(y, x) through maddubs. */
AVX2 static inline __m256i dot_i8_to_i32(__m256i x, __m256i y) {
    const __m256i ax = _mm256_sign_epi8(x, x);
    const __m256i sy = _mm256_sign_epi8(y, x);
    const __m256i p16 = _mm256_maddubs_epi16(ax, sy);
    return _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
}

/* The same products through one vpdpbusd (ggml's mul_sum_i8_pairs_float where the host has AVX512-VNNI with
 * AVX512VL): |x| as the unsigned operand, sign(y, x) as the signed one, summed in fours into int32 lanes. The int32
 * lane sums equal the maddubs / madd pair's, so the output is bit-identical to the AVX2 path. */
#define VNNI __attribute__((target("avx2,fma,f16c,avx512f,avx512vl,avx512vnni")))

VNNI static float dot_q8_0_vnni(int64_t n, const blk_q8_0 *x, const blk_q8_0 *y) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t ib = 0; ib < n / 32; ++ib) {
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(x[ib].d) * _cvtsh_ss(y[ib].d));
        const __m256i qx = _mm256_loadu_si256((const __m256i *)x[ib].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        const __m256i s = _mm256_dpbusd_epi32(_mm256_setzero_si256(), _mm256_sign_epi8(qx, qx),
                                              _mm256_sign_epi8(qy, qx));
        acc = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(s), acc);
    }
    return hsum8(acc);
}

AVX2 static float dot_q8_0(int64_t n, const blk_q8_0 *x, const blk_q8_0 *y) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t ib = 0; ib < n / 32; ++ib) {
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(x[ib].d) * _cvtsh_ss(y[ib].d));
        const __m256i qx = _mm256_loadu_si256((const __m256i *)x[ib].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        acc = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(dot_i8_to_i32(qx, qy)), acc);
    }
    return hsum8(acc);
}

AVX2 static float dot_q4_K(int64_t n, const blk_q4_K *x, const blk_q8_K *y) {
    __m256 acc = _mm256_setzero_ps();
    float acc_m = 0.0f;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    for (int64_t i = 0; i < n / 256; ++i) {
        uint8_t sc[8], mn[8];
        q4k_scales_mins(x[i].scales, sc, mn);
        int msum = 0;
        for (int j = 0; j < 16; j++) msum += y[i].bsums[j] * mn[j / 2];
        const float d = _cvtsh_ss(x[i].d) * y[i].d;
        const float dmin = _cvtsh_ss(x[i].dmin) * y[i].d;
        __m256i sumi = _mm256_setzero_si256();
        const uint8_t *q4 = x[i].qs;
        const int8_t *q8 = y[i].qs;
        for (int j = 0; j < 4; ++j) {
            const __m256i q4bits = _mm256_loadu_si256((const __m256i *)q4);
            const __m256i lo = _mm256_and_si256(q4bits, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q4bits, 4), m4);
            const __m256i y0 = _mm256_loadu_si256((const __m256i *)q8);
            const __m256i y1 = _mm256_loadu_si256((const __m256i *)(q8 + 32));
            __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, y0), _mm256_set1_epi16(sc[2 * j]));
            __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, y1), _mm256_set1_epi16(sc[2 * j + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
            q4 += 32;
            q8 += 64;
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
        acc_m += dmin * (float)msum;
    }
    return hsum8(acc) - acc_m;
}

AVX2 static float dot_q6_K(int64_t n, const blk_q6_K *x, const blk_q8_K *y) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i m4 = _mm256_set1_epi8(0xF);
    const __m256i m2 = _mm256_set1_epi8(3);
    for (int64_t i = 0; i < n / 256; ++i) {
        const float d = _cvtsh_ss(x[i].d) * y[i].d;
        const uint8_t *ql = x[i].ql;
        const uint8_t *qh = x[i].qh;
        const int8_t *q8 = y[i].qs;
        __m256i sumi = _mm256_setzero_si256();
        for (int half = 0; half < 2; ++half) {
            const __m256i l0 = _mm256_loadu_si256((const __m256i *)ql);
            const __m256i l1 = _mm256_loadu_si256((const __m256i *)(ql + 32));
            const __m256i h = _mm256_loadu_si256((const __m256i *)qh);
            __m256i q[4];
            q[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(h, m2), 4));
            q[1] = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 2), m2), 4));
            q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 4), m2), 4));
            q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 6), m2), 4));
            for (int k = 0; k < 4; k++) {
                const __m256i yk = _mm256_loadu_si256((const __m256i *)(q8 + 32 * k));
                /* (q - 32) . y = q . y - 32 * sum(y): maddubs on the unsigned 6-bit codes, then the offset. */
                const __m256i p = _mm256_maddubs_epi16(q[k], yk);
                const __m256i off = _mm256_maddubs_epi16(_mm256_set1_epi8(32), yk);
                const __m256i p16 = _mm256_sub_epi16(p, off);
                const int s0 = x[i].scales[half * 8 + 2 * k], s1 = x[i].scales[half * 8 + 2 * k + 1];
                const __m256i scv = _mm256_setr_epi16((short)s0, (short)s0, (short)s0, (short)s0, (short)s0, (short)s0,
                                                      (short)s0, (short)s0, (short)s1, (short)s1, (short)s1, (short)s1,
                                                      (short)s1, (short)s1, (short)s1, (short)s1);
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(p16, scv));
            }
            ql += 64;
            qh += 32;
            q8 += 128;
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum8(acc);
}

int cpf_have_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
}

static int have_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl");
}

/* The instruction set the Q8_0 dot runs on here: 2 = AVX512-VNNI (vpdpbusd), 1 = AVX2 (maddubs + madd). K-quant dots
 * are AVX2 on every host, as in ggml's x86 quants.c. */
int cpf_q8_0_isa(void) { return have_vnni() ? 2 : 1; }

static float dot_any(int type, int64_t n, const void *x, const void *y) {
    static int vnni = -1;
    if (vnni < 0) vnni = have_vnni();
    switch (type) {
        case ORC_TYPE_Q8_0:
            return vnni ? dot_q8_0_vnni(n, (const blk_q8_0 *)x, (const blk_q8_0 *)y)
                        : dot_q8_0(n, (const blk_q8_0 *)x, (const blk_q8_0 *)y);
        case ORC_TYPE_Q4_K: return dot_q4_K(n, (const blk_q4_K *)x, (const blk_q8_K *)y);
        case ORC_TYPE_Q6_K: return dot_q6_K(n, (const blk_q6_K *)x, (const blk_q8_K *)y);
        default: return NAN;
    }
}

/* ggml_compute_forward_mul_mat for 2-D src0 [K, N] and src1 [K, M]; nthreads OpenMP threads. Returns 0 on success. */
int cpf_mul_mat(const orc_tensor *src0, const orc_tensor *src1, orc_tensor *dst, int nthreads) {
    if (!cpf_have_avx2()) return -3;
    const int vdt = orc_vec_dot_type(src0->type);
    if (vdt < 0 || src1->type != ORC_TYPE_F32 || dst->type != ORC_TYPE_F32) return -1;
    const int64_t K = src0->ne[0], N = src0->ne[1], M = src1->ne[1];
    if (src1->ne[0] != K || src0->ne[2] != 1 || src1->ne[2] != 1 || src0->ne[3] != 1 || src1->ne[3] != 1) return -1;
    const size_t qrow = orc_row_size(vdt, K);
    uint8_t *wq = (uint8_t *)malloc(qrow * (size_t)M);
    if (!wq) return -1;
    for (int64_t m = 0; m < M; m++) {
        const float *x = (const float *)((const char *)src1->data + m * src1->nb[1]);
        if (vdt == ORC_TYPE_Q8_0) orc_quantize_row_q8_0(x, wq + m * qrow, K, ORC_ROUND_X86);
        else orc_quantize_row_q8_K(x, wq + m * qrow, K);
    }
    const int64_t chunk = 16;
    const int64_t nchunks = (N + chunk - 1) / chunk;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
    for (int64_t c = 0; c < nchunks; c++) {
        const int64_t n0 = c * chunk, n1 = n0 + chunk < N ? n0 + chunk : N;
        for (int64_t m = 0; m < M; m++) {
            float *y = (float *)((char *)dst->data + m * dst->nb[1]);
            for (int64_t n = n0; n < n1; n++)
                y[n] = dot_any(src0->type, K, (const char *)src0->data + n * src0->nb[1], wq + m * qrow);
        }
    }
    free(wq);
    return 0;
}

/* ggml_compute_forward_flash_attn_ext_f16 for F16 K / V as ggml-cpu runs it: the (q row, head) pairs split across
 * threads; per pair q rounded to fp16, each score an F16C dot of the key row with q summed in fp32
 * (ggml_vec_dot_f16), the online softmax, and the V accumulator kept in fp16 (ggml_vec_scale_f16 / ggml_vec_mad_f16:
 * converted to fp32, scaled or multiply-added, converted back, eight channels at a time). Layouts as
 * orc_flash_attn_ext: q [n_head][n_q][D], k, v [n_kv_head][n_kv][D], mask [n_q][n_kv] f16, dst [n_q][n_head][D].
 * D a multiple of 8. Returns 0 on success. */
AVX2 static float dot_f16_row(const uint16_t *a, const uint16_t *b, int D) {
    __m256 acc = _mm256_setzero_ps();
    for (int d = 0; d < D; d += 8) {
        const __m256 x = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(a + d)));
        const __m256 y = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(b + d)));
        acc = _mm256_fmadd_ps(x, y, acc);
    }
    return hsum8(acc);
}

AVX2 static void fa_pair(const float *qr, const uint16_t *k, const uint16_t *v, const uint16_t *mr, float *out, int D,
                         int64_t n_kv, float scale, uint16_t *qh, uint16_t *acc) {
    for (int d = 0; d < D; d += 8)
        _mm_storeu_si128((__m128i *)(qh + d), _mm256_cvtps_ph(_mm256_loadu_ps(qr + d), _MM_FROUND_TO_NEAREST_INT));
    for (int d = 0; d < D; d++) acc[d] = 0;
    float S = 0.0f, M = -INFINITY;
    for (int64_t j = 0; j < n_kv; j++) {
        const float mv = mr ? _cvtsh_ss(mr[j]) : 0.0f;
        if (mv == -INFINITY) continue;
        const float s = dot_f16_row(k + j * D, qh, D) * scale + mv;
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            const float Mold = M;
            M = s;
            ms = expf(Mold - M);
            const __m256 f = _mm256_set1_ps(ms);
            for (int d = 0; d < D; d += 8) {
                const __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(acc + d)));
                _mm_storeu_si128((__m128i *)(acc + d), _mm256_cvtps_ph(_mm256_mul_ps(a, f), _MM_FROUND_TO_NEAREST_INT));
            }
        } else {
            vs = expf(s - M);
        }
        const __m256 f = _mm256_set1_ps(vs);
        const uint16_t *vr = v + j * D;
        for (int d = 0; d < D; d += 8) {
            const __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(acc + d)));
            const __m256 x = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(vr + d)));
            _mm_storeu_si128((__m128i *)(acc + d), _mm256_cvtps_ph(_mm256_fmadd_ps(x, f, a), _MM_FROUND_TO_NEAREST_INT));
        }
        S = S * ms + vs;
    }
    const float inv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int d = 0; d < D; d++) out[d] = _cvtsh_ss(acc[d]) * inv;
}

int cpf_flash_attn_ext(const float *q, const uint16_t *k, const uint16_t *v, const uint16_t *mask, float *dst, int D,
                       int64_t n_q, int64_t n_head, int64_t n_kv, int64_t n_kv_head, float scale, int nthreads) {
    if (!cpf_have_avx2()) return -3;
    if (n_kv_head < 1 || n_head % n_kv_head != 0 || D % 8 != 0 || D > 1024) return -1;
    const int64_t g = n_head / n_kv_head;
#pragma omp parallel num_threads(nthreads)
    {
        uint16_t qh[1024], acc[1024];
#pragma omp for schedule(dynamic, 1)
        for (int64_t p = 0; p < n_q * n_head; p++) {
            const int64_t i = p / n_head, h = p % n_head, hk = h / g;
            fa_pair(q + (h * n_q + i) * D, k + hk * n_kv * D, v + hk * n_kv * D, mask ? mask + i * n_kv : NULL,
                    dst + (i * n_head + h) * D, D, n_kv, scale, qh, acc);
        }
    }
    return 0;
}
