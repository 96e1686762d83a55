/*
 * libmx -- an MI355X (gfx950) device for ggml's quantized MUL_MAT, MUL_MAT_ID and GET_ROWS, with the ops either side
 * of them in a decoder step (ARGMAX, RMS_NORM, ADD, MUL, SwiGLU, RoPE, SET_ROWS, FLASH_ATTN_EXT) and a GGUF loader.
 *
 * The C ABI below is the drop-in boundary. speech.cpp reaches these ops through ggml's backend plugin interface
 * (ggml-backend-impl.h: ggml_backend_reg_i / ggml_backend_device_i / ggml_backend_i / ggml_backend_buffer_type_i /
 * ggml_backend_buffer_i); each entry point names the ggml hook it serves and the speech.cpp call site that reaches that
 * hook. Plain C types only: device pointers, sizes and a ggml-shaped tensor descriptor.
 *
 * Conventions
 *  - Status codes mirror ggml_status: 0 success, -1 failed, -2 allocation failed; -3 / -4 are invalid / unsupported
 *    arguments, which a ggml adapter reports as GGML_STATUS_FAILED (src/common/graph.cpp:13-31 maps them to the
 *    Device and OutOfMemory faults). No entry point aborts on bad input; the message is in mx_last_error().
 *  - Tensors follow ggml order: ne[0] is the fastest axis, nb[] are byte strides.
 *  - Quantized tensors (Q8_0, Q4_K, Q5_K, Q6_K) held by this library are stored in its own device layout: each tensor's
 *    allocation is split into planes (quants, scales, super-block scales) so every plane is 256-byte aligned and every
 *    row of quants is contiguous. mx_tensor_set / mx_tensor_get take and return ggml's own block bytes (GGUF layout),
 *    at any byte offset and size, so ggml and GGUF never see the device layout. Float and integer tensors are plain.
 *  - One mx_backend is driven by one thread at a time (include/speech.h:27-30: one request per model at a time).
 *    Work is queued on the backend's stream; results are ready after mx_backend_synchronize().
 */
#ifndef MX_H
#define MX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MX_API __attribute__((visibility("default")))

/* ggml_status values plus argument errors. */
enum {
    MX_SUCCESS = 0,
    MX_FAILED = -1,
    MX_ALLOC_FAILED = -2,
    MX_INVALID = -3,
    MX_UNSUPPORTED = -4,
};

/* ggml_type values (ggml.h enum ggml_type). */
enum {
    MX_TYPE_F32 = 0,
    MX_TYPE_F16 = 1,
    MX_TYPE_Q8_0 = 8,
    MX_TYPE_Q8_1 = 9,
    MX_TYPE_Q4_K = 12,
    MX_TYPE_Q5_K = 13,
    MX_TYPE_Q6_K = 14,
    MX_TYPE_Q8_K = 15,
    MX_TYPE_I32 = 26,
};

/* The ops this device computes (the ggml adapter maps GGML_OP_GET_ROWS / GGML_OP_MUL_MAT / GGML_OP_MUL_MAT_ID /
 * GGML_OP_ARGMAX, and the decoder layer's GGML_OP_RMS_NORM / GGML_OP_ADD / GGML_OP_MUL / GGML_OP_GLU (swiglu) /
 * GGML_OP_SET_ROWS; ROPE and FLASH_ATTN_EXT carry parameters and have supports functions of their own). */
enum {
    MX_OP_GET_ROWS = 1,
    MX_OP_MUL_MAT = 2,
    MX_OP_MUL_MAT_ID = 3,
    MX_OP_ARGMAX = 4,
    MX_OP_RMS_NORM = 5,
    MX_OP_ADD = 6,
    MX_OP_MUL = 7,
    MX_OP_SWIGLU = 8,
    MX_OP_SET_ROWS = 9,
};

/* Rounding of the activation quantizers.
 * MX_ROUND_REF: ggml-quants.c quantize_row_q8_{0,1}_ref (d = amax/127, q = roundf(x * (1/d))). The default.
 * MX_ROUND_X86: ggml-cpu's x86 quantize_row_q8_0 / _q8_1 (q = round-half-even(x * (127/amax))).
 * Q8_K (the activation type of Q4_K / Q6_K weights) has a single form, quantize_row_q8_K_ref. */
enum {
    MX_ROUND_REF = 0,
    MX_ROUND_X86 = 1,
};

/* A ggml tensor as the backend sees it (ggml.h struct ggml_tensor: type, ne, nb, data). `data` is a device address
 * inside a buffer from mx_buffer_alloc (or any device memory for float / int tensors). */
typedef struct mx_tensor {
    int32_t type;
    int32_t pad_;
    int64_t ne[4];
    uint64_t nb[4];
    void *data;
} mx_tensor;

typedef struct mx_backend mx_backend;
typedef struct mx_graph mx_graph;
typedef struct mx_event mx_event;

/* ---------------------------------------------------------------------------------------------------------------
 * Device and backend: ggml_backend_reg_i.get_device_count / ggml_backend_device_i.{get_name, get_description,
 * get_memory, init_backend} and ggml_backend_i.{free, synchronize}. Called from src/common/backend.cpp:70-120
 * (enumeration, find_device, start_device), src/api/speech.cpp:339 and src/engines/drama3-engine.cpp:57 (memory).
 * ------------------------------------------------------------------------------------------------------------- */
MX_API int mx_device_count(void);
MX_API int mx_device_description(int device, char *buf, size_t len);
MX_API int mx_device_memory(int device, size_t *free_bytes, size_t *total_bytes);
MX_API mx_backend *mx_backend_init(int device);
MX_API void mx_backend_free(mx_backend *be);
/* The hipStream_t the backend queues its work on. */
MX_API void *mx_backend_stream(mx_backend *be);
/* Waits for the queued work. Reports an index out of range met by GET_ROWS / MUL_MAT_ID since the last call as
 * MX_INVALID (ggml's CPU backend asserts on it, ggml-cpu.c get_rows / mul_mat_id; this device never aborts). */
MX_API int mx_backend_synchronize(mx_backend *be);
/* Activation rounding used by mx_mul_mat / mx_mul_mat_id from now on (MX_ROUND_REF by default). */
MX_API int mx_backend_set_rounding(mx_backend *be, int rounding);

/* Kernel choices of a backend's products. No counterpart in speech.cpp or ggml's backend interface: this is the
 * device's own test and measurement control (ggml's GPU backends read process-wide environment switches for the same
 * purpose). Every option is 0 by default, which lets the dispatcher pick per product; a forced choice sends every
 * product it covers to one kernel, so a test can reach each kernel the dispatcher may pick, in one process. A product
 * the forced kernel cannot compute fails with MX_UNSUPPORTED (or MX_FAILED for a tile the kernel lacks) instead of
 * going elsewhere. Values outside those listed are refused with MX_INVALID.
 *   MX_OPT_GEMM_Q8_0          Q8_0 at M > 8: 0 as picked (the int8 MFMA GEMM where K % 128 == 0, else the fp16
 *                             dequantizing GEMM where K % 64 == 0), 1 the int8 MFMA GEMM, 2 the fp16 dequantizing GEMM
 *   MX_OPT_GEMM_KQUANT        Q4_K / Q6_K at M > 8: 0 as picked (scale-split int8 for Q4_K, fp16 dequantizing for
 *                             Q6_K), 1 the VALU-scaled int8 GEMM
 *   MX_OPT_GEMM_TILE_M / _N   the GEMM's tile (0 0: picked per product): the Q4_K GEMM 128 x 128, 64 x 128, 128 x 64
 *                             or 64 x 64; the fp16 dequantizing GEMM 128 x 128, 128 x 64 or 64 x 64, and for Q8_0,
 *                             Q5_K and Q6_K also 64 x 128 and 32 x 128; the int8 Q8_0 GEMM 64 x 64, 64 x 128 or
 *                             128 x 128; the fp16 GEMM over MUL_MAT_ID's expert chunks 32 x 128, 32 x 64 or 64 x 64
 *   MX_OPT_GEMM_SPLIT         K splits of the fp16 dequantizing GEMM and the int8 Q8_0 GEMM, 0 (picked) .. 64
 *   MX_OPT_MATVEC_LPR         lanes per weight row of the mat-vec: 0 (picked), 16, 32, 64
 *   MX_OPT_MMID_KERNEL        MUL_MAT_ID with many pairs: 0 as picked (Q4_K: the grouped int8 MFMA product; Q8_0,
 *                             Q5_K, Q6_K: the fp16 dequantizing GEMM over chunks of each expert's pairs from one /
 *                             three pairs per expert on average, else the experts kernel), 1 the experts kernel, 2 the
 *                             grouped product (Q4_K int8, the other types the fp16 GEMM over the chunks)
 *   MX_OPT_MMID_MATVEC_PAIRS  MUL_MAT_ID runs as one mat-vec launch up to this many (token, slot) pairs (16; 0..4096)
 *   MX_OPT_MMID_CHUNK         pairs per chunk of an expert's pairs in the grouped Q4_K product: 0 as picked (16 when
 *                             the pairs average at most four per expert, else 32), 16 (one 16-row tile per chunk),
 *                             32 (two tiles sharing each decoded weight fragment) */
enum {
    MX_OPT_GEMM_Q8_0 = 1,
    MX_OPT_GEMM_KQUANT = 2,
    MX_OPT_GEMM_TILE_M = 3,
    MX_OPT_GEMM_TILE_N = 4,
    MX_OPT_GEMM_SPLIT = 5,
    MX_OPT_MATVEC_LPR = 6,
    MX_OPT_MMID_KERNEL = 7,
    MX_OPT_MMID_MATVEC_PAIRS = 8,
    MX_OPT_MMID_CHUNK = 9,
};
MX_API int mx_backend_set_option(mx_backend *be, int option, int64_t value);
MX_API int mx_backend_get_option(mx_backend *be, int option, int64_t *value);
/* The last error message of the calling thread ("" if none). */
MX_API const char *mx_last_error(void);

/* ---------------------------------------------------------------------------------------------------------------
 * Buffer type and buffers: ggml_backend_buffer_type_i.{get_alignment, get_max_size, get_alloc_size, alloc_buffer} and
 * ggml_backend_buffer_i.{get_base, free_buffer, clear, set_tensor, get_tensor, memset_tensor, cpy_tensor}.
 * Reached from src/common/model-file.cpp:222-268 (ggml_backend_alloc_ctx_tensors, set_usage WEIGHTS, tensor_set in
 * 16 MB pieces at increasing offsets) and src/common/qwen3-decoder.cpp:160,204,225,250,282,442.
 * ------------------------------------------------------------------------------------------------------------- */
MX_API size_t mx_buft_alignment(void);
MX_API size_t mx_buft_max_size(void);
/* Bytes the tensor takes in this device's layout (>= ggml_nbytes). */
MX_API size_t mx_tensor_alloc_size(const mx_tensor *t);
MX_API int mx_buffer_alloc(mx_backend *be, size_t size, void **base);
MX_API int mx_buffer_free(mx_backend *be, void *base);
MX_API int mx_buffer_clear(mx_backend *be, void *base, size_t size, uint8_t value);
/* Writes `size` bytes of the tensor's ggml-layout bytes starting at byte `offset` (any offset, any size). */
MX_API int mx_tensor_set(mx_backend *be, const mx_tensor *t, const void *host, size_t offset, size_t size);
/* Reads ggml-layout bytes [offset, offset + size) of the tensor into host memory. */
MX_API int mx_tensor_get(mx_backend *be, const mx_tensor *t, void *host, size_t offset, size_t size);
/* Sets ggml-layout bytes [offset, offset + size) of the tensor to `value`. */
MX_API int mx_tensor_memset(mx_backend *be, const mx_tensor *t, uint8_t value, size_t offset, size_t size);
/* Copies a whole tensor between two tensors of the same type and shape held by this device; the copy has landed
 * when the call returns (ggml's cpy_tensor contract), so work on any stream may read dst next. */
MX_API int mx_tensor_copy(mx_backend *be, const mx_tensor *src, const mx_tensor *dst);

/* ---------------------------------------------------------------------------------------------------------------
 * Ops: ggml_backend_device_i.supports_op and the nodes ggml_backend_i.graph_compute runs.
 *   GET_ROWS:    src/common/qwen3-decoder.cpp:464,483,499; src/families/qwen3-tts/talker.cpp:55,63,91;
 *                src/families/drama3/text-model.cpp:253,255
 *   MUL_MAT:     src/common/qwen3-decoder.cpp:362-364,403,406-407,410,426; src/common/graph.h:15-19
 *   MUL_MAT_ID:  src/common/graph.h:21-26 from src/families/drama3/text-model.cpp:198-221
 * Shapes follow ggml exactly:
 *   mx_get_rows(src0 [K, R, A, B] quantized, ids [n, A, B] I32) -> dst [K, n, A, B] F32 (n A B < 2^31 rows)
 *   mx_mul_mat(src0 [K, N, A, B] quantized, src1 [K, M, A*r2, B*r3] F32) -> dst [N, M, A*r2, B*r3] F32
 *   mx_mul_mat_id(as [K, N, E] quantized, b [K, 1 or k, T] F32, ids [k, T] I32) -> dst [N, k, T] F32
 * All products accumulate each block's integer sum exactly and sum across blocks in fp32, whatever the tensor's
 * requested precision (ggml_prec_set_acc, src/common/graph.h:10-26).
 * ------------------------------------------------------------------------------------------------------------- */
MX_API int mx_supports_op(int op, const mx_tensor *src0, const mx_tensor *src1, const mx_tensor *src2,
                          const mx_tensor *dst);
MX_API int mx_get_rows(mx_backend *be, const mx_tensor *src0, const mx_tensor *ids, const mx_tensor *dst);
MX_API int mx_mul_mat(mx_backend *be, const mx_tensor *src0, const mx_tensor *src1, const mx_tensor *dst);
MX_API int mx_mul_mat_id(mx_backend *be, const mx_tensor *as, const mx_tensor *b, const mx_tensor *ids,
                         const mx_tensor *dst);
/* Several MUL_MAT_ID nodes that read the same b and ids, as a backend's graph_compute may fuse them: the gate and up
 * experts of a MoE FFN (src/families/drama3/text-model.cpp:208-209, TextModel::experts). Each dst[i] = as[i] routed by
 * ids over b, exactly as n separate mx_mul_mat_id calls compute it; one prep launch (bucketing, the rows'
 * quantization) serves all n, and Q4_K experts take one grouped launch for all of them. 1..4 products whose experts
 * share type and shape and whose dst share shape and strides. */
MX_API int mx_mul_mat_id_group(mx_backend *be, int n, const mx_tensor *const *as, const mx_tensor *b,
                               const mx_tensor *ids, const mx_tensor *const *dst);
/* MUL_MAT_ID that allocates nothing. No counterpart in speech.cpp or ggml's backend interface: for callers that
 * cannot allocate device memory -- code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * The same products as mx_mul_mat_id, on the same kernels and with the same results, but its scratch (the bucketing
 * tables, the quantized activation rows, the chunk list) lives in a static device array of MX_NOALLOC_SCRATCH_BYTES
 * that each GPU holds from the first mx_backend_init on it until the process ends; the call itself calls no
 * allocator. A call needing more scratch (mx_mul_mat_id_noalloc_bytes; SIZE_MAX for inputs MUL_MAT_ID does not
 * take) fails with MX_UNSUPPORTED. Every call on one GPU shares that GPU's array, which keeps the last call's contents
 * (each call writes everything it reads before reading it): calls that overlap on one GPU -- two streams, two
 * backends -- race. */
#define MX_NOALLOC_SCRATCH_BYTES (16u << 20)
MX_API size_t mx_mul_mat_id_noalloc_bytes(const mx_tensor *as, const mx_tensor *b, const mx_tensor *ids);
MX_API int mx_mul_mat_id_noalloc(mx_backend *be, const mx_tensor *as, const mx_tensor *b, const mx_tensor *ids,
                                 const mx_tensor *dst);
/* ARGMAX: dst[r] = the index of the largest value of row r of src, the first of equal ones, as speech.cpp's ggml
 * fork computes GGML_OP_ARGMAX (src/families/fastconformer/decoder.cpp:56-62 first_argmax states the rule; the
 * decoder's greedy pick, src/common/qwen3-decoder.cpp:426-429,501, reads back these four bytes per row instead of the
 * logits). A NaN never compares greater: at index 0 it keeps index 0, elsewhere it is passed over.
 *   mx_argmax(src [n, R] F32, rows 16-byte aligned) -> dst [R] I32 */
MX_API int mx_argmax(mx_backend *be, const mx_tensor *src, const mx_tensor *dst);
/* ---------------------------------------------------------------------------------------------------------------
 * The decoder layer's other ops, so a layer runs on the device without CPU round trips (src/common/qwen3-decoder.cpp
 * Qwen3Decoder::layers :350-410, outputs :422-438): f32 rows with ne0 contiguous, any row strides.
 *   mx_rms_norm(src [n, ...]) -> dst: ggml_rms_norm (:361,368-369,409,424); w [n] F32 or NULL multiplies the result
 *     as the ggml_mul by the norm weight that follows it does (fused, same roundings).
 *   mx_binary(MX_OP_ADD | MX_OP_MUL, a, b) -> dst: ggml_add (:405,411) / ggml_mul, b repeated over a's shape.
 *   mx_swiglu(a, b) -> dst: ggml_swiglu_split (:411), silu(a) * b.
 *   mx_rope(src [n, heads, rows], pos [rows] I32) -> dst: ggml_rope_ext (:375-376) in GGML_ROPE_TYPE_NEOX with
 *     freq_factors NULL, ext_factor 0, attn_factor 1 (the decoder's arguments); other modes are unsupported.
 *   mx_set_rows(src [n, rows] F32, idx [rows] I32 or I64) -> dst F16 rows: ggml_set_rows (:373,378) writing the new
 *     keys and values into the f16 KV cache at their positions; an index out of range is reported by
 *     mx_backend_synchronize as MX_INVALID and leaves the cache as it was.
 *   mx_flash_attn_ext(q [D, n_q, n_head] F32, k, v [D, n_kv, n_kv_head] F16, mask [n_kv, >= n_q] F16 or NULL)
 *     -> dst [D, n_head, n_q] F32: ggml_flash_attn_ext (:394-397) with max_bias 0 and no softcap; D 64 or 128;
 *     q rounded to fp16 as ggml does, scores and the V sum in fp32 (the GGML_PREC_F32 the decoder sets).
 * ------------------------------------------------------------------------------------------------------------- */
MX_API int mx_rms_norm(mx_backend *be, const mx_tensor *src, const mx_tensor *dst, float eps, const mx_tensor *w);
MX_API int mx_binary(mx_backend *be, int op, const mx_tensor *a, const mx_tensor *b, const mx_tensor *dst);
MX_API int mx_swiglu(mx_backend *be, const mx_tensor *a, const mx_tensor *b, const mx_tensor *dst);
MX_API int mx_supports_rope(const mx_tensor *src, const mx_tensor *pos, const mx_tensor *dst, int n_dims, int mode,
                            float ext_factor, float attn_factor);
MX_API int mx_rope(mx_backend *be, const mx_tensor *src, const mx_tensor *pos, const mx_tensor *dst, int n_dims,
                   int mode, float freq_base, float freq_scale, float ext_factor, float attn_factor);
MX_API int mx_set_rows(mx_backend *be, const mx_tensor *src, const mx_tensor *idx, const mx_tensor *dst);
/* The attention block's per-head work between the q/k/v products and attention (qwen3-decoder.cpp:366-378) in one
 * launch, each value as the separate ops compute it: q_out = rope(mul(rms_norm(q), q_norm)); the keys
 * rope(mul(rms_norm(k), k_norm)) and the values v written into the f16 caches at row pos[r] (set_rows). q, k, v:
 * [128, heads, rows] F32 (views of the products' outputs), q_norm / k_norm [128], pos [rows] I32, caches
 * [heads_kv * 128, capacity] F16. Head size 128, NEOX over all of it, ext_factor 0, attn_factor 1; else
 * MX_UNSUPPORTED and the ops run separately. A position outside the caches is reported by mx_backend_synchronize. */
MX_API int mx_qk_norm_rope_kv(mx_backend *be, const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                              const mx_tensor *q_norm, const mx_tensor *k_norm, const mx_tensor *pos,
                              const mx_tensor *q_out, const mx_tensor *k_cache, const mx_tensor *v_cache, float eps,
                              int n_dims, int mode, float freq_base, float freq_scale, float ext_factor,
                              float attn_factor);
/* One decode row's attention with the q / k norms, RoPE and KV-cache stores before it, in one launch: no single ggml
 * op -- mx_qk_norm_rope_kv(q, k, v, q_norm, k_norm, pos, q_out, k_cache, v_cache, ...) followed by
 * mx_flash_attn_ext(q_out viewed [128, 1, heads], k_view, v_view, mask, dst, scale) (qwen3-decoder.cpp:366-397), for
 * a caller or graph_compute that recognises the pair. Every value as those two compute it; the roped q is not written
 * out. One row (pos holds one position), head size 128, 1, 2 or 4 q heads per kv head, k_view / v_view the caches
 * read from row 0 ([128, n_kv, heads_kv], head stride 256 bytes); anything else returns MX_UNSUPPORTED and the two
 * calls run separately. */
MX_API int mx_attn_decode(mx_backend *be, const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                          const mx_tensor *q_norm, const mx_tensor *k_norm, const mx_tensor *pos,
                          const mx_tensor *k_cache, const mx_tensor *v_cache, const mx_tensor *k_view,
                          const mx_tensor *v_view, const mx_tensor *mask, const mx_tensor *dst, float eps, int n_dims,
                          int mode, float freq_base, float freq_scale, float ext_factor, float attn_factor,
                          float scale);
MX_API int mx_supports_flash_attn_ext(const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                                      const mx_tensor *mask, const mx_tensor *dst, float max_bias,
                                      float logit_softcap);
MX_API int mx_flash_attn_ext(mx_backend *be, const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                             const mx_tensor *mask, const mx_tensor *dst, float scale);

/* A product fused with the ops the decoder puts around it, each computed exactly as the separate op computes it (the
 * same roundings), for a graph_compute that recognises the sequence:
 *   norm_w:   src1 columns become mul(rms_norm(src1, norm_eps), norm_w) first (qwen3-decoder.cpp:361-363 before
 *             q/k/v, :409-411 before gate/up);
 *   glu_b:    src1 columns become swiglu(src1, glu_b) first (ggml_swiglu_split(gate, up) before down, :411);
 *   residual: dst[i] = add(residual[i], product) (:405,411 the residual stream; residual[i] may be dst[i]).
 * n products (1..4) share src1 as in mx_mul_mat_group; quantized weights, at most 8 columns (the mat-vec path);
 * anything else returns MX_UNSUPPORTED and the ops run separately. glu_b has src1's layout, residual[i] dst[i]'s. */
typedef struct mx_fusion {
    const mx_tensor *norm_w;            /* F32 [K] or NULL */
    float norm_eps;
    const mx_tensor *glu_b;             /* F32 like src1, or NULL */
    const mx_tensor *const *residual;   /* n entries (each may be NULL), or NULL */
} mx_fusion;
MX_API int mx_mul_mat_fused(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                            const mx_tensor *const *dst, const mx_fusion *f);

/* Several MUL_MAT nodes that read the same src1 (q/k/v, or gate/up) in one launch, as a backend's graph_compute
 * may fuse them. Each dst[i] = src0[i] x src1, exactly as n separate mx_mul_mat calls compute it. */
MX_API int mx_mul_mat_group(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                            const mx_tensor *const *dst);

/* The activation quantizer the products use, exposed on its own: `nrows` rows of `k` floats (row stride
 * `x_row_stride` bytes, device memory) to ggml blocks of `type` (MX_TYPE_Q8_0, MX_TYPE_Q8_1 or MX_TYPE_Q8_K),
 * row after row, at `out` (device memory). ggml-cpu's src1 conversion (type_traits_cpu[vec_dot_type].from_float). */
MX_API int mx_quantize_act(mx_backend *be, int type, int rounding, const float *x, int64_t k, int64_t nrows,
                           size_t x_row_stride, void *out);

/* ---------------------------------------------------------------------------------------------------------------
 * Measurement: no counterpart in speech.cpp or ggml. Peak micro-benchmarks launched on the backend's stream, for the
 * practical ceilings the products' roofline fractions are read beside (the caller times them with mx_event_*).
 *   mx_peak_read: one streaming read of `bytes` at `src` (device memory, 16-byte aligned, a multiple of 16 bytes) by
 *                 `workgroups` (1..65536) of 256 threads, `loads` (1, 2, 4, 8 or 16) 16-byte loads in flight per
 *                 thread, nontemporal when `nontemporal` is set; nothing is written.
 *   mx_peak_mfma: `workgroups` (1..65536) of four waves, each issuing `iters` (1..1e7) rounds of eight independent
 *                 MFMAs on register operands: kind 0 v_mfma_i32_32x32x32_i8 (65,536 int8 ops each), kind 1
 *                 v_mfma_f32_32x32x16_f16 (32,768 flops each).
 * ------------------------------------------------------------------------------------------------------------- */
MX_API int mx_peak_read(mx_backend *be, const void *src, size_t bytes, int workgroups, int loads, int nontemporal);
MX_API int mx_peak_mfma(mx_backend *be, int kind, int workgroups, int iters);

/* ---------------------------------------------------------------------------------------------------------------
 * Replay of a fixed sequence of ops with one launch (the role CUDA graphs play inside ggml-cuda's graph_compute;
 * the kept decode-step graph of src/common/qwen3-decoder.cpp:187-208,462-490). Between mx_graph_begin and
 * mx_graph_end the ops are recorded, not run; mx_graph_launch replays them on the backend's stream. Record after one
 * eager run of the same ops so every scratch buffer has its final size. A recorded graph holds the address of the
 * backend's scratch: once a later op grows the scratch (and frees the old one), mx_graph_launch refuses every graph
 * recorded before that with MX_FAILED, and the caller records it again. A graph launches only on the backend that
 * recorded it (MX_INVALID otherwise).
 * ------------------------------------------------------------------------------------------------------------- */
MX_API int mx_graph_begin(mx_backend *be);
MX_API int mx_graph_end(mx_backend *be, mx_graph **graph);
MX_API int mx_graph_launch(mx_backend *be, mx_graph *graph);
/* The number of nodes (kernel launches) a recorded graph holds; 0 for a null graph. */
MX_API size_t mx_graph_nodes(const mx_graph *graph);
/* Waits for the graph's replays on its backend's stream, then frees it; free graphs before their backend. */
MX_API void mx_graph_free(mx_graph *graph);

/* ---------------------------------------------------------------------------------------------------------------
 * Events on the backend's stream: ggml_backend_device_i.{event_new, event_free, event_synchronize} and
 * ggml_backend_i.event_record, plus the elapsed time between two recorded events (for timing on that stream).
 * ------------------------------------------------------------------------------------------------------------- */
MX_API mx_event *mx_event_new(mx_backend *be);
MX_API int mx_event_record(mx_backend *be, mx_event *ev);
MX_API int mx_event_synchronize(mx_event *ev);
MX_API int mx_event_elapsed_ms(mx_event *start, mx_event *end, float *ms);
MX_API void mx_event_free(mx_event *ev);

/* ---------------------------------------------------------------------------------------------------------------
 * Host-side weight quantization: ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, imatrix = NULL), the
 * `speech quantize` path (src/common/quantize.cpp:164-182). ggml block bytes out; returns bytes written, 0 on error.
 * ------------------------------------------------------------------------------------------------------------- */
MX_API size_t mx_quantize_chunk(int type, const float *src, void *dst, int64_t start, int64_t nrows,
                                int64_t n_per_row);
/* Seeded N(mean, stddev) rows (splitmix64 -> xoshiro256** -> Box-Muller in double), row r from its own stream, and
 * the same rows quantized straight to `type` with `nthreads` threads: synthetic weights without a float copy. */
MX_API void mx_fill_normal_rows(uint64_t seed, int64_t row0, int64_t nrows, int64_t n_per_row, float mean,
                                float stddev, float *out);
MX_API size_t mx_quantize_normal_rows(int type, uint64_t seed, int64_t row0, int64_t nrows, int64_t n_per_row,
                                      float mean, float stddev, void *dst, int nthreads);

/* ---------------------------------------------------------------------------------------------------------------
 * GGUF model files straight into the buffer type, for a caller without a ggml context: the parse ggml's
 * gguf_init_from_file(no_alloc = true) gives speech.cpp's ModelFile::open (src/common/model-file.cpp:35-47,136-160),
 * and ModelFile::load (src/common/model-file.cpp:251-268), which reads each tensor from the file in 16 MB pieces and
 * sets each piece on the device at its offset (ggml_backend_tensor_set; here mx_tensor_set). GGUF versions 2 and 3.
 * Every ggml type a speech.cpp file stores (src/common/storage.cpp:30-89: F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, including
 * the Q8_0 / F16 fallbacks inside K-quant files) is read; other known ggml types are held as plain bytes.
 * mx_gguf_open returns NULL on a file it cannot open or parse (mx_last_error says which); strings returned point into
 * the mx_gguf and live until mx_gguf_close. Value types are GGUF's: 0 u8 .. 12 f64, 8 string, 9 array.
 * ------------------------------------------------------------------------------------------------------------- */
typedef struct mx_gguf mx_gguf;
typedef struct mx_gguf_tensor_info {
    const char *name;
    int32_t type;      /* ggml_type */
    int32_t n_dims;
    int64_t ne[4];     /* ggml order; axes past n_dims are 1 */
    uint64_t offset;   /* from the start of the data section (gguf_get_tensor_offset) */
    uint64_t nbytes;   /* ggml_nbytes of the contiguous tensor */
} mx_gguf_tensor_info;

MX_API mx_gguf *mx_gguf_open(const char *path);
MX_API void mx_gguf_close(mx_gguf *f);
MX_API uint64_t mx_gguf_data_offset(const mx_gguf *f);            /* gguf_get_data_offset */
MX_API int64_t mx_gguf_n_tensors(const mx_gguf *f);               /* gguf_get_n_tensors */
MX_API int mx_gguf_get_tensor(const mx_gguf *f, int64_t i, mx_gguf_tensor_info *out);
MX_API int64_t mx_gguf_find_tensor(const mx_gguf *f, const char *name);  /* gguf_find_tensor; -1 if absent */
MX_API int64_t mx_gguf_n_keys(const mx_gguf *f);                  /* gguf_get_n_kv */
MX_API const char *mx_gguf_key(const mx_gguf *f, int64_t id);     /* gguf_get_key */
MX_API int64_t mx_gguf_find_key(const mx_gguf *f, const char *key);      /* gguf_find_key; -1 if absent */
MX_API int mx_gguf_key_type(const mx_gguf *f, int64_t id);        /* gguf_get_kv_type; -1 if no such key */
MX_API int mx_gguf_get_str(const mx_gguf *f, int64_t id, const char **out, size_t *len);
MX_API int mx_gguf_get_int(const mx_gguf *f, int64_t id, int64_t *out);   /* any integer or bool value */
MX_API int mx_gguf_get_float(const mx_gguf *f, int64_t id, double *out);  /* f32 or f64 */
MX_API int mx_gguf_get_arr(const mx_gguf *f, int64_t id, int *elem_type, uint64_t *n, const void **data);
MX_API int mx_gguf_get_arr_str(const mx_gguf *f, int64_t id, uint64_t i, const char **out, size_t *len);
/* Reads tensor i into dst (same type and ne; allocated with mx_tensor_alloc_size) in 16 MB pieces. */
MX_API int mx_gguf_load_tensor(mx_backend *be, const mx_gguf *f, int64_t i, const mx_tensor *dst);

#ifdef __cplusplus
}
#endif
#endif
