// A declaration subset of ggml's public header, ggml.h: the types, constants and functions the MI355X backend and its
// test host use, and nothing else. ggml itself is not part of this repository (speech.cpp builds it from the
// nyosegawa/ggml fork of ggml v0.27.0, `.gitmodules:1-4`, a submodule absent from the reference snapshot), so these
// declarations restate ggml's interface as the backend was written against it: ggml's names, its struct layout for
// ggml_tensor, and its numbering of ggml_type (fixed by the GGUF format) and ggml_op.
//
// The integration build compiles the backend against the fork's own headers instead (ggml/include), where the
// static_asserts in ggml-mi355x.cpp check the fork's ggml_tensor and interface tables against the layout the backend
// was written for. ggml_op numbering moves between ggml versions as ops are added; the backend never trusts it: its
// registry compares ggml_op_name / ggml_type_name / ggml_glu_op_name of every value it uses with what the linked ggml
// reports, and a tensor it creates through ggml_new_tensor_2d with the fields it reads, before it registers a device.
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifndef GGML_API
#define GGML_API __attribute__((visibility("default")))
#endif

#define GGML_MAX_DIMS 4
#define GGML_MAX_PARAMS 2048
#define GGML_MAX_SRC 10
#define GGML_MAX_NAME 64
#define GGML_MAX_OP_PARAMS 64
#define GGML_MEM_ALIGN 16

#define GGML_ROPE_TYPE_NEOX 2

#ifdef __cplusplus
extern "C" {
#endif

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED = -1,
    GGML_STATUS_SUCCESS = 0,
    GGML_STATUS_ABORTED = 1,
};

// The values GGUF files store (ggml_type is part of the file format): only those the backend names.
enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_Q8_K = 15,
    GGML_TYPE_I32 = 26,
    GGML_TYPE_I64 = 27,
};

enum ggml_prec {
    GGML_PREC_DEFAULT = 0,
    GGML_PREC_F32 = 10,
};

// ggml's op numbering (the order of ggml.h's enum, ADD_ID and GLU included). Checked at run time by the backend's
// registry against ggml_op_name of the linked ggml.
enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_DUP,
    GGML_OP_ADD,
    GGML_OP_ADD_ID,
    GGML_OP_ADD1,
    GGML_OP_ACC,
    GGML_OP_SUB,
    GGML_OP_MUL,
    GGML_OP_DIV,
    GGML_OP_SQR,
    GGML_OP_SQRT,
    GGML_OP_LOG,
    GGML_OP_SIN,
    GGML_OP_COS,
    GGML_OP_SUM,
    GGML_OP_SUM_ROWS,
    GGML_OP_MEAN,
    GGML_OP_ARGMAX,
    GGML_OP_COUNT_EQUAL,
    GGML_OP_REPEAT,
    GGML_OP_REPEAT_BACK,
    GGML_OP_CONCAT,
    GGML_OP_SILU_BACK,
    GGML_OP_NORM,
    GGML_OP_RMS_NORM,
    GGML_OP_RMS_NORM_BACK,
    GGML_OP_GROUP_NORM,
    GGML_OP_L2_NORM,
    GGML_OP_MUL_MAT,
    GGML_OP_MUL_MAT_ID,
    GGML_OP_OUT_PROD,
    GGML_OP_SCALE,
    GGML_OP_SET,
    GGML_OP_CPY,
    GGML_OP_CONT,
    GGML_OP_RESHAPE,
    GGML_OP_VIEW,
    GGML_OP_PERMUTE,
    GGML_OP_TRANSPOSE,
    GGML_OP_GET_ROWS,
    GGML_OP_GET_ROWS_BACK,
    GGML_OP_SET_ROWS,
    GGML_OP_DIAG,
    GGML_OP_DIAG_MASK_INF,
    GGML_OP_DIAG_MASK_ZERO,
    GGML_OP_SOFT_MAX,
    GGML_OP_SOFT_MAX_BACK,
    GGML_OP_ROPE,
    GGML_OP_ROPE_BACK,
    GGML_OP_CLAMP,
    GGML_OP_CONV_TRANSPOSE_1D,
    GGML_OP_IM2COL,
    GGML_OP_IM2COL_BACK,
    GGML_OP_IM2COL_3D,
    GGML_OP_CONV_2D,
    GGML_OP_CONV_3D,
    GGML_OP_CONV_2D_DW,
    GGML_OP_CONV_TRANSPOSE_2D,
    GGML_OP_POOL_1D,
    GGML_OP_POOL_2D,
    GGML_OP_POOL_2D_BACK,
    GGML_OP_UPSCALE,
    GGML_OP_PAD,
    GGML_OP_PAD_REFLECT_1D,
    GGML_OP_ROLL,
    GGML_OP_ARANGE,
    GGML_OP_TIMESTEP_EMBEDDING,
    GGML_OP_ARGSORT,
    GGML_OP_LEAKY_RELU,
    GGML_OP_FLASH_ATTN_EXT,
    GGML_OP_FLASH_ATTN_BACK,
    GGML_OP_SSM_CONV,
    GGML_OP_SSM_SCAN,
    GGML_OP_WIN_PART,
    GGML_OP_WIN_UNPART,
    GGML_OP_GET_REL_POS,
    GGML_OP_ADD_REL_POS,
    GGML_OP_RWKV_WKV6,
    GGML_OP_GATED_LINEAR_ATTN,
    GGML_OP_RWKV_WKV7,
    GGML_OP_UNARY,
    GGML_OP_MAP_CUSTOM1,
    GGML_OP_MAP_CUSTOM2,
    GGML_OP_MAP_CUSTOM3,
    GGML_OP_CUSTOM,
    GGML_OP_CROSS_ENTROPY_LOSS,
    GGML_OP_CROSS_ENTROPY_LOSS_BACK,
    GGML_OP_OPT_STEP_ADAMW,
    GGML_OP_OPT_STEP_SGD,
    GGML_OP_GLU,
    GGML_OP_COUNT,
};

enum ggml_glu_op {
    GGML_GLU_OP_REGLU,
    GGML_GLU_OP_GEGLU,
    GGML_GLU_OP_SWIGLU,
    GGML_GLU_OP_SWIGLU_OAI,
    GGML_GLU_OP_GEGLU_ERF,
    GGML_GLU_OP_GEGLU_QUICK,
    GGML_GLU_OP_COUNT,
};

enum ggml_log_level {
    GGML_LOG_LEVEL_NONE = 0,
    GGML_LOG_LEVEL_DEBUG = 1,
    GGML_LOG_LEVEL_INFO = 2,
    GGML_LOG_LEVEL_WARN = 3,
    GGML_LOG_LEVEL_ERROR = 4,
    GGML_LOG_LEVEL_CONT = 5,
};

enum ggml_tensor_flag {
    GGML_TENSOR_FLAG_INPUT = 1,
    GGML_TENSOR_FLAG_OUTPUT = 2,
    GGML_TENSOR_FLAG_PARAM = 4,
    GGML_TENSOR_FLAG_LOSS = 8,
};

struct ggml_backend_buffer;
struct ggml_context;
struct ggml_cgraph;

// n-dimensional tensor: ne elements and nb bytes per dimension; a view reads view_src's memory at view_offs.
struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer *buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t nb[GGML_MAX_DIMS];
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor *src[GGML_MAX_SRC];
    struct ggml_tensor *view_src;
    size_t view_offs;
    void *data;
    char name[GGML_MAX_NAME];
    void *extra;
    char padding[8];
};

struct ggml_init_params {
    size_t mem_size;
    void *mem_buffer;
    bool no_alloc;
};

typedef uint8_t ggml_guid[16];
typedef ggml_guid *ggml_guid_t;

// ----------------------------------------------------------------------------------------------- type traits
GGML_API int64_t ggml_blck_size(enum ggml_type type);
GGML_API size_t ggml_type_size(enum ggml_type type);
GGML_API size_t ggml_row_size(enum ggml_type type, int64_t ne);
GGML_API const char *ggml_type_name(enum ggml_type type);
GGML_API bool ggml_is_quantized(enum ggml_type type);

GGML_API const char *ggml_op_name(enum ggml_op op);
GGML_API const char *ggml_op_desc(const struct ggml_tensor *t);
GGML_API const char *ggml_glu_op_name(enum ggml_glu_op op);
GGML_API enum ggml_glu_op ggml_get_glu_op(const struct ggml_tensor *tensor);

// ----------------------------------------------------------------------------------------------- tensors
GGML_API int64_t ggml_nelements(const struct ggml_tensor *tensor);
GGML_API int64_t ggml_nrows(const struct ggml_tensor *tensor);
GGML_API size_t ggml_nbytes(const struct ggml_tensor *tensor);
GGML_API bool ggml_is_empty(const struct ggml_tensor *tensor);
GGML_API bool ggml_is_contiguous(const struct ggml_tensor *tensor);

GGML_API struct ggml_context *ggml_init(struct ggml_init_params params);
GGML_API void ggml_free(struct ggml_context *ctx);

GGML_API struct ggml_tensor *ggml_new_tensor_1d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0);
GGML_API struct ggml_tensor *ggml_new_tensor_2d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                                int64_t ne1);
GGML_API struct ggml_tensor *ggml_new_tensor_3d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                                int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor *ggml_set_name(struct ggml_tensor *tensor, const char *name);
GGML_API const char *ggml_get_name(const struct ggml_tensor *tensor);
GGML_API void ggml_set_input(struct ggml_tensor *tensor);
GGML_API void ggml_set_output(struct ggml_tensor *tensor);

// ----------------------------------------------------------------------------------------------- operations
GGML_API struct ggml_tensor *ggml_add(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_mul(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_argmax(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API struct ggml_tensor *ggml_rms_norm(struct ggml_context *ctx, struct ggml_tensor *a, float eps);
GGML_API struct ggml_tensor *ggml_mul_mat(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_mul_mat_id(struct ggml_context *ctx, struct ggml_tensor *as, struct ggml_tensor *b,
                                             struct ggml_tensor *ids);
GGML_API struct ggml_tensor *ggml_reshape_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                             int64_t ne1);
GGML_API struct ggml_tensor *ggml_reshape_3d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                             int64_t ne2);
GGML_API struct ggml_tensor *ggml_view_3d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                          int64_t ne2, size_t nb1, size_t nb2, size_t offset);
GGML_API struct ggml_tensor *ggml_permute(struct ggml_context *ctx, struct ggml_tensor *a, int axis0, int axis1,
                                          int axis2, int axis3);
GGML_API struct ggml_tensor *ggml_get_rows(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_set_rows(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b,
                                           struct ggml_tensor *c);
GGML_API struct ggml_tensor *ggml_rope_ext(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b,
                                           struct ggml_tensor *c, int n_dims, int mode, int n_ctx_orig,
                                           float freq_base, float freq_scale, float ext_factor, float attn_factor,
                                           float beta_fast, float beta_slow);
GGML_API struct ggml_tensor *ggml_flash_attn_ext(struct ggml_context *ctx, struct ggml_tensor *q,
                                                 struct ggml_tensor *k, struct ggml_tensor *v, struct ggml_tensor *mask,
                                                 float scale, float max_bias, float logit_softcap);
GGML_API void ggml_flash_attn_ext_set_prec(struct ggml_tensor *a, enum ggml_prec prec);
GGML_API struct ggml_tensor *ggml_swiglu_split(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);

// ----------------------------------------------------------------------------------------------- graphs
GGML_API struct ggml_cgraph *ggml_new_graph(struct ggml_context *ctx);
GGML_API struct ggml_cgraph *ggml_new_graph_custom(struct ggml_context *ctx, size_t size, bool grads);
GGML_API void ggml_build_forward_expand(struct ggml_cgraph *cgraph, struct ggml_tensor *tensor);
GGML_API int ggml_graph_n_nodes(struct ggml_cgraph *cgraph);
GGML_API struct ggml_tensor *ggml_graph_node(struct ggml_cgraph *cgraph, int i);

#ifdef __cplusplus
}
#endif
