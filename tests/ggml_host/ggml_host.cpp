// A stand-in for ggml's core and its backend dispatch, to drive the MI355X ggml backend (libggml-mi355x.so) in tests
// the way speech.cpp drives a backend: registry -> device -> buffer type -> buffers -> tensors placed and uploaded ->
// graphs built with ggml's op constructors -> graph_compute.
//
// ggml is not part of this repository, nor of the reference snapshot (speech.cpp's ggml is an absent submodule), so
// this file restates the part of ggml's public C API that speech.cpp's graph code and a backend call, from ggml's
// documented semantics: tensor shapes and byte strides, views (view_src / view_offs), the op parameters a backend
// reads (ggml.c's op constructors), the depth-first order in which ggml_build_forward_expand lists nodes, and
// ggml-backend.cpp's dispatch into a backend's interface tables. It computes nothing: every node is the backend's.
// It is test infrastructure only; the product links the real ggml.
#include <cassert>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-impl.h"

#define HOST_CHECK(c)                                                                          \
    do {                                                                                       \
        if (!(c)) {                                                                            \
            std::fprintf(stderr, "ggml host: %s:%d: check failed: %s\n", __FILE__, __LINE__, #c); \
            std::abort();                                                                      \
        }                                                                                      \
    } while (0)

struct ggml_context {
    bool no_alloc = true;
    std::vector<ggml_tensor *> tensors;
    std::vector<void *> host_data;
    std::vector<ggml_cgraph *> graphs;
};


namespace {

struct Traits {
    const char *name;
    int64_t blck;
    size_t size;
    bool quantized;
};

Traits traits(ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return {"f32", 1, 4, false};
        case GGML_TYPE_F16: return {"f16", 1, 2, false};
        case GGML_TYPE_Q8_0: return {"q8_0", 32, 34, true};
        case GGML_TYPE_Q4_K: return {"q4_K", 256, 144, true};
        case GGML_TYPE_Q5_K: return {"q5_K", 256, 176, true};
        case GGML_TYPE_Q6_K: return {"q6_K", 256, 210, true};
        case GGML_TYPE_Q8_K: return {"q8_K", 256, 292, true};
        case GGML_TYPE_I32: return {"i32", 1, 4, false};
        case GGML_TYPE_I64: return {"i64", 1, 8, false};
    }
    return {nullptr, 0, 0, false};
}

const char *const kOpNames[GGML_OP_COUNT] = {
    "NONE", "DUP", "ADD", "ADD_ID", "ADD1", "ACC", "SUB", "MUL", "DIV", "SQR", "SQRT", "LOG", "SIN", "COS", "SUM",
    "SUM_ROWS", "MEAN", "ARGMAX", "COUNT_EQUAL", "REPEAT", "REPEAT_BACK", "CONCAT", "SILU_BACK", "NORM", "RMS_NORM",
    "RMS_NORM_BACK", "GROUP_NORM", "L2_NORM", "MUL_MAT", "MUL_MAT_ID", "OUT_PROD", "SCALE", "SET", "CPY", "CONT",
    "RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE", "GET_ROWS", "GET_ROWS_BACK", "SET_ROWS", "DIAG", "DIAG_MASK_INF",
    "DIAG_MASK_ZERO", "SOFT_MAX", "SOFT_MAX_BACK", "ROPE", "ROPE_BACK", "CLAMP", "CONV_TRANSPOSE_1D", "IM2COL",
    "IM2COL_BACK", "IM2COL_3D", "CONV_2D", "CONV_3D", "CONV_2D_DW", "CONV_TRANSPOSE_2D", "POOL_1D", "POOL_2D",
    "POOL_2D_BACK", "UPSCALE", "PAD", "PAD_REFLECT_1D", "ROLL", "ARANGE", "TIMESTEP_EMBEDDING", "ARGSORT",
    "LEAKY_RELU", "FLASH_ATTN_EXT", "FLASH_ATTN_BACK", "SSM_CONV", "SSM_SCAN", "WIN_PART", "WIN_UNPART",
    "GET_REL_POS", "ADD_REL_POS", "RWKV_WKV6", "GATED_LINEAR_ATTN", "RWKV_WKV7", "UNARY", "MAP_CUSTOM1",
    "MAP_CUSTOM2", "MAP_CUSTOM3", "CUSTOM", "CROSS_ENTROPY_LOSS", "CROSS_ENTROPY_LOSS_BACK", "OPT_STEP_ADAMW",
    "OPT_STEP_SGD", "GLU"};

const char *const kGluNames[GGML_GLU_OP_COUNT] = {"REGLU", "GEGLU", "SWIGLU", "SWIGLU_OAI", "GEGLU_ERF",
                                                  "GEGLU_QUICK"};

std::string g_last_log;

// ggml_new_tensor_impl: ne given, nb contiguous for the type; a view of a view resolves to the base tensor.
ggml_tensor *new_tensor(ggml_context *ctx, ggml_type type, int n_dims, const int64_t *ne, ggml_tensor *view_src,
                        size_t view_offs) {
    HOST_CHECK(traits(type).name && n_dims >= 1 && n_dims <= GGML_MAX_DIMS);
    if (view_src && view_src->view_src) {
        view_offs += view_src->view_offs;
        view_src = view_src->view_src;
    }
    auto *t = new ggml_tensor;
    std::memset(t, 0, sizeof *t);
    t->type = type;
    for (int i = 0; i < GGML_MAX_DIMS; i++) t->ne[i] = i < n_dims ? ne[i] : 1;
    HOST_CHECK(t->ne[0] % traits(type).blck == 0);
    t->nb[0] = traits(type).size;
    t->nb[1] = t->nb[0] * (size_t)(t->ne[0] / traits(type).blck);
    for (int i = 2; i < GGML_MAX_DIMS; i++) t->nb[i] = t->nb[i - 1] * (size_t)t->ne[i - 1];
    t->view_src = view_src;
    t->view_offs = view_offs;
    if (view_src) {
        if (view_src->data) t->data = (char *)view_src->data + view_offs;
    } else if (!ctx->no_alloc) {
        void *p = std::calloc(1, ggml_nbytes(t) + 1);
        ctx->host_data.push_back(p);
        t->data = p;
    }
    ctx->tensors.push_back(t);
    return t;
}

ggml_tensor *dup_tensor(ggml_context *ctx, const ggml_tensor *a) { return new_tensor(ctx, a->type, 4, a->ne, nullptr, 0); }

ggml_tensor *view_tensor(ggml_context *ctx, ggml_tensor *a) {
    ggml_tensor *t = new_tensor(ctx, a->type, 4, a->ne, a, 0);
    for (int i = 0; i < GGML_MAX_DIMS; i++) t->nb[i] = a->nb[i];
    return t;
}

void set_f32(ggml_tensor *t, int i, float v) { std::memcpy(&t->op_params[i], &v, sizeof v); }

// ggml_visit_parents: depth-first over the sources, each tensor listed once (a node or a leaf) after its sources; a
// tensor's use count goes up once per node that names it as a source, over the whole graph.
void visit(ggml_cgraph *g, ggml_tensor *t) {
    const size_t slot = ggml_hash_find(&g->visited_hash_set, t);
    HOST_CHECK(slot != GGML_HASHSET_FULL);
    if (ggml_bitset_get(g->visited_hash_set.used, slot)) return;
    g->visited_hash_set.keys[slot] = t;
    g->visited_hash_set.used[slot >> 5] |= 1u << (slot & 31);
    g->use_counts[slot] = 0;
    for (int s = 0; s < GGML_MAX_SRC; s++) {
        if (!t->src[s]) continue;
        visit(g, t->src[s]);
        g->use_counts[ggml_hash_find(&g->visited_hash_set, t->src[s])]++;
    }
    if (t->op == GGML_OP_NONE && !(t->flags & GGML_TENSOR_FLAG_PARAM)) {
        HOST_CHECK(g->n_leafs < g->size);
        g->leafs[g->n_leafs++] = t;
    } else {
        HOST_CHECK(g->n_nodes < g->size);
        g->nodes[g->n_nodes++] = t;
    }
}

void free_graph(ggml_cgraph *g) {
    delete[] g->nodes;
    delete[] g->leafs;
    delete[] g->use_counts;
    delete[] g->visited_hash_set.used;
    delete[] g->visited_hash_set.keys;
    delete g;
}

ggml_backend_buffer_t buffer_of(const ggml_tensor *t) { return t->view_src ? t->view_src->buffer : t->buffer; }

}  // namespace

extern "C" {

// ------------------------------------------------------------------------------------------------- core
int64_t ggml_blck_size(ggml_type type) { return traits(type).blck; }
size_t ggml_type_size(ggml_type type) { return traits(type).size; }
size_t ggml_row_size(ggml_type type, int64_t ne) { return traits(type).size * (size_t)ne / (size_t)traits(type).blck; }
const char *ggml_type_name(ggml_type type) { return traits(type).name; }
bool ggml_is_quantized(ggml_type type) { return traits(type).quantized; }
#ifdef GGML_HOST_WITHOUT_ADD_ID
// A ggml from before ADD_ID joined the op list: every later op is numbered one lower than in the headers.
const char *ggml_op_name(ggml_op op) {
    if (op < 0 || op >= GGML_OP_COUNT - 1) return nullptr;
    return kOpNames[op < GGML_OP_ADD_ID ? op : op + 1];
}
#else
const char *ggml_op_name(ggml_op op) { return op >= 0 && op < GGML_OP_COUNT ? kOpNames[op] : nullptr; }
#endif
const char *ggml_glu_op_name(ggml_glu_op op) { return op >= 0 && op < GGML_GLU_OP_COUNT ? kGluNames[op] : nullptr; }
ggml_glu_op ggml_get_glu_op(const ggml_tensor *t) { return (ggml_glu_op)t->op_params[0]; }
const char *ggml_op_desc(const ggml_tensor *t) {
    return t->op == GGML_OP_GLU ? ggml_glu_op_name(ggml_get_glu_op(t)) : ggml_op_name(t->op);
}

int64_t ggml_nelements(const ggml_tensor *t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t ggml_nrows(const ggml_tensor *t) { return t->ne[1] * t->ne[2] * t->ne[3]; }
bool ggml_is_empty(const ggml_tensor *t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] == 0) return true;
    return false;
}
size_t ggml_nbytes(const ggml_tensor *t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] <= 0) return 0;
    const int64_t blck = traits(t->type).blck;
    size_t n;
    if (blck == 1) {
        n = traits(t->type).size;
        for (int i = 0; i < GGML_MAX_DIMS; i++) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    } else {
        n = (size_t)t->ne[0] * t->nb[0] / (size_t)blck;
        for (int i = 1; i < GGML_MAX_DIMS; i++) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    }
    return n;
}
bool ggml_is_contiguous(const ggml_tensor *t) {
    size_t next = traits(t->type).size;
    if (t->nb[0] != next) return false;
    next = t->nb[0] * (size_t)(t->ne[0] / traits(t->type).blck);
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] != 1 && t->nb[i] != next) return false;
        next *= (size_t)t->ne[i];
    }
    return true;
}

ggml_context *ggml_init(ggml_init_params params) {
    auto *ctx = new ggml_context;
    ctx->no_alloc = params.no_alloc;
    return ctx;
}

void ggml_free(ggml_context *ctx) {
    if (!ctx) return;
    for (ggml_tensor *t : ctx->tensors) delete t;
    for (void *p : ctx->host_data) std::free(p);
    for (ggml_cgraph *g : ctx->graphs) free_graph(g);
    delete ctx;
}

ggml_tensor *ggml_new_tensor_1d(ggml_context *ctx, ggml_type type, int64_t ne0) {
    return new_tensor(ctx, type, 1, &ne0, nullptr, 0);
}
ggml_tensor *ggml_new_tensor_2d(ggml_context *ctx, ggml_type type, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return new_tensor(ctx, type, 2, ne, nullptr, 0);
}
ggml_tensor *ggml_new_tensor_3d(ggml_context *ctx, ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return new_tensor(ctx, type, 3, ne, nullptr, 0);
}
ggml_tensor *ggml_set_name(ggml_tensor *t, const char *name) {
    std::snprintf(t->name, sizeof t->name, "%s", name);
    return t;
}
const char *ggml_get_name(const ggml_tensor *t) { return t->name; }
void ggml_set_input(ggml_tensor *t) { t->flags |= GGML_TENSOR_FLAG_INPUT; }
void ggml_set_output(ggml_tensor *t) { t->flags |= GGML_TENSOR_FLAG_OUTPUT; }

// ------------------------------------------------------------------------------------------------- ops
static ggml_tensor *binary(ggml_context *ctx, ggml_op op, ggml_tensor *a, ggml_tensor *b) {
    for (int i = 0; i < GGML_MAX_DIMS; i++) HOST_CHECK(a->ne[i] % b->ne[i] == 0);  // b repeats over a
    ggml_tensor *r = dup_tensor(ctx, a);
    r->op = op;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}
ggml_tensor *ggml_add(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b) { return binary(ctx, GGML_OP_ADD, a, b); }
ggml_tensor *ggml_mul(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b) { return binary(ctx, GGML_OP_MUL, a, b); }

ggml_tensor *ggml_argmax(ggml_context *ctx, ggml_tensor *a) {
    HOST_CHECK(a->ne[2] == 1 && a->ne[3] == 1);
    ggml_tensor *r = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, a->ne[1]);
    r->op = GGML_OP_ARGMAX;
    r->src[0] = a;
    return r;
}

ggml_tensor *ggml_rms_norm(ggml_context *ctx, ggml_tensor *a, float eps) {
    ggml_tensor *r = dup_tensor(ctx, a);
    set_f32(r, 0, eps);
    r->op = GGML_OP_RMS_NORM;
    r->src[0] = a;
    return r;
}

ggml_tensor *ggml_mul_mat(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b) {
    HOST_CHECK(a->ne[0] == b->ne[0] && b->ne[2] % a->ne[2] == 0 && b->ne[3] % a->ne[3] == 0);
    const int64_t ne[4] = {a->ne[1], b->ne[1], b->ne[2], b->ne[3]};
    ggml_tensor *r = new_tensor(ctx, GGML_TYPE_F32, 4, ne, nullptr, 0);
    r->op = GGML_OP_MUL_MAT;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

ggml_tensor *ggml_mul_mat_id(ggml_context *ctx, ggml_tensor *as, ggml_tensor *b, ggml_tensor *ids) {
    HOST_CHECK(ids->type == GGML_TYPE_I32 && as->ne[3] == 1 && b->ne[3] == 1 && ids->ne[2] == 1 && ids->ne[3] == 1);
    HOST_CHECK(ids->ne[1] == b->ne[2] && as->ne[0] == b->ne[0] && ids->ne[0] % b->ne[1] == 0);
    const int64_t ne[4] = {as->ne[1], ids->ne[0], b->ne[2], 1};
    ggml_tensor *r = new_tensor(ctx, GGML_TYPE_F32, 4, ne, nullptr, 0);
    r->op = GGML_OP_MUL_MAT_ID;
    r->src[0] = as;
    r->src[1] = b;
    r->src[2] = ids;
    return r;
}

static ggml_tensor *reshape(ggml_context *ctx, ggml_tensor *a, int n, const int64_t *ne) {
    HOST_CHECK(ggml_is_contiguous(a));
    int64_t total = 1;
    for (int i = 0; i < n; i++) total *= ne[i];
    HOST_CHECK(total == ggml_nelements(a));
    ggml_tensor *r = new_tensor(ctx, a->type, n, ne, a, 0);
    r->op = GGML_OP_RESHAPE;
    r->src[0] = a;
    return r;
}
ggml_tensor *ggml_reshape_2d(ggml_context *ctx, ggml_tensor *a, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return reshape(ctx, a, 2, ne);
}
ggml_tensor *ggml_reshape_3d(ggml_context *ctx, ggml_tensor *a, int64_t ne0, int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return reshape(ctx, a, 3, ne);
}

ggml_tensor *ggml_view_3d(ggml_context *ctx, ggml_tensor *a, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1,
                          size_t nb2, size_t offset) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    ggml_tensor *r = new_tensor(ctx, a->type, 3, ne, a, offset);
    r->nb[1] = nb1;
    r->nb[2] = nb2;
    r->nb[3] = nb2 * (size_t)ne2;
    std::memcpy(r->op_params, &offset, sizeof offset);
    r->op = GGML_OP_VIEW;
    r->src[0] = a;
    return r;
}

ggml_tensor *ggml_permute(ggml_context *ctx, ggml_tensor *a, int axis0, int axis1, int axis2, int axis3) {
    const int ax[4] = {axis0, axis1, axis2, axis3};
    ggml_tensor *r = view_tensor(ctx, a);
    for (int i = 0; i < 4; i++) {
        HOST_CHECK(ax[i] >= 0 && ax[i] < 4);
        r->ne[ax[i]] = a->ne[i];
        r->nb[ax[i]] = a->nb[i];
    }
    r->op = GGML_OP_PERMUTE;
    r->src[0] = a;
    for (int i = 0; i < 4; i++) r->op_params[i] = ax[i];
    return r;
}

ggml_tensor *ggml_get_rows(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b) {
    HOST_CHECK(b->type == GGML_TYPE_I32 && a->ne[2] == b->ne[1]);
    const int64_t ne[4] = {a->ne[0], b->ne[0], b->ne[1], b->ne[2]};
    ggml_tensor *r = new_tensor(ctx, a->type == GGML_TYPE_I32 ? GGML_TYPE_I32 : GGML_TYPE_F32, 4, ne, nullptr, 0);
    r->op = GGML_OP_GET_ROWS;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

ggml_tensor *ggml_set_rows(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b, ggml_tensor *c) {
    HOST_CHECK(a->ne[0] == b->ne[0] && b->ne[1] == c->ne[0] && (c->type == GGML_TYPE_I64 || c->type == GGML_TYPE_I32));
    ggml_tensor *r = view_tensor(ctx, a);
    r->op = GGML_OP_SET_ROWS;
    r->src[0] = b;
    r->src[1] = c;
    return r;
}

ggml_tensor *ggml_rope_ext(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b, ggml_tensor *c, int n_dims, int mode,
                           int n_ctx_orig, float freq_base, float freq_scale, float ext_factor, float attn_factor,
                           float beta_fast, float beta_slow) {
    HOST_CHECK(b->type == GGML_TYPE_I32 && b->ne[0] == a->ne[2]);
    ggml_tensor *r = dup_tensor(ctx, a);
    r->op_params[0] = 0;
    r->op_params[1] = n_dims;
    r->op_params[2] = mode;
    r->op_params[3] = 0;
    r->op_params[4] = n_ctx_orig;
    set_f32(r, 5, freq_base);
    set_f32(r, 6, freq_scale);
    set_f32(r, 7, ext_factor);
    set_f32(r, 8, attn_factor);
    set_f32(r, 9, beta_fast);
    set_f32(r, 10, beta_slow);
    r->op = GGML_OP_ROPE;
    r->src[0] = a;
    r->src[1] = b;
    r->src[2] = c;
    return r;
}

ggml_tensor *ggml_flash_attn_ext(ggml_context *ctx, ggml_tensor *q, ggml_tensor *k, ggml_tensor *v, ggml_tensor *mask,
                                 float scale, float max_bias, float logit_softcap) {
    HOST_CHECK(q->ne[0] == k->ne[0] && k->ne[1] == v->ne[1] && q->ne[2] % k->ne[2] == 0);
    const int64_t ne[4] = {v->ne[0], q->ne[2], q->ne[1], q->ne[3]};
    ggml_tensor *r = new_tensor(ctx, GGML_TYPE_F32, 4, ne, nullptr, 0);
    set_f32(r, 0, scale);
    set_f32(r, 1, max_bias);
    set_f32(r, 2, logit_softcap);
    r->op = GGML_OP_FLASH_ATTN_EXT;
    r->src[0] = q;
    r->src[1] = k;
    r->src[2] = v;
    r->src[3] = mask;
    return r;
}

void ggml_flash_attn_ext_set_prec(ggml_tensor *a, ggml_prec prec) { a->op_params[3] = (int32_t)prec; }

ggml_tensor *ggml_swiglu_split(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b) {
    HOST_CHECK(a->ne[0] == b->ne[0] && ggml_nelements(a) == ggml_nelements(b));
    ggml_tensor *r = dup_tensor(ctx, a);
    r->op_params[0] = GGML_GLU_OP_SWIGLU;
    r->op_params[1] = 0;
    r->op = GGML_OP_GLU;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

// ------------------------------------------------------------------------------------------------- graphs
ggml_cgraph *ggml_new_graph_custom(ggml_context *ctx, size_t size, bool grads) {
    HOST_CHECK(!grads && size > 0);
    auto *g = new ggml_cgraph;
    std::memset(g, 0, sizeof *g);
    g->size = (int)size;
    g->nodes = new ggml_tensor *[size]();
    g->leafs = new ggml_tensor *[size]();
    const size_t slots = 2 * size + 1;  // at most 2 size tensors (nodes and leafs) in an open-addressing set
    g->use_counts = new int32_t[slots]();
    g->visited_hash_set.size = slots;
    g->visited_hash_set.used = new ggml_bitset_t[(slots + 31) / 32]();
    g->visited_hash_set.keys = new ggml_tensor *[slots]();
    g->order = GGML_CGRAPH_EVAL_ORDER_LEFT_TO_RIGHT;
    ctx->graphs.push_back(g);
    return g;
}
ggml_cgraph *ggml_new_graph(ggml_context *ctx) { return ggml_new_graph_custom(ctx, 16384, false); }
ggml_cgraph ggml_graph_view(ggml_cgraph *g, int i0, int i1) {
    HOST_CHECK(0 <= i0 && i0 <= i1 && i1 <= g->n_nodes);
    ggml_cgraph v = *g;
    v.size = 0;
    v.n_nodes = i1 - i0;
    v.n_leafs = 0;
    v.nodes = g->nodes + i0;
    v.grads = nullptr;
    v.grad_accs = nullptr;
    v.leafs = nullptr;
    return v;
}
void ggml_build_forward_expand(ggml_cgraph *g, ggml_tensor *t) { visit(g, t); }
int ggml_graph_n_nodes(ggml_cgraph *g) { return g->n_nodes; }
ggml_tensor *ggml_graph_node(ggml_cgraph *g, int i) {
    if (i < 0) i += g->n_nodes;
    HOST_CHECK(i >= 0 && i < g->n_nodes);
    return g->nodes[i];
}

void ggml_log_internal(ggml_log_level level, const char *format, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, format);
    std::vsnprintf(buf, sizeof buf, format, ap);
    va_end(ap);
    if (level == GGML_LOG_LEVEL_ERROR || level == GGML_LOG_LEVEL_WARN) g_last_log = buf;
    std::fputs(buf, stderr);
}

// The last error or warning a backend logged through ggml_log_internal (test inspection only).
const char *ggml_host_last_log(void) { return g_last_log.c_str(); }
void ggml_host_clear_log(void) { g_last_log.clear(); }

// ------------------------------------------------------------------------------------------------- buffers
ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, ggml_backend_buffer_i iface,
                                               void *context, size_t size) {
    return new ggml_backend_buffer{iface, buft, context, size, GGML_BACKEND_BUFFER_USAGE_ANY};
}

void ggml_backend_buffer_free(ggml_backend_buffer_t buffer) {
    if (!buffer) return;
    if (buffer->iface.free_buffer) buffer->iface.free_buffer(buffer);
    delete buffer;
}

void *ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer) {
    if (buffer->size == 0) return nullptr;
    void *base = buffer->iface.get_base(buffer);
    HOST_CHECK(base);
    return base;
}

size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer) { return buffer->size; }
ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer) { return buffer->buft; }
void ggml_backend_buffer_set_usage(ggml_backend_buffer_t buffer, ggml_backend_buffer_usage usage) {
    buffer->usage = usage;
}

ggml_status ggml_backend_buffer_init_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor) {
    return buffer->iface.init_tensor ? buffer->iface.init_tensor(buffer, tensor) : GGML_STATUS_SUCCESS;
}

void ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    if (buffer->size == 0) return;
    buffer->iface.clear(buffer, value);
}

const char *ggml_backend_buft_name(ggml_backend_buffer_type_t buft) { return buft->iface.get_name(buft); }

ggml_backend_buffer_t ggml_backend_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    if (size == 0) return ggml_backend_buffer_init(buft, {}, nullptr, 0);
    return buft->iface.alloc_buffer(buft, size);
}

size_t ggml_backend_buft_get_alignment(ggml_backend_buffer_type_t buft) { return buft->iface.get_alignment(buft); }
size_t ggml_backend_buft_get_max_size(ggml_backend_buffer_type_t buft) {
    return buft->iface.get_max_size ? buft->iface.get_max_size(buft) : SIZE_MAX;
}
size_t ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft, const ggml_tensor *tensor) {
    if (!buft->iface.get_alloc_size) return ggml_nbytes(tensor);
    const size_t n = buft->iface.get_alloc_size(buft, tensor);
    HOST_CHECK(n >= ggml_nbytes(tensor));
    return n;
}
bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft) {
    return buft->iface.is_host ? buft->iface.is_host(buft) : false;
}
ggml_backend_dev_t ggml_backend_buft_get_device(ggml_backend_buffer_type_t buft) { return buft->device; }

size_t ggml_backend_buffer_get_alloc_size(ggml_backend_buffer_t buffer, const ggml_tensor *tensor) {
    return ggml_backend_buft_get_alloc_size(buffer->buft, tensor);
}

// ------------------------------------------------------------------------------------------------- tensors
ggml_status ggml_backend_tensor_alloc(ggml_backend_buffer_t buffer, ggml_tensor *tensor, void *addr) {
    HOST_CHECK(!tensor->buffer && !tensor->data && !tensor->view_src);
    char *base = (char *)ggml_backend_buffer_get_base(buffer);
    HOST_CHECK((char *)addr >= base &&
               (char *)addr + ggml_backend_buffer_get_alloc_size(buffer, tensor) <= base + buffer->size);
    tensor->buffer = buffer;
    tensor->data = addr;
    return ggml_backend_buffer_init_tensor(buffer, tensor);
}

ggml_status ggml_backend_view_init(ggml_tensor *tensor) {
    HOST_CHECK(tensor->view_src && tensor->view_src->buffer && tensor->view_src->data);
    tensor->buffer = tensor->view_src->buffer;
    tensor->data = (char *)tensor->view_src->data + tensor->view_offs;
    return ggml_backend_buffer_init_tensor(tensor->buffer, tensor);
}

void ggml_backend_tensor_set(ggml_tensor *tensor, const void *data, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = buffer_of(tensor);
    if (size == 0) return;
    HOST_CHECK(buf && tensor->data && data && offset + size <= ggml_nbytes(tensor));
    buf->iface.set_tensor(buf, tensor, data, offset, size);
}

void ggml_backend_tensor_get(const ggml_tensor *tensor, void *data, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = buffer_of(tensor);
    if (size == 0) return;
    HOST_CHECK(buf && tensor->data && data && offset + size <= ggml_nbytes(tensor));
    buf->iface.get_tensor(buf, tensor, data, offset, size);
}

void ggml_backend_tensor_memset(ggml_tensor *tensor, uint8_t value, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = buffer_of(tensor);
    if (size == 0) return;
    HOST_CHECK(buf && tensor->data && buf->iface.memset_tensor && offset + size <= ggml_nbytes(tensor));
    buf->iface.memset_tensor(buf, tensor, value, offset, size);
}

void ggml_backend_tensor_copy(ggml_tensor *src, ggml_tensor *dst) {
    HOST_CHECK(ggml_nbytes(src) == ggml_nbytes(dst));
    if (src == dst) return;
    ggml_backend_buffer_t db = buffer_of(dst);
    if (db->iface.cpy_tensor && db->iface.cpy_tensor(db, src, dst)) return;
    std::vector<uint8_t> tmp(ggml_nbytes(src));
    ggml_backend_tensor_get(src, tmp.data(), 0, tmp.size());
    ggml_backend_tensor_set(dst, tmp.data(), 0, tmp.size());
}

// ------------------------------------------------------------------------------------------------- backends
const char *ggml_backend_name(ggml_backend_t backend) { return backend->iface.get_name(backend); }
void ggml_backend_free(ggml_backend_t backend) {
    if (backend) backend->iface.free(backend);
}
ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t backend) { return backend->device; }
void ggml_backend_synchronize(ggml_backend_t backend) {
    if (backend->iface.synchronize) backend->iface.synchronize(backend);
}
ggml_status ggml_backend_graph_compute_async(ggml_backend_t backend, ggml_cgraph *cgraph) {
    return backend->iface.graph_compute(backend, cgraph);
}
ggml_status ggml_backend_graph_compute(ggml_backend_t backend, ggml_cgraph *cgraph) {
    const ggml_status st = ggml_backend_graph_compute_async(backend, cgraph);
    ggml_backend_synchronize(backend);
    return st;
}
// Nodes [i0, i1) of a graph computed as ggml_backend_sched computes one split of it: a view sharing the whole graph's
// use counts, handed to the backend's graph_compute.
ggml_status ggml_host_graph_compute_split(ggml_backend_t backend, ggml_cgraph *cgraph, int i0, int i1) {
    ggml_cgraph view = ggml_graph_view(cgraph, i0, i1);
    return ggml_backend_graph_compute(backend, &view);
}
bool ggml_backend_supports_op(ggml_backend_t backend, const ggml_tensor *op) {
    return ggml_backend_dev_supports_op(backend->device, op);
}

ggml_backend_event_t ggml_backend_event_new(ggml_backend_dev_t device) {
    return device && device->iface.event_new ? device->iface.event_new(device) : nullptr;
}
void ggml_backend_event_free(ggml_backend_event_t event) {
    if (event) event->device->iface.event_free(event->device, event);
}
void ggml_backend_event_record(ggml_backend_event_t event, ggml_backend_t backend) {
    HOST_CHECK(backend->iface.event_record);
    backend->iface.event_record(backend, event);
}
void ggml_backend_event_synchronize(ggml_backend_event_t event) {
    HOST_CHECK(event->device->iface.event_synchronize);
    event->device->iface.event_synchronize(event->device, event);
}

// ------------------------------------------------------------------------------------------------- devices
const char *ggml_backend_dev_name(ggml_backend_dev_t d) { return d->iface.get_name(d); }
const char *ggml_backend_dev_description(ggml_backend_dev_t d) { return d->iface.get_description(d); }
void ggml_backend_dev_memory(ggml_backend_dev_t d, size_t *free, size_t *total) { d->iface.get_memory(d, free, total); }
enum ggml_backend_dev_type ggml_backend_dev_type(ggml_backend_dev_t d) { return d->iface.get_type(d); }
void ggml_backend_dev_get_props(ggml_backend_dev_t d, ggml_backend_dev_props *props) {
    std::memset(props, 0, sizeof *props);
    d->iface.get_props(d, props);
}
ggml_backend_reg_t ggml_backend_dev_backend_reg(ggml_backend_dev_t d) { return d->reg; }
ggml_backend_t ggml_backend_dev_init(ggml_backend_dev_t d, const char *params) {
    return d->iface.init_backend(d, params);
}
ggml_backend_buffer_type_t ggml_backend_dev_buffer_type(ggml_backend_dev_t d) { return d->iface.get_buffer_type(d); }
bool ggml_backend_dev_supports_op(ggml_backend_dev_t d, const ggml_tensor *op) { return d->iface.supports_op(d, op); }
bool ggml_backend_dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t buft) {
    return d->iface.supports_buft(d, buft);
}
bool ggml_backend_dev_offload_op(ggml_backend_dev_t d, const ggml_tensor *op) {
    return d->iface.offload_op ? d->iface.offload_op(d, op) : false;
}

// ------------------------------------------------------------------------------------------------- registries
const char *ggml_backend_reg_name(ggml_backend_reg_t reg) { return reg->iface.get_name(reg); }
size_t ggml_backend_reg_dev_count(ggml_backend_reg_t reg) { return reg->iface.get_device_count(reg); }
ggml_backend_dev_t ggml_backend_reg_dev_get(ggml_backend_reg_t reg, size_t index) {
    return reg->iface.get_device(reg, index);
}
void *ggml_backend_reg_get_proc_address(ggml_backend_reg_t reg, const char *name) {
    return reg->iface.get_proc_address ? reg->iface.get_proc_address(reg, name) : nullptr;
}

}  // extern "C"
