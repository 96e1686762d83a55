// ggml backend for the MI355X: the reg / device / backend / buffer-type / buffer interfaces of ggml-backend-impl.h,
// each hook a thin call into libmx's C ABI (include/mx.h).
//
// Built against the ggml that speech.cpp vendors (the nyosegawa/ggml fork on upstream v0.27.0, `.gitmodules:1-4`);
// ggml's headers are not part of this repository. speech.cpp reaches these hooks from:
//   device selection   src/common/backend.cpp:70-120 (ggml_backend_dev_count/get/type/name/init)
//   weight buffers     src/common/model-file.cpp:222-268 (alloc_ctx_tensors, set_usage WEIGHTS, tensor_set pieces)
//   compute            src/common/graph.cpp:96-110 (gallocr + graph_compute, or ggml_backend_sched over {this, CPU})
//   capability probes  src/common/qwen3-decoder.cpp:73-83,550 (ggml_backend_supports_op)
//
// Quantized tensors in this buffer type are stored in libmx's planar device layout; set_tensor / get_tensor /
// memset_tensor translate ggml-layout bytes at any offset, so ggml, GGUF loading and tensor copies see ggml's layout.
// A quantized view with an offset cannot be addressed in that layout: supports_op declines it and init_tensor reports it.
#include "ggml-mi355x.h"

#include <algorithm>
#include <cstddef>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-impl.h"
#include "mx.h"

// ------------------------------------------------------------------------------------ the layout written against
// The fields of ggml_tensor and the slots of the five interface tables this backend reads and fills, as ggml lays them
// out on LP64 (ggml.h, ggml-backend-impl.h). Built against another ggml whose headers moved any of them, the build
// stops here instead of reading the wrong field or filling the wrong slot.
static_assert(sizeof(void *) == 8, "LP64 only");
static_assert(offsetof(ggml_tensor, type) == 0 && offsetof(ggml_tensor, buffer) == 8 &&
                  offsetof(ggml_tensor, ne) == 16 && offsetof(ggml_tensor, nb) == 48 &&
                  offsetof(ggml_tensor, op) == 80 && offsetof(ggml_tensor, op_params) == 84 &&
                  offsetof(ggml_tensor, flags) == 148 && offsetof(ggml_tensor, src) == 152 &&
                  offsetof(ggml_tensor, view_src) == 232 && offsetof(ggml_tensor, view_offs) == 240 &&
                  offsetof(ggml_tensor, data) == 248 && offsetof(ggml_tensor, name) == 256 &&
                  offsetof(ggml_tensor, extra) == 320 && sizeof(ggml_tensor) == 336,
              "ggml_tensor differs from the layout this backend was written for");
static_assert(GGML_MAX_DIMS == 4 && GGML_MAX_SRC == 10 && GGML_MAX_OP_PARAMS == 64 && GGML_MAX_NAME == 64,
              "ggml's tensor limits differ");
#define MI355X_SLOT(T, f, i) (offsetof(T, f) == (i) * sizeof(void *))
static_assert(sizeof(ggml_backend_buffer_type_i) == 6 * sizeof(void *) &&
                  MI355X_SLOT(ggml_backend_buffer_type_i, get_name, 0) &&
                  MI355X_SLOT(ggml_backend_buffer_type_i, alloc_buffer, 1) &&
                  MI355X_SLOT(ggml_backend_buffer_type_i, get_alignment, 2) &&
                  MI355X_SLOT(ggml_backend_buffer_type_i, get_max_size, 3) &&
                  MI355X_SLOT(ggml_backend_buffer_type_i, get_alloc_size, 4) &&
                  MI355X_SLOT(ggml_backend_buffer_type_i, is_host, 5),
              "ggml_backend_buffer_type_i differs");
static_assert(sizeof(ggml_backend_buffer_i) == 9 * sizeof(void *) && MI355X_SLOT(ggml_backend_buffer_i, free_buffer, 0) &&
                  MI355X_SLOT(ggml_backend_buffer_i, get_base, 1) && MI355X_SLOT(ggml_backend_buffer_i, init_tensor, 2) &&
                  MI355X_SLOT(ggml_backend_buffer_i, memset_tensor, 3) &&
                  MI355X_SLOT(ggml_backend_buffer_i, set_tensor, 4) && MI355X_SLOT(ggml_backend_buffer_i, get_tensor, 5) &&
                  MI355X_SLOT(ggml_backend_buffer_i, cpy_tensor, 6) && MI355X_SLOT(ggml_backend_buffer_i, clear, 7) &&
                  MI355X_SLOT(ggml_backend_buffer_i, reset, 8),
              "ggml_backend_buffer_i differs");
static_assert(sizeof(ggml_backend_i) == 14 * sizeof(void *) && MI355X_SLOT(ggml_backend_i, get_name, 0) &&
                  MI355X_SLOT(ggml_backend_i, free, 1) && MI355X_SLOT(ggml_backend_i, set_tensor_async, 2) &&
                  MI355X_SLOT(ggml_backend_i, get_tensor_async, 3) && MI355X_SLOT(ggml_backend_i, cpy_tensor_async, 4) &&
                  MI355X_SLOT(ggml_backend_i, synchronize, 5) && MI355X_SLOT(ggml_backend_i, graph_plan_create, 6) &&
                  MI355X_SLOT(ggml_backend_i, graph_plan_free, 7) && MI355X_SLOT(ggml_backend_i, graph_plan_update, 8) &&
                  MI355X_SLOT(ggml_backend_i, graph_plan_compute, 9) && MI355X_SLOT(ggml_backend_i, graph_compute, 10) &&
                  MI355X_SLOT(ggml_backend_i, event_record, 11) && MI355X_SLOT(ggml_backend_i, event_wait, 12) &&
                  MI355X_SLOT(ggml_backend_i, graph_optimize, 13),
              "ggml_backend_i differs");
static_assert(sizeof(ggml_backend_device_i) == 15 * sizeof(void *) && MI355X_SLOT(ggml_backend_device_i, get_name, 0) &&
                  MI355X_SLOT(ggml_backend_device_i, get_description, 1) &&
                  MI355X_SLOT(ggml_backend_device_i, get_memory, 2) && MI355X_SLOT(ggml_backend_device_i, get_type, 3) &&
                  MI355X_SLOT(ggml_backend_device_i, get_props, 4) && MI355X_SLOT(ggml_backend_device_i, init_backend, 5) &&
                  MI355X_SLOT(ggml_backend_device_i, get_buffer_type, 6) &&
                  MI355X_SLOT(ggml_backend_device_i, get_host_buffer_type, 7) &&
                  MI355X_SLOT(ggml_backend_device_i, buffer_from_host_ptr, 8) &&
                  MI355X_SLOT(ggml_backend_device_i, supports_op, 9) &&
                  MI355X_SLOT(ggml_backend_device_i, supports_buft, 10) &&
                  MI355X_SLOT(ggml_backend_device_i, offload_op, 11) && MI355X_SLOT(ggml_backend_device_i, event_new, 12) &&
                  MI355X_SLOT(ggml_backend_device_i, event_free, 13) &&
                  MI355X_SLOT(ggml_backend_device_i, event_synchronize, 14),
              "ggml_backend_device_i differs");
static_assert(sizeof(ggml_backend_reg_i) == 4 * sizeof(void *) && MI355X_SLOT(ggml_backend_reg_i, get_name, 0) &&
                  MI355X_SLOT(ggml_backend_reg_i, get_device_count, 1) && MI355X_SLOT(ggml_backend_reg_i, get_device, 2) &&
                  MI355X_SLOT(ggml_backend_reg_i, get_proc_address, 3),
              "ggml_backend_reg_i differs");
static_assert(offsetof(ggml_backend_buffer, iface) == 0 && offsetof(ggml_backend_buffer, buft) == 72 &&
                  offsetof(ggml_backend_buffer, context) == 80 && offsetof(ggml_backend_buffer, size) == 88 &&
                  offsetof(ggml_backend_buffer, usage) == 96 && offsetof(ggml_backend_buffer_type, device) == 48 &&
                  offsetof(ggml_backend_buffer_type, context) == 56 && offsetof(ggml_backend, iface) == 8 &&
                  offsetof(ggml_backend, device) == 120 && offsetof(ggml_backend, context) == 128 &&
                  offsetof(ggml_backend_device, reg) == 120 && offsetof(ggml_backend_device, context) == 128 &&
                  offsetof(ggml_backend_reg, iface) == 8 && offsetof(ggml_backend_reg, context) == 40 &&
                  offsetof(ggml_backend_event, context) == 8,
              "the structs that carry ggml's interface tables differ");
#undef MI355X_SLOT

namespace {

struct DeviceCtx {
    int device = 0;
    std::string name;
    std::string description;
    mx_backend *io = nullptr;  // the stream buffer transfers run on
    ggml_backend_buffer_type buft{};
};

struct BufferCtx {
    DeviceCtx *dev = nullptr;
    void *base = nullptr;
    size_t size = 0;
};

// What one tensor of a node contributes to the key of a graph: every field a launch reads -- its type, shape, byte
// strides, data address and view offset -- and its flags (a graph output is never fused away).
struct TensorKey {
    int32_t type;
    int32_t flags;
    int64_t ne[4];
    uint64_t nb[4];
    const void *data;
    uint64_t view_offs;
};

// One node of a graph, to recognise a graph computed again with the same tensors: the node (with its operation
// parameters: eps, RoPE's dims / mode / bases, attention's scale), its first five sources, and how many nodes of the
// whole graph read it (what decides the fusions it can take part in).
struct NodeKey {
    int32_t op;
    int32_t uses;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    TensorKey t[6];
    bool operator==(const NodeKey &o) const { return std::memcmp(this, &o, sizeof(NodeKey)) == 0; }
};

// A graph seen before and how often in a row it came again, with its recording once it has one.
struct SeenGraph {
    std::vector<NodeKey> keys;
    int repeats = 0;
    mx_graph *replay = nullptr;  // recorded from the third identical computation on
    uint64_t last_use = 0;
};
constexpr size_t kSeenGraphs = 8;  // the graphs a backend keeps recordings of: the splits of a scheduled step

// What a backend's graph_compute did, for tests and tuning: graphs computed eagerly / recorded / replayed, then the
// fusions run as one launch -- norm into products, SwiGLU and residual around a product, a decode row's attention
// block, a prefill block's norms + RoPE + stores (its attention separate) -- and fusions libmx declined.
enum Count {
    kEager, kRecorded, kReplayed, kNormProducts, kProductOut, kAttention, kAttentionRows, kDeclined, kExpertsGroup,
    kCounts
};

struct BackendCtx {
    DeviceCtx *dev = nullptr;
    mx_backend *be = nullptr;
    std::vector<SeenGraph> seen;  // at most kSeenGraphs, the least recently computed dropped first
    uint64_t clock = 0;
    int64_t counts[kCounts] = {};
};

mx_tensor desc(const ggml_tensor *t) {
    mx_tensor d;
    std::memset(&d, 0, sizeof d);
    d.type = (int32_t)t->type;
    for (int i = 0; i < 4; i++) {
        d.ne[i] = t->ne[i];
        d.nb[i] = t->nb[i];
    }
    d.data = t->data;
    return d;
}

// Operation parameters as ggml stores them in op_params (ggml.c: ggml_rms_norm_impl eps at 0; ggml_rope_impl n_dims
// at 1, mode at 2, freq_base .. attn_factor at 5..8; ggml_flash_attn_ext scale, max_bias, logit_softcap at 0..2;
// ggml_glu_impl the GLU op at 0 and `swapped` at 1).
float op_f32(const ggml_tensor *t, int i) {
    float v;
    std::memcpy(&v, &t->op_params[i], sizeof v);
    return v;
}

// The descriptor of a tensor the scheduler is still planning (no memory yet): an aligned placeholder address, so that
// libmx checks shapes, strides and alignment as it will find them (this buffer type's allocations are 256-aligned).
mx_tensor planned(const ggml_tensor *t) {
    alignas(256) static const char placeholder[256] = {};
    mx_tensor d = desc(t);
    if (!d.data) d.data = (void *)placeholder;
    return d;
}

enum ggml_status to_status(int rc) {
    if (rc == MX_SUCCESS) return GGML_STATUS_SUCCESS;
    if (rc == MX_ALLOC_FAILED) return GGML_STATUS_ALLOC_FAILED;
    return GGML_STATUS_FAILED;
}

bool report(int rc, const char *what) {
    if (rc != MX_SUCCESS) GGML_LOG_ERROR("%s: %s: %s\n", __func__, what, mx_last_error());
    return rc == MX_SUCCESS;
}

// ------------------------------------------------------------------------------------------------------ buffer
void buffer_free(ggml_backend_buffer_t buffer) {
    auto *ctx = (BufferCtx *)buffer->context;
    report(mx_buffer_free(ctx->dev->io, ctx->base), "free buffer");
    delete ctx;
}

void *buffer_get_base(ggml_backend_buffer_t buffer) { return ((BufferCtx *)buffer->context)->base; }

enum ggml_status buffer_init_tensor(ggml_backend_buffer_t, ggml_tensor *tensor) {
    if (tensor->view_src && ggml_is_quantized(tensor->type) && tensor->view_offs != 0) {
        GGML_LOG_ERROR("%s: %s: a quantized view at an offset cannot be addressed in the MI355X layout\n", __func__,
                       tensor->name);
        return GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

void buffer_memset_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor, uint8_t value, size_t offset,
                          size_t size) {
    const mx_tensor d = desc(tensor);
    report(mx_tensor_memset(((BufferCtx *)buffer->context)->dev->io, &d, value, offset, size), "memset_tensor");
}

void buffer_set_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor, const void *data, size_t offset,
                       size_t size) {
    const mx_tensor d = desc(tensor);
    report(mx_tensor_set(((BufferCtx *)buffer->context)->dev->io, &d, data, offset, size), "set_tensor");
}

void buffer_get_tensor(ggml_backend_buffer_t buffer, const ggml_tensor *tensor, void *data, size_t offset,
                       size_t size) {
    const mx_tensor d = desc(tensor);
    report(mx_tensor_get(((BufferCtx *)buffer->context)->dev->io, &d, data, offset, size), "get_tensor");
}

bool buffer_is_ours(ggml_backend_buffer_t buffer);

bool buffer_cpy_tensor(ggml_backend_buffer_t buffer, const ggml_tensor *src, ggml_tensor *dst) {
    if (!src->buffer || !buffer_is_ours(src->buffer)) return false;  // ggml copies through the host instead
    const mx_tensor s = desc(src), d = desc(dst);
    return report(mx_tensor_copy(((BufferCtx *)buffer->context)->dev->io, &s, &d), "cpy_tensor");
}

void buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    auto *ctx = (BufferCtx *)buffer->context;
    report(mx_buffer_clear(ctx->dev->io, ctx->base, ctx->size, value), "clear");
}

const ggml_backend_buffer_i kBufferIface = {
    /* .free_buffer   = */ buffer_free,
    /* .get_base      = */ buffer_get_base,
    /* .init_tensor   = */ buffer_init_tensor,
    /* .memset_tensor = */ buffer_memset_tensor,
    /* .set_tensor    = */ buffer_set_tensor,
    /* .get_tensor    = */ buffer_get_tensor,
    /* .cpy_tensor    = */ buffer_cpy_tensor,
    /* .clear         = */ buffer_clear,
    /* .reset         = */ nullptr,
};

bool buffer_is_ours(ggml_backend_buffer_t buffer) { return buffer->iface.get_base == buffer_get_base; }

// ------------------------------------------------------------------------------------------------- buffer type
const char *buft_get_name(ggml_backend_buffer_type_t) { return "MI355X"; }

ggml_backend_buffer_t buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    auto *dev = (DeviceCtx *)buft->context;
    void *base = nullptr;
    if (!report(mx_buffer_alloc(dev->io, size, &base), "alloc_buffer")) return nullptr;
    auto *ctx = new BufferCtx{dev, base, size};
    return ggml_backend_buffer_init(buft, kBufferIface, ctx, size);
}

size_t buft_get_alignment(ggml_backend_buffer_type_t) { return mx_buft_alignment(); }
size_t buft_get_max_size(ggml_backend_buffer_type_t) { return mx_buft_max_size(); }

size_t buft_get_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor *tensor) {
    const mx_tensor d = desc(tensor);
    const size_t n = mx_tensor_alloc_size(&d);
    return n ? n : ggml_nbytes(tensor);
}

bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

const ggml_backend_buffer_type_i kBuftIface = {
    /* .get_name       = */ buft_get_name,
    /* .alloc_buffer   = */ buft_alloc_buffer,
    /* .get_alignment  = */ buft_get_alignment,
    /* .get_max_size   = */ buft_get_max_size,
    /* .get_alloc_size = */ buft_get_alloc_size,
    /* .is_host        = */ buft_is_host,
};

// ----------------------------------------------------------------------------------------------------- backend
const char *backend_get_name(ggml_backend_t backend) { return ((BackendCtx *)backend->context)->dev->name.c_str(); }

void backend_free(ggml_backend_t backend) {
    auto *ctx = (BackendCtx *)backend->context;
    for (SeenGraph &g : ctx->seen) mx_graph_free(g.replay);
    mx_backend_free(ctx->be);
    delete ctx;
    delete backend;
}

void backend_synchronize(ggml_backend_t backend) {
    report(mx_backend_synchronize(((BackendCtx *)backend->context)->be), "synchronize");
}

bool is_noop(const ggml_tensor *node) {
    return ggml_is_empty(node) || node->op == GGML_OP_NONE || node->op == GGML_OP_RESHAPE ||
           node->op == GGML_OP_VIEW || node->op == GGML_OP_PERMUTE || node->op == GGML_OP_TRANSPOSE;
}

// One node on the device through its C-ABI entry point.
int run_node(BackendCtx *ctx, const ggml_tensor *node) {
    switch (node->op) {
        case GGML_OP_MUL_MAT: {
            const mx_tensor s0 = desc(node->src[0]), s1 = desc(node->src[1]), d = desc(node);
            return mx_mul_mat(ctx->be, &s0, &s1, &d);
        }
        case GGML_OP_MUL_MAT_ID: {
            const mx_tensor as = desc(node->src[0]), b = desc(node->src[1]), ids = desc(node->src[2]), d = desc(node);
            return mx_mul_mat_id(ctx->be, &as, &b, &ids, &d);
        }
        case GGML_OP_GET_ROWS: {
            const mx_tensor s0 = desc(node->src[0]), ids = desc(node->src[1]), d = desc(node);
            return mx_get_rows(ctx->be, &s0, &ids, &d);
        }
        case GGML_OP_ARGMAX: {
            const mx_tensor s0 = desc(node->src[0]), d = desc(node);
            return mx_argmax(ctx->be, &s0, &d);
        }
        case GGML_OP_RMS_NORM: {
            const mx_tensor s0 = desc(node->src[0]), d = desc(node);
            return mx_rms_norm(ctx->be, &s0, &d, op_f32(node, 0), nullptr);
        }
        case GGML_OP_ADD:
        case GGML_OP_MUL: {
            const mx_tensor a = desc(node->src[0]), b = desc(node->src[1]), d = desc(node);
            return mx_binary(ctx->be, node->op == GGML_OP_ADD ? MX_OP_ADD : MX_OP_MUL, &a, &b, &d);
        }
        case GGML_OP_GLU: {
            const mx_tensor a = desc(node->src[0]), b = desc(node->src[1]), d = desc(node);
            return mx_swiglu(ctx->be, &a, &b, &d);
        }
        case GGML_OP_ROPE: {
            const mx_tensor x = desc(node->src[0]), pos = desc(node->src[1]), d = desc(node);
            return mx_rope(ctx->be, &x, &pos, &d, node->op_params[1], node->op_params[2], op_f32(node, 5),
                           op_f32(node, 6), op_f32(node, 7), op_f32(node, 8));
        }
        case GGML_OP_SET_ROWS: {
            const mx_tensor src = desc(node->src[0]), idx = desc(node->src[1]), d = desc(node);
            return mx_set_rows(ctx->be, &src, &idx, &d);
        }
        case GGML_OP_FLASH_ATTN_EXT: {
            const mx_tensor q = desc(node->src[0]), k = desc(node->src[1]), v = desc(node->src[2]), d = desc(node);
            const mx_tensor m = node->src[3] ? desc(node->src[3]) : mx_tensor{};
            return mx_flash_attn_ext(ctx->be, &q, &k, &v, node->src[3] ? &m : nullptr, &d, op_f32(node, 0));
        }
        default:
            GGML_LOG_ERROR("%s: op %s is not computed by the MI355X backend\n", __func__, ggml_op_desc(node));
            return MX_UNSUPPORTED;
    }
}

// MUL_MATs that read one src1 with one weight type, as one launch (members of different shape classes: one at a time).
int run_products(BackendCtx *ctx, const std::vector<const ggml_tensor *> &group) {
    if (group.size() == 1) return run_node(ctx, group[0]);
    std::vector<mx_tensor> w, y;
    for (const ggml_tensor *g : group) {
        w.push_back(desc(g->src[0]));
        y.push_back(desc(g));
    }
    std::vector<const mx_tensor *> wp, yp;
    for (size_t k = 0; k < group.size(); k++) {
        wp.push_back(&w[k]);
        yp.push_back(&y[k]);
    }
    const mx_tensor s1 = desc(group[0]->src[1]);
    int rc = mx_mul_mat_group(ctx->be, (int)group.size(), wp.data(), &s1, yp.data());
    if (rc != MX_UNSUPPORTED) return rc;
    rc = MX_SUCCESS;
    for (size_t k = 0; k < group.size() && rc == MX_SUCCESS; k++) rc = mx_mul_mat(ctx->be, wp[k], &s1, yp[k]);
    return rc;
}

// ------------------------------------------------------------------------------------------ fusions of a graph
// What the plan of a graph knows about it: each node's position, for each tensor the nodes of this graph that read
// it, and each node's use count over the whole graph ggml built. Under ggml_backend_sched the graph is one split (a
// view of the whole graph's nodes, sharing its use counts): a node of a later split may read a tensor this one
// computes, and only the whole graph's count shows it.
struct GraphInfo {
    ggml_cgraph *graph;
    std::vector<const ggml_tensor *> nodes;
    std::unordered_map<const ggml_tensor *, int> index;
    std::unordered_map<const ggml_tensor *, std::vector<int>> readers;

    explicit GraphInfo(ggml_cgraph *cgraph) : graph(cgraph) {
        const int n = ggml_graph_n_nodes(cgraph);
        for (int i = 0; i < n; i++) {
            const ggml_tensor *t = ggml_graph_node(cgraph, i);
            nodes.push_back(t);
            index[t] = i;
            for (int s = 0; s < GGML_MAX_SRC; s++)
                if (t->src[s]) readers[t->src[s]].push_back(i);
        }
    }
    // whether t is computed here and every node of the whole graph that reads it is among this graph's `n` readers
    bool read_here_only(const ggml_tensor *t, size_t n) const {
        const int i = pos(t);
        return i >= 0 && ggml_node_get_use_count(graph, i) == (int)n;
    }
    // the one node that reads t, if exactly one node of the whole graph does and t is not a graph output (a fusion
    // need not write t then)
    const ggml_tensor *sole_reader(const ggml_tensor *t) const {
        if (!t || (t->flags & GGML_TENSOR_FLAG_OUTPUT)) return nullptr;
        auto it = readers.find(t);
        if (it == readers.end() || it->second.size() != 1 || !read_here_only(t, 1)) return nullptr;
        return nodes[it->second[0]];
    }
    int pos(const ggml_tensor *t) const {
        auto it = index.find(t);
        return it == index.end() ? -1 : it->second;
    }
};

// A step of the plan: one node, a group of products, or a fusion over several nodes (roles below, in graph order).
enum class StepKind { Node, Products, NormProducts, ProductOut, Attention, Experts };
struct Step {
    StepKind kind;
    std::vector<const ggml_tensor *> nodes;
};

// Whether every node of [first, last] that computes anything is one of the step's own.
bool covers_range(const GraphInfo &gi, int first, int last, const std::vector<const ggml_tensor *> &own) {
    for (int i = first; i <= last; i++) {
        const ggml_tensor *t = gi.nodes[i];
        if (is_noop(t)) continue;
        bool found = false;
        for (const ggml_tensor *o : own) found = found || o == t;
        if (!found) return false;
    }
    return true;
}

bool is_vector_of(const ggml_tensor *w, int64_t n) {
    return w && w->type == GGML_TYPE_F32 && w->ne[0] == n && w->ne[1] == 1 && w->ne[2] == 1 && w->ne[3] == 1;
}

bool is_head_permute(const ggml_tensor *t) {
    return t && t->op == GGML_OP_PERMUTE && t->op_params[0] == 0 && t->op_params[1] == 2 && t->op_params[2] == 1 &&
           t->op_params[3] == 3;
}

// RMS_NORM -> MUL by a weight vector -> 1..4 MUL_MATs that read it (qwen3-decoder.cpp:361-363 before q/k/v, :409-411
// before gate/up, :426-427 before the output head). Roles: {norm, mul, products...}.
bool match_norm_products(const GraphInfo &gi, int i, Step &st) {
    const ggml_tensor *norm = gi.nodes[i];
    const ggml_tensor *mul = gi.sole_reader(norm);
    if (!mul || mul->op != GGML_OP_MUL || mul->src[0] != norm || !is_vector_of(mul->src[1], norm->ne[0])) return false;
    if (mul->flags & GGML_TENSOR_FLAG_OUTPUT) return false;
    auto it = gi.readers.find(mul);
    if (it == gi.readers.end() || it->second.empty() || it->second.size() > 4) return false;
    if (!gi.read_here_only(mul, it->second.size())) return false;
    std::vector<const ggml_tensor *> own{norm, mul};
    int last = gi.pos(mul);
    for (int r : it->second) {
        const ggml_tensor *p = gi.nodes[r];
        if (p->op != GGML_OP_MUL_MAT || p->src[1] != mul || p->src[0]->type != gi.nodes[it->second[0]]->src[0]->type)
            return false;
        own.push_back(p);
        last = std::max(last, r);
    }
    if (!covers_range(gi, i, last, own)) return false;
    st = Step{StepKind::NormProducts, own};
    return true;
}

// [GLU swiglu(gate, up) ->] MUL_MAT -> ADD with the residual stream (qwen3-decoder.cpp:405 attn_o, :411 ffn_down).
// Roles: {glu or nullptr, product, add}.
bool match_product_out(const GraphInfo &gi, int i, Step &st) {
    const ggml_tensor *first = gi.nodes[i];
    const ggml_tensor *glu = nullptr, *prod = first;
    if (first->op == GGML_OP_GLU) {
        if (ggml_get_glu_op(first) != GGML_GLU_OP_SWIGLU || !first->src[1] || first->op_params[1] != 0) return false;
        glu = first;
        prod = gi.sole_reader(glu);
        if (!prod || prod->op != GGML_OP_MUL_MAT || prod->src[1] != glu) return false;
    }
    if (prod->op != GGML_OP_MUL_MAT) return false;
    const ggml_tensor *add = gi.sole_reader(prod);
    if (!add || add->op != GGML_OP_ADD || (add->src[0] != prod && add->src[1] != prod)) return false;
    std::vector<const ggml_tensor *> own{prod, add};
    if (glu) own.push_back(glu);
    if (!covers_range(gi, i, gi.pos(add), own)) return false;
    st = Step{StepKind::ProductOut, {glu, prod, add}};
    return true;
}

// The attention block of one layer from the q head norm on (qwen3-decoder.cpp:366-397): RMS_NORM x q_norm and
// x k_norm, NEOX RoPE of both at pos, SET_ROWS of v and of the roped k into the caches, FLASH_ATTN_EXT over the
// caches' head views. Roles: {q norm, q mul, k norm, k mul, v set_rows, q rope, k rope, k set_rows, attention}.
bool match_attention(const GraphInfo &gi, int i, Step &st) {
    const ggml_tensor *nq = gi.nodes[i];
    const ggml_tensor *mq = gi.sole_reader(nq);
    if (!mq || mq->op != GGML_OP_MUL || mq->src[0] != nq) return false;
    const ggml_tensor *rq = gi.sole_reader(mq);
    if (!rq || rq->op != GGML_OP_ROPE || rq->src[0] != mq || rq->src[2]) return false;
    const ggml_tensor *qh = gi.sole_reader(rq);
    if (!is_head_permute(qh) || qh->src[0] != rq) return false;
    const ggml_tensor *fa = gi.sole_reader(qh);
    if (!fa || fa->op != GGML_OP_FLASH_ATTN_EXT || fa->src[0] != qh || fa->src[4]) return false;
    const ggml_tensor *kh = fa->src[1], *vh = fa->src[2], *pos = rq->src[1];
    if (!is_head_permute(kh) || !is_head_permute(vh) || !kh->view_src || !vh->view_src) return false;
    const ggml_tensor *kc = kh->view_src, *vc = vh->view_src;
    // the stores into the two caches at the same positions, between the q norm and the attention
    const ggml_tensor *sk = nullptr, *sv = nullptr;
    const int ifa = gi.pos(fa);
    for (int j = i + 1; j < ifa; j++) {
        const ggml_tensor *t = gi.nodes[j];
        if (t->op != GGML_OP_SET_ROWS || t->src[1] != pos) continue;
        if (t->view_src == kc && t->view_offs == kh->view_offs) sk = t;
        if (t->view_src == vc && t->view_offs == vh->view_offs) sv = t;
    }
    if (!sk || !sv) return false;
    const ggml_tensor *k2 = sk->src[0];  // the roped k as cache rows
    if (!k2 || k2->op != GGML_OP_RESHAPE || !gi.sole_reader(k2)) return false;
    const ggml_tensor *rk = k2->src[0];
    if (!rk || rk->op != GGML_OP_ROPE || gi.sole_reader(rk) != k2 || rk->src[1] != pos || rk->src[2]) return false;
    const ggml_tensor *mk = rk->src[0];
    if (!mk || mk->op != GGML_OP_MUL || gi.sole_reader(mk) != rk) return false;
    const ggml_tensor *nk = mk->src[0];
    if (!nk || nk->op != GGML_OP_RMS_NORM || gi.sole_reader(nk) != mk) return false;
    if (std::memcmp(&nq->op_params[0], &nk->op_params[0], 4) != 0 ||
        std::memcmp(&rq->op_params[1], &rk->op_params[1], 10 * sizeof(int32_t)) != 0)
        return false;
    const std::vector<const ggml_tensor *> own{nq, mq, nk, mk, sv, rq, rk, sk, fa};
    const int first = std::min(i, gi.pos(nk));
    if (first != i || !covers_range(gi, first, ifa, own)) return false;
    st = Step{StepKind::Attention, own};
    return true;
}

bool same_ne(const ggml_tensor *a, const ggml_tensor *b) {
    return a->ne[0] == b->ne[0] && a->ne[1] == b->ne[1] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3];
}

// Whether the bytes two tensors' data span, [data, data + nbytes), meet.
bool overlaps(const ggml_tensor *a, const ggml_tensor *b) {
    if (!a || !b || !a->data || !b->data) return false;
    const uint8_t *a0 = (const uint8_t *)a->data, *b0 = (const uint8_t *)b->data;
    return a0 < b0 + ggml_nbytes(b) && b0 < a0 + ggml_nbytes(a);
}

// MUL_MAT_ID at i and later MUL_MAT_IDs that read the same rows and ids with experts of the same type and shape (the
// gate and up experts of text-model.cpp:208-209; ggml's graph order puts silu(gate) between them). Run together at
// i: a later product reads nothing computed after i (its experts are a weight, its rows and ids are i's, which no
// node between them writes), and its output may not share memory with any tensor a node between them reads or
// writes (the allocator reuses freed memory in graph order). Roles: {products...}.
bool match_experts(const GraphInfo &gi, int i, const std::vector<bool> &taken, Step &st) {
    const ggml_tensor *a = gi.nodes[i];
    std::vector<const ggml_tensor *> own{a};
    for (int j = i + 1; j < (int)gi.nodes.size() && own.size() < 4; j++) {
        const ggml_tensor *b = gi.nodes[j];
        if (taken[j] || b->op != GGML_OP_MUL_MAT_ID || b->src[1] != a->src[1] || b->src[2] != a->src[2]) continue;
        const ggml_tensor *wa = a->src[0], *wb = b->src[0];
        if (wb->type != wa->type || !same_ne(wa, wb) || !same_ne(a, b)) continue;
        if (gi.pos(wb) >= 0) continue;  // experts computed by the graph itself
        bool clear = !overlaps(b, a->src[1]) && !overlaps(b, a->src[2]);
        for (int k = i + 1; k < j && clear; k++) {
            const ggml_tensor *n = gi.nodes[k];
            // n writes neither b's output nor its rows and ids (an in-place op or a view over them), and reads no
            // memory b writes
            clear = !overlaps(b, n) && !overlaps(n, a->src[1]) && !overlaps(n, a->src[2]);
            for (int s = 0; s < GGML_MAX_SRC && clear; s++) clear = !overlaps(b, n->src[s]);
        }
        for (const ggml_tensor *o : own) clear = clear && !overlaps(b, o);
        if (!clear) continue;
        own.push_back(b);
    }
    if (own.size() < 2) return false;
    st = Step{StepKind::Experts, own};
    return true;
}

std::vector<Step> plan_graph(const GraphInfo &gi) {
    std::vector<Step> plan;
    std::vector<bool> taken(gi.nodes.size(), false);
    for (int i = 0; i < (int)gi.nodes.size(); i++) {
        const ggml_tensor *t = gi.nodes[i];
        if (taken[i] || is_noop(t)) continue;
        Step st;
        bool fused = false;
        if (t->op == GGML_OP_RMS_NORM) fused = match_attention(gi, i, st) || match_norm_products(gi, i, st);
        if (!fused && (t->op == GGML_OP_GLU || t->op == GGML_OP_MUL_MAT)) fused = match_product_out(gi, i, st);
        if (!fused && t->op == GGML_OP_MUL_MAT_ID) fused = match_experts(gi, i, taken, st);
        if (fused) {
            for (const ggml_tensor *n : st.nodes)
                if (n) taken[gi.pos(n)] = true;
            plan.push_back(std::move(st));
            continue;
        }
        if (t->op == GGML_OP_MUL_MAT) {  // consecutive products of one src1 and weight type: one launch
            Step g{StepKind::Products, {t}};
            for (int j = i + 1; j < (int)gi.nodes.size() && g.nodes.size() < 4; j++) {
                const ggml_tensor *nx = gi.nodes[j];
                if (taken[j] || nx->op != GGML_OP_MUL_MAT || nx->src[1] != t->src[1] || nx->src[0]->type != t->src[0]->type)
                    break;
                g.nodes.push_back(nx);
                taken[j] = true;
            }
            plan.push_back(std::move(g));
            continue;
        }
        plan.push_back(Step{StepKind::Node, {t}});
    }
    return plan;
}

mx_tensor heads_of(const ggml_tensor *rows) {  // [n_heads * 128, n_rows] as [128, n_heads, n_rows]
    mx_tensor d = desc(rows);
    d.ne[2] = rows->ne[1];
    d.ne[1] = rows->ne[0] / 128;
    d.ne[0] = 128;
    d.nb[2] = rows->nb[1];
    d.nb[1] = 128 * rows->nb[0];
    d.nb[3] = d.nb[2] * (size_t)d.ne[2];
    return d;
}

// The nodes of a fusion one at a time (what the fused entry point declined), products still grouped.
int run_unfused(BackendCtx *ctx, const Step &st) {
    std::vector<const ggml_tensor *> group;
    for (const ggml_tensor *n : st.nodes) {
        if (!n) continue;
        if (n->op == GGML_OP_MUL_MAT && (group.empty() || n->src[1] == group[0]->src[1])) {
            group.push_back(n);
            continue;
        }
        int rc = group.empty() ? MX_SUCCESS : run_products(ctx, group);
        group.clear();
        if (rc == MX_SUCCESS && n->op == GGML_OP_MUL_MAT) {
            group.push_back(n);
            continue;
        }
        if (rc == MX_SUCCESS) rc = run_node(ctx, n);
        if (rc != MX_SUCCESS) return rc;
    }
    return group.empty() ? MX_SUCCESS : run_products(ctx, group);
}

int run_step(BackendCtx *ctx, const Step &st) {
    switch (st.kind) {
        case StepKind::Node: return run_node(ctx, st.nodes[0]);
        case StepKind::Products: return run_products(ctx, st.nodes);
        case StepKind::Experts: {
            const int n = (int)st.nodes.size();
            std::vector<mx_tensor> w(n), y(n);
            std::vector<const mx_tensor *> wp(n), yp(n);
            for (int k = 0; k < n; k++) {
                w[k] = desc(st.nodes[k]->src[0]);
                y[k] = desc(st.nodes[k]);
                wp[k] = &w[k];
                yp[k] = &y[k];
            }
            const mx_tensor b = desc(st.nodes[0]->src[1]), ids = desc(st.nodes[0]->src[2]);
            const int rc = mx_mul_mat_id_group(ctx->be, n, wp.data(), &b, &ids, yp.data());
            ctx->counts[rc == MX_UNSUPPORTED ? kDeclined : kExpertsGroup]++;
            if (rc != MX_UNSUPPORTED) return rc;
            for (const ggml_tensor *e : st.nodes) {
                const int r = run_node(ctx, e);
                if (r != MX_SUCCESS) return r;
            }
            return MX_SUCCESS;
        }
        case StepKind::NormProducts: {
            const ggml_tensor *norm = st.nodes[0], *mul = st.nodes[1];
            const int n = (int)st.nodes.size() - 2;
            std::vector<mx_tensor> w(n), y(n);
            std::vector<const mx_tensor *> wp(n), yp(n);
            for (int k = 0; k < n; k++) {
                w[k] = desc(st.nodes[2 + k]->src[0]);
                y[k] = desc(st.nodes[2 + k]);
                wp[k] = &w[k];
                yp[k] = &y[k];
            }
            const mx_tensor x = desc(norm->src[0]), nw = desc(mul->src[1]);
            const mx_fusion f{&nw, op_f32(norm, 0), nullptr, nullptr};
            const int rc = mx_mul_mat_fused(ctx->be, n, wp.data(), &x, yp.data(), &f);
            ctx->counts[rc == MX_UNSUPPORTED ? kDeclined : kNormProducts]++;
            return rc == MX_UNSUPPORTED ? run_unfused(ctx, st) : rc;
        }
        case StepKind::ProductOut: {
            const ggml_tensor *glu = st.nodes[0], *prod = st.nodes[1], *add = st.nodes[2];
            const ggml_tensor *res = add->src[0] == prod ? add->src[1] : add->src[0];
            const mx_tensor w = desc(prod->src[0]), d = desc(add), r = desc(res);
            const mx_tensor x = glu ? desc(glu->src[0]) : desc(prod->src[1]);
            const mx_tensor b = glu ? desc(glu->src[1]) : mx_tensor{};
            const mx_tensor *wp = &w, *dp = &d, *rp = &r;
            const mx_fusion f{nullptr, 0.0f, glu ? &b : nullptr, &rp};
            const int rc = mx_mul_mat_fused(ctx->be, 1, &wp, &x, &dp, &f);
            ctx->counts[rc == MX_UNSUPPORTED ? kDeclined : kProductOut]++;
            return rc == MX_UNSUPPORTED ? run_unfused(ctx, st) : rc;
        }
        case StepKind::Attention: {
            const ggml_tensor *nq = st.nodes[0], *mq = st.nodes[1], *nk = st.nodes[2], *mk = st.nodes[3];
            const ggml_tensor *sv = st.nodes[4], *rq = st.nodes[5], *sk = st.nodes[7], *fa = st.nodes[8];
            const mx_tensor q = desc(nq->src[0]), k = desc(nk->src[0]), v = heads_of(sv->src[0]);
            const mx_tensor qw = desc(mq->src[1]), kw = desc(mk->src[1]), pos = desc(rq->src[1]);
            const mx_tensor kc = desc(sk), vc = desc(sv);  // the caches, as the stores see them
            const mx_tensor kv = desc(fa->src[1]), vv = desc(fa->src[2]), d = desc(fa);
            const mx_tensor m = fa->src[3] ? desc(fa->src[3]) : mx_tensor{};
            const float eps = op_f32(nq, 0);
            const int n_dims = rq->op_params[1], mode = rq->op_params[2];
            const float base = op_f32(rq, 5), fscale = op_f32(rq, 6), ext = op_f32(rq, 7), attn = op_f32(rq, 8);
            int rc = mx_attn_decode(ctx->be, &q, &k, &v, &qw, &kw, &pos, &kc, &vc, &kv, &vv, fa->src[3] ? &m : nullptr,
                                    &d, eps, n_dims, mode, base, fscale, ext, attn, op_f32(fa, 0));
            if (rc != MX_UNSUPPORTED) {
                ctx->counts[kAttention]++;
                return rc;
            }
            // several rows (a prefill block): the norms, RoPE and stores in one launch, then the attention
            const mx_tensor qo = desc(rq);
            rc = mx_qk_norm_rope_kv(ctx->be, &q, &k, &v, &qw, &kw, &pos, &qo, &kc, &vc, eps, n_dims, mode, base, fscale,
                                    ext, attn);
            ctx->counts[rc == MX_UNSUPPORTED ? kDeclined : kAttentionRows]++;
            if (rc == MX_SUCCESS) return run_node(ctx, fa);
            return rc == MX_UNSUPPORTED ? run_unfused(ctx, st) : rc;
        }
    }
    return MX_FAILED;
}

// Runs a graph's nodes in order, as the steps of its plan: consecutive MUL_MATs that read the same src1 (q/k/v,
// gate/up) as one launch, and the decoder's fusions -- norm x weight into the products that read it, SwiGLU and the
// residual ADD into the product between them, a decode row's q/k norms, RoPE, cache stores and attention into one
// launch -- where every intermediate they skip is read by no other node and is not a graph output. A fusion libmx
// declines (shapes its fused kernels do not take) runs as its separate nodes.
int run_nodes(BackendCtx *ctx, ggml_cgraph *cgraph) {
    const GraphInfo gi(cgraph);
    for (const Step &st : plan_graph(gi)) {
        const int rc = run_step(ctx, st);
        if (rc != MX_SUCCESS) {
            const ggml_tensor *n = st.nodes.back();
            GGML_LOG_ERROR("%s: %s (%s): %s\n", __func__, n->name, ggml_op_desc(n), mx_last_error());
            return rc;
        }
    }
    return MX_SUCCESS;
}

void key_of(const ggml_tensor *t, TensorKey &k) {
    if (!t) return;  // stays zero
    k.type = (int32_t)t->type;
    k.flags = t->flags;
    for (int d = 0; d < 4; d++) {
        k.ne[d] = t->ne[d];
        k.nb[d] = (uint64_t)t->nb[d];
    }
    k.data = t->data;
    k.view_offs = (uint64_t)t->view_offs;
}

std::vector<NodeKey> keys_of(ggml_cgraph *cgraph) {
    std::vector<NodeKey> keys;
    for (int i = 0; i < ggml_graph_n_nodes(cgraph); i++) {
        const ggml_tensor *t = ggml_graph_node(cgraph, i);
        NodeKey k;
        std::memset(&k, 0, sizeof k);
        k.op = (int32_t)t->op;
        k.uses = ggml_node_get_use_count(cgraph, i);
        std::memcpy(k.op_params, t->op_params, sizeof k.op_params);
        key_of(t, k.t[0]);
        for (int s = 0; s < 5; s++) key_of(t->src[s], k.t[s + 1]);
        keys.push_back(k);
    }
    return keys;
}

// The same graph over the same tensors computed again (the kept decode-step graph, src/common/qwen3-decoder.cpp:
// 187-208; each split of a step ggml_backend_sched computes, src/families/drama3/text-model.cpp:91-97) is recorded
// once its scratch has its final size and replayed with one launch from then on. Graphs are told apart by every
// node's op, parameters and whole-graph use count and every tensor's type, shape, strides, address and view offset;
// the backend keeps the last kSeenGraphs of them, each with its own count and recording (a dropped one is freed;
// mx_graph_free waits for a replay still in flight). A recording libmx refuses because the scratch grew since
// (MX_FAILED) is recorded again on the next identical computation.
enum ggml_status backend_graph_compute(ggml_backend_t backend, ggml_cgraph *cgraph) {
    auto *ctx = (BackendCtx *)backend->context;
    std::vector<NodeKey> keys = keys_of(cgraph);
    SeenGraph *g = nullptr;
    for (SeenGraph &e : ctx->seen)
        if (e.keys == keys) g = &e;
    if (g) {
        g->repeats++;
    } else {
        if (ctx->seen.size() >= kSeenGraphs) {
            auto oldest = std::min_element(ctx->seen.begin(), ctx->seen.end(), [](const SeenGraph &a, const SeenGraph &b) {
                return a.last_use < b.last_use;
            });
            mx_graph_free(oldest->replay);
            ctx->seen.erase(oldest);
        }
        ctx->seen.push_back(SeenGraph{std::move(keys), 0, nullptr, 0});
        g = &ctx->seen.back();
    }
    g->last_use = ++ctx->clock;
    if (g->replay) {
        const int rc = mx_graph_launch(ctx->be, g->replay);
        if (rc == MX_SUCCESS) {
            ctx->counts[kReplayed]++;
            return GGML_STATUS_SUCCESS;
        }
        mx_graph_free(g->replay);  // recorded before the scratch grew: compute eagerly, record again next time
        g->replay = nullptr;
        g->repeats = 1;
    }
    if (g->repeats >= 2) {
        int rc = mx_graph_begin(ctx->be);
        if (rc == MX_SUCCESS) {
            const int run = run_nodes(ctx, cgraph);
            mx_graph *rec = nullptr;
            rc = mx_graph_end(ctx->be, &rec);
            if (run == MX_SUCCESS && rc == MX_SUCCESS) {
                g->replay = rec;
                ctx->counts[kRecorded]++;
                return to_status(mx_graph_launch(ctx->be, rec));
            }
            mx_graph_free(rec);
        }
        g->repeats = -1000000;  // not recordable: compute it eagerly from now on
    }
    ctx->counts[kEager]++;
    return to_status(run_nodes(ctx, cgraph));
}

void backend_event_record(ggml_backend_t backend, ggml_backend_event_t event) {
    report(mx_event_record(((BackendCtx *)backend->context)->be, (mx_event *)event->context), "event_record");
}

const ggml_backend_i kBackendIface = {
    /* .get_name           = */ backend_get_name,
    /* .free               = */ backend_free,
    /* .set_tensor_async   = */ nullptr,
    /* .get_tensor_async   = */ nullptr,
    /* .cpy_tensor_async   = */ nullptr,
    /* .synchronize        = */ backend_synchronize,
    /* .graph_plan_create  = */ nullptr,
    /* .graph_plan_free    = */ nullptr,
    /* .graph_plan_update  = */ nullptr,
    /* .graph_plan_compute = */ nullptr,
    /* .graph_compute      = */ backend_graph_compute,
    /* .event_record       = */ backend_event_record,
    /* .event_wait         = */ nullptr,
    /* .graph_optimize     = */ nullptr,
};

ggml_guid_t backend_guid() {
    static ggml_guid guid = {0x6d, 0x69, 0x33, 0x35, 0x35, 0x78, 0x2d, 0x71,
                             0x75, 0x61, 0x6e, 0x74, 0x2d, 0x6d, 0x6d, 0x31};
    return &guid;
}

// ------------------------------------------------------------------------------------------------------ device
const char *dev_get_name(ggml_backend_dev_t dev) { return ((DeviceCtx *)dev->context)->name.c_str(); }
const char *dev_get_description(ggml_backend_dev_t dev) { return ((DeviceCtx *)dev->context)->description.c_str(); }

void dev_get_memory(ggml_backend_dev_t dev, size_t *free, size_t *total) {
    report(mx_device_memory(((DeviceCtx *)dev->context)->device, free, total), "get_memory");
}

enum ggml_backend_dev_type dev_get_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_get_props(ggml_backend_dev_t dev, ggml_backend_dev_props *props) {
    props->name = dev_get_name(dev);
    props->description = dev_get_description(dev);
    props->type = dev_get_type(dev);
    dev_get_memory(dev, &props->memory_free, &props->memory_total);
    props->caps.async = true;
    props->caps.host_buffer = false;
    props->caps.buffer_from_host_ptr = false;
    props->caps.events = true;
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t dev, const char *) {
    auto *dctx = (DeviceCtx *)dev->context;
    mx_backend *be = mx_backend_init(dctx->device);
    if (!be) {
        GGML_LOG_ERROR("%s: %s\n", __func__, mx_last_error());
        return nullptr;
    }
    auto *ctx = new BackendCtx();
    ctx->dev = dctx;
    ctx->be = be;
    return new ggml_backend{backend_guid(), kBackendIface, dev, ctx};
}

ggml_backend_buffer_type_t dev_get_buffer_type(ggml_backend_dev_t dev) { return &((DeviceCtx *)dev->context)->buft; }

bool in_our_buffer(const ggml_tensor *t, ggml_backend_dev_t dev) {
    return t && t->buffer && t->buffer->buft == dev_get_buffer_type(dev);
}

// True exactly for MUL_MAT / MUL_MAT_ID / GET_ROWS whose weight lives in this device's buffer type -- Q8_0, Q4_K,
// Q5_K, Q6_K for all three; F16 / F32 (the storages of storage.cpp:52-89 besides the K-quants) for MUL_MAT and
// GET_ROWS --, for ARGMAX over f32 logits in it (the greedy pick after the head, qwen3-decoder.cpp:428,501), and for
// the decoder layer's RMS_NORM, ADD, MUL, GLU (swiglu), ROPE (NEOX), SET_ROWS and FLASH_ATTN_EXT over a KV cache in
// it, with the shapes, strides and parameters libmx computes; everything else stays on the CPU backend.
bool dev_supports_op(ggml_backend_dev_t dev, const ggml_tensor *op) {
    // the decoder layer's other ops (qwen3-decoder.cpp:350-410): f32 rows wherever they live (the scheduler copies
    // inputs), except the KV cache, which SET_ROWS writes and FLASH_ATTN_EXT reads in place and must be this device's
    switch (op->op) {
        case GGML_OP_RMS_NORM: {
            const mx_tensor s0 = planned(op->src[0]), d = planned(op);
            return mx_supports_op(MX_OP_RMS_NORM, &s0, nullptr, nullptr, &d) != 0;
        }
        case GGML_OP_ADD:
        case GGML_OP_MUL: {
            const mx_tensor a = planned(op->src[0]), b = planned(op->src[1]), d = planned(op);
            return mx_supports_op(op->op == GGML_OP_ADD ? MX_OP_ADD : MX_OP_MUL, &a, &b, nullptr, &d) != 0;
        }
        case GGML_OP_GLU: {
            // the split form ggml_swiglu_split(a, b), not swapped
            if (ggml_get_glu_op(op) != GGML_GLU_OP_SWIGLU || !op->src[1] || op->op_params[1] != 0) return false;
            const mx_tensor a = planned(op->src[0]), b = planned(op->src[1]), d = planned(op);
            return mx_supports_op(MX_OP_SWIGLU, &a, &b, nullptr, &d) != 0;
        }
        case GGML_OP_ROPE: {
            if (op->src[2]) return false;  // frequency factors
            const mx_tensor x = planned(op->src[0]), pos = planned(op->src[1]), d = planned(op);
            return mx_supports_rope(&x, &pos, &d, op->op_params[1], op->op_params[2], op_f32(op, 7), op_f32(op, 8)) != 0;
        }
        case GGML_OP_SET_ROWS: {
            if (!in_our_buffer(op->view_src ? op->view_src : op, dev)) return false;
            const mx_tensor src = planned(op->src[0]), idx = planned(op->src[1]), d = planned(op);
            return mx_supports_op(MX_OP_SET_ROWS, &src, &idx, nullptr, &d) != 0;
        }
        case GGML_OP_FLASH_ATTN_EXT: {
            if (op->src[4] || !in_our_buffer(op->src[1], dev) || !in_our_buffer(op->src[2], dev)) return false;  // sinks
            const mx_tensor q = planned(op->src[0]), k = planned(op->src[1]), v = planned(op->src[2]), d = planned(op);
            const mx_tensor m = op->src[3] ? planned(op->src[3]) : mx_tensor{};
            return mx_supports_flash_attn_ext(&q, &k, &v, op->src[3] ? &m : nullptr, &d, op_f32(op, 1),
                                              op_f32(op, 2)) != 0;
        }
        default: break;
    }
    if (op->op == GGML_OP_ARGMAX) {
        const ggml_tensor *x = op->src[0];
        if (!in_our_buffer(x, dev)) return false;
        mx_tensor s0 = desc(x), d = desc(op);
        alignas(256) static const char placeholder[256] = {};
        if (!s0.data) s0.data = (void *)placeholder;
        if (!d.data) d.data = (void *)placeholder;
        return mx_supports_op(MX_OP_ARGMAX, &s0, nullptr, nullptr, &d) != 0;
    }
    if (op->op != GGML_OP_MUL_MAT && op->op != GGML_OP_MUL_MAT_ID && op->op != GGML_OP_GET_ROWS) return false;
    const ggml_tensor *w = op->src[0];
    if (!in_our_buffer(w, dev) || (w->view_src && w->view_offs != 0)) return false;
    const mx_tensor s0 = desc(w), d = desc(op);
    const mx_tensor s1 = op->src[1] ? desc(op->src[1]) : mx_tensor{};
    const mx_tensor s2 = op->src[2] ? desc(op->src[2]) : mx_tensor{};
    // src1 / src2 / dst have no data yet while the scheduler plans: libmx checks their alignment with a placeholder
    // aligned address (this buffer type's allocations are 256-byte aligned).
    mx_tensor p1 = s1, p2 = s2, pd = d, p0 = s0;
    alignas(256) static const char placeholder[256] = {};
    if (!p0.data) p0.data = (void *)placeholder;
    if (!p1.data) p1.data = (void *)placeholder;
    if (!p2.data) p2.data = (void *)placeholder;
    if (!pd.data) pd.data = (void *)placeholder;
    const int mxop = op->op == GGML_OP_MUL_MAT ? MX_OP_MUL_MAT : (op->op == GGML_OP_MUL_MAT_ID ? MX_OP_MUL_MAT_ID : MX_OP_GET_ROWS);
    return mx_supports_op(mxop, &p0, op->src[1] ? &p1 : nullptr, op->src[2] ? &p2 : nullptr, &pd) != 0;
}

bool dev_supports_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft) { return buft == dev_get_buffer_type(dev); }

bool dev_offload_op(ggml_backend_dev_t, const ggml_tensor *) { return false; }

ggml_backend_event_t dev_event_new(ggml_backend_dev_t dev) {
    mx_event *e = mx_event_new(((DeviceCtx *)dev->context)->io);
    if (!e) return nullptr;
    return new ggml_backend_event{dev, e};
}

void dev_event_free(ggml_backend_dev_t, ggml_backend_event_t event) {
    mx_event_free((mx_event *)event->context);
    delete event;
}

void dev_event_synchronize(ggml_backend_dev_t, ggml_backend_event_t event) {
    report(mx_event_synchronize((mx_event *)event->context), "event_synchronize");
}

const ggml_backend_device_i kDeviceIface = {
    /* .get_name             = */ dev_get_name,
    /* .get_description      = */ dev_get_description,
    /* .get_memory           = */ dev_get_memory,
    /* .get_type             = */ dev_get_type,
    /* .get_props            = */ dev_get_props,
    /* .init_backend         = */ dev_init_backend,
    /* .get_buffer_type      = */ dev_get_buffer_type,
    /* .get_host_buffer_type = */ nullptr,
    /* .buffer_from_host_ptr = */ nullptr,
    /* .supports_op          = */ dev_supports_op,
    /* .supports_buft        = */ dev_supports_buft,
    /* .offload_op           = */ dev_offload_op,
    /* .event_new            = */ dev_event_new,
    /* .event_free           = */ dev_event_free,
    /* .event_synchronize    = */ dev_event_synchronize,
};

// ------------------------------------------------------------------------------------------------ the linked ggml
// Whether the ggml this library runs in numbers ops, types and GLU ops, lays out a tensor and places operation
// parameters as the headers this backend was built with. ggml_op values move between ggml versions as ops are added,
// so a backend built against other headers than its host's would otherwise run the wrong op. Checked once by the
// registry, before it registers any device; the first difference is logged.
bool differs(const char *what, const char *want, const char *got) {
    GGML_LOG_ERROR("ggml_backend_mi355x_reg: the linked ggml has %s '%s' where this backend was built with '%s': no "
                   "MI355X device is registered\n", what, got ? got : "(null)", want);
    return false;
}

bool linked_ggml_matches() {
    static const struct {
        ggml_op op;
        const char *name;
    } ops[] = {{GGML_OP_NONE, "NONE"},         {GGML_OP_ADD, "ADD"},
               {GGML_OP_MUL, "MUL"},           {GGML_OP_ARGMAX, "ARGMAX"},
               {GGML_OP_RMS_NORM, "RMS_NORM"}, {GGML_OP_MUL_MAT, "MUL_MAT"},
               {GGML_OP_MUL_MAT_ID, "MUL_MAT_ID"}, {GGML_OP_RESHAPE, "RESHAPE"},
               {GGML_OP_VIEW, "VIEW"},         {GGML_OP_PERMUTE, "PERMUTE"},
               {GGML_OP_TRANSPOSE, "TRANSPOSE"}, {GGML_OP_GET_ROWS, "GET_ROWS"},
               {GGML_OP_SET_ROWS, "SET_ROWS"}, {GGML_OP_ROPE, "ROPE"},
               {GGML_OP_FLASH_ATTN_EXT, "FLASH_ATTN_EXT"}, {GGML_OP_GLU, "GLU"}};
    for (const auto &o : ops) {
        const char *got = ggml_op_name(o.op);
        if (!got || std::strcmp(got, o.name) != 0) return differs("op", o.name, got);
    }
    static const struct {
        ggml_type type;
        const char *name;
    } types[] = {{GGML_TYPE_F32, "f32"},   {GGML_TYPE_F16, "f16"},   {GGML_TYPE_Q8_0, "q8_0"}, {GGML_TYPE_Q4_K, "q4_K"},
                 {GGML_TYPE_Q5_K, "q5_K"}, {GGML_TYPE_Q6_K, "q6_K"}, {GGML_TYPE_I32, "i32"}};
    for (const auto &t : types) {
        const char *got = ggml_type_name(t.type);
        if (!got || std::strcmp(got, t.name) != 0) return differs("type", t.name, got);
    }
    const char *glu = ggml_glu_op_name(GGML_GLU_OP_SWIGLU);
    if (!glu || std::strcmp(glu, "SWIGLU") != 0) return differs("GLU op", "SWIGLU", glu);
    // tensors made by the linked ggml, read through this backend's view of ggml_tensor
    ggml_init_params ip{1024 * 1024, nullptr, true};
    ggml_context *ctx = ggml_init(ip);
    if (!ctx) return differs("ggml_init result", "a context", nullptr);
    bool ok = true;
    ggml_tensor *w = ggml_new_tensor_2d(ctx, GGML_TYPE_Q8_0, 64, 3);
    ggml_set_name(w, "mi355x-abi");
    ok = ok && w->type == GGML_TYPE_Q8_0 && w->ne[0] == 64 && w->ne[1] == 3 && w->ne[2] == 1 && w->ne[3] == 1 &&
         w->nb[0] == 34 && w->nb[1] == 68 && w->nb[2] == 204 && w->op == GGML_OP_NONE && !w->data && !w->view_src &&
         !w->buffer && std::strcmp(w->name, "mi355x-abi") == 0 && ggml_nbytes(w) == 204;
    if (!ok) differs("ggml_tensor layout", "ggml.h's", "another");
    ggml_tensor *x = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, 128, 2, 1);
    ggml_tensor *pos = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, 1);
    if (ok) {
        ggml_tensor *n = ggml_rms_norm(ctx, x, 0.5f);
        ggml_tensor *r = ggml_rope_ext(ctx, x, pos, nullptr, 128, GGML_ROPE_TYPE_NEOX, 0, 1e6f, 1.0f, 0.0f, 1.0f, 0.0f,
                                       0.0f);
        ggml_tensor *g = ggml_swiglu_split(ctx, x, x);
        ok = n->op == GGML_OP_RMS_NORM && op_f32(n, 0) == 0.5f && r->op == GGML_OP_ROPE && r->op_params[1] == 128 &&
             r->op_params[2] == GGML_ROPE_TYPE_NEOX && op_f32(r, 5) == 1e6f && op_f32(r, 6) == 1.0f &&
             op_f32(r, 8) == 1.0f && r->src[0] == x && r->src[1] == pos && g->op == GGML_OP_GLU &&
             ggml_get_glu_op(g) == GGML_GLU_OP_SWIGLU && g->op_params[1] == 0 && g->src[1] == x;
        if (!ok) differs("operation parameters", "ggml.c's", "others");
    }
    if (ok) {
        // a graph's layout and use counts, read as the fusions read them: n is read twice, m once, a not at all;
        // a view of the last two nodes (one split of the graph) sees the same counts
        ggml_tensor *n = ggml_rms_norm(ctx, x, 0.5f);
        ggml_tensor *m = ggml_mul(ctx, n, n);
        ggml_tensor *a = ggml_add(ctx, m, x);
        ggml_cgraph *g = ggml_new_graph_custom(ctx, 16, false);
        ok = g != nullptr;
        if (ok) {
            ggml_build_forward_expand(g, a);
            // nodes [1, 3) as ggml_graph_view forms a split: the same hash set and use counts
            ggml_cgraph v = *g;
            v.size = 0;
            v.n_nodes = 2;
            v.n_leafs = 0;
            v.nodes = g->nodes + 1;
            v.leafs = nullptr;
            ok = ggml_graph_n_nodes(g) == 3 && g->n_nodes == 3 && g->nodes[0] == n && g->nodes[1] == m &&
                 g->nodes[2] == a && ggml_node_get_use_count(g, 0) == 2 && ggml_node_get_use_count(g, 1) == 1 &&
                 ggml_node_get_use_count(g, 2) == 0 && v.n_nodes == 2 && v.nodes[0] == m &&
                 ggml_node_get_use_count(&v, 0) == 1;
        }
        if (!ok) differs("graph layout or use counts", "ggml-impl.h's", "others");
    }
    ggml_free(ctx);
    return ok;
}

bool linked_ggml_ok() {
    static const bool ok = linked_ggml_matches();
    return ok;
}

// -------------------------------------------------------------------------------------------------------- reg
struct RegCtx {
    std::vector<std::unique_ptr<DeviceCtx>> ctxs;
    std::vector<ggml_backend_device> devices;
};

const char *reg_get_name(ggml_backend_reg_t) { return "MI355X"; }
size_t reg_get_device_count(ggml_backend_reg_t reg) { return ((RegCtx *)reg->context)->devices.size(); }
ggml_backend_dev_t reg_get_device(ggml_backend_reg_t reg, size_t index) {
    auto *ctx = (RegCtx *)reg->context;
    return index < ctx->devices.size() ? &ctx->devices[index] : nullptr;
}
// A backend's counters (enum Count, in that order) into out[0 .. n).
void backend_counters(ggml_backend_t backend, int64_t *out, int n) {
    const auto *ctx = (const BackendCtx *)backend->context;
    for (int i = 0; i < n && i < kCounts; i++) out[i] = ctx->counts[i];
}

// The steps graph_compute would run a graph as (no device needed): each step's kind (StepKind, in that order) and
// its first node's index; returns the number of steps, of which at most max are written.
int graph_plan(ggml_cgraph *cgraph, int32_t *kinds, int32_t *first, int max) {
    const GraphInfo gi(cgraph);
    const std::vector<Step> plan = plan_graph(gi);
    for (int i = 0; i < (int)plan.size() && i < max; i++) {
        kinds[i] = (int32_t)plan[i].kind;
        const ggml_tensor *n = plan[i].nodes[0] ? plan[i].nodes[0] : plan[i].nodes[1];
        first[i] = gi.pos(n);
    }
    return (int)plan.size();
}

// The backend's own functions, by name:
//   "ggml_backend_mi355x_abi_ok"    bool (*)(void): whether the linked ggml matched the headers this backend was built
//                                   with (no device is registered otherwise);
//   "ggml_backend_mi355x_counters"  void (*)(ggml_backend_t, int64_t *out, int n): what graph_compute did;
//   "ggml_backend_mi355x_plan"      int (*)(ggml_cgraph *, int32_t *kinds, int32_t *first, int max): its plan of a graph.
void *reg_get_proc_address(ggml_backend_reg_t, const char *name) {
    if (name && std::strcmp(name, "ggml_backend_mi355x_abi_ok") == 0) return (void *)&linked_ggml_ok;
    if (name && std::strcmp(name, "ggml_backend_mi355x_counters") == 0) return (void *)&backend_counters;
    if (name && std::strcmp(name, "ggml_backend_mi355x_plan") == 0) return (void *)&graph_plan;
    return nullptr;
}

const ggml_backend_reg_i kRegIface = {
    /* .get_name         = */ reg_get_name,
    /* .get_device_count = */ reg_get_device_count,
    /* .get_device       = */ reg_get_device,
    /* .get_proc_address = */ reg_get_proc_address,
};

}  // namespace

ggml_backend_reg_t ggml_backend_mi355x_reg(void) {
    static ggml_backend_reg reg;
    static std::once_flag once;
    std::call_once(once, [] {
        auto *ctx = new RegCtx();
        const int n = linked_ggml_ok() ? mx_device_count() : 0;
        ctx->devices.reserve(n);
        for (int i = 0; i < n; i++) {
            auto dctx = std::make_unique<DeviceCtx>();
            dctx->device = i;
            dctx->name = "MI355X" + std::to_string(i);
            char desc[256] = {0};
            mx_device_description(i, desc, sizeof desc);
            dctx->description = desc;
            dctx->io = mx_backend_init(i);
            if (!dctx->io) {
                GGML_LOG_ERROR("%s: device %d: %s\n", __func__, i, mx_last_error());
                continue;
            }
            ctx->devices.push_back(ggml_backend_device{kDeviceIface, &reg, dctx.get()});
            dctx->buft = ggml_backend_buffer_type{kBuftIface, &ctx->devices.back(), dctx.get()};
            ctx->ctxs.push_back(std::move(dctx));
        }
        reg = ggml_backend_reg{GGML_BACKEND_API_VERSION, kRegIface, ctx};
    });
    return &reg;
}

GGML_BACKEND_DL_IMPL(ggml_backend_mi355x_reg)
