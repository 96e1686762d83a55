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

#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-impl.h"
#include "mx.h"

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
// strides, data address and view offset.
struct TensorKey {
    int32_t type;
    int32_t pad_;
    int64_t ne[4];
    uint64_t nb[4];
    const void *data;
    uint64_t view_offs;
};

// One step of the last graph computed, to recognise a graph computed again with the same tensors: the node (with its
// operation parameters: eps, RoPE's dims / mode / bases, attention's scale) and its first five sources.
struct NodeKey {
    int32_t op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    TensorKey t[6];
    bool operator==(const NodeKey &o) const { return std::memcmp(this, &o, sizeof(NodeKey)) == 0; }
};

struct BackendCtx {
    DeviceCtx *dev = nullptr;
    mx_backend *be = nullptr;
    std::vector<NodeKey> last;   // the previous graph's nodes
    int repeats = 0;             // how many times in a row it came again
    mx_graph *replay = nullptr;  // recorded from the third identical graph on
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
    mx_graph_free(ctx->replay);
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

// Runs the graph's nodes in order. Consecutive MUL_MATs that read the same src1 (q/k/v, gate/up) go to the device as
// one launch.
int run_nodes(BackendCtx *ctx, ggml_cgraph *cgraph) {
    const int n = ggml_graph_n_nodes(cgraph);
    for (int i = 0; i < n; i++) {
        ggml_tensor *node = ggml_graph_node(cgraph, i);
        if (is_noop(node)) continue;
        int rc = MX_SUCCESS;
        switch (node->op) {
            case GGML_OP_MUL_MAT: {
                std::vector<ggml_tensor *> group{node};
                for (int j = i + 1; j < n && group.size() < 4; j++) {
                    ggml_tensor *nx = ggml_graph_node(cgraph, j);
                    if (nx->op != GGML_OP_MUL_MAT || nx->src[1] != node->src[1] || nx->src[0]->type != node->src[0]->type)
                        break;
                    group.push_back(nx);
                }
                if (group.size() == 1) {
                    const mx_tensor s0 = desc(node->src[0]), s1 = desc(node->src[1]), d = desc(node);
                    rc = mx_mul_mat(ctx->be, &s0, &s1, &d);
                } else {
                    std::vector<mx_tensor> w, y;
                    for (ggml_tensor *g : group) {
                        w.push_back(desc(g->src[0]));
                        y.push_back(desc(g));
                    }
                    std::vector<const mx_tensor *> wp, yp;
                    for (size_t k = 0; k < group.size(); k++) {
                        wp.push_back(&w[k]);
                        yp.push_back(&y[k]);
                    }
                    const mx_tensor s1 = desc(node->src[1]);
                    rc = mx_mul_mat_group(ctx->be, (int)group.size(), wp.data(), &s1, yp.data());
                    if (rc == MX_UNSUPPORTED) {  // members of different shape classes: one at a time
                        rc = MX_SUCCESS;
                        for (size_t k = 0; k < group.size() && rc == MX_SUCCESS; k++)
                            rc = mx_mul_mat(ctx->be, wp[k], &s1, yp[k]);
                    }
                    i += (int)group.size() - 1;
                }
                break;
            }
            case GGML_OP_MUL_MAT_ID: {
                const mx_tensor as = desc(node->src[0]), b = desc(node->src[1]), ids = desc(node->src[2]), d = desc(node);
                rc = mx_mul_mat_id(ctx->be, &as, &b, &ids, &d);
                break;
            }
            case GGML_OP_GET_ROWS: {
                const mx_tensor s0 = desc(node->src[0]), ids = desc(node->src[1]), d = desc(node);
                rc = mx_get_rows(ctx->be, &s0, &ids, &d);
                break;
            }
            case GGML_OP_ARGMAX: {
                const mx_tensor s0 = desc(node->src[0]), d = desc(node);
                rc = mx_argmax(ctx->be, &s0, &d);
                break;
            }
            case GGML_OP_RMS_NORM: {
                const mx_tensor s0 = desc(node->src[0]), d = desc(node);
                rc = mx_rms_norm(ctx->be, &s0, &d, op_f32(node, 0), nullptr);
                break;
            }
            case GGML_OP_ADD:
            case GGML_OP_MUL: {
                const mx_tensor a = desc(node->src[0]), b = desc(node->src[1]), d = desc(node);
                rc = mx_binary(ctx->be, node->op == GGML_OP_ADD ? MX_OP_ADD : MX_OP_MUL, &a, &b, &d);
                break;
            }
            case GGML_OP_GLU: {
                const mx_tensor a = desc(node->src[0]), b = desc(node->src[1]), d = desc(node);
                rc = mx_swiglu(ctx->be, &a, &b, &d);
                break;
            }
            case GGML_OP_ROPE: {
                const mx_tensor x = desc(node->src[0]), pos = desc(node->src[1]), d = desc(node);
                rc = mx_rope(ctx->be, &x, &pos, &d, node->op_params[1], node->op_params[2], op_f32(node, 5),
                             op_f32(node, 6), op_f32(node, 7), op_f32(node, 8));
                break;
            }
            case GGML_OP_SET_ROWS: {
                const mx_tensor src = desc(node->src[0]), idx = desc(node->src[1]), d = desc(node);
                rc = mx_set_rows(ctx->be, &src, &idx, &d);
                break;
            }
            case GGML_OP_FLASH_ATTN_EXT: {
                const mx_tensor q = desc(node->src[0]), k = desc(node->src[1]), v = desc(node->src[2]), d = desc(node);
                const mx_tensor m = node->src[3] ? desc(node->src[3]) : mx_tensor{};
                rc = mx_flash_attn_ext(ctx->be, &q, &k, &v, node->src[3] ? &m : nullptr, &d, op_f32(node, 0));
                break;
            }
            default:
                GGML_LOG_ERROR("%s: op %s is not computed by the MI355X backend\n", __func__, ggml_op_desc(node));
                return MX_UNSUPPORTED;
        }
        if (rc != MX_SUCCESS) {
            GGML_LOG_ERROR("%s: %s (%s): %s\n", __func__, node->name, ggml_op_desc(node), mx_last_error());
            return rc;
        }
    }
    return MX_SUCCESS;
}

void key_of(const ggml_tensor *t, TensorKey &k) {
    if (!t) return;  // stays zero
    k.type = (int32_t)t->type;
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
        std::memcpy(k.op_params, t->op_params, sizeof k.op_params);
        key_of(t, k.t[0]);
        for (int s = 0; s < 5; s++) key_of(t->src[s], k.t[s + 1]);
        keys.push_back(k);
    }
    return keys;
}

// The same graph over the same tensors computed again (the kept decode-step graph, src/common/qwen3-decoder.cpp:
// 187-208) is recorded once its scratch has its final size and replayed with one launch from then on. A graph that
// differs in any node's op, parameters, or any tensor's type, shape, strides, address or view offset is computed
// eagerly and the recording dropped (mx_graph_free waits for a replay still in flight). A recording libmx refuses
// because the scratch grew since (MX_FAILED) is recorded again on the next identical graph.
enum ggml_status backend_graph_compute(ggml_backend_t backend, ggml_cgraph *cgraph) {
    auto *ctx = (BackendCtx *)backend->context;
    std::vector<NodeKey> keys = keys_of(cgraph);
    if (keys == ctx->last) {
        ctx->repeats++;
    } else {
        ctx->last = std::move(keys);
        ctx->repeats = 0;
        mx_graph_free(ctx->replay);
        ctx->replay = nullptr;
    }
    if (ctx->replay) {
        const int rc = mx_graph_launch(ctx->be, ctx->replay);
        if (rc == MX_SUCCESS) return GGML_STATUS_SUCCESS;
        mx_graph_free(ctx->replay);  // recorded before the scratch grew: compute eagerly, record again next time
        ctx->replay = nullptr;
        ctx->repeats = 1;
    }
    if (ctx->repeats >= 2) {
        int rc = mx_graph_begin(ctx->be);
        if (rc == MX_SUCCESS) {
            const int run = run_nodes(ctx, cgraph);
            mx_graph *g = nullptr;
            rc = mx_graph_end(ctx->be, &g);
            if (run == MX_SUCCESS && rc == MX_SUCCESS) {
                ctx->replay = g;
                return to_status(mx_graph_launch(ctx->be, g));
            }
            mx_graph_free(g);
        }
        ctx->repeats = -1000000;  // not recordable: compute it eagerly from now on
    }
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
void *reg_get_proc_address(ggml_backend_reg_t, const char *) { return nullptr; }

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
        const int n = mx_device_count();
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
