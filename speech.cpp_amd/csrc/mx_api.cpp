// libmx C ABI: device, backend, buffers and the three ops. See include/mx.h for the contract of each entry point.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "mx_common.h"
#include "mx_dot.h"
#include "mx_error.h"

struct mx_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    int rounding = MX_ROUND_REF;
    int *err = nullptr;              // device word: bit 0 GET_ROWS index, bit 1 MUL_MAT_ID expert, bit 2 SET_ROWS index
                                     // out of range
    void *scratch = nullptr;         // grows on demand outside graph capture
    size_t scratch_size = 0;
    uint64_t scratch_gen = 0;        // counts scratch reallocations: a graph recorded before one holds a freed address
    uint8_t *staging = nullptr;      // device staging for ggml-layout uploads and downloads
    size_t staging_size = 0;
    bool capturing = false;
    mx::Options opt;                 // kernel choices (mx_backend_set_option)
};

struct mx_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    const mx_backend *be = nullptr;  // the backend whose stream and scratch the recorded kernels use
    uint64_t scratch_gen = 0;        // be->scratch_gen when recorded
};

struct mx_event {
    int device = 0;
    hipEvent_t ev = nullptr;
};

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

}  // namespace

int mx::set_error(int code, const char *msg) {
    g_error = msg ? msg : "";
    return code;
}

namespace {

int hip_fail(hipError_t e, const char *what) {
    return fail(e == hipErrorOutOfMemory ? MX_ALLOC_FAILED : MX_FAILED, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_OK(expr, what)                          \
    do {                                            \
        hipError_t e_ = (expr);                     \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

constexpr size_t kStagingPiece = 64ull << 20;  // bytes per upload / download piece
constexpr size_t kMaxLds = 64 * 1024;         // LDS a product kernel may ask for

// ggml's block geometry (ggml-common.h). Types this device does not compute (Q4_0 ... Q3_K, integers, F64, BF16) are
// held as plain bytes, so a model file's every tensor can live in the buffer type.
int64_t blck(int type) {
    switch (type) {
        case 2: case 3: case 6: case 7:                               // Q4_0, Q4_1, Q5_0, Q5_1
        case MX_TYPE_Q8_0: case MX_TYPE_Q8_1: return 32;
        case 10: case 11:                                             // Q2_K, Q3_K
        case MX_TYPE_Q4_K: case MX_TYPE_Q5_K: case MX_TYPE_Q6_K: case MX_TYPE_Q8_K: return 256;
        case MX_TYPE_F32: case MX_TYPE_F16: case MX_TYPE_I32:
        case 24: case 25: case 27: case 28: case 30: return 1;       // I8, I16, I64, F64, BF16
        default: return 0;
    }
}
size_t tsize(int type) {
    switch (type) {
        case 24: return 1;
        case MX_TYPE_F16: case 25: case 30: return 2;
        case MX_TYPE_F32: case MX_TYPE_I32: return 4;
        case 27: case 28: return 8;
        case 2: return 18;
        case 3: return 20;
        case 6: return 22;
        case 7: return 24;
        case MX_TYPE_Q8_0: return 34;
        case MX_TYPE_Q8_1: return 36;
        case 10: return 84;
        case 11: return 110;
        case MX_TYPE_Q4_K: return 144;
        case MX_TYPE_Q5_K: return 176;
        case MX_TYPE_Q6_K: return 210;
        case MX_TYPE_Q8_K: return 292;
        default: return 0;
    }
}

int64_t nelements(const mx_tensor *t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

// ggml_nbytes
size_t nbytes(const mx_tensor *t) {
    const int64_t b = blck(t->type);
    if (nelements(t) == 0 || b == 0) return 0;
    size_t n = b == 1 ? tsize(t->type) : (size_t)(t->ne[0] / b) * t->nb[0];
    if (b == 1) {
        for (int i = 0; i < 4; i++) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    } else {
        for (int i = 1; i < 4; i++) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    }
    return n;
}

bool contiguous(const mx_tensor *t) {
    const int64_t b = blck(t->type);
    if (b == 0 || t->ne[0] % b != 0) return false;
    if (t->nb[0] != tsize(t->type)) return false;
    const uint64_t row = (uint64_t)(t->ne[0] / b) * tsize(t->type);
    return t->nb[1] == row && t->nb[2] == row * (uint64_t)t->ne[1] && t->nb[3] == t->nb[2] * (uint64_t)t->ne[2];
}

bool shape_ok(const mx_tensor *t) {
    for (int i = 0; i < 4; i++)
        if (t->ne[i] < 0) return false;
    return true;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// A quantized weight this device computes from: Q8_0 / Q4_K / Q5_K / Q6_K, whole blocks, contiguous (the planar
// layout is a function of type and shape only).
bool weight_ok(const mx_tensor *w) {
    return w && mx::is_quantized(w->type) && shape_ok(w) && contiguous(w) && w->data && nelements(w) > 0;
}

// An F16 / F32 weight for MUL_MAT and GET_ROWS: contiguous ggml rows read with 16-byte loads (rows of a multiple of
// 8 halves or 4 floats, 16-byte aligned data).
bool float_weight_ok(const mx_tensor *w) {
    if (!w || (w->type != MX_TYPE_F16 && w->type != MX_TYPE_F32) || !shape_ok(w) || !contiguous(w) || !w->data ||
        nelements(w) == 0 || !aligned16(w->data))
        return false;
    return w->ne[0] % (w->type == MX_TYPE_F16 ? 8 : 4) == 0;
}

// F32 activations read with 16-byte loads: contiguous rows, 16-byte aligned rows and slices.
bool f32_rows_ok(const mx_tensor *x) {
    return x && x->type == MX_TYPE_F32 && shape_ok(x) && x->nb[0] == 4 && x->nb[1] % 16 == 0 && x->nb[2] % 16 == 0 &&
           x->nb[3] % 16 == 0 && aligned16(x->data) && x->ne[0] % 4 == 0;
}

// The scratch of the entry point that allocates nothing (mx_mul_mat_id_noalloc): a static device array, one copy per
// GPU, held until the process ends. Host code never passes `scratch` itself to a kernel (in host code the name is a
// stand-in, not a device address): mx_backend_init looks up each device's copy once, with that device current, and
// the entry point uses that address.
constexpr int kNoAllocDevices = 64;
std::mutex g_noalloc_mu;
bool g_noalloc_done[kNoAllocDevices] = {};
void *g_noalloc_ptr[kNoAllocDevices] = {};

}  // namespace

static __device__ __align__(256) uint8_t scratch[MX_NOALLOC_SCRATCH_BYTES];

namespace {

// With `device` current: its copy of `scratch`, looked up on the first call for the device.
void noalloc_setup(int device) {
    if (device < 0 || device >= kNoAllocDevices) return;
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (g_noalloc_done[device]) return;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_noalloc_ptr[device] = e == hipSuccess ? p : nullptr;
    g_noalloc_done[device] = true;
}

void *noalloc_scratch(int device) {
    if (device < 0 || device >= kNoAllocDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    return g_noalloc_ptr[device];
}

int check_be(mx_backend *be) {
    if (!be) return fail(MX_INVALID, "null backend");
    if (hipSetDevice(be->device) != hipSuccess) return fail(MX_FAILED, "cannot select device %d", be->device);
    return MX_SUCCESS;
}

int ensure_scratch(mx_backend *be, size_t bytes) {
    if (bytes <= be->scratch_size) return MX_SUCCESS;
    if (be->capturing)
        return fail(MX_FAILED, "an op needs %zu bytes of scratch while a graph is recorded; run it once before recording",
                    bytes);
    HIP_OK(hipStreamSynchronize(be->stream), "synchronize before growing scratch");
    if (be->scratch) HIP_OK(hipFree(be->scratch), "free scratch");
    be->scratch = nullptr;
    be->scratch_size = 0;
    const size_t size = std::max<size_t>(mx::align_up(bytes + bytes / 2, 1 << 20), 1 << 20);
    be->scratch_gen++;  // graphs recorded before this point hold the freed address
    HIP_OK(hipMalloc(&be->scratch, size), "allocate scratch");
    be->scratch_size = size;
    return MX_SUCCESS;
}

int ensure_staging(mx_backend *be) {
    if (be->staging) return MX_SUCCESS;
    HIP_OK(hipMalloc(&be->staging, kStagingPiece), "allocate staging");
    be->staging_size = kStagingPiece;
    return MX_SUCCESS;
}

int no_capture(mx_backend *be, const char *what) {
    if (be->capturing) return fail(MX_FAILED, "%s cannot be recorded in a graph", what);
    return MX_SUCCESS;
}

}  // namespace

extern "C" {

MX_API const char *mx_last_error(void) { return g_error.c_str(); }

MX_API int mx_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

MX_API int mx_device_description(int device, char *buf, size_t len) {
    hipDeviceProp_t p;
    HIP_OK(hipGetDeviceProperties(&p, device), "device properties");
    if (buf && len) snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return MX_SUCCESS;
}

MX_API int mx_device_memory(int device, size_t *free_bytes, size_t *total_bytes) {
    HIP_OK(hipSetDevice(device), "select device");
    size_t f = 0, t = 0;
    HIP_OK(hipMemGetInfo(&f, &t), "memory info");
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return MX_SUCCESS;
}

MX_API mx_backend *mx_backend_init(int device) {
    if (device < 0 || device >= mx_device_count()) {
        fail(MX_INVALID, "no device %d", device);
        return nullptr;
    }
    if (hipSetDevice(device) != hipSuccess) {
        fail(MX_FAILED, "cannot select device %d", device);
        return nullptr;
    }
    noalloc_setup(device);
    mx_backend *be = new mx_backend();
    be->device = device;
    if (hipStreamCreateWithFlags(&be->stream, hipStreamNonBlocking) != hipSuccess ||
        hipMalloc(&be->err, 256) != hipSuccess || hipMemset(be->err, 0, 256) != hipSuccess) {
        fail(MX_FAILED, "cannot create the backend of device %d", device);
        mx_backend_free(be);
        return nullptr;
    }
    return be;
}

MX_API void mx_backend_free(mx_backend *be) {
    if (!be) return;
    // Teardown: errors here have no one to report to.
    (void)hipSetDevice(be->device);
    if (be->stream) (void)hipStreamSynchronize(be->stream);
    if (be->scratch) (void)hipFree(be->scratch);
    if (be->staging) (void)hipFree(be->staging);
    if (be->err) (void)hipFree(be->err);
    if (be->stream) (void)hipStreamDestroy(be->stream);
    delete be;
}

MX_API void *mx_backend_stream(mx_backend *be) { return be ? (void *)be->stream : nullptr; }

MX_API int mx_backend_set_option(mx_backend *be, int option, int64_t value) {
    if (!be) return fail(MX_INVALID, "null backend");
    mx::Options &o = be->opt;
    auto in = [&](std::initializer_list<int64_t> ok) {
        for (int64_t v : ok)
            if (v == value) return true;
        return false;
    };
    switch (option) {
        case MX_OPT_GEMM_Q8_0:
            if (!in({0, 1, 2})) break;
            o.gemm_q8_0 = (int)value;
            return MX_SUCCESS;
        case MX_OPT_GEMM_KQUANT:
            if (!in({0, 1})) break;
            o.gemm_kquant = (int)value;
            return MX_SUCCESS;
        case MX_OPT_GEMM_TILE_M:
        case MX_OPT_GEMM_TILE_N:
            if (!in({0, 64, 128}) && !(option == MX_OPT_GEMM_TILE_M && value == 32)) break;
            (option == MX_OPT_GEMM_TILE_M ? o.tile_m : o.tile_n) = (int)value;
            return MX_SUCCESS;
        case MX_OPT_GEMM_SPLIT:
            if (value < 0 || value > 64) break;
            o.split = (int)value;
            return MX_SUCCESS;
        case MX_OPT_MATVEC_LPR:
            if (!in({0, 16, 32, 64})) break;
            o.matvec_lpr = (int)value;
            return MX_SUCCESS;
        case MX_OPT_MMID_KERNEL:
            if (!in({0, 1, 2})) break;
            o.mmid_kernel = (int)value;
            return MX_SUCCESS;
        case MX_OPT_MMID_MATVEC_PAIRS:
            if (value < 0 || value > 4096) break;
            o.mmid_matvec_pairs = value;
            return MX_SUCCESS;
        case MX_OPT_MMID_CHUNK:
            if (!in({0, 16, 32})) break;
            o.mmid_chunk = (int)value;
            return MX_SUCCESS;
        default:
            return fail(MX_INVALID, "unknown option %d", option);
    }
    return fail(MX_INVALID, "option %d cannot take the value %lld", option, (long long)value);
}

MX_API int mx_backend_get_option(mx_backend *be, int option, int64_t *value) {
    if (!be || !value) return fail(MX_INVALID, "null argument");
    const mx::Options &o = be->opt;
    switch (option) {
        case MX_OPT_GEMM_Q8_0: *value = o.gemm_q8_0; return MX_SUCCESS;
        case MX_OPT_GEMM_KQUANT: *value = o.gemm_kquant; return MX_SUCCESS;
        case MX_OPT_GEMM_TILE_M: *value = o.tile_m; return MX_SUCCESS;
        case MX_OPT_GEMM_TILE_N: *value = o.tile_n; return MX_SUCCESS;
        case MX_OPT_GEMM_SPLIT: *value = o.split; return MX_SUCCESS;
        case MX_OPT_MATVEC_LPR: *value = o.matvec_lpr; return MX_SUCCESS;
        case MX_OPT_MMID_KERNEL: *value = o.mmid_kernel; return MX_SUCCESS;
        case MX_OPT_MMID_MATVEC_PAIRS: *value = o.mmid_matvec_pairs; return MX_SUCCESS;
        case MX_OPT_MMID_CHUNK: *value = o.mmid_chunk; return MX_SUCCESS;
        default: return fail(MX_INVALID, "unknown option %d", option);
    }
}

MX_API int mx_backend_set_rounding(mx_backend *be, int rounding) {
    if (!be) return fail(MX_INVALID, "null backend");
    if (rounding != MX_ROUND_REF && rounding != MX_ROUND_X86) return fail(MX_INVALID, "unknown rounding %d", rounding);
    be->rounding = rounding;
    return MX_SUCCESS;
}

MX_API int mx_backend_synchronize(mx_backend *be) {
    int rc = check_be(be);
    if (rc) return rc;
    if ((rc = no_capture(be, "synchronize"))) return rc;
    HIP_OK(hipStreamSynchronize(be->stream), "synchronize");
    int flag = 0;
    HIP_OK(hipMemcpy(&flag, be->err, sizeof flag, hipMemcpyDeviceToHost), "read error word");
    if (flag) {
        const int zero = 0;
        HIP_OK(hipMemcpy(be->err, &zero, sizeof zero, hipMemcpyHostToDevice), "clear error word");
        return fail(MX_INVALID, "%s%s%s", (flag & 1) ? "GET_ROWS met a row index out of range; its rows are zero. " : "",
                    (flag & 2) ? "MUL_MAT_ID met an expert index out of range; its pairs were skipped. " : "",
                    (flag & 4) ? "SET_ROWS met a row index out of range; those rows were not written." : "");
    }
    return MX_SUCCESS;
}

// ------------------------------------------------------------------------------------------------------ buffers
MX_API size_t mx_buft_alignment(void) { return mx::PLANE_ALIGN; }
MX_API size_t mx_buft_max_size(void) { return SIZE_MAX; }

MX_API size_t mx_tensor_alloc_size(const mx_tensor *t) {
    if (!t || !shape_ok(t)) return 0;
    if (mx::is_quantized(t->type)) return mx::planes_of(t->type, nelements(t)).total;
    return nbytes(t);
}

MX_API int mx_buffer_alloc(mx_backend *be, size_t size, void **base) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!base) return fail(MX_INVALID, "null base pointer");
    *base = nullptr;
    HIP_OK(hipMalloc(base, std::max<size_t>(size, 1)), "allocate buffer");
    return MX_SUCCESS;
}

MX_API int mx_buffer_free(mx_backend *be, void *base) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!base) return MX_SUCCESS;
    HIP_OK(hipStreamSynchronize(be->stream), "synchronize before free");
    HIP_OK(hipFree(base), "free buffer");
    return MX_SUCCESS;
}

MX_API int mx_buffer_clear(mx_backend *be, void *base, size_t size, uint8_t value) {
    int rc = check_be(be);
    if (rc) return rc;
    if ((rc = no_capture(be, "buffer clear"))) return rc;
    HIP_OK(hipMemsetAsync(base, value, size, be->stream), "clear buffer");
    HIP_OK(hipStreamSynchronize(be->stream), "synchronize clear");
    return MX_SUCCESS;
}

static int tensor_range_ok(const mx_tensor *t, size_t offset, size_t size) {
    if (!t || !t->data || !shape_ok(t)) return fail(MX_INVALID, "invalid tensor");
    if (blck(t->type) == 0) return fail(MX_UNSUPPORTED, "unknown tensor type %d", t->type);
    if (mx::is_quantized(t->type) && !contiguous(t)) return fail(MX_UNSUPPORTED, "quantized tensors must be contiguous");
    const size_t n = nbytes(t);
    if (offset > n || size > n - offset) return fail(MX_INVALID, "bytes [%zu, %zu) lie outside the tensor's %zu", offset,
                                                     offset + size, n);
    return MX_SUCCESS;
}

MX_API int mx_tensor_set(mx_backend *be, const mx_tensor *t, const void *host, size_t offset, size_t size) {
    int rc = check_be(be);
    if (rc || (rc = no_capture(be, "tensor_set")) || (rc = tensor_range_ok(t, offset, size))) return rc;
    if (size == 0) return MX_SUCCESS;
    if (!host) return fail(MX_INVALID, "null host pointer");
    if (!mx::is_quantized(t->type)) {
        HIP_OK(hipMemcpyAsync((uint8_t *)t->data + offset, host, size, hipMemcpyHostToDevice, be->stream), "upload");
        HIP_OK(hipStreamSynchronize(be->stream), "synchronize upload");
        return MX_SUCCESS;
    }
    if ((rc = ensure_staging(be))) return rc;
    const mx::Planes pl = mx::planes_of(t->type, nelements(t));
    const mx::SegMap map = mx::segmap_of(t->type, pl);
    for (size_t done = 0; done < size;) {
        const size_t piece = std::min(size - done, be->staging_size);
        HIP_OK(hipMemcpyAsync(be->staging, (const uint8_t *)host + done, piece, hipMemcpyHostToDevice, be->stream),
               "upload piece");
        HIP_OK(mx::launch_scatter(map, (uint8_t *)t->data, be->staging, offset + done, piece, be->stream), "scatter");
        done += piece;
    }
    HIP_OK(hipStreamSynchronize(be->stream), "synchronize upload");
    return MX_SUCCESS;
}

MX_API int mx_tensor_get(mx_backend *be, const mx_tensor *t, void *host, size_t offset, size_t size) {
    int rc = check_be(be);
    if (rc || (rc = no_capture(be, "tensor_get")) || (rc = tensor_range_ok(t, offset, size))) return rc;
    if (size == 0) return MX_SUCCESS;
    if (!host) return fail(MX_INVALID, "null host pointer");
    if (!mx::is_quantized(t->type)) {
        HIP_OK(hipMemcpyAsync(host, (const uint8_t *)t->data + offset, size, hipMemcpyDeviceToHost, be->stream),
               "download");
        HIP_OK(hipStreamSynchronize(be->stream), "synchronize download");
        return MX_SUCCESS;
    }
    if ((rc = ensure_staging(be))) return rc;
    const mx::Planes pl = mx::planes_of(t->type, nelements(t));
    const mx::SegMap map = mx::segmap_of(t->type, pl);
    for (size_t done = 0; done < size;) {
        const size_t piece = std::min(size - done, be->staging_size);
        HIP_OK(mx::launch_gather(map, (const uint8_t *)t->data, be->staging, offset + done, piece, be->stream), "gather");
        HIP_OK(hipMemcpyAsync((uint8_t *)host + done, be->staging, piece, hipMemcpyDeviceToHost, be->stream),
               "download piece");
        HIP_OK(hipStreamSynchronize(be->stream), "synchronize download");
        done += piece;
    }
    return MX_SUCCESS;
}

MX_API int mx_tensor_memset(mx_backend *be, const mx_tensor *t, uint8_t value, size_t offset, size_t size) {
    int rc = check_be(be);
    if (rc || (rc = no_capture(be, "tensor_memset")) || (rc = tensor_range_ok(t, offset, size))) return rc;
    if (size == 0) return MX_SUCCESS;
    if (!mx::is_quantized(t->type)) {
        HIP_OK(hipMemsetAsync((uint8_t *)t->data + offset, value, size, be->stream), "memset");
    } else {
        const mx::Planes pl = mx::planes_of(t->type, nelements(t));
        const mx::SegMap map = mx::segmap_of(t->type, pl);
        for (size_t done = 0; done < size;) {
            const size_t piece = std::min<size_t>(size - done, 1ull << 30);
            HIP_OK(mx::launch_fill(map, (uint8_t *)t->data, value, offset + done, piece, be->stream), "fill");
            done += piece;
        }
    }
    HIP_OK(hipStreamSynchronize(be->stream), "synchronize memset");
    return MX_SUCCESS;
}

MX_API int mx_tensor_copy(mx_backend *be, const mx_tensor *src, const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!src || !dst || !src->data || !dst->data) return fail(MX_INVALID, "invalid tensor");
    if (src->type != dst->type || nelements(src) != nelements(dst)) return fail(MX_INVALID, "tensors differ");
    if (mx::is_quantized(src->type) && (!contiguous(src) || !contiguous(dst)))
        return fail(MX_UNSUPPORTED, "quantized tensors must be contiguous");
    const size_t n = mx::is_quantized(src->type) ? mx::planes_of(src->type, nelements(src)).total : nbytes(src);
    if (!mx::is_quantized(src->type) && (!contiguous(src) || !contiguous(dst)))
        return fail(MX_UNSUPPORTED, "only contiguous copies");
    if ((rc = no_capture(be, "tensor_copy"))) return rc;
    HIP_OK(hipMemcpyAsync(dst->data, src->data, n, hipMemcpyDeviceToDevice, be->stream), "copy tensor");
    // complete on return, as ggml's cpy_tensor is: a compute on another stream may read dst next
    HIP_OK(hipStreamSynchronize(be->stream), "synchronize copy");
    return MX_SUCCESS;
}

// f32 rows: ne0 contiguous floats, rows anywhere (the layer ops index rows at byte strides).
static bool f32_any(const mx_tensor *t) {
    return t && t->type == MX_TYPE_F32 && shape_ok(t) && t->nb[0] == 4 && t->data && ((uintptr_t)t->data & 3) == 0 &&
           t->nb[1] % 4 == 0 && t->nb[2] % 4 == 0 && t->nb[3] % 4 == 0;
}
static bool same_shape(const mx_tensor *a, const mx_tensor *b) {
    return a->ne[0] == b->ne[0] && a->ne[1] == b->ne[1] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3];
}
static mx::RowsArgs rows_of(const mx_tensor *src, const mx_tensor *dst) {
    mx::RowsArgs r{};
    r.src = src->data;
    r.dst = dst->data;
    r.ne0 = src->ne[0];
    r.ne1 = src->ne[1];
    r.ne2 = src->ne[2];
    r.nrows = src->ne[1] * src->ne[2] * src->ne[3];
    r.s_nb1 = (int64_t)src->nb[1];
    r.s_nb2 = (int64_t)src->nb[2];
    r.s_nb3 = (int64_t)src->nb[3];
    r.d_nb1 = (int64_t)dst->nb[1];
    r.d_nb2 = (int64_t)dst->nb[2];
    r.d_nb3 = (int64_t)dst->nb[3];
    return r;
}

// The row-wise layer ops: RMS_NORM (src0, optional weight src1), ADD / MUL (a = src0, b = src1), SWIGLU (a, b),
// SET_ROWS (src0 rows, src1 indices, dst f16 rows).
static int supports_layer_op(int op, const mx_tensor *src0, const mx_tensor *src1, const mx_tensor *dst) {
    switch (op) {
        case MX_OP_RMS_NORM:
            if (!f32_any(src0) || !f32_any(dst) || !same_shape(src0, dst) || src0->ne[0] < 1) return 0;
            return !src1 || (f32_any(src1) && src1->ne[0] == src0->ne[0] && nelements(src1) == src1->ne[0]);
        case MX_OP_ADD:
        case MX_OP_MUL:
            if (!f32_any(src0) || !f32_any(src1) || !f32_any(dst) || !same_shape(src0, dst)) return 0;
            for (int i = 0; i < 4; i++)
                if (src1->ne[i] < 1 || src0->ne[i] % src1->ne[i] != 0) return 0;
            return 1;
        case MX_OP_SWIGLU:
            return f32_any(src0) && f32_any(src1) && f32_any(dst) && same_shape(src0, src1) && same_shape(src0, dst) &&
                   src0->ne[2] == 1 && src0->ne[3] == 1;
        case MX_OP_SET_ROWS: {
            if (!f32_any(src0) || src0->ne[2] != 1 || src0->ne[3] != 1) return 0;
            if (!src1 || (src1->type != MX_TYPE_I32 && src1->type != 27) || !src1->data || !shape_ok(src1) ||
                src1->ne[0] != src0->ne[1] || nelements(src1) != src1->ne[0] || src1->nb[0] != (src1->type == 27 ? 8u : 4u))
                return 0;
            return dst && dst->type == MX_TYPE_F16 && shape_ok(dst) && dst->nb[0] == 2 && dst->data &&
                   ((uintptr_t)dst->data & 1) == 0 && dst->ne[0] == src0->ne[0] && dst->ne[2] == 1 && dst->ne[3] == 1 &&
                   dst->nb[1] % 2 == 0;
        }
        default: return 0;
    }
}

// ---------------------------------------------------------------------------------------------------------- ops
MX_API int mx_supports_op(int op, const mx_tensor *src0, const mx_tensor *src1, const mx_tensor *src2,
                          const mx_tensor *dst) {
    if (op >= MX_OP_RMS_NORM && op <= MX_OP_SET_ROWS) return supports_layer_op(op, src0, src1, dst);
    if (op == MX_OP_ARGMAX) {  // f32 rows in, one I32 per row out
        if (!src0 || src0->type != MX_TYPE_F32 || !shape_ok(src0) || src0->nb[0] != 4 || src0->nb[1] % 16 != 0 ||
            !src0->data || !aligned16(src0->data) || src0->ne[2] != 1 || src0->ne[3] != 1)
            return 0;
        if (src0->ne[0] < 1 || src0->ne[0] >= ((int64_t)1 << 31) || src0->ne[1] > 0x7FFFFFFF) return 0;
        return dst && dst->type == MX_TYPE_I32 && shape_ok(dst) && dst->nb[0] == 4 && dst->ne[0] == src0->ne[1] &&
               dst->ne[1] == 1 && dst->ne[2] == 1 && dst->ne[3] == 1 && dst->data && ((uintptr_t)dst->data & 3) == 0;
    }
    const bool fw = op != MX_OP_MUL_MAT_ID && float_weight_ok(src0);  // routed experts are quantized
    if (!(weight_ok(src0) || fw) || !dst || dst->type != MX_TYPE_F32 || !shape_ok(dst) || dst->nb[0] != 4) return 0;
    const int64_t K = src0->ne[0];
    switch (op) {
        case MX_OP_GET_ROWS: {
            const mx_tensor *ids = src1;
            if (!ids || ids->type != MX_TYPE_I32 || !shape_ok(ids) || ids->ne[3] != 1) return 0;
            if (src0->ne[2] != ids->ne[1] || src0->ne[3] != ids->ne[2]) return 0;
            if (ids->ne[0] * ids->ne[1] * ids->ne[2] >= ((int64_t)1 << 31)) return 0;  // rows are indexed with 32 bits
            if (dst->ne[0] != K || dst->ne[1] != ids->ne[0] || dst->ne[2] != ids->ne[1] || dst->ne[3] != ids->ne[2]) return 0;
            return aligned16(dst->data) && dst->nb[1] % 16 == 0 && dst->nb[2] % 16 == 0 && dst->nb[3] % 16 == 0;
        }
        case MX_OP_MUL_MAT: {
            if (!f32_rows_ok(src1) || src1->ne[0] != K) return 0;
            if (src0->ne[2] == 0 || src0->ne[3] == 0) return 0;
            if (src1->ne[2] % src0->ne[2] != 0 || src1->ne[3] % src0->ne[3] != 0) return 0;
            if (src1->ne[2] * src1->ne[3] > mx::MAX_BATCH) return 0;
            if (dst->ne[0] != src0->ne[1] || dst->ne[1] != src1->ne[1] || dst->ne[2] != src1->ne[2] ||
                dst->ne[3] != src1->ne[3])
                return 0;
            return mx::act_lds_bytes(src0->type, K, 1) <= kMaxLds;
        }
        case MX_OP_MUL_MAT_ID: {
            const mx_tensor *b = src1, *ids = src2;
            if (!f32_rows_ok(b) || !ids || ids->type != MX_TYPE_I32 || !shape_ok(ids)) return 0;
            if (src0->ne[3] != 1 || b->ne[0] != K || b->ne[3] != 1 || ids->ne[2] != 1 || ids->ne[3] != 1) return 0;
            const int64_t n_ids = ids->ne[0], T = ids->ne[1];
            if (b->ne[2] != T || (b->ne[1] != 1 && b->ne[1] != n_ids)) return 0;
            if (dst->ne[0] != src0->ne[1] || dst->ne[1] != n_ids || dst->ne[2] != T || dst->ne[3] != 1) return 0;
            // experts' pair counters live in LDS (4 bytes each); pairs are indexed with 32 bits
            if (src0->ne[2] > 8192 || n_ids * T >= ((int64_t)1 << 31)) return 0;
            return mx::act_lds_bytes(src0->type, K, mx::MAX_COLS) <= kMaxLds;
        }
        default: return 0;
    }
}

MX_API int mx_get_rows(mx_backend *be, const mx_tensor *src0, const mx_tensor *ids, const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!mx_supports_op(MX_OP_GET_ROWS, src0, ids, nullptr, dst))
        return fail(MX_UNSUPPORTED, "GET_ROWS: unsupported types, shapes or strides");
    const mx::Planes pl = mx::planes_of(src0->type, nelements(src0));
    mx::GetRowsArgs a{};
    a.type = src0->type;
    a.w = mx::wplanes(src0->data, pl);
    a.K = src0->ne[0];
    a.R = src0->ne[1];
    a.n_ids0 = ids->ne[0];
    a.n_ids1 = ids->ne[1];
    a.n_ids2 = ids->ne[2];
    a.src_mat_rows1 = src0->ne[1];
    a.src_mat_rows2 = src0->ne[1] * src0->ne[2];
    a.ids = (const int32_t *)ids->data;
    a.ids_nb0 = (int64_t)ids->nb[0];
    a.ids_nb1 = (int64_t)ids->nb[1];
    a.ids_nb2 = (int64_t)ids->nb[2];
    a.dst = (float *)dst->data;
    a.dst_nb1 = (int64_t)dst->nb[1];
    a.dst_nb2 = (int64_t)dst->nb[2];
    a.dst_nb3 = (int64_t)dst->nb[3];
    a.err = be->err;
    HIP_OK(mx::launch_get_rows(a, be->stream), "GET_ROWS launch");
    return MX_SUCCESS;
}

static int max_cols(int type, int64_t K) {
    int nc = mx::MAX_COLS;
    while (nc > 1 && mx::act_lds_bytes(type, K, nc) > kMaxLds) nc--;
    return nc;
}

// The first planar row of matrix (i02, i03) of a weight, as plane pointers.
static mx::WPlanes matrix_planes(const mx_tensor *w, int64_t mat) {
    const mx::Planes pl = mx::planes_of(w->type, nelements(w));
    mx::WPlanes p = mx::wplanes(w->data, pl);
    const int64_t blocks = mat * w->ne[1] * (w->ne[0] / mx::type_info(w->type)->blk_elems);
    p.p0 += blocks * pl.per_blk[0];
    p.p1 += blocks * pl.per_blk[1];
    if (p.p2) p.p2 += blocks * pl.per_blk[2];
    if (p.p3) p.p3 += blocks * pl.per_blk[3];
    return p;
}

// M > 8 on Q8_0 weights (int8 MFMA): per batch slice, src1 quantized once into scratch, then one launch over every
// weight sharing it (plus the reduce when K is split).
static int gemm_group(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                      const mx_tensor *const *dst) {
    const mx_tensor *w0 = src0[0];
    const int64_t K = w0->ne[0], M = src1->ne[1];
    int64_t Ns[4];
    for (int i = 0; i < n; i++) Ns[i] = src0[i]->ne[1];
    int rc = ensure_scratch(be, mx::gemm_scratch_bytes(n, Ns, M, K, be->opt));
    if (rc) return rc;
    const int64_t r2 = src1->ne[2] / w0->ne[2], r3 = src1->ne[3] / w0->ne[3];
    for (int64_t i13 = 0; i13 < src1->ne[3]; i13++)
        for (int64_t i12 = 0; i12 < src1->ne[2]; i12++) {
            const float *x = (const float *)((const uint8_t *)src1->data + i12 * src1->nb[2] + i13 * src1->nb[3]);
            HIP_OK(mx::launch_gemm_quant(w0->type, be->rounding, x, (int64_t)(src1->nb[1] / 4), M, K, be->scratch,
                                         be->stream),
                   "GEMM activation quantization");
            mx::WPlanes w[4];
            int64_t N[4], ldy[4];
            float *y[4];
            for (int i = 0; i < n; i++) {
                w[i] = matrix_planes(src0[i], i12 / r2 + (i13 / r3) * src0[i]->ne[2]);
                N[i] = src0[i]->ne[1];
                y[i] = (float *)((uint8_t *)dst[i]->data + i12 * dst[i]->nb[2] + i13 * dst[i]->nb[3]);
                ldy[i] = (int64_t)(dst[i]->nb[1] / 4);
            }
            HIP_OK(mx::launch_gemm(w0->type, n, w, N, y, ldy, M, K, be->scratch, be->opt, be->stream), "GEMM launch");
        }
    return MX_SUCCESS;
}

// M > 8 on K-quant weights: per batch slice and weight, Q8_K activations into scratch and one MFMA GEMM.
static int gemm_kq_group(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                         const mx_tensor *const *dst) {
    const mx_tensor *w0 = src0[0];
    const int64_t K = w0->ne[0], M = src1->ne[1];
    int rc = ensure_scratch(be, mx::gemm_kq_act_bytes(M, K));
    if (rc) return rc;
    const int64_t r2 = src1->ne[2] / w0->ne[2], r3 = src1->ne[3] / w0->ne[3];
    for (int64_t i13 = 0; i13 < src1->ne[3]; i13++)
        for (int64_t i12 = 0; i12 < src1->ne[2]; i12++) {
            const float *x = (const float *)((const uint8_t *)src1->data + i12 * src1->nb[2] + i13 * src1->nb[3]);
            HIP_OK(mx::launch_gemm_kq_quant(x, (int64_t)(src1->nb[1] / 4), M, K, be->scratch, be->stream),
                   "K-quant GEMM activation quantization");
            for (int i = 0; i < n; i++) {
                const int64_t mat = i12 / r2 + (i13 / r3) * src0[i]->ne[2];
                float *y = (float *)((uint8_t *)dst[i]->data + i12 * dst[i]->nb[2] + i13 * dst[i]->nb[3]);
                HIP_OK(mx::launch_gemm_kq(src0[i]->type, matrix_planes(src0[i], mat), M, src0[i]->ne[1], K, be->scratch,
                                          y, (int64_t)(dst[i]->nb[1] / 4), be->stream),
                       "K-quant GEMM launch");
            }
        }
    return MX_SUCCESS;
}

// M > 8 on Q4_K weights: per batch slice, activations quantized once, then one launch for the whole group.
static int gemm_q4k_group(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                          const mx_tensor *const *dst) {
    const mx_tensor *w0 = src0[0];
    const int64_t K = w0->ne[0], M = src1->ne[1];
    int rc = ensure_scratch(be, mx::gemm_q4k_act_bytes(M, K));
    if (rc) return rc;
    const int64_t r2 = src1->ne[2] / w0->ne[2], r3 = src1->ne[3] / w0->ne[3];
    for (int64_t i13 = 0; i13 < src1->ne[3]; i13++)
        for (int64_t i12 = 0; i12 < src1->ne[2]; i12++) {
            const float *x = (const float *)((const uint8_t *)src1->data + i12 * src1->nb[2] + i13 * src1->nb[3]);
            HIP_OK(mx::launch_gemm_q4k_quant(x, (int64_t)(src1->nb[1] / 4), M, K, be->scratch, be->stream),
                   "Q4_K GEMM activation quantization");
            mx::WPlanes w[4];
            int64_t N[4], ldy[4];
            float *y[4];
            for (int i = 0; i < n; i++) {
                w[i] = matrix_planes(src0[i], i12 / r2 + (i13 / r3) * src0[i]->ne[2]);
                N[i] = src0[i]->ne[1];
                y[i] = (float *)((uint8_t *)dst[i]->data + i12 * dst[i]->nb[2] + i13 * dst[i]->nb[3]);
                ldy[i] = (int64_t)(dst[i]->nb[1] / 4);
            }
            HIP_OK(mx::launch_gemm_q4k(n, w, N, y, ldy, M, K, be->scratch, be->opt, be->stream),
                   "Q4_K GEMM launch");
        }
    return MX_SUCCESS;
}

// M > 8 on Q8_0 weights through the dequantizing fp16 GEMM: per batch slice, activations quantized once (as fp16 of
// their Q8_0 values), then one launch for the whole group.
static int gemm_dq_group(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                         const mx_tensor *const *dst) {
    const mx_tensor *w0 = src0[0];
    const int64_t K = w0->ne[0], M = src1->ne[1];
    int64_t Ns[4];
    for (int i = 0; i < n; i++) Ns[i] = src0[i]->ne[1];
    int rc = ensure_scratch(be, mx::gemm_dq_scratch_bytes(w0->type, n, Ns, M, K, be->opt));
    if (rc) return rc;
    const int64_t r2 = src1->ne[2] / w0->ne[2], r3 = src1->ne[3] / w0->ne[3];
    for (int64_t i13 = 0; i13 < src1->ne[3]; i13++)
        for (int64_t i12 = 0; i12 < src1->ne[2]; i12++) {
            const float *x = (const float *)((const uint8_t *)src1->data + i12 * src1->nb[2] + i13 * src1->nb[3]);
            HIP_OK(mx::launch_gemm_dq_act(w0->type, be->rounding, x, (int64_t)(src1->nb[1] / 4), M, K, be->scratch,
                                          be->stream),
                   "GEMM activation quantization");
            mx::WPlanes w[4];
            int64_t N[4], ldy[4];
            float *y[4];
            for (int i = 0; i < n; i++) {
                w[i] = matrix_planes(src0[i], i12 / r2 + (i13 / r3) * src0[i]->ne[2]);
                N[i] = src0[i]->ne[1];
                y[i] = (float *)((uint8_t *)dst[i]->data + i12 * dst[i]->nb[2] + i13 * dst[i]->nb[3]);
                ldy[i] = (int64_t)(dst[i]->nb[1] / 4);
            }
            HIP_OK(mx::launch_gemm_dq(w0->type, n, w, N, y, ldy, M, K, be->scratch, be->opt, be->stream),
                   "GEMM launch");
        }
    return MX_SUCCESS;
}

// Products sharing src1: n problems (n <= 4) of the same type and K, each with its own rows and dst; `f` (validated
// by mx_mul_mat_fused, mat-vec path only) fuses the neighbouring norm / SwiGLU / residual ADD.
static int matvec_group(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                        const mx_tensor *const *dst, const mx_fusion *f = nullptr) {
    const mx_tensor *w0 = src0[0];
    mx::MatvecArgs a{};
    a.type = w0->type;
    a.rounding = be->rounding;
    a.K = w0->ne[0];
    a.x_col_stride = (int64_t)(src1->nb[1] / 4);
    a.nbatch = (int)(src1->ne[2] * src1->ne[3]);
    a.ne12 = (int)src1->ne[2];
    a.ne02 = (int)w0->ne[2];
    a.r2 = (int)(src1->ne[2] / w0->ne[2]);
    a.r3 = (int)(src1->ne[3] / w0->ne[3]);
    a.x_b2 = (int64_t)(src1->nb[2] / 4);
    a.x_b3 = (int64_t)(src1->nb[3] / 4);
    a.y_b2 = (int64_t)(dst[0]->nb[2] / 4);
    a.y_b3 = (int64_t)(dst[0]->nb[3] / 4);
    a.nprob = n;
    const int64_t M = src1->ne[1];
    a.lpr = be->opt.matvec_lpr;
    if (f) {
        a.glu_b = f->glu_b ? (const float *)f->glu_b->data : nullptr;
        a.norm_w = f->norm_w ? (const float *)f->norm_w->data : nullptr;
        a.norm_eps = f->norm_eps;
    }
    if (M > mx::MAX_COLS) {
        // The GEMM each weight type takes at M > 8 (a backend's options may force another one; a product the forced
        // kernel cannot compute is refused rather than sent elsewhere, so a test of a forced kernel tests it).
        const mx::Options &o = be->opt;
        bool fits = true;  // every weight's rows within 32-bit element offsets
        for (int i = 0; i < n; i++) fits = fits && src0[i]->ne[1] * a.K < ((int64_t)1 << 31);
        if (a.type == MX_TYPE_Q8_0 && o.gemm_q8_0 != 2) {  // the int8 GEMM: picked wherever it can take the product
            if (fits && mx::gemm_supported(a.type, M, a.K)) return gemm_group(be, n, src0, src1, dst);
            if (o.gemm_q8_0 == 1)
                return fail(MX_UNSUPPORTED, "int8 Q8_0 GEMM: K must be a multiple of 128 (and M K, N K below 2^31)");
        }
        if (a.type == MX_TYPE_Q8_0 && o.gemm_q8_0 == 2 && !(fits && mx::gemm_dq_supported(a.type, M, a.K)))
            return fail(MX_UNSUPPORTED, "fp16 Q8_0 GEMM: K must be a multiple of 64 (and M K, N K below 2^31)");
        if ((a.type == MX_TYPE_Q4_K || a.type == MX_TYPE_Q6_K) && o.gemm_kquant == 1) {
            if (!mx::gemm_kq_supported(a.type, a.K)) return fail(MX_UNSUPPORTED, "int8 K-quant GEMM: K % 256");
            return gemm_kq_group(be, n, src0, src1, dst);
        }
        if (fits && mx::gemm_dq_supported(a.type, M, a.K)) return gemm_dq_group(be, n, src0, src1, dst);
        if (a.type == MX_TYPE_Q4_K && a.K % 256 == 0) return gemm_q4k_group(be, n, src0, src1, dst);
        if (mx::gemm_kq_supported(a.type, a.K)) return gemm_kq_group(be, n, src0, src1, dst);
    }
    const int ncmax = max_cols(a.type, a.K);
    for (int64_t m0 = 0; m0 < M; m0 += ncmax) {
        a.ncols = (int)std::min<int64_t>(ncmax, M - m0);
        a.x = (const float *)src1->data + m0 * a.x_col_stride;
        for (int i = 0; i < n; i++) {
            const mx::Planes pl = mx::planes_of(src0[i]->type, nelements(src0[i]));
            a.prob[i].w = mx::wplanes(src0[i]->data, pl);
            a.prob[i].N = src0[i]->ne[1];
            a.prob[i].row0 = 0;
            a.prob[i].y_col_stride = (int64_t)(dst[i]->nb[1] / 4);
            a.prob[i].y = (float *)dst[i]->data + m0 * a.prob[i].y_col_stride;
            a.prob[i].res = f && f->residual && f->residual[i]
                                ? (const float *)f->residual[i]->data + m0 * a.prob[i].y_col_stride
                                : nullptr;
        }
        HIP_OK(mx::launch_matvec(a, be->stream), "MUL_MAT launch");
    }
    return MX_SUCCESS;
}

MX_API int mx_mul_mat(mx_backend *be, const mx_tensor *src0, const mx_tensor *src1, const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!mx_supports_op(MX_OP_MUL_MAT, src0, src1, nullptr, dst))
        return fail(MX_UNSUPPORTED, "MUL_MAT: unsupported types, shapes or strides");
    if (nelements(dst) == 0) return MX_SUCCESS;
    return matvec_group(be, 1, &src0, src1, &dst);
}

MX_API int mx_mul_mat_group(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                            const mx_tensor *const *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (n <= 0 || !src0 || !dst) return fail(MX_INVALID, "empty group");
    for (int i = 0; i < n; i++) {
        if (!mx_supports_op(MX_OP_MUL_MAT, src0[i], src1, nullptr, dst[i]))
            return fail(MX_UNSUPPORTED, "MUL_MAT group member %d: unsupported types, shapes or strides", i);
        if (src0[i]->type != src0[0]->type || src0[i]->ne[2] != 1 || src0[i]->ne[3] != 1 || src1->ne[2] != 1 ||
            src1->ne[3] != 1)
            return fail(MX_UNSUPPORTED, "MUL_MAT group members must be 2-D products of one weight type");
    }
    for (int i0 = 0; i0 < n; i0 += 4) {
        const int k = std::min(4, n - i0);
        if ((rc = matvec_group(be, k, src0 + i0, src1, dst + i0))) return rc;
    }
    return MX_SUCCESS;
}

static bool same_layout(const mx_tensor *a, const mx_tensor *b) {
    return a && b && a->type == b->type && same_shape(a, b) && a->nb[0] == b->nb[0] && a->nb[1] == b->nb[1] &&
           a->nb[2] == b->nb[2] && a->nb[3] == b->nb[3];
}

MX_API int mx_mul_mat_fused(mx_backend *be, int n, const mx_tensor *const *src0, const mx_tensor *src1,
                            const mx_tensor *const *dst, const mx_fusion *f) {
    int rc = check_be(be);
    if (rc) return rc;
    if (n <= 0 || n > 4 || !src0 || !dst || !f) return fail(MX_INVALID, "fused product: 1 to 4 products and a fusion");
    for (int i = 0; i < n; i++) {
        if (!weight_ok(src0[i]) || !mx_supports_op(MX_OP_MUL_MAT, src0[i], src1, nullptr, dst[i]))
            return fail(MX_UNSUPPORTED, "fused product %d: unsupported types, shapes or strides", i);
        if (src0[i]->type != src0[0]->type || src0[i]->ne[0] != src0[0]->ne[0])
            return fail(MX_UNSUPPORTED, "fused products must share the weight type and K");
        if (f->residual && f->residual[i] && !same_layout(f->residual[i], dst[i]))
            return fail(MX_UNSUPPORTED, "fused residual %d must have dst's shape and strides", i);
    }
    const int64_t K = src0[0]->ne[0];
    if (src1->ne[1] > mx::MAX_COLS || src1->ne[2] * src1->ne[3] > mx::MAX_BATCH)
        return fail(MX_UNSUPPORTED, "fusions run on the mat-vec path: at most %d columns", mx::MAX_COLS);
    if (f->norm_w && (!f32_any(f->norm_w) || nelements(f->norm_w) != K || !aligned16(f->norm_w->data)))
        return fail(MX_UNSUPPORTED, "the norm weight must be K contiguous floats, 16-byte aligned");
    if (f->glu_b && !same_layout(f->glu_b, src1)) return fail(MX_UNSUPPORTED, "glu_b must have src1's layout");
    if (nelements(src1) == 0) return MX_SUCCESS;
    return matvec_group(be, n, src0, src1, dst, f);
}

// The launch arguments of a MUL_MAT_ID (scratch not yet carved).
static void mmid_args(mx_backend *be, const mx_tensor *as, const mx_tensor *b, const mx_tensor *ids,
                      const mx_tensor *dst, mx::MulMatIdArgs &a) {
    const mx::Planes pl = mx::planes_of(as->type, nelements(as));
    a = mx::MulMatIdArgs{};
    a.type = as->type;
    a.rounding = be->rounding;
    a.w = mx::wplanes(as->data, pl);
    a.K = as->ne[0];
    a.N = as->ne[1];
    a.E = as->ne[2];
    a.n_ids = ids->ne[0];
    a.T = ids->ne[1];
    a.b = (const float *)b->data;
    a.b_ne1 = b->ne[1];
    a.b_nb1 = (int64_t)b->nb[1];
    a.b_nb2 = (int64_t)b->nb[2];
    a.ids = (const int32_t *)ids->data;
    a.ids_nb0 = (int64_t)ids->nb[0];
    a.ids_nb1 = (int64_t)ids->nb[1];
    a.dst = (float *)dst->data;
    a.dst_nb1 = (int64_t)dst->nb[1];
    a.dst_nb2 = (int64_t)dst->nb[2];
    a.nprob = 1;
    a.wg[0] = a.w;
    a.dstg[0] = a.dst;
    a.generic = be->opt.mmid_kernel;
    a.chunk = mx::mmid_chunk_for(a.n_ids * a.T, a.E, be->opt.mmid_chunk);
    a.matvec_pairs = be->opt.mmid_matvec_pairs;
    a.lpr = be->opt.matvec_lpr;
    a.tile_m = be->opt.tile_m;
    a.tile_n = be->opt.tile_n;
    a.err = be->err;
}

MX_API int mx_mul_mat_id(mx_backend *be, const mx_tensor *as, const mx_tensor *b, const mx_tensor *ids,
                         const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!mx_supports_op(MX_OP_MUL_MAT_ID, as, b, ids, dst))
        return fail(MX_UNSUPPORTED, "MUL_MAT_ID: unsupported types, shapes or strides");
    mx::MulMatIdArgs a;
    mmid_args(be, as, b, ids, dst, a);
    if (a.n_ids * a.T == 0) return MX_SUCCESS;
    const size_t need = mx::mul_mat_id_scratch(&a, nullptr);
    if ((rc = ensure_scratch(be, need))) return rc;
    mx::mul_mat_id_scratch(&a, be->scratch);
    HIP_OK(mx::launch_mul_mat_id(a, be->stream), "MUL_MAT_ID launch");
    return MX_SUCCESS;
}

MX_API int mx_mul_mat_id_group(mx_backend *be, int n, const mx_tensor *const *as, const mx_tensor *b,
                               const mx_tensor *ids, const mx_tensor *const *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (n <= 0 || n > 4 || !as || !dst) return fail(MX_INVALID, "MUL_MAT_ID group: 1 to 4 products");
    for (int i = 0; i < n; i++) {
        if (!mx_supports_op(MX_OP_MUL_MAT_ID, as[i], b, ids, dst[i]))
            return fail(MX_UNSUPPORTED, "MUL_MAT_ID group member %d: unsupported types, shapes or strides", i);
        if (as[i]->type != as[0]->type || !same_shape(as[i], as[0]) || !same_layout(dst[i], dst[0]))
            return fail(MX_UNSUPPORTED, "MUL_MAT_ID group members must share the expert type and shape, and dst's "
                                        "shape and strides");
    }
    mx::MulMatIdArgs a;
    mmid_args(be, as[0], b, ids, dst[0], a);
    if (a.n_ids * a.T == 0) return MX_SUCCESS;
    a.nprob = n;
    for (int i = 0; i < n; i++) {
        a.wg[i] = mx::wplanes(as[i]->data, mx::planes_of(as[i]->type, nelements(as[i])));
        a.dstg[i] = (float *)dst[i]->data;
    }
    const size_t need = mx::mul_mat_id_scratch(&a, nullptr);
    if ((rc = ensure_scratch(be, need))) return rc;
    mx::mul_mat_id_scratch(&a, be->scratch);
    HIP_OK(mx::launch_mul_mat_id(a, be->stream), "MUL_MAT_ID group launch");
    return MX_SUCCESS;
}

MX_API size_t mx_mul_mat_id_noalloc_bytes(const mx_tensor *as, const mx_tensor *b, const mx_tensor *ids) {
    // inputs it cannot size read as needing more than any scratch holds, never as fitting
    if (!as || !b || !ids || !mx::is_quantized(as->type) || !shape_ok(as) || !shape_ok(b) || !shape_ok(ids) ||
        b->type != MX_TYPE_F32 || ids->type != MX_TYPE_I32 || b->ne[0] != as->ne[0] || ids->ne[1] != b->ne[2] ||
        (b->ne[1] != 1 && b->ne[1] != ids->ne[0]))
        return SIZE_MAX;
    mx::MulMatIdArgs a{};
    a.type = as->type;
    a.K = as->ne[0];
    a.N = as->ne[1];
    a.E = as->ne[2];
    a.n_ids = ids->ne[0];
    a.T = ids->ne[1];
    a.b_ne1 = b->ne[1];
    return mx::mul_mat_id_scratch(&a, nullptr);
}

MX_API int mx_mul_mat_id_noalloc(mx_backend *be, const mx_tensor *as, const mx_tensor *b, const mx_tensor *ids,
                                 const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!mx_supports_op(MX_OP_MUL_MAT_ID, as, b, ids, dst))
        return fail(MX_UNSUPPORTED, "MUL_MAT_ID: unsupported types, shapes or strides");
    mx::MulMatIdArgs a;
    mmid_args(be, as, b, ids, dst, a);
    if (a.n_ids * a.T == 0) return MX_SUCCESS;
    void *ptr = noalloc_scratch(be->device);
    if (!ptr) return fail(MX_FAILED, "MUL_MAT_ID without allocating: device %d has no address for its static scratch",
                          be->device);
    const size_t need = mx::mul_mat_id_scratch(&a, nullptr);
    if (need > MX_NOALLOC_SCRATCH_BYTES)
        return fail(MX_UNSUPPORTED, "MUL_MAT_ID without allocating needs %zu bytes of scratch, above its %u", need,
                    (unsigned)MX_NOALLOC_SCRATCH_BYTES);
    // every table and row the kernels read from the scratch is written by the prep launch first: nothing to clear
    mx::mul_mat_id_scratch(&a, ptr);
    HIP_OK(mx::launch_mul_mat_id(a, be->stream), "MUL_MAT_ID launch");
    return MX_SUCCESS;
}

MX_API int mx_argmax(mx_backend *be, const mx_tensor *src, const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!mx_supports_op(MX_OP_ARGMAX, src, nullptr, nullptr, dst))
        return fail(MX_UNSUPPORTED, "ARGMAX: unsupported types, shapes or strides");
    const int parts = mx::argmax_parts(src->ne[0], src->ne[1]);
    if (parts > 1 && (rc = ensure_scratch(be, (size_t)src->ne[1] * (size_t)parts * 8))) return rc;
    HIP_OK(mx::launch_argmax((const float *)src->data, src->ne[0], src->ne[1], (int64_t)src->nb[1],
                             (int32_t *)dst->data, (int64_t)dst->nb[0], be->scratch, be->stream),
           "ARGMAX launch");
    return MX_SUCCESS;
}

MX_API int mx_rms_norm(mx_backend *be, const mx_tensor *src, const mx_tensor *dst, float eps, const mx_tensor *w) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!supports_layer_op(MX_OP_RMS_NORM, src, w, dst)) return fail(MX_UNSUPPORTED, "RMS_NORM: unsupported tensors");
    HIP_OK(mx::launch_rms_norm(rows_of(src, dst), eps, w ? (const float *)w->data : nullptr, be->stream),
           "RMS_NORM launch");
    return MX_SUCCESS;
}

MX_API int mx_binary(mx_backend *be, int op, const mx_tensor *a, const mx_tensor *b, const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if ((op != MX_OP_ADD && op != MX_OP_MUL) || !supports_layer_op(op, a, b, dst))
        return fail(MX_UNSUPPORTED, "ADD / MUL: unsupported op or tensors");
    mx::BinaryArgs x{};
    x.op = op == MX_OP_ADD ? 0 : 1;
    x.a = (const float *)a->data;
    x.b = (const float *)b->data;
    x.dst = (float *)dst->data;
    for (int i = 0; i < 4; i++) {
        x.ne[i] = a->ne[i];
        x.a_nb[i] = (int64_t)a->nb[i];
        x.b_ne[i] = b->ne[i];
        x.b_nb[i] = (int64_t)b->nb[i];
        x.d_nb[i] = (int64_t)dst->nb[i];
    }
    HIP_OK(mx::launch_binary(x, be->stream), "ADD / MUL launch");
    return MX_SUCCESS;
}

MX_API int mx_swiglu(mx_backend *be, const mx_tensor *a, const mx_tensor *b, const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!supports_layer_op(MX_OP_SWIGLU, a, b, dst)) return fail(MX_UNSUPPORTED, "SWIGLU: unsupported tensors");
    HIP_OK(mx::launch_swiglu(rows_of(a, dst), (const float *)b->data, (int64_t)b->nb[1], be->stream), "SWIGLU launch");
    return MX_SUCCESS;
}

MX_API int mx_supports_rope(const mx_tensor *src, const mx_tensor *pos, const mx_tensor *dst, int n_dims, int mode,
                            float ext_factor, float attn_factor) {
    if (!f32_any(src) || !f32_any(dst) || !same_shape(src, dst) || src->ne[3] != 1) return 0;
    if (!pos || pos->type != MX_TYPE_I32 || !pos->data || pos->nb[0] != 4 || pos->ne[0] != src->ne[2] ||
        nelements(pos) != pos->ne[0])
        return 0;
    // GGML_ROPE_TYPE_NEOX (2) with the decoder's plain arguments
    return mode == 2 && n_dims > 0 && n_dims % 2 == 0 && n_dims <= src->ne[0] && ext_factor == 0.0f &&
           attn_factor == 1.0f;
}

MX_API int mx_rope(mx_backend *be, const mx_tensor *src, const mx_tensor *pos, const mx_tensor *dst, int n_dims,
                   int mode, float freq_base, float freq_scale, float ext_factor, float attn_factor) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!mx_supports_rope(src, pos, dst, n_dims, mode, ext_factor, attn_factor))
        return fail(MX_UNSUPPORTED, "ROPE: unsupported mode, parameters or tensors");
    // ggml_compute_forward_rope: theta_scale = powf(freq_base, -2.0f/n_dims), on the host as ggml-cpu forms it
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    HIP_OK(mx::launch_rope_neox(rows_of(src, dst), (const int32_t *)pos->data, n_dims, theta_scale, freq_scale,
                                be->stream),
           "ROPE launch");
    return MX_SUCCESS;
}

MX_API int mx_set_rows(mx_backend *be, const mx_tensor *src, const mx_tensor *idx, const mx_tensor *dst) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!supports_layer_op(MX_OP_SET_ROWS, src, idx, dst)) return fail(MX_UNSUPPORTED, "SET_ROWS: unsupported tensors");
    mx::RowsArgs r = rows_of(src, dst);
    HIP_OK(mx::launch_set_rows_f16(r, idx->data, idx->type == 27, dst->ne[1], be->err, be->stream), "SET_ROWS launch");
    return MX_SUCCESS;
}

// Validation and arguments of the q / k norm + RoPE + KV store step (mx_qk_norm_rope_kv; mx_attn_decode).
static int qkv_post_args(mx_backend *be, const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                         const mx_tensor *q_norm, const mx_tensor *k_norm, const mx_tensor *pos, const mx_tensor *q_out,
                         const mx_tensor *k_cache, const mx_tensor *v_cache, float eps, int n_dims, int mode,
                         float freq_base, float freq_scale, float ext_factor, float attn_factor, mx::QkvPostArgs *a) {
    auto heads = [](const mx_tensor *t) { return f32_any(t) && t->ne[0] == 128 && t->ne[3] == 1; };
    auto cache = [](const mx_tensor *c, int64_t nkv) {
        return c && c->type == MX_TYPE_F16 && shape_ok(c) && c->nb[0] == 2 && c->data && ((uintptr_t)c->data & 1) == 0 &&
               c->ne[0] == nkv * 128 && c->ne[2] == 1 && c->ne[3] == 1 && c->nb[1] % 2 == 0;
    };
    auto norm = [](const mx_tensor *w) { return f32_any(w) && w->ne[0] == 128 && nelements(w) == 128; };
    if (!heads(q) || !heads(k) || !heads(v) || !heads(q_out) || !same_shape(q, q_out) || !same_shape(k, v) ||
        k->ne[2] != q->ne[2] || !norm(q_norm) || !norm(k_norm) || !cache(k_cache, k->ne[1]) ||
        !cache(v_cache, k->ne[1]) || n_dims != 128 || mode != 2 || ext_factor != 0.0f || attn_factor != 1.0f)
        return fail(MX_UNSUPPORTED, "q/k norm + RoPE + KV store: head size 128, NEOX over all of it, f16 caches");
    if (!pos || pos->type != MX_TYPE_I32 || !pos->data || pos->nb[0] != 4 || pos->ne[0] != q->ne[2] ||
        nelements(pos) != pos->ne[0])
        return fail(MX_UNSUPPORTED, "q/k norm + RoPE + KV store: one I32 position per row");
    a->q = (const float *)q->data;
    a->k = (const float *)k->data;
    a->v = (const float *)v->data;
    a->qw = (const float *)q_norm->data;
    a->kw = (const float *)k_norm->data;
    a->pos = (const int32_t *)pos->data;
    a->q_out = (float *)q_out->data;
    a->kc = k_cache->data;
    a->vc = v_cache->data;
    a->nq = q->ne[1];
    a->nkv = k->ne[1];
    a->cache_rows = std::min(k_cache->ne[1], v_cache->ne[1]);
    a->q_nb1 = (int64_t)q->nb[1];
    a->q_nb2 = (int64_t)q->nb[2];
    a->k_nb1 = (int64_t)k->nb[1];
    a->k_nb2 = (int64_t)k->nb[2];
    a->v_nb1 = (int64_t)v->nb[1];
    a->v_nb2 = (int64_t)v->nb[2];
    a->qo_nb1 = (int64_t)q_out->nb[1];
    a->qo_nb2 = (int64_t)q_out->nb[2];
    a->kc_nb1 = (int64_t)k_cache->nb[1];
    a->vc_nb1 = (int64_t)v_cache->nb[1];
    a->eps = eps;
    a->theta_scale = powf(freq_base, -2.0f / (float)n_dims);  // as ggml-cpu forms it
    a->freq_scale = freq_scale;
    a->err = be->err;
    return MX_SUCCESS;
}

MX_API int mx_qk_norm_rope_kv(mx_backend *be, const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                              const mx_tensor *q_norm, const mx_tensor *k_norm, const mx_tensor *pos,
                              const mx_tensor *q_out, const mx_tensor *k_cache, const mx_tensor *v_cache, float eps,
                              int n_dims, int mode, float freq_base, float freq_scale, float ext_factor,
                              float attn_factor) {
    int rc = check_be(be);
    if (rc) return rc;
    mx::QkvPostArgs a{};
    if ((rc = qkv_post_args(be, q, k, v, q_norm, k_norm, pos, q_out, k_cache, v_cache, eps, n_dims, mode, freq_base,
                            freq_scale, ext_factor, attn_factor, &a)))
        return rc;
    HIP_OK(mx::launch_qkv_post(a, q->ne[2], be->stream), "q/k norm + RoPE + KV store launch");
    return MX_SUCCESS;
}

MX_API int mx_supports_flash_attn_ext(const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                                      const mx_tensor *mask, const mx_tensor *dst, float max_bias,
                                      float logit_softcap) {
    if (max_bias != 0.0f || logit_softcap != 0.0f) return 0;
    if (!f32_any(q) || q->ne[3] != 1) return 0;
    const int64_t D = q->ne[0];
    if (D != 64 && D != 128) return 0;
    for (const mx_tensor *t : {k, v}) {
        if (!t || t->type != MX_TYPE_F16 || !shape_ok(t) || t->nb[0] != 2 || !t->data || t->ne[0] != D ||
            t->ne[3] != 1 || !aligned16(t->data) || t->nb[1] % 16 != 0 || t->nb[2] % 16 != 0)
            return 0;
    }
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[2] < 1 || q->ne[2] % k->ne[2] != 0) return 0;
    if (mask && (mask->type != MX_TYPE_F16 || !shape_ok(mask) || mask->nb[0] != 2 || !mask->data ||
                 mask->ne[0] < k->ne[1] || mask->ne[1] < q->ne[1] || mask->ne[2] != 1 || mask->ne[3] != 1 ||
                 ((uintptr_t)mask->data & 1)))
        return 0;
    // the permuted output: dst [D, n_head, n_q] contiguous
    return dst && dst->type == MX_TYPE_F32 && dst->ne[0] == D && dst->ne[1] == q->ne[2] && dst->ne[2] == q->ne[1] &&
           dst->ne[3] == 1 && contiguous(dst) && dst->data && q->ne[1] <= 65535 && q->ne[2] <= 65535;
}

// Validation, arguments and scratch of an attention launch (mx_flash_attn_ext; mx_attn_decode).
static int fa_args(mx_backend *be, const mx_tensor *q, const mx_tensor *k, const mx_tensor *v, const mx_tensor *mask,
                   const mx_tensor *dst, float scale, mx::FaArgs *a) {
    if (!mx_supports_flash_attn_ext(q, k, v, mask, dst, 0.0f, 0.0f))
        return fail(MX_UNSUPPORTED, "FLASH_ATTN_EXT: unsupported tensors");
    a->q = (const float *)q->data;
    a->k = k->data;
    a->v = v->data;
    a->mask = mask ? mask->data : nullptr;
    a->dst = (float *)dst->data;
    a->D = (int)q->ne[0];
    a->n_q = q->ne[1];
    a->n_head = q->ne[2];
    a->n_kv = k->ne[1];
    a->gqa = q->ne[2] / k->ne[2];
    a->q_nb1 = (int64_t)q->nb[1];
    a->q_nb2 = (int64_t)q->nb[2];
    a->k_nb1 = (int64_t)k->nb[1];
    a->k_nb2 = (int64_t)k->nb[2];
    a->v_nb1 = (int64_t)v->nb[1];
    a->v_nb2 = (int64_t)v->nb[2];
    a->m_nb1 = mask ? (int64_t)mask->nb[1] : 0;
    a->scale = scale;
    a->nsplit = mx::fa_splits(a->n_q, a->n_head, a->n_kv, a->gqa, a->D);
    a->split_len = ((a->n_kv + 63) / 64 + a->nsplit - 1) / a->nsplit * 64;  // whole 64-position blocks per split
    if (a->nsplit > 1) {
        const size_t need = (size_t)a->n_q * (size_t)a->n_head * (size_t)a->nsplit * (size_t)(a->D + 2) * 4;
        int rc = ensure_scratch(be, need);
        if (rc) return rc;
        a->part = (float *)be->scratch;
    }
    return MX_SUCCESS;
}

MX_API int mx_flash_attn_ext(mx_backend *be, const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                             const mx_tensor *mask, const mx_tensor *dst, float scale) {
    int rc = check_be(be);
    if (rc) return rc;
    mx::FaArgs a{};
    if ((rc = fa_args(be, q, k, v, mask, dst, scale, &a))) return rc;
    HIP_OK(mx::launch_flash_attn(a, be->stream), "FLASH_ATTN_EXT launch");
    return MX_SUCCESS;
}

MX_API int mx_attn_decode(mx_backend *be, const mx_tensor *q, const mx_tensor *k, const mx_tensor *v,
                          const mx_tensor *q_norm, const mx_tensor *k_norm, const mx_tensor *pos,
                          const mx_tensor *k_cache, const mx_tensor *v_cache, const mx_tensor *k_view,
                          const mx_tensor *v_view, const mx_tensor *mask, const mx_tensor *dst, float eps, int n_dims,
                          int mode, float freq_base, float freq_scale, float ext_factor, float attn_factor,
                          float scale) {
    int rc = check_be(be);
    if (rc) return rc;
    mx::QkvPostArgs pa{};
    // the roped q is not written: q stands in for q_out in the checks
    if ((rc = qkv_post_args(be, q, k, v, q_norm, k_norm, pos, q, k_cache, v_cache, eps, n_dims, mode, freq_base,
                            freq_scale, ext_factor, attn_factor, &pa)))
        return rc;
    if (q->ne[2] != 1) return fail(MX_UNSUPPORTED, "fused attention: one decode row");
    for (const mx_tensor *t : {k_view, v_view})
        if (!t || t->ne[2] != k->ne[1] || t->nb[2] != 256) return fail(MX_UNSUPPORTED, "fused attention: cache views");
    if (k_view->data != k_cache->data || v_view->data != v_cache->data || k_view->nb[1] != k_cache->nb[1] ||
        v_view->nb[1] != v_cache->nb[1])
        return fail(MX_UNSUPPORTED, "fused attention: the views must read the caches from row 0");
    mx_tensor qa = *q;  // q as the attention reads it: [128, 1 row, heads]
    qa.ne[1] = 1;
    qa.ne[2] = q->ne[1];
    qa.nb[1] = q->nb[2];
    qa.nb[2] = q->nb[1];
    mx::FaArgs a{};
    if ((rc = fa_args(be, &qa, k_view, v_view, mask, dst, scale, &a))) return rc;
    if (a.gqa != 1 && a.gqa != 2 && a.gqa != 4) return fail(MX_UNSUPPORTED, "fused attention: 1, 2 or 4 q heads per kv head");
    if (a.n_kv < 1) return fail(MX_UNSUPPORTED, "fused attention: the cache views hold no position");
    HIP_OK(mx::launch_attn_decode(a, pa, be->stream), "fused attention launch");
    return MX_SUCCESS;
}

MX_API int mx_peak_read(mx_backend *be, const void *src, size_t bytes, int workgroups, int loads, int nontemporal) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!src || !aligned16(src) || bytes % 16 != 0) return fail(MX_INVALID, "peak read: 16-byte aligned whole chunks");
    if (workgroups < 1 || workgroups > 65536) return fail(MX_INVALID, "peak read: 1 to 65536 workgroups");
    if (loads != 1 && loads != 2 && loads != 4 && loads != 8 && loads != 16)
        return fail(MX_INVALID, "peak read: 1, 2, 4, 8 or 16 loads in flight");
    if ((rc = ensure_scratch(be, (size_t)workgroups * 4))) return rc;
    HIP_OK(mx::launch_peak_read(src, (int64_t)bytes, workgroups, loads, nontemporal != 0, (int *)be->scratch,
                                be->stream),
           "peak read launch");
    return MX_SUCCESS;
}

MX_API int mx_peak_mfma(mx_backend *be, int kind, int workgroups, int iters) {
    int rc = check_be(be);
    if (rc) return rc;
    if (kind != 0 && kind != 1) return fail(MX_INVALID, "peak mfma: kind 0 (int8) or 1 (fp16)");
    if (workgroups < 1 || workgroups > 65536 || iters < 1 || iters > 10000000)
        return fail(MX_INVALID, "peak mfma: 1 to 65536 workgroups, 1 to 1e7 rounds");
    if ((rc = ensure_scratch(be, (size_t)workgroups * 4))) return rc;
    HIP_OK(mx::launch_peak_mfma(kind, workgroups, iters, (int *)be->scratch, be->stream), "peak mfma launch");
    return MX_SUCCESS;
}

MX_API int mx_quantize_act(mx_backend *be, int type, int rounding, const float *x, int64_t k, int64_t nrows,
                           size_t x_row_stride, void *out) {
    int rc = check_be(be);
    if (rc) return rc;
    if (type != MX_TYPE_Q8_0 && type != MX_TYPE_Q8_1 && type != MX_TYPE_Q8_K)
        return fail(MX_UNSUPPORTED, "activation type %d", type);
    if (rounding != MX_ROUND_REF && rounding != MX_ROUND_X86) return fail(MX_INVALID, "unknown rounding %d", rounding);
    if (k < 0 || nrows < 0 || k % blck(type) != 0) return fail(MX_INVALID, "k must be a multiple of the block size");
    if (!aligned16(x) || x_row_stride % 16 != 0) return fail(MX_INVALID, "x rows must be 16-byte aligned");
    if ((type == MX_TYPE_Q8_K) && ((uintptr_t)out & 3)) return fail(MX_INVALID, "Q8_K output must be 4-byte aligned");
    HIP_OK(mx::launch_quantize_act(type, rounding, x, k, nrows, (int64_t)(x_row_stride / 4), out, be->stream),
           "quantize launch");
    return MX_SUCCESS;
}

// ------------------------------------------------------------------------------------------------------ graphs
MX_API int mx_graph_begin(mx_backend *be) {
    int rc = check_be(be);
    if (rc) return rc;
    if (be->capturing) return fail(MX_FAILED, "a graph is already being recorded");
    HIP_OK(hipStreamBeginCapture(be->stream, hipStreamCaptureModeThreadLocal), "begin capture");
    be->capturing = true;
    return MX_SUCCESS;
}

MX_API int mx_graph_end(mx_backend *be, mx_graph **graph) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!be->capturing) return fail(MX_FAILED, "no graph is being recorded");
    be->capturing = false;
    hipGraph_t g = nullptr;
    HIP_OK(hipStreamEndCapture(be->stream, &g), "end capture");
    mx_graph *out = new mx_graph();
    out->graph = g;
    out->be = be;
    out->scratch_gen = be->scratch_gen;
    hipError_t e = hipGraphInstantiate(&out->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        delete out;
        return hip_fail(e, "instantiate graph");
    }
    *graph = out;
    return MX_SUCCESS;
}

MX_API size_t mx_graph_nodes(const mx_graph *graph) {
    size_t n = 0;
    if (!graph || hipGraphGetNodes(graph->graph, nullptr, &n) != hipSuccess) return 0;
    return n;
}

MX_API int mx_graph_launch(mx_backend *be, mx_graph *graph) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!graph) return fail(MX_INVALID, "null graph");
    if (graph->be != be) return fail(MX_INVALID, "the graph was recorded on another backend");
    if (graph->scratch_gen != be->scratch_gen)
        return fail(MX_FAILED, "the graph was recorded before an op grew the backend's scratch (its kernels hold the "
                               "freed buffer); record it again");
    HIP_OK(hipGraphLaunch(graph->exec, be->stream), "launch graph");
    return MX_SUCCESS;
}

MX_API void mx_graph_free(mx_graph *graph) {
    if (!graph) return;
    // a replay may still be running on the recording backend's stream: let it finish before its exec goes
    if (graph->be && graph->be->stream) {
        (void)hipSetDevice(graph->be->device);
        (void)hipStreamSynchronize(graph->be->stream);
    }
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
}

// ------------------------------------------------------------------------------------------------------ events
MX_API mx_event *mx_event_new(mx_backend *be) {
    if (check_be(be)) return nullptr;
    mx_event *e = new mx_event();
    e->device = be->device;
    if (hipEventCreate(&e->ev) != hipSuccess) {
        fail(MX_FAILED, "cannot create an event");
        delete e;
        return nullptr;
    }
    return e;
}

MX_API int mx_event_record(mx_backend *be, mx_event *ev) {
    int rc = check_be(be);
    if (rc) return rc;
    if (!ev) return fail(MX_INVALID, "null event");
    HIP_OK(hipEventRecord(ev->ev, be->stream), "record event");
    return MX_SUCCESS;
}

MX_API int mx_event_synchronize(mx_event *ev) {
    if (!ev) return fail(MX_INVALID, "null event");
    HIP_OK(hipEventSynchronize(ev->ev), "synchronize event");
    return MX_SUCCESS;
}

MX_API int mx_event_elapsed_ms(mx_event *start, mx_event *end, float *ms) {
    if (!start || !end || !ms) return fail(MX_INVALID, "null argument");
    HIP_OK(hipEventElapsedTime(ms, start->ev, end->ev), "elapsed time");
    return MX_SUCCESS;
}

MX_API void mx_event_free(mx_event *ev) {
    if (!ev) return;
    (void)hipEventDestroy(ev->ev);
    delete ev;
}

}  // extern "C"
