// One decode step of a Qwen3 decoder (src/common/qwen3-decoder.cpp Qwen3Decoder::step :462-490, the layers of
// ::layers :350-410 and the head of ::outputs :422-438) as one persistent launch: GET_ROWS of the token, per layer
// RMS_NORM x attn_norm, the q / k / v products, q / k head norms + NEOX RoPE, SET_ROWS of the new key and value into
// the f16 caches, flash attention over positions 0..p, attn_o + residual, RMS_NORM x ffn_norm, gate / up, SwiGLU,
// down + residual; then the final norm, the output head and ARGMAX (the first of equal values). Q8_0 weights.
//
// Why one launch. A decode step is a chain of ~170 dependent phases whose products each stream 1-7 MB: launched one
// by one, each pays a launch (~1.7 us) plus a cold weight fetch (~1.2 us) before it can start. Here one workgroup per
// CU stays resident for the whole step, and
//   - every phase's weights (its rows of the product, or its split of the KV cache) are copied into LDS by
//     buffer-to-LDS DMA while the workgroup still waits for the phase's input, so a phase starts with its weights on
//     chip and the weight stream is off the dependency chain;
//   - a phase's outputs travel to the next phase as 8-byte words (32-bit tag, 32-bit value) written and polled with
//     agent-scope atomic accesses (coherent across the XCDs' L2s, no cache write-back or fence): a word is valid when
//     its tag is this step's tag for that phase, so a consumer needs no separate flag and no barrier. One phase's
//     all-to-all costs ~1.5-2 us on MI355X (measured with 256 workgroups).
// Tags: epoch * 1024 + phase + 1, epoch a device counter the last workgroup advances at the end of the step; words of
// an earlier step (or phase) never carry the current tag. A buffer is rewritten six phases after it is read, and a
// workgroup reaches phase v + 2 only after every workgroup has finished phase v, so no word is overwritten while
// read.
//
// Phases of layer l (6 l + k): 0 norm + q/k/v rows; 1 attention over one (kv head, position split); 2 merge of the
// splits (8 channels per workgroup); 3 attn_o rows + residual; 4 norm + gate/up rows + SwiGLU; 5 down rows + residual.
// Then the head (norm + output rows + local argmax) and the pick (workgroup 0).
//
// Arithmetic as the separate kernels (and ggml-cpu): activations quantized to Q8_0 blocks (REF or x86 rounding),
// exact int32 block sums, fp32 (d_w d_x) * isum summed in fp32; RMS norm squares summed in double; q / k norms and
// RoPE as k_qkv_post; attention as k_fa_gqa (q rounded to fp16, fp32 scores, online softmax, fp32 V accumulator) and
// the merge of k_fa_merge; SwiGLU x / (1 + expf(-x)) * g; residual adds in fp32. Only the order of fp32 sums differs.
//
// Every wait is bounded (spin_limit polls); a workgroup that times out sets bit 3 of the error word and the step
// ends early for every workgroup (each times out in turn), which mx_backend_synchronize reports.
#include "mx_common.h"
#include "mx_device.h"

#pragma clang fp contract(off)

#include "mx_layer.h"

namespace mx {

typedef int dv4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void dec_lds;

constexpr int DT = DEC_THREADS, DW = DEC_THREADS / 64;
constexpr int NSLOT = 3;
constexpr int KVC = 64;                       // positions per attention chunk: K and V rows of 256 bytes, one slot
// NG groups of four inputs per thread and NC 16-code chunks per lane and row cover products of K <= 2048 NG and
// K <= 1024 NC: one instance, for inputs up to DEC_KMAX.
constexpr int HD = 128;

// LDS carve, bytes
constexpr int L_SLOT = 0;                                 // NSLOT * DEC_SLOT
constexpr int L_XQ = NSLOT * DEC_SLOT;                    // int8 [DEC_KMAX] quantized input
constexpr int L_XD = L_XQ + DEC_KMAX;                     // float [DEC_KMAX / 32] its block scales
constexpr int L_HB = L_XD + DEC_KMAX / 8;                 // float [DEC_HMAX] residual stream
constexpr int L_QS = L_HB + DEC_HMAX * 4;                 // float [4][128] q heads (fp16 values)
constexpr int L_PS = L_QS + 4 * HD * 4;                   // float [4][64] scores / weights
constexpr int L_ACC = L_PS + 4 * KVC * 4;                 // float [DT * 2] P.V partial sums
constexpr int L_KN = L_ACC + DT * 2 * 4;                  // uint16 [2][128] the new key and value
constexpr int L_RED = L_KN + 2 * HD * 2;                  // double [DW] / (float, int) [DW] reductions
constexpr int L_SM = L_RED + DW * 8;                      // float [3][4]: running max, sum, rescale per head
constexpr int L_END = L_SM + 12 * 4;

size_t decode_lds_bytes() { return (size_t)L_END; }

// ------------------------------------------------------------------------------------------------ exchange words
__device__ __forceinline__ uint64_t ll_ld(const uint64_t *p) {
    return __hip_atomic_load((uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_st(uint64_t *p, uint32_t tag, float v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

struct LL {
    int qkv, part, att, h1, g, h2, arg, total;
};
__host__ __device__ inline LL ll_layout(const DecArgs &a, int grid) {
    LL o;
    o.qkv = 0;
    o.part = o.qkv + a.Q + 2 * a.KV;
    o.att = o.part + a.nkv * a.S * a.gqa * (HD + 2);
    o.h1 = o.att + a.Q;
    o.g = o.h1 + a.H;
    o.h2 = o.g + a.F;
    o.arg = o.h2 + a.H;
    o.total = o.arg + 2 * grid;
    return o;
}
size_t decode_ll_words(const DecArgs &a, int grid) { return (size_t)ll_layout(a, grid).total; }

// Thread t's groups of four words t, t + DT, ... of buf[0, n) (n % 4 == 0) into v[], once every word carries `tag`.
// False after spin_limit polls.
template <int NG>
__device__ __forceinline__ bool ll_poll4(const uint64_t *buf, int n, uint32_t tag, float4 (&v)[NG], int limit) {
    const int t = threadIdx.x, ng = n / 4;
    for (int spins = 0;; spins++) {
        uint64_t w[NG][4];
#pragma unroll
        for (int j = 0; j < NG; j++) {
            const int g = t + DT * j;
            if (g < ng) {
#pragma unroll
                for (int e = 0; e < 4; e++) w[j][e] = ll_ld(buf + 4 * g + e);
            }
        }
        bool ok = true;
#pragma unroll
        for (int j = 0; j < NG; j++) {
            const int g = t + DT * j;
            if (g < ng) {
#pragma unroll
                for (int e = 0; e < 4; e++) ok = ok && (uint32_t)(w[j][e] >> 32) == tag;
                v[j] = make_float4(__uint_as_float((uint32_t)w[j][0]), __uint_as_float((uint32_t)w[j][1]),
                                   __uint_as_float((uint32_t)w[j][2]), __uint_as_float((uint32_t)w[j][3]));
            }
        }
        if (ok) return true;
        if (spins >= limit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

// Up to N words at p[off[i]] (i < n), polled together.
template <int N>
__device__ __forceinline__ bool ll_pollv(const uint64_t *p, const int (&off)[N], int n, uint32_t tag, float (&v)[N],
                                         int limit) {
    for (int spins = 0;; spins++) {
        uint64_t w[N];
#pragma unroll
        for (int i = 0; i < N; i++)
            if (i < n) w[i] = ll_ld(p + off[i]);
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; i++)
            if (i < n) {
                ok = ok && (uint32_t)(w[i] >> 32) == tag;
                v[i] = __uint_as_float((uint32_t)w[i]);
            }
        if (ok) return true;
        if (spins >= limit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

__device__ __forceinline__ void vm_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Every wave's copies and polls landed, and the workgroup agrees that its polls succeeded: a failed poll in any
// thread ends the step for the whole workgroup.
__device__ __forceinline__ bool sync_ok(bool mine, int *abort_flag) {
    vm_wait_all();
    if (!mine) *abort_flag = 1;
    __syncthreads();
    return *abort_flag == 0;
}

// -------------------------------------------------------------------------------------------------- weight items
// Item 5 l + k of the step: k = 0 q/k/v rows, 1 KV split, 2 attn_o rows, 3 gate/up rows, 4 down rows of layer l.
// A product item lays its rows' codes out back to back in the slot, then their fp16 scales.
struct Seg {
    Q8p w;
    int row0, n;
};
struct MvItem {
    Seg seg[3];  // empty segments have n = 0
    int nrows, K;
};

// The layer table through the constant address space: its fields come in by scalar loads, which no wait for the
// copies in flight (vmcnt) has to cover.
typedef const __attribute__((address_space(4))) DecLayer *ConstLayers;
__device__ __forceinline__ ConstLayers const_layers(const DecArgs &a) { return (ConstLayers)(uintptr_t)a.layers; }
template <typename T>
__device__ __forceinline__ Q8p q8of(const T &x) {
    return Q8p{x.q, x.d};
}

__device__ __forceinline__ MvItem mv_item(const DecArgs &a, int layer, int kind, int wg) {
    const auto &L = const_layers(a)[layer];
    MvItem it{};
    if (kind == 0) {  // q, k, v rows of the concatenated [q | k | v] outputs
        it.K = a.H;
        const int N = a.Q + 2 * a.KV, r0 = min(N, wg * a.r_qkv), r1 = min(N, r0 + a.r_qkv);
        const int b1 = a.Q, b2 = a.Q + a.KV;
        it.seg[0] = Seg{q8of(L.wq), r0, max(0, min(r1, b1) - r0)};
        it.seg[1] = Seg{q8of(L.wk), max(r0, b1) - b1, max(0, min(r1, b2) - max(r0, b1))};
        it.seg[2] = Seg{q8of(L.wv), max(r0, b2) - b2, max(0, r1 - max(r0, b2))};
        it.nrows = r1 - r0;
    } else if (kind == 2 || kind == 4) {
        it.K = kind == 2 ? a.Q : a.F;
        const int rr = kind == 2 ? a.r_o : a.r_d;
        const int r0 = min(a.H, wg * rr), r1 = min(a.H, r0 + rr);
        it.seg[0] = Seg{kind == 2 ? q8of(L.wo) : q8of(L.wd), r0, r1 - r0};
        it.nrows = r1 - r0;
    } else {  // gate rows, then the same up rows
        it.K = a.H;
        const int r0 = min(a.F, wg * a.r_f), r1 = min(a.F, r0 + a.r_f);
        it.seg[0] = Seg{q8of(L.wg), r0, r1 - r0};
        it.seg[1] = Seg{q8of(L.wu), r0, r1 - r0};
        it.nrows = 2 * (r1 - r0);
    }
    return it;
}

// Copies `bytes` (a multiple of 16) from src to LDS byte address dst, 1 KB per wave instruction; instruction i of the
// item goes to wave i % DW.
__device__ __forceinline__ void dma_copy(const uint8_t *src, uint32_t dst, int bytes, int &instr, int wave,
                                         int lane) {
    const int n = (bytes + 1023) / 1024;
    for (int i = 0; i < n; i++, instr++) {
        if (instr % DW != wave) continue;
        if (1024 * i + 16 * lane < bytes)
            __builtin_amdgcn_global_load_lds((const void *)(src + 1024 * i + 16 * lane),
                                             (dec_lds *)(uintptr_t)(dst + 1024 * i), 16, 0, 0);
    }
}

// The attention split of workgroup wg: kv head, positions [j0, j1) of 0..p.
struct Split {
    int hk, s, j0, j1;
    bool on;
};
__device__ __forceinline__ Split split_of(const DecArgs &a, int wg, int p) {
    Split sp{};
    sp.on = wg < a.nkv * a.S;
    if (!sp.on) return sp;
    sp.hk = wg / a.S;
    sp.s = wg % a.S;
    const int n = p + 1, len = (n + a.S - 1) / a.S;
    sp.j0 = min(n, sp.s * len);
    sp.j1 = min(n, sp.j0 + len);
    return sp;
}

// K rows then V rows of `np` positions from j0 (256 bytes of kv head hk each), four rows per instruction.
__device__ __forceinline__ void dma_kv(const DecArgs &a, const uint16_t *kc, const uint16_t *vc, const Split &sp,
                                       uint32_t dst, int &instr, int wave, int lane) {
    const int np = min(KVC, sp.j1 - sp.j0);
    const int n = (np + 3) / 4;
    for (int c = 0; c < 2; c++) {
        const uint16_t *base = (c == 0 ? kc : vc) + (int64_t)sp.hk * HD;
        for (int i = 0; i < n; i++, instr++) {
            if (instr % DW != wave) continue;
            const int row = 4 * i + (lane >> 4);
            if (row < np)
                __builtin_amdgcn_global_load_lds(
                    (const void *)((const uint8_t *)(base + (int64_t)(sp.j0 + row) * a.KV) + 16 * (lane & 15)),
                    (dec_lds *)(uintptr_t)(dst + c * (KVC * 256) + 1024 * i), 16, 0, 0);
        }
    }
}

__device__ __forceinline__ void issue_item(const DecArgs &a, int item, uint32_t lds0, int wg, int p, int wave,
                                           int lane) {
    const int layer = item / 5, kind = item % 5;
    if (layer >= a.n_layer) return;
    const uint32_t dst = lds0 + L_SLOT + (uint32_t)(item % NSLOT) * DEC_SLOT;
    int instr = 0;
    if (kind == 1) {
        const Split sp = split_of(a, wg, p);
        if (sp.on && sp.j1 > sp.j0) {
            const auto &L = const_layers(a)[layer];
            dma_kv(a, L.kc, L.vc, sp, dst, instr, wave, lane);
        }
        return;
    }
    const MvItem it = mv_item(a, layer, kind, wg);
    int rows = 0;
#pragma unroll
    for (int t = 0; t < 3; t++) {
        const Seg &s = it.seg[t];
        if (s.n <= 0) continue;
        dma_copy(s.w.q + (int64_t)s.row0 * it.K, dst + rows * it.K, s.n * it.K, instr, wave, lane);
        dma_copy(s.w.d + (int64_t)s.row0 * (it.K / 16), dst + it.nrows * it.K + rows * (it.K / 16), s.n * (it.K / 16),
                 instr, wave, lane);
        rows += s.n;
    }
}

// -------------------------------------------------------------------------------------------------- product parts
// Quantizes the input held by the threads (group g = t + DT j: elements 4g..4g+3 in v[j]) into xq / xd: Q8_0 blocks,
// eight consecutive threads per block, scales rounded to fp16 as the dot reads them.
template <int NG>
__device__ __forceinline__ void quantize_input(const float4 (&v)[NG], int K, int rounding, uint8_t *lds) {
    int8_t *xq = (int8_t *)(lds + L_XQ);
    float *xd = (float *)(lds + L_XD);
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NG; j++) {
        const int g = t + DT * j;
        if (DT * j >= K / 4) break;  // uniform
        float d;
        int sum;
        const float4 x = g < K / 4 ? v[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        const int q = quant32_lane(x, rounding, &d, &sum);
        if (g < K / 4) {
            *(int *)(xq + 4 * g) = q;
            if ((g & 7) == 0) xd[g >> 3] = h2f(f2h(d));
        }
    }
}

// v[] *= rms-norm scale, then * w (ggml_rms_norm then ggml_mul): squares summed in double over the workgroup.
template <int NG>
__device__ __forceinline__ void rms_norm_input(float4 (&v)[NG], int K, const float *w, float eps, uint8_t *lds) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < NG; j++) {
        if (t + DT * j < K / 4) {
            const float4 x = v[j];
            ss += (double)(x.x * x.x);
            ss += (double)(x.y * x.y);
            ss += (double)(x.z * x.z);
            ss += (double)(x.w * x.w);
        }
    }
    ss = wave_sum_d(ss);
    double *red = (double *)(lds + L_RED);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < DW; i++) tot += red[i];
    const float mean = (float)(tot / (double)K);
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int j = 0; j < NG; j++) {
        const int g = t + DT * j;
        if (g < K / 4) {
            const float4 wv = *(const float4 *)(w + 4 * g);
            v[j].x = (v[j].x * scale) * wv.x;
            v[j].y = (v[j].y * scale) * wv.y;
            v[j].z = (v[j].z * scale) * wv.z;
            v[j].w = (v[j].w * scale) * wv.w;
        }
    }
    __syncthreads();  // red is reused
}

// The lane's input chunks (chunk c = lane + 64 i: 16 codes, and its block's scale) into registers.
template <int NC>
struct XChunks {
    dv4i q[NC];
    float d[NC];
};
template <int NC>
__device__ __forceinline__ void load_xchunks(XChunks<NC> &x, int K, const uint8_t *lds, int lane) {
    const int nc = K / 16;
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = lane + 64 * i;
        if (64 * i >= nc) break;  // uniform
        const int cc = c < nc ? c : 0;
        x.q[i] = *(const dv4i *)(lds + L_XQ + 16 * cc);
        x.d[i] = ((const float *)(lds + L_XD))[cc >> 1];
    }
}

// Row dot from LDS (codes at qa, scales at sa: byte addresses), the weights read by inline assembly: a DMA of the next
// item may be in flight, and the compiler would otherwise wait for it before any LDS read. Exact in lane 63.
template <int NC>
__device__ __forceinline__ float row_dot(uint32_t qa, uint32_t sa, int K, const XChunks<NC> &x, int lane) {
    const int nc = K / 16;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; i++) {
        if (64 * i >= nc) break;  // uniform
        const int c = lane + 64 * i;
        const bool valid = c < nc;
        const int cc = valid ? c : 0;
        dv4i q;
        uint32_t d;
        asm volatile("ds_read_b128 %0, %2\n\tds_read_u16 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(q), "=&v"(d)
                     : "v"(qa + 16 * cc), "v"(sa + 2 * (cc >> 1))
                     : "memory");
        int s = 0;
        s = __builtin_amdgcn_sdot4(q.x, x.q[i].x, s, false);
        s = __builtin_amdgcn_sdot4(q.y, x.q[i].y, s, false);
        s = __builtin_amdgcn_sdot4(q.z, x.q[i].z, s, false);
        s = __builtin_amdgcn_sdot4(q.w, x.q[i].w, s, false);
        s += dpp_i<dpp::XOR1>(0, s);  // the block's other half (chunks 2b, 2b + 1 sit in lanes 2j, 2j + 1)
        if (valid && (lane & 1) == 0) acc += (float)s * (h2f((uint16_t)d) * x.d[i]);
    }
    return sum_lanes<64>(acc);
}


// The head's rows [r0, r0 + nr) of this workgroup, rows wave, wave + DW, ... per wave, B rows' loads in flight per
// wave: logits to global memory and the wave's first largest non-NaN value (lane 63). K = 1024 NCH.
template <int NCH, int NC>
__device__ __forceinline__ void head_rows(const DecArgs &a, const XChunks<NC> &xc, int r0, int nr, int wave, int lane,
                                          float &best, int &bi, float *first) {
    constexpr int B = 8 / NCH;
    const int K = 1024 * NCH;
    for (int i0 = wave; i0 < nr; i0 += DW * B) {
        dv4i q[B][NCH];
        uint16_t d[B][NCH];
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int64_t n = r0 + min(i0 + DW * b, nr - 1);
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                const int ch = lane + 64 * c;
                q[b][c] = *(const dv4i *)(a.out.q + n * K + 16 * ch);
                d[b][c] = *(const uint16_t *)(a.out.d + n * (K / 16) + 2 * (ch >> 1));
            }
        }
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int i = i0 + DW * b;
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                int s = 0;
                s = __builtin_amdgcn_sdot4(q[b][c].x, xc.q[c].x, s, false);
                s = __builtin_amdgcn_sdot4(q[b][c].y, xc.q[c].y, s, false);
                s = __builtin_amdgcn_sdot4(q[b][c].z, xc.q[c].z, s, false);
                s = __builtin_amdgcn_sdot4(q[b][c].w, xc.q[c].w, s, false);
                s += dpp_i<dpp::XOR1>(0, s);
                if ((lane & 1) == 0) acc += (float)s * (h2f(d[b][c]) * xc.d[c]);
            }
            const float y = sum_lanes<64>(acc);
            if (i < nr && lane == 63) {
                a.logits[r0 + i] = y;
                if (r0 + i == 0) *first = y;
                if (!(y != y) && (bi < 0 || y > best)) {
                    best = y;
                    bi = r0 + i;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------------ the kernel
template <int NG, int NC>
__global__ __launch_bounds__(DT) void k_decode_step(DecArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wg = blockIdx.x, G = gridDim.x;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(dec_lds *)lds;
    const LL o = ll_layout(a, G);
    const int32_t tok = *a.token, p = *a.pos;
    if (tok < 0 || tok >= a.V || p < 0 || p >= a.cache_rows) {  // the same for every workgroup: nothing runs
        if (wg == 0 && tid == 0) atomicOr(a.err, (tok < 0 || tok >= a.V) ? 1 : 4);
        return;
    }
    const uint32_t E = *a.epoch;
#define tag(phase) (E * 1024u + (uint32_t)(phase) + 1u)
    __shared__ int abort_flag;
    if (tid == 0) abort_flag = 0;

    // items 0..2 go out first; issue_upto(last) sends every item up to `last` not sent yet
    int next_item = 0;
    const int n_items = 5 * a.n_layer;
#define issue_upto(last)                                                          \
    for (; next_item <= (last) && next_item < n_items; next_item++) issue_item(a, next_item, lds0, wg, p, wave, lane)
    issue_upto(2);

    // GET_ROWS of the token: every workgroup dequantizes the row itself (d * q, as dequantize_row_q8_0)
    float4 v[NG];
#pragma unroll
    for (int j = 0; j < NG; j++) {
        const int g = tid + DT * j;
        if (g < a.H / 4) {
            const int64_t e = (int64_t)tok * a.H + 4 * g;
            const int q = *(const int *)(a.emb.q + e);
            const float d = h2f(*(const uint16_t *)(a.emb.d + (e / 32) * 2));
            v[j] = make_float4(d * (float)(int8_t)(q & 0xFF), d * (float)(int8_t)((q >> 8) & 0xFF),
                               d * (float)(int8_t)((q >> 16) & 0xFF), d * (float)(int8_t)(q >> 24));
        }
    }
    vm_wait_all();
    __syncthreads();

    float *hb = (float *)(lds + L_HB);
    XChunks<NC> xc;
    bool ok = true;


    for (int l = 0; l < a.n_layer; l++) {
        const auto &L = const_layers(a)[l];
        const int ph = 6 * l;
        // ---------------------------------------------------------------- phase 0: norm + q / k / v rows
        ok = true;
        if (l > 0) ok = ll_poll4(a.ll + o.h2, a.H, tag(ph - 1), v, a.spin_limit);
        if (!sync_ok(ok, &abort_flag)) break;
#pragma unroll
        for (int j = 0; j < NG; j++)
            if (tid + DT * j < a.H / 4) *(float4 *)(hb + 4 * (tid + DT * j)) = v[j];
        rms_norm_input(v, a.H, L.attn_norm, a.eps, lds);
        quantize_input(v, a.H, a.rounding, lds);
        __syncthreads();
        load_xchunks(xc, a.H, lds, lane);
        issue_upto(5 * l + 2);  // in flight during the rows: nothing below reads LDS outside inline assembly
        {
            const int item = 5 * l;
            const MvItem it = mv_item(a, l, 0, wg);
            const uint32_t slot = lds0 + L_SLOT + (uint32_t)(item % NSLOT) * DEC_SLOT;
            const int r0 = wg * a.r_qkv;
            for (int i = wave; i < it.nrows; i += DW) {
                const float y = row_dot(slot + i * it.K, slot + it.nrows * it.K + i * (it.K / 16), it.K, xc, lane);
                if (lane == 63) ll_st(a.ll + o.qkv + r0 + i, tag(ph), y);
            }
        }
        // ---------------------------------------------------------------- phase 1: attention split
        {
            const Split sp = split_of(a, wg, p);
            const int G_ = a.gqa;
            float x0 = 0.f, x1 = 0.f, w0 = 0.f, w1 = 0.f;
            const bool owner = sp.on && p >= sp.j0 && p < sp.j1;
            ok = true;
            if (sp.on && wave < G_) {  // q head hk * gqa + wave: lane holds channels lane, lane + 64
                w0 = L.q_norm[lane];
                w1 = L.q_norm[lane + 64];
                const int off[2] = {lane, lane + 64};
                float xv[2];
                ok = ll_pollv<2>(a.ll + o.qkv + (sp.hk * G_ + wave) * HD, off, 2, tag(ph), xv, a.spin_limit);
                x0 = xv[0];
                x1 = xv[1];
            }
            float k0 = 0.f, k1 = 0.f, vv0 = 0.f, vv1 = 0.f, kw0 = 0.f, kw1 = 0.f;
            if (owner && wave == 4) {  // the new key and value
                kw0 = L.k_norm[lane];
                kw1 = L.k_norm[lane + 64];
                const int kb = a.Q + sp.hk * HD, vb = a.Q + a.KV + sp.hk * HD;
                const int off[4] = {kb + lane, kb + lane + 64, vb + lane, vb + lane + 64};
                float kv[4];
                ok = ll_pollv<4>(a.ll + o.qkv, off, 4, tag(ph), kv, a.spin_limit);
                k0 = kv[0];
                k1 = kv[1];
                vv0 = kv[2];
                vv1 = kv[3];
            }
            if (!sync_ok(ok, &abort_flag)) break;
            float *qs = (float *)(lds + L_QS);
            uint16_t *kn = (uint16_t *)(lds + L_KN);
            if (sp.on && wave < G_) {
                float o0, o1;
                qk_norm_rope(x0, x1, w0, w1, p, a.eps, a.theta_scale, a.freq_scale, lane, o0, o1);
                qs[wave * HD + lane] = h2f(f2h(o0));  // ggml converts q to K's f16 first
                qs[wave * HD + lane + 64] = h2f(f2h(o1));
            }
            if (owner && wave == 4) {
                float o0, o1;
                qk_norm_rope(k0, k1, kw0, kw1, p, a.eps, a.theta_scale, a.freq_scale, lane, o0, o1);
                const uint16_t h0 = f2h(o0), h1 = f2h(o1), e0 = f2h(vv0), e1 = f2h(vv1);
                uint16_t *kc = L.kc + (int64_t)p * a.KV + sp.hk * HD, *vc = L.vc + (int64_t)p * a.KV + sp.hk * HD;
                kc[lane] = h0;  // SET_ROWS of the new key and value (no other workgroup reads row p in this step)
                kc[lane + 64] = h1;
                vc[lane] = e0;
                vc[lane + 64] = e1;
                kn[lane] = h0;
                kn[lane + 64] = h1;
                kn[HD + lane] = e0;
                kn[HD + lane + 64] = e1;
            }
            float *ps = (float *)(lds + L_PS);
            float *sm = (float *)(lds + L_SM);  // [0..3] running max, [4..7] sum, [8..11] rescale
            if (tid < 4) {
                sm[tid] = -INFINITY;
                sm[4 + tid] = 0.0f;
            }
            const uint32_t slot = (uint32_t)(L_SLOT + ((5 * l + 1) % NSLOT) * DEC_SLOT);
            uint8_t *Ks = lds + slot, *Vs = lds + slot + KVC * 256;
            // roles: scores (head gs, position js, part ts of T); P.V (head gv, channel pair cp, positions part pv)
            const int T = DT / (G_ * 64), CPT = HD / T;
            const int pair = tid / T, gs = pair / 64, js = pair % 64, ts = tid % T;
            const int TPH = DT / G_, gv = tid / TPH, cp = (tid % TPH) % 64, pv = (tid % TPH) / 64, PP = TPH / 64;
            const int PLEN = KVC / PP;
            float acc0 = 0.f, acc1 = 0.f;
            if (sp.on) {
                for (int base = sp.j0; base < sp.j1; base += KVC) {
                    const int np = min(KVC, sp.j1 - base);
                    if (base > sp.j0) {  // later chunks (contexts past 64 S positions): plain loads into the slot
                        __syncthreads();
                        const uint16_t *kb = L.kc + (int64_t)sp.hk * HD, *vb = L.vc + (int64_t)sp.hk * HD;
                        for (int e = tid; e < 2 * KVC * 16; e += DT) {
                            const int c = e / (KVC * 16), row = (e / 16) % KVC, seg = e % 16;
                            if (row < np)
                                *(uint4 *)(lds + slot + c * KVC * 256 + row * 256 + 16 * seg) =
                                    *(const uint4 *)((const uint8_t *)((c == 0 ? kb : vb) + (int64_t)(base + row) * a.KV) +
                                                     16 * seg);
                        }
                    }
                    __syncthreads();
                    if (owner && p >= base && p < base + np && tid < 64) {  // the new row from registers of wave 4
                        *(uint32_t *)(Ks + (p - base) * 256 + 4 * tid) = *(const uint32_t *)(kn + 2 * tid);
                        *(uint32_t *)(Vs + (p - base) * 256 + 4 * tid) = *(const uint32_t *)(kn + HD + 2 * tid);
                    }
                    __syncthreads();
                    {  // scores
                        const uint8_t *kr = Ks + js * 256 + ts * CPT * 2;
                        const float *qv = qs + gs * HD + ts * CPT;
                        float d0 = 0.0f;
                        for (int c = 0; c < CPT / 8; c++) {
                            const uint4 w = *(const uint4 *)(kr + 16 * c);
                            const float4 qa = *(const float4 *)(qv + 8 * c), qb = *(const float4 *)(qv + 8 * c + 4);
                            d0 = fmaf(h2f((uint16_t)(w.x & 0xFFFF)), qa.x, d0);
                            d0 = fmaf(h2f((uint16_t)(w.x >> 16)), qa.y, d0);
                            d0 = fmaf(h2f((uint16_t)(w.y & 0xFFFF)), qa.z, d0);
                            d0 = fmaf(h2f((uint16_t)(w.y >> 16)), qa.w, d0);
                            d0 = fmaf(h2f((uint16_t)(w.z & 0xFFFF)), qb.x, d0);
                            d0 = fmaf(h2f((uint16_t)(w.z >> 16)), qb.y, d0);
                            d0 = fmaf(h2f((uint16_t)(w.w & 0xFFFF)), qb.z, d0);
                            d0 = fmaf(h2f((uint16_t)(w.w >> 16)), qb.w, d0);
                        }
                        for (int off = 1; off < T; off <<= 1) d0 += __shfl_xor(d0, off, 64);
                        if (ts == 0) ps[gs * KVC + js] = js < np ? d0 * a.scale : -INFINITY;
                    }
                    __syncthreads();
                    if (wave < G_) {  // online softmax, one wave per head
                        const float sv = ps[wave * KVC + lane];
                        const float mc = wave_max_f(sv);
                        const float Mold = sm[wave];
                        float r = 1.0f, pj = 0.0f, Mn = Mold;
                        if (mc != -INFINITY) {
                            Mn = fmaxf(Mold, mc);
                            r = expf(Mold - Mn);
                            pj = sv == -INFINITY ? 0.0f : expf(sv - Mn);
                        }
                        const float sum = wave_sum_f(pj);
                        ps[wave * KVC + lane] = pj;
                        if (lane == 0) {
                            sm[8 + wave] = r;
                            sm[wave] = Mn;
                            sm[4 + wave] = sm[4 + wave] * r + sum;
                        }
                    }
                    __syncthreads();
                    {  // P.V
                        const float r = sm[8 + gv];
                        acc0 *= r;
                        acc1 *= r;
                        for (int t = 0; t < PLEN; t++) {
                            const int j = pv * PLEN + t;
                            if (j >= np) break;  // rows past the chunk hold other bytes (possibly NaN patterns)
                            const float pj = ps[gv * KVC + j];
                            const uint32_t v2 = *(const uint32_t *)(Vs + j * 256 + 4 * cp);
                            acc0 = fmaf(pj, h2f((uint16_t)(v2 & 0xFFFF)), acc0);
                            acc1 = fmaf(pj, h2f((uint16_t)(v2 >> 16)), acc1);
                        }
                    }
                }
            }
            float *accs = (float *)(lds + L_ACC);
            __syncthreads();
            accs[(pv * G_ + gv) * HD + 2 * cp] = acc0;
            accs[(pv * G_ + gv) * HD + 2 * cp + 1] = acc1;
            __syncthreads();
            if (sp.on) {  // this split's (max, sum, channels) per head
                for (int e = tid; e < G_ * (HD + 2); e += DT) {
                    const int g = e / (HD + 2), c = e % (HD + 2);
                    float val;
                    if (c == 0) val = sm[g];
                    else if (c == 1) val = sm[4 + g];
                    else {
                        val = 0.0f;
                        for (int pp = 0; pp < PP; pp++) val += accs[(pp * G_ + g) * HD + (c - 2)];
                    }
                    ll_st(a.ll + o.part + ((sp.hk * a.S + sp.s) * G_ + g) * (HD + 2) + c, tag(ph + 1), val);
                }
            }
            issue_upto(5 * l + 3);
        }
        // ---------------------------------------------------------------- phase 2: merge of the splits
        {
            const int o0 = wg * a.r_m;
            const int nd = max(0, min(a.r_m, a.Q - o0));
            const int h = o0 / HD, hk = h / a.gqa, g = h % a.gqa, d0 = o0 % HD;
            float ms = -INFINITY, ss = 0.0f, vals[8];
            ok = true;
            if (wave == 0 && nd > 0 && lane < a.S) {
                int off[10];
                float pv[10];
                off[0] = 0;
                off[1] = 1;
                for (int d = 0; d < 8; d++) off[2 + d] = 2 + d0 + d;
                ok = ll_pollv<10>(a.ll + o.part + ((hk * a.S + lane) * a.gqa + g) * (HD + 2), off, 2 + nd, tag(ph + 1),
                                  pv, a.spin_limit);
                ms = pv[0];
                ss = pv[1];
                for (int d = 0; d < 8; d++) vals[d] = pv[2 + d];
            }
            if (!sync_ok(ok, &abort_flag)) break;
            if (wave == 0 && nd > 0) {
                const float M = wave_max_f(ms);
                const float w = (ms == -INFINITY) ? 0.0f : expf(ms - M);
                const float S = wave_sum_f(ss * w);
                const float inv = S == 0.0f ? 0.0f : 1.0f / S;
                for (int d = 0; d < 8; d++) {
                    if (d >= nd) break;
                    const float accd = wave_sum_f(lane < a.S ? vals[d] * w : 0.0f);
                    if (lane == 0) ll_st(a.ll + o.att + o0 + d, tag(ph + 2), accd * inv);
                }
            }
            issue_upto(5 * l + 4);  // down goes out (after the merge: its shuffles would otherwise wait for it)
        }
        // ---------------------------------------------------------------- phase 3: attn_o rows + residual
        ok = ll_poll4(a.ll + o.att, a.Q, tag(ph + 2), v, a.spin_limit);
        if (!sync_ok(ok, &abort_flag)) break;
        quantize_input(v, a.Q, a.rounding, lds);
        __syncthreads();
        load_xchunks(xc, a.Q, lds, lane);
        {
            const int r0 = wg * a.r_o;
            const int nr = max(0, min(a.r_o, a.H - r0));
            float res[4];
#pragma unroll
            for (int i = 0; i < 4; i++) res[i] = (wave + DW * i < nr) ? hb[r0 + wave + DW * i] : 0.0f;
            issue_upto(5 * l + 4);
            const uint32_t slot = lds0 + L_SLOT + (uint32_t)((5 * l + 2) % NSLOT) * DEC_SLOT;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = wave + DW * u;
                if (i >= nr) break;
                const float y = row_dot(slot + i * a.Q, slot + nr * a.Q + i * (a.Q / 16), a.Q, xc, lane);
                if (lane == 63) ll_st(a.ll + o.h1 + r0 + i, tag(ph + 3), res[u] + y);
            }
        }
        // ---------------------------------------------------------------- phase 4: norm + gate / up rows + SwiGLU
        ok = ll_poll4(a.ll + o.h1, a.H, tag(ph + 3), v, a.spin_limit);
        if (!sync_ok(ok, &abort_flag)) break;
#pragma unroll
        for (int j = 0; j < NG; j++)
            if (tid + DT * j < a.H / 4) *(float4 *)(hb + 4 * (tid + DT * j)) = v[j];
        rms_norm_input(v, a.H, L.ffn_norm, a.eps, lds);
        quantize_input(v, a.H, a.rounding, lds);
        __syncthreads();
        load_xchunks(xc, a.H, lds, lane);
        issue_upto(5 * l + 5);
        {
            const int r0 = wg * a.r_f;
            const int nr = max(0, min(a.r_f, a.F - r0));
            const uint32_t slot = lds0 + L_SLOT + (uint32_t)((5 * l + 3) % NSLOT) * DEC_SLOT;
            const int rows = 2 * nr;
            for (int i = wave; i < nr; i += DW) {
                const float gt = row_dot(slot + i * a.H, slot + rows * a.H + i * (a.H / 16), a.H, xc, lane);
                const float up = row_dot(slot + (nr + i) * a.H, slot + rows * a.H + (nr + i) * (a.H / 16), a.H, xc,
                                         lane);
                if (lane == 63) ll_st(a.ll + o.g + r0 + i, tag(ph + 4), gt / (1.0f + expf(-gt)) * up);
            }
        }
        // ---------------------------------------------------------------- phase 5: down rows + residual
        ok = ll_poll4(a.ll + o.g, a.F, tag(ph + 4), v, a.spin_limit);
        if (!sync_ok(ok, &abort_flag)) break;
        quantize_input(v, a.F, a.rounding, lds);
        __syncthreads();
        load_xchunks(xc, a.F, lds, lane);
        {
            const int r0 = wg * a.r_d;
            const int nr = max(0, min(a.r_d, a.H - r0));
            float res[4];
#pragma unroll
            for (int i = 0; i < 4; i++) res[i] = (wave + DW * i < nr) ? hb[r0 + wave + DW * i] : 0.0f;
            issue_upto(5 * l + 6);
            const uint32_t slot = lds0 + L_SLOT + (uint32_t)((5 * l + 4) % NSLOT) * DEC_SLOT;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = wave + DW * u;
                if (i >= nr) break;
                const float y = row_dot(slot + i * a.F, slot + nr * a.F + i * (a.F / 16), a.F, xc, lane);
                if (lane == 63) ll_st(a.ll + o.h2 + r0 + i, tag(ph + 5), res[u] + y);
            }
        }
    }

    // -------------------------------------------------------------------- head: norm + output rows + local argmax
    const int ph = 6 * a.n_layer;
    if (abort_flag == 0) {
        ok = ll_poll4(a.ll + o.h2, a.H, tag(ph - 1), v, a.spin_limit);
        if (sync_ok(ok, &abort_flag)) {
            rms_norm_input(v, a.H, a.out_norm, a.eps, lds);
            quantize_input(v, a.H, a.rounding, lds);
            __syncthreads();
            load_xchunks(xc, a.H, lds, lane);
            const int r0 = wg * a.r_v;
            const int nr = max(0, min(a.r_v, a.V - r0));
            float best = 0.0f;
            int bi = -1;  // the first of the largest non-NaN values of this wave's rows (rows ascend)
            float *first = (float *)(lds + L_SM);  // logits[0], kept for the pick (workgroup 0 computes it)
            if (a.H == 1024) head_rows<1, NC>(a, xc, r0, nr, wave, lane, best, bi, first);
            else if (NC >= 2 && a.H == 2048) head_rows<(NC >= 2 ? 2 : 1), NC>(a, xc, r0, nr, wave, lane, best, bi, first);
            else if (NC >= 3 && a.H == 3072) head_rows<(NC >= 3 ? 3 : 1), NC>(a, xc, r0, nr, wave, lane, best, bi, first);
            else if (NC >= 4) head_rows<(NC >= 4 ? 4 : 1), NC>(a, xc, r0, nr, wave, lane, best, bi, first);
            // across the waves: the largest value, the smaller index on ties (rows of wave w are r0 + w + 8 k)
            float *rv = (float *)(lds + L_RED);
            int *ri = (int *)(lds + L_RED + DW * 4);
            if (lane == 63) {
                rv[wave] = best;
                ri[wave] = bi;
            }
            __syncthreads();
            if (tid == 0) {
                float bv = 0.0f;
                int bx = -1;
                for (int w = 0; w < DW; w++) {
                    if (ri[w] < 0) continue;
                    if (bx < 0 || rv[w] > bv || (rv[w] == bv && ri[w] < bx)) {
                        bv = rv[w];
                        bx = ri[w];
                    }
                }
                ll_st(a.ll + o.arg + 2 * wg, tag(ph), bv);
                ll_st(a.ll + o.arg + 2 * wg + 1, tag(ph), __int_as_float(bx));
            }
            // ------------------------------------------------------------ pick (workgroup 0)
            if (wg == 0) {
                float bv = 0.0f, ix = 0.0f;
                bool good = true;
                if (tid < G) {
                    const int off[2] = {2 * tid, 2 * tid + 1};
                    float pr[2];
                    good = ll_pollv<2>(a.ll + o.arg, off, 2, tag(ph), pr, a.spin_limit);
                    bv = pr[0];
                    ix = pr[1];
                }
                float *pv = (float *)(lds + L_ACC);
                int *pi = (int *)(lds + L_ACC + DT * 4);
                if (tid < G) {
                    pv[tid] = bv;
                    pi[tid] = __float_as_int(ix);
                }
                if (sync_ok(good, &abort_flag) && tid == 0) {
                    // ggml's rule over the whole row: a NaN at index 0 keeps index 0; elsewhere NaNs never win
                    int bx = -1;
                    float bvv = 0.0f;
                    const float f0 = *(const float *)(lds + L_SM);
                    if (f0 != f0) {
                        bx = 0;
                    } else {
                        for (int w = 0; w < G; w++) {
                            if (pi[w] < 0) continue;
                            if (bx < 0 || pv[w] > bvv) {  // workgroups hold ascending rows: ties keep the earlier
                                bvv = pv[w];
                                bx = pi[w];
                            }
                        }
                    }
                    *a.pick = bx < 0 ? 0 : bx;
                    *a.epoch = E + 1;
                }
            }
        }
    }
    vm_wait_all();
    if (abort_flag && tid == 0) atomicOr(a.err, 8);
#undef tag
#undef issue_upto
}

template <int NG, int NC>
static hipError_t launch_inst(const DecArgs &a, int grid, bool cooperative, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_decode_step<NG, NC>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)L_END);
        if (e != hipSuccess) return e;
        attr = true;
    }
    if (cooperative) {
        DecArgs arg = a;
        void *params[] = {&arg};
        return hipLaunchCooperativeKernel((const void *)k_decode_step<NG, NC>, dim3((unsigned)grid), dim3(DT), params,
                                          (unsigned)L_END, s);
    }
    hipLaunchKernelGGL((k_decode_step<NG, NC>), dim3((unsigned)grid), dim3(DT), L_END, s, a);
    return hipGetLastError();
}

hipError_t launch_decode_step(const DecArgs &a, int grid, bool cooperative, hipStream_t s) {
    const int kmax = a.H > a.Q ? (a.H > a.F ? a.H : a.F) : (a.Q > a.F ? a.Q : a.F);
    if (kmax > DEC_KMAX) return hipErrorInvalidValue;
    return launch_inst<DEC_KMAX / 4 / DT, DEC_KMAX / 1024>(a, grid, cooperative, s);
}

}  // namespace mx
