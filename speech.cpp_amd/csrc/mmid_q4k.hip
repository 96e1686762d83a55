// MUL_MAT_ID on Q4_K experts as a grouped product: dst[:, s, t] = as[ids[s, t]] . quant(b[:, s % b_ne1, t]).
//
// The prep launch cuts each expert's (token, slot) pairs into chunks of up to 32, the rows of two 16-row MFMA tiles
// (or, when the pairs average at most four per expert, of up to 16: one tile, in a kernel form without the second).
// A workgroup takes one chunk and a few blocks of 128 of the expert's weight rows (dst columns); wave w owns columns
// 16 w .. 16 w + 15 of each block and streams their super-blocks block after block, so each weight byte leaves HBM
// once per 32 pairs of its expert, and each decoded weight fragment feeds both 16-row tiles (a chunk of at most 16
// pairs runs the one-tile form).
//
// The weights stream through a ring of two stages per wave in LDS, filled by global_load_lds copies issued one step
// ahead (no registers held for them). Deeper rings were slower at every depth tried (us per 64-expert top-4 layer,
// gate + up + down, at 16 / 256 tokens: two-tile chunks with 2 stages 81.6 / 118.9, 3 stages 82.5 / 119.0, 4 stages
// 85.4 / 119.4; one-tile chunks at 16 tokens with 2 stages 78.9, 3 stages 80.3, 6 stages 89.3, and two workgroups
// per CU 85.1): the weight stream does not wait on latency. The chunk's activation operands (K <= 2048) are loaded into LDS once per
// workgroup and shared by its eight waves and all its column blocks.
//
// Arithmetic per 256-element super-block, as ggml-cpu's vec_dot_q4_K_q8_K (and the Q4_K prefill GEMM):
//   y += dx * (d * sum_j sc_j * S_j  -  dmin * sum_j mn_j * bsum_j)
// In MFMA step q (q = 0..3) lane group g (lanes 16 g .. 16 g + 15) carries elements 64 q + 16 g .. + 15 of its column
// and of its activation row: code bytes 32 q + 16 (g & 1) .. + 15, low nibbles for g < 2 (sub-block 2 q), high
// nibbles for g >= 2 (sub-block 2 q + 1). So a step's activation loads are 64 contiguous bytes of each row, and A and B
// agree on which element every (lane group, byte) slot carries. The codes are scaled by the 3-bit halves of their
// own 6-bit scale (sc = 8 hi + lo; hi * q and lo * q are at most 105), so two MFMA chains give sum_j hi_j S_j and
// sum_j lo_j S_j exactly. The min term is one v_mfma_f32_16x16x16_f16 on [64 h_j | l_j] (bsum_j = 64 h_j + l_j)
// against the mins, exact.
#include "mx_common.h"
#include "mx_device.h"

namespace mx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// Two u16 lanes of two codes each times (s, s): each byte's product stays below 256, so bytes do not interact.
__device__ __forceinline__ int mq_pk_mul(int codes, uint32_t s2) {
    int r;
    asm("v_pk_mul_lo_u16 %0, %1, %2" : "=v"(r) : "v"(codes), "v"(s2));
    return r;
}

constexpr int MQ_W = 8;              // waves per workgroup
constexpr int MQ_COLS = 16 * MQ_W;   // dst columns per column block: 16 per wave
static_assert(MMID_CHUNK == 32 && MMID_CHUNK_SMALL == 16, "a chunk is one or two 16-row MFMA tiles");

constexpr int MQ_STAGE = 2304;  // one stage: 16 columns x (128 code bytes + 12 scale bytes + d | dmin)


// Keeps the memory ops before it ahead of the ones after it (the wait counts depend on their issue order).
__device__ __forceinline__ void mq_order() { asm volatile("" ::: "memory"); }

// LDS of a workgroup whose chunks have up to NGMAX 16-row tiles and whose waves stream through rings of S stages: per
// wave a ring of S weight stages, then the chunk's activation operands for up to MQ_KSEG super-blocks (one segment
// of K), laid out as the lanes read them (tile g = rows 16 g .. 16 g + 15):
//   codes   [sb][g][q][grp][fr] x 16 bytes: row 16 g + fr, elements 256 sb + 64 q + 16 grp .. + 15
//   sums    [sb][g][fr] x 32 bytes: that row's split sub-block sums [64 h_j | l_j] (fp16)
//   scales  [sb][g][fr] floats: that row's Q8_K scale
constexpr int MQ_KSEG = 8;
template <int NGMAX, int S>
struct MqMap {
    static constexpr int RING = MQ_W * S * MQ_STAGE;
    static constexpr int AQ_SB = 4096 * NGMAX, A16_SB = 512 * NGMAX, ADX_SB = 64 * NGMAX;  // per super-block
    static constexpr int AQ = RING, A16 = AQ + MQ_KSEG * AQ_SB, ADX = A16 + MQ_KSEG * A16_SB;
    static constexpr int SIZE = ADX + MQ_KSEG * ADX_SB;
    static_assert(SIZE <= 160 * 1024, "one workgroup per CU");
};

// One wave's view of its work: the weight stream (ncb column blocks x nsb super-blocks).
struct MqLane {
    const uint8_t *qe, *se;  // the expert's code plane (+ 32 grp) and this lane's scale word source
    int sstride;             // bytes between blocks of the scale source (12 or 4)
    int col0, scol0;         // column of this lane's codes / of its scale word in column block 0
    int nmax;                // last column
    int nsb, nsteps, lane, fr, grp;
    uint8_t *ring;           // this wave's ring (uniform)
    uint32_t ring_lds, a_lds;  // LDS byte addresses of the ring and of the activation operands
};

// Segment `seg` of the chunk's activation operands, as thread t = 256 g + u (g < NGMAX) brings it to LDS: pieces of
// row 16 g + (t & 15) (arow: its activation row). Loads past the segment repeat its last super-block; only the stores
// are conditional.
struct MqSeg {
    v4i codes[MQ_KSEG];  // u = (q, grp, fr): elements 64 q + 16 grp .. + 15 of each super-block
    v4i sums;            // u = (sb, half, fr): 8 of the 16 split sums of super-block sb
    float scale;         // u = (sb, fr): the Q8_K scale of super-block sb
};
__device__ __forceinline__ MqSeg mq_seg_load(const MulMatIdArgs &a, int arow, int seg, int nsb) {
    const int u = threadIdx.x & 255;
    const int sb0 = MQ_KSEG * seg, last = min(MQ_KSEG, nsb - sb0) - 1;
    MqSeg r;
    const int8_t *xs = a.xq + arow * (int)a.K + sb0 * 256 + 64 * (u >> 6) + 16 * ((u >> 4) & 3);
#pragma unroll
    for (int i = 0; i < MQ_KSEG; i++) r.codes[i] = *(const v4i *)(xs + min(i, last) * 256);
    r.sums = *(const v4i *)(a.x16 + (arow * nsb + sb0 + min(u >> 5, last)) * 16 + 8 * ((u >> 4) & 1));
    r.scale = a.xd[arow * nsb + sb0 + min((u >> 4) & 7, last)];
    return r;
}
// The stores go through inline assembly: the compiler would otherwise order them after every copy in flight into
// the (disjoint) ring, since it cannot tell the two LDS regions apart.
template <typename Map>
__device__ __forceinline__ void mq_seg_store(const MqSeg &r, uint8_t *smem, int seg, int nsb) {
    const int g = threadIdx.x >> 8, u = threadIdx.x & 255, fr = u & 15;
    const int n = min(MQ_KSEG, nsb - MQ_KSEG * seg);
    const uint32_t base = (uint32_t)(uintptr_t)(lds_void *)smem;
#pragma unroll
    for (int i = 0; i < MQ_KSEG; i++)
        if (i < n)
            asm volatile("ds_write_b128 %0, %1" ::"v"(base + Map::AQ + i * Map::AQ_SB + g * 4096 + 16 * u),
                         "v"(r.codes[i])
                         : "memory");
    if ((u >> 5) < n)
        asm volatile("ds_write_b128 %0, %1" ::"v"(base + Map::A16 + (u >> 5) * Map::A16_SB + g * 512 + fr * 32 +
                                                  ((u >> 4) & 1) * 16),
                     "v"(r.sums) : "memory");
    if ((u >> 4) < n)
        asm volatile("ds_write_b32 %0, %1" ::"v"(base + Map::ADX + (u >> 4) * Map::ADX_SB + g * 64 + fr * 4),
                     "v"(r.scale)
                     : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Where the next copy comes from: column block cb (its per-lane sources at qcb / scb) and super-block sb.
struct MqCursor {
    const uint8_t *qcb, *scb;
    int cb, sb;
};
__device__ __forceinline__ void mq_seek(const MqLane &c, MqCursor &k, int cb) {
    const int64_t qcol = min(c.col0 + MQ_COLS * cb, c.nmax), scol = min(c.scol0 + MQ_COLS * cb, c.nmax);
    k.qcb = c.qe + qcol * c.nsb * 128;
    k.scb = c.se + scol * c.nsb * c.sstride;
    k.cb = cb;
}

// Copies the cursor's super-block of the wave's 16 columns into ring stage SLOT (3 vector memory ops) and advances
// the cursor; past the last step it stays on the last one, so the copies after the end repeat it. (Nontemporal copies
// measured 8-11 % slower here: T = 16 86 -> 96 us, T = 256 120 -> 128 us.)
template <int SLOT>
__device__ __forceinline__ void mq_copy(const MqLane &c, MqCursor &k, int ncb) {
    uint8_t *st = c.ring + SLOT * MQ_STAGE;
    __builtin_amdgcn_global_load_lds((const void *)(k.qcb + k.sb * 128), (lds_void *)st, 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void *)(k.qcb + k.sb * 128 + 16), (lds_void *)(st + 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void *)(k.scb + k.sb * c.sstride), (lds_void *)(st + 2048), 4, 0, 0);
    if (k.sb + 1 < c.nsb) {
        k.sb++;
    } else if (k.cb + 1 < ncb) {
        k.sb = 0;
        mq_seek(c, k, k.cb + 1);
    }
}

// Step of the wave's stream: super-block sb (sbl within the loaded segment) of its column block, weights in ring
// stage SLOT of S, for NG 16-row tiles of the chunk. Each step issues the copies S - 1 steps ahead (3 ops) and then
// waits for its own, which were issued S - 1 copies (3 (S - 1) ops) earlier. Operands are read from LDS in one block
// with the compiler kept out of it: it cannot see that the copies waited for wrote there.
template <typename Map, int S, int SLOT, int NG>
__device__ __forceinline__ void mq_step(const MqLane &c, MqCursor &k, int ncb, int sbl, float (&acc)[NG][4]) {
    mq_copy<(SLOT + S - 1) % S>(c, k, ncb);
    wait_vm<3 * (S - 1)>();
    const uint32_t st = c.ring_lds + SLOT * MQ_STAGE;
    const uint32_t aq = c.a_lds + Map::AQ - Map::RING + sbl * Map::AQ_SB + 16 * c.lane;
    const uint32_t a16 = c.a_lds + Map::A16 - Map::RING + sbl * Map::A16_SB + 32 * c.fr + 8 * c.grp;
    const uint32_t adx = c.a_lds + Map::ADX - Map::RING + sbl * Map::ADX_SB + 16 * c.grp;
    v4i w[4];       // code bytes 32 q + 16 (grp & 1) .. + 15 of column fr
    uint4 sv;       // its scale words 0..2, d | dmin
    v4i xa[NG][4];  // activation bytes 64 q + 16 grp .. + 15 of row 16 g + fr
    v4h s16[NG];    // that row's split sums 4 grp .. 4 grp + 3
    v4f dxv[NG];    // Q8_K scales of rows 16 g + 4 grp .. + 3
    if constexpr (NG == 1) {
        asm volatile(
            "ds_read_b128 %0, %11\n"
            "ds_read_b128 %1, %11 offset:256\n"
            "ds_read_b128 %2, %11 offset:512\n"
            "ds_read_b128 %3, %11 offset:768\n"
            "ds_read_b128 %4, %12 offset:2048\n"
            "ds_read_b128 %5, %13\n"
            "ds_read_b128 %6, %13 offset:1024\n"
            "ds_read_b128 %7, %13 offset:2048\n"
            "ds_read_b128 %8, %13 offset:3072\n"
            "ds_read_b64 %9, %14\n"
            "ds_read_b128 %10, %15\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(sv), "=&v"(xa[0][0]), "=&v"(xa[0][1]),
              "=&v"(xa[0][2]), "=&v"(xa[0][3]), "=&v"(s16[0]), "=&v"(dxv[0])  // early clobber: no output may share
            : "v"(st + 1024 * (c.grp & 1) + 16 * c.fr), "v"(st + 16 * c.fr), "v"(aq), "v"(a16), "v"(adx)  // an address
            : "memory");
    } else {
        asm volatile(
            "ds_read_b128 %0, %17\n"
            "ds_read_b128 %1, %17 offset:256\n"
            "ds_read_b128 %2, %17 offset:512\n"
            "ds_read_b128 %3, %17 offset:768\n"
            "ds_read_b128 %4, %18 offset:2048\n"
            "ds_read_b128 %5, %19\n"
            "ds_read_b128 %6, %19 offset:1024\n"
            "ds_read_b128 %7, %19 offset:2048\n"
            "ds_read_b128 %8, %19 offset:3072\n"
            "ds_read_b128 %9, %19 offset:4096\n"
            "ds_read_b128 %10, %19 offset:5120\n"
            "ds_read_b128 %11, %19 offset:6144\n"
            "ds_read_b128 %12, %19 offset:7168\n"
            "ds_read_b64 %13, %20\n"
            "ds_read_b64 %14, %20 offset:512\n"
            "ds_read_b128 %15, %21\n"
            "ds_read_b128 %16, %21 offset:64\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(sv), "=&v"(xa[0][0]), "=&v"(xa[0][1]),
              "=&v"(xa[0][2]), "=&v"(xa[0][3]), "=&v"(xa[NG - 1][0]), "=&v"(xa[NG - 1][1]), "=&v"(xa[NG - 1][2]),
              "=&v"(xa[NG - 1][3]), "=&v"(s16[0]), "=&v"(s16[NG - 1]), "=&v"(dxv[0]), "=&v"(dxv[NG - 1])
            : "v"(st + 1024 * (c.grp & 1) + 16 * c.fr), "v"(st + 16 * c.fr), "v"(aq), "v"(a16), "v"(adx)
            : "memory");
    }

    const int grp = c.grp, hi = grp >> 1;
    const v4i mask = {0x0F0F0F0F, 0x0F0F0F0F, 0x0F0F0F0F, 0x0F0F0F0F};
    // The 6-bit scales and mins of four sub-blocks at a time from the packed words (get_scale_min_k4 for j < 4 and
    // for j >= 4): sub-blocks 0..3 in the bytes of the *_lo4 words, 4..7 in those of the *_hi4 words.
    const uint32_t sc_lo4 = sv.x & 0x3F3F3F3Fu, sc_hi4 = (sv.z & 0x0F0F0F0Fu) | ((sv.x >> 2) & 0x30303030u);
    const uint32_t mn4 = (grp & 1) ? (((sv.z >> 4) & 0x0F0F0F0Fu) | ((sv.y >> 2) & 0x30303030u)) : (sv.y & 0x3F3F3F3Fu);
    // mins of sub-blocks (4 grp + i) mod 8, matching the [64 h | l] halves this lane group carries
    v4h b16;
#pragma unroll
    for (int i = 0; i < 4; i++) b16[i] = (_Float16)(float)__builtin_amdgcn_ubfe(mn4, 8 * i, 8);
    const float d = h2f((uint16_t)(sv.w & 0xFFFF)), dmin = h2f((uint16_t)(sv.w >> 16));
    v4i ih[NG], il[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) ih[g] = il[g] = (v4i){0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < 4; q++) {  // codes scaled by the hi / lo halves of their sub-block's scale
        const uint32_t sc = __builtin_amdgcn_ubfe(q < 2 ? sc_lo4 : sc_hi4, 8 * (hi + 2 * (q & 1)), 8);  // j = 2 q + hi
        const uint32_t h = (sc >> 3) * 0x10001u, l = (sc & 7) * 0x10001u;
        const v4i cq = (w[q] >> (4 * hi)) & mask;
        const v4i bh = {mq_pk_mul(cq.x, h), mq_pk_mul(cq.y, h), mq_pk_mul(cq.z, h), mq_pk_mul(cq.w, h)};
        const v4i bl = {mq_pk_mul(cq.x, l), mq_pk_mul(cq.y, l), mq_pk_mul(cq.z, l), mq_pk_mul(cq.w, l)};
#pragma unroll
        for (int g = 0; g < NG; g++) {
            ih[g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[g][q], bh, ih[g], 0, 0, 0);
            il[g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[g][q], bl, il[g], 0, 0, 0);
        }
    }
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const v4f mt = __builtin_amdgcn_mfma_f32_16x16x16f16(s16[g], b16, (v4f){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {  // output row 16 g + 4 grp + i
            const int v = (ih[g][i] << 3) + il[g][i];
            acc[g][i] = fmaf(dxv[g][i], fmaf(-dmin, mt[i], d * (float)v), acc[g][i]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // steps do not interleave: one step's operands live at a time
}

// Steps SLOT .. S - 1 of one turn of the ring (steps it + SLOT, ...), each while steps remain.
template <typename Map, int S, int SLOT, int NG, typename F>
__device__ __forceinline__ void mq_turn(const MqLane &c, MqCursor &k, int ncb, int it, int &sb, float (&acc)[NG][4],
                                        F &finish) {
    if constexpr (SLOT < S) {
        if (SLOT > 0 && it + SLOT >= c.nsteps) return;
        mq_step<Map, S, SLOT, NG>(c, k, ncb, sb, acc);
        finish();
        mq_turn<Map, S, SLOT + 1, NG>(c, k, ncb, it, sb, acc, finish);
    }
}
// Copies SLOT .. S - 2 of the ring's prologue.
template <int S, int SLOT>
__device__ __forceinline__ void mq_prologue(const MqLane &c, MqCursor &k, int ncb) {
    if constexpr (SLOT < S - 1) {
        mq_copy<SLOT>(c, k, ncb);
        mq_prologue<S, SLOT + 1>(c, k, ncb);
    }
}

// One workgroup's share with NG 16-row tiles (NG = 1 when the chunk has at most 16 pairs).
template <typename Map, int S, int NG>
__device__ __forceinline__ void mq_run(const MulMatIdArgs &a, MqLane &c, uint8_t *smem, int p0, int cnt, int ncb,
                                       float *dst) {
    const unsigned n_ids = (unsigned)a.n_ids;
    // lane fr carries row 16 g + fr of tile g (rows past the chunk repeat its last pair; their sums are dropped)
    int pair[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) pair[g] = a.pairs[p0 + min(16 * g + c.fr, cnt - 1)];
    // the activation row thread t brings to LDS: row 16 (t >> 8) + (t & 15) of the chunk (threads of a tile the
    // kernel form lacks bring nothing)
    const bool seg_thread = (int)(threadIdx.x >> 8) < Map::AQ_SB / 4096;
    int arow;
    {
        const int pr = a.pairs[p0 + min(16 * (int)(threadIdx.x >> 8) + c.fr, cnt - 1)];
        const unsigned pt = (unsigned)pr / n_ids, ps = (unsigned)pr - pt * n_ids;
        arow = (int)(pt * (unsigned)a.b_ne1 + (a.b_ne1 == 1 ? 0u : ps));
    }

    // activation operands of the first segment (their loads go out ahead of the copies), then the ring's prologue
    MqCursor k;
    k.sb = 0;
    mq_seek(c, k, 0);
    {
        MqSeg seg0;
        if (seg_thread) seg0 = mq_seg_load(a, arow, 0, c.nsb);
        mq_order();
        mq_prologue<S, 0>(c, k, ncb);
        if (seg_thread) mq_seg_store<Map>(seg0, smem, 0, c.nsb);  // its wait leaves the copies in flight
    }
    __syncthreads();

    float acc[NG][4];
#pragma unroll
    for (int g = 0; g < NG; g++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[g][i] = 0.f;
    int sb = 0, cb = 0;
    // after each step: a column block is finished when its last super-block is
    auto finish = [&]() {
        if (++sb < c.nsb) return;
        const int col = c.col0 + MQ_COLS * cb;
#pragma unroll
        for (int g = 0; g < NG; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = 4 * c.grp + i;
                const unsigned pi = (unsigned)__shfl(pair[g], row, 64);  // lane `row` holds that row's pair
                if (16 * g + row < cnt && col <= c.nmax) {
                    const unsigned t = pi / n_ids, s = pi - t * n_ids;
                    float *y = (float *)((uint8_t *)dst + (int64_t)s * a.dst_nb1 + (int64_t)t * a.dst_nb2);
                    y[col] = acc[g][i];
                }
                acc[g][i] = 0.f;
            }
        sb = 0;
        cb++;
    };
#pragma unroll 1
    for (int it = 0; it < c.nsteps; it += S) mq_turn<Map, S, 0, NG>(c, k, ncb, it, sb, acc, finish);
    wait_vm<0>();  // no copy may still be landing in LDS when the workgroup ends
}

// Grid: one workgroup per CU. The work is nprob x ntiles x nblk units (a product, a chunk and one block of MQ_COLS
// columns); workgroup b takes the contiguous units [b U / G, (b + 1) U / G), chunk by chunk, so every CU gets the
// same number of column blocks to within one. Within a unit wave w owns columns 16 w .. 16 w + 15 of the block and streams super-blocks
// 0 .. nsb - 1 (nsb <= MQ_KSEG); a block's sums are written when its last super-block is done. NGMAX = 1: the host
// cut the pairs into chunks of at most 16.
template <int NGMAX, int S>
__global__ __launch_bounds__(64 * MQ_W) void k_mmid_q4k(MulMatIdArgs a) {
    using Map = MqMap<NGMAX, S>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // The argument block's fields on the way to the first weight copy, requested together into scalar registers (left
    // to the compiler, they came in over several round trips in a row, between the tile count's and the tiles' loads).
    asm volatile("" ::"s"(a.N), "s"(a.K), "s"(a.nprob), "s"(a.ntiles), "s"(a.tiles), "s"(a.pairs), "s"(a.n_ids),
                 "s"(a.b_ne1), "s"(a.xq), "s"(a.x16), "s"(a.xd));
    asm volatile("" ::"s"(a.wg[0].p0), "s"(a.wg[0].p1), "s"(a.wg[0].p2), "s"(a.dstg[0]), "s"(a.dst_nb1),
                 "s"(a.dst_nb2));
    const int N = (int)a.N;
    const int nblk = (N + MQ_COLS - 1) / MQ_COLS;
    const int64_t per = (int64_t)a.ntiles[0] * nblk;  // units of one product
    const int64_t units = per * a.nprob;
    const int u1 = (int)((blockIdx.x + 1) * units / gridDim.x);
    for (int u = (int)(blockIdx.x * units / gridDim.x); u < u1;) {
        const int pr = (int)(u / per), ur = u - pr * (int)per;
        const int chunk = ur / nblk, cb0 = ur - chunk * nblk, ncb = min(nblk - cb0, u1 - u);
        // uniform selection keeps the kernel-argument arrays out of private memory
        const WPlanes w = pr == 0 ? a.wg[0] : (pr == 1 ? a.wg[1] : (pr == 2 ? a.wg[2] : a.wg[3]));
        float *dst = pr == 0 ? a.dstg[0] : (pr == 1 ? a.dstg[1] : (pr == 2 ? a.dstg[2] : a.dstg[3]));
        const int p0 = a.tiles[3 * chunk], cnt = a.tiles[3 * chunk + 1], e = a.tiles[3 * chunk + 2];
        MqLane c;
        c.lane = threadIdx.x & 63;
        c.fr = c.lane & 15;
        c.grp = c.lane >> 4;
        c.nsb = (int)(a.K / 256);
        c.nsteps = ncb * c.nsb;
        // Copy sources: lane l brings code bytes 32 grp + 16 h (h = 0, 1) of column fr, and scale word l & 3 of
        // column l >> 2 (words 0..2: the 12 scale bytes, word 3: d | dmin). They land at stage + 1024 h + 16 l and
        // stage + 2048 + 4 l: bytes 32 q + 16 h of column fr sit at stage + 1024 h + 256 q + 16 fr, its scale words at
        // stage + 2048 + 16 fr.
        const int64_t eblk = (int64_t)e * N * c.nsb;
        c.nmax = N - 1;
        c.col0 = cb0 * MQ_COLS + wave * 16 + c.fr;
        c.scol0 = cb0 * MQ_COLS + wave * 16 + (c.lane >> 2);
        c.qe = w.p0 + eblk * 128 + 32 * c.grp;
        const int sw = c.lane & 3;
        c.sstride = sw < 3 ? 12 : 4;
        c.se = sw < 3 ? w.p1 + eblk * 12 + 4 * sw : w.p2 + eblk * 4;
        c.ring = smem + wave * S * MQ_STAGE;
        c.ring_lds = (uint32_t)(uintptr_t)(lds_void *)c.ring;
        c.a_lds = (uint32_t)(uintptr_t)(lds_void *)(smem + Map::RING);
        if (NGMAX > 1 && cnt > 16) mq_run<Map, S, NGMAX>(a, c, smem, p0, cnt, ncb, dst);
        else mq_run<Map, S, 1>(a, c, smem, p0, cnt, ncb, dst);
        u += ncb;
        __syncthreads();  // every wave is done with this chunk's activation operands before the next one's land
    }
}

// Workgroups: one per CU of the current device.
static int mq_grid() {
    static const int n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            return 256;
        return cus;
    }();
    return n;
}

bool mmid_q4k_supported(const MulMatIdArgs &a) {
    return a.type == MX_TYPE_Q4_K && a.K % 256 == 0 && a.K / 256 <= MQ_KSEG &&
           a.T * a.b_ne1 * a.K < ((int64_t)1 << 31) && a.N < ((int64_t)1 << 31) - MQ_COLS;
}

template <int NGMAX, int S>
static hipError_t launch_form(const MulMatIdArgs &a, hipStream_t s) {
    constexpr size_t lds = MqMap<NGMAX, S>::SIZE;
    static bool attr = false;
    if (!attr) {
        const hipError_t err = hipFuncSetAttribute((const void *)k_mmid_q4k<NGMAX, S>,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) return err;
        attr = true;
    }
    hipLaunchKernelGGL((k_mmid_q4k<NGMAX, S>), dim3((unsigned)mq_grid()), dim3(64 * MQ_W), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_mmid_q4k(const MulMatIdArgs &a, hipStream_t s) {
    if (!mmid_q4k_supported(a)) return hipErrorInvalidValue;
    if (a.chunk == MMID_CHUNK_SMALL) return launch_form<1, 2>(a, s);
    if (a.chunk == MMID_CHUNK) return launch_form<2, 2>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace mx
