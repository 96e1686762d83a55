// Prefill products on K-quant weights (Q4_K, Q6_K) with Q8_K activations, on int8 MFMA.
//
// ggml-cpu's vec_dot_q4_K_q8_K / _q6_K_q8_K per 256-element super-block of weight row n and activation row m:
//   Q4_K: y += dx*d * sum_j sc_j * S_j  -  dx*dmin * sum_j mn_j * bsum32_j     (8 sub-blocks of 32)
//   Q6_K: y += dx*d * sum_j sc_j * S_j                                          (16 sub-blocks of 16; codes q - 32)
// where S_j is the exact int32 dot of sub-block j's codes with the activation quants.
//
// One LDS stage is one super-block (256 of K). Each wave owns a 32 x 32 tile of Y; per sub-block one
// v_mfma_i32_32x32x32_i8 gives S_j for the whole tile (Q6_K: two, each with the other 16 codes of the 32 zeroed, since
// its scales cover 16), folded into an int32 accumulator with the sub-block's integer scale (exact: |I| < 2^31). The
// Q4_K min term is a K = 8 product of integers, exact in fp32, on v_mfma_f32_32x32x2_f32. Float scales are applied once
// per super-block, in ggml's order: (fp16(d) * dx) * I.
#include "mx_common.h"
#include "mx_device.h"

namespace mx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int KQS = 256;          // K per stage: one super-block
constexpr int KQROW = KQS + 16;   // padded LDS row (bytes)

// Activation rows -> Q8_K: int8 quants [M][K], fp32 d [M][K/256], fp32 sums of 32 quants [M][K/32].
__global__ __launch_bounds__(256) void k_gemm_quant_q8k(const float *x, int64_t x_stride, int64_t K, int8_t *xq,
                                                        float *xd, float *xs32) {
    const int64_t m = blockIdx.x;  // rows on x: grid.y holds at most 65,535
    const int lane = threadIdx.x & 63;
    const int64_t sb = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6);
    if (sb * 256 >= K) return;  // whole wave
    const float4 v = *(const float4 *)(x + m * x_stride + sb * 256 + 4 * lane);
    float d;
    int bs16;
    const int q = quant256_wave(v, lane, &d, &bs16);
    const int bs32 = bs16 + dpp_i<dpp::HALF_MIRROR>(0, bs16);  // lanes 8j..8j+7 hold sub-block j
    *(int *)(xq + m * K + sb * 256 + 4 * lane) = q;
    if (lane == 0) xd[m * (K / 256) + sb] = d;
    if ((lane & 7) == 0) xs32[m * (K / 32) + sb * 8 + (lane >> 3)] = (float)bs32;
}

struct KqArgs {
    WPlanes w;
    int64_t M, N, K;
    const int8_t *xq;
    const float *xd;
    const float *xs32;
    float *y;
    int64_t ldy;
};

// 16 packed Q4_K code bytes (bytes 16t..16t+15 of a super-block's 128) -> 32 int8 codes at their element positions:
// low nibbles are elements 64(t/2) + 16(t%2) + i, high nibbles the same + 32.
__device__ __forceinline__ void unpack_q4k(v4i p, v4i &lo, v4i &hi) {
    lo = v4i{p.x & 0x0F0F0F0F, p.y & 0x0F0F0F0F, p.z & 0x0F0F0F0F, p.w & 0x0F0F0F0F};
    hi = v4i{(p.x >> 4) & 0x0F0F0F0F, (p.y >> 4) & 0x0F0F0F0F, (p.z >> 4) & 0x0F0F0F0F, (p.w >> 4) & 0x0F0F0F0F};
}

template <int TYPE>
__global__ __launch_bounds__(256) void k_gemm_kq(KqArgs a) {
    constexpr int BM = 64, BN = 64;
    __shared__ __align__(16) int8_t xs[BM * KQROW];
    __shared__ __align__(16) int8_t ws[BN * KQROW];
    __shared__ float dxs[BM];          // activation d of the super-block
    __shared__ float x32s[8][BM];      // activation sums of 32 (Q4_K min term)
    __shared__ float dws[BN], dmws[BN];
    __shared__ int scs[TYPE == MX_TYPE_Q4_K ? 8 : 16][BN];  // integer sub-block scales
    __shared__ float mns[8][BN];       // Q4_K mins

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int64_t K = a.K, nsb = K / 256;
    const int fr = lane & 31, fk = (lane >> 5) * 16;

    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;

    for (int64_t sb = 0; sb < nsb; sb++) {
        __syncthreads();
        // ---- stage the super-block: activations (4 threads per 256-byte row, 4 x 16 B each)
        {
            const int r = tid >> 2, c = (tid & 3) * 64;
            int64_t m = m0 + r;
            m = m < a.M ? m : a.M - 1;
            const int8_t *src = a.xq + m * K + sb * 256 + c;
#pragma unroll
            for (int p = 0; p < 4; p++) *(v4i *)(xs + r * KQROW + c + 16 * p) = *(const v4i *)(src + 16 * p);
        }
        if (tid < BM) {
            int64_t m = m0 + tid;
            m = m < a.M ? m : a.M - 1;
            dxs[tid] = a.xd[m * nsb + sb];
            if (TYPE == MX_TYPE_Q4_K)
#pragma unroll
                for (int j = 0; j < 8; j++) x32s[j][tid] = a.xs32[m * (K / 32) + sb * 8 + j];
        }
        // ---- weights: unpack codes to int8, scales to integers
        {
            const int r = tid >> 2;  // 4 threads per row
            int64_t n = n0 + r;
            n = n < a.N ? n : a.N - 1;
            const int64_t blk = n * nsb + sb;
            int8_t *dst = ws + r * KQROW;
            if (TYPE == MX_TYPE_Q4_K) {
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int t = (tid & 3) * 2 + u;  // 16-byte chunk t of the 128 code bytes
                    v4i lo, hi;
                    unpack_q4k(*(const v4i *)(a.w.p0 + blk * 128 + 16 * t), lo, hi);
                    const int e = 64 * (t >> 1) + 16 * (t & 1);
                    *(v4i *)(dst + e) = lo;
                    *(v4i *)(dst + e + 32) = hi;
                }
            } else {
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int t = (tid & 3) * 2 + u;  // 16-byte chunk t of the 128 ql bytes
                    const int h = t >> 2, q = t & 3;
                    const v4i ql = *(const v4i *)(a.w.p0 + blk * 128 + 64 * h + 16 * q);
                    const v4i qh = *(const v4i *)(a.w.p1 + blk * 64 + 32 * h + 16 * (q & 1));
                    const int sh = 2 * (q >> 1);
                    const int e = 128 * h + 32 * (q >> 1) + 16 * (q & 1);
                    v4i lo, hi;
                    lo.x = ((ql.x & 0x0F0F0F0F) | (((qh.x >> sh) & 0x03030303) << 4));
                    lo.y = ((ql.y & 0x0F0F0F0F) | (((qh.y >> sh) & 0x03030303) << 4));
                    lo.z = ((ql.z & 0x0F0F0F0F) | (((qh.z >> sh) & 0x03030303) << 4));
                    lo.w = ((ql.w & 0x0F0F0F0F) | (((qh.w >> sh) & 0x03030303) << 4));
                    hi.x = (((ql.x >> 4) & 0x0F0F0F0F) | (((qh.x >> (sh + 4)) & 0x03030303) << 4));
                    hi.y = (((ql.y >> 4) & 0x0F0F0F0F) | (((qh.y >> (sh + 4)) & 0x03030303) << 4));
                    hi.z = (((ql.z >> 4) & 0x0F0F0F0F) | (((qh.z >> (sh + 4)) & 0x03030303) << 4));
                    hi.w = (((ql.w >> 4) & 0x0F0F0F0F) | (((qh.w >> (sh + 4)) & 0x03030303) << 4));
                    // codes 0..63 -> code - 32 in each byte (no byte borrows: every code is at least 0)
                    const v4i off = {0x20202020, 0x20202020, 0x20202020, 0x20202020};
                    lo = ((lo | (v4i){(int)0x80808080, (int)0x80808080, (int)0x80808080, (int)0x80808080}) - off) ^
                         (v4i){(int)0x80808080, (int)0x80808080, (int)0x80808080, (int)0x80808080};
                    hi = ((hi | (v4i){(int)0x80808080, (int)0x80808080, (int)0x80808080, (int)0x80808080}) - off) ^
                         (v4i){(int)0x80808080, (int)0x80808080, (int)0x80808080, (int)0x80808080};
                    *(v4i *)(dst + e) = lo;
                    *(v4i *)(dst + e + 64) = hi;
                }
            }
            if ((tid & 3) == 0) {
                if (TYPE == MX_TYPE_Q4_K) {
                    const uint8_t *s = a.w.p1 + blk * 12;
                    const uint32_t dm = *(const uint32_t *)(a.w.p2 + blk * 4);
                    dws[r] = h2f((uint16_t)(dm & 0xFFFF));
                    dmws[r] = h2f((uint16_t)(dm >> 16));
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        int sc, mn;
                        if (j < 4) {
                            sc = s[j] & 63;
                            mn = s[j + 4] & 63;
                        } else {
                            sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
                            mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
                        }
                        scs[j][r] = sc;
                        mns[j][r] = (float)mn;
                    }
                } else {
                    const int8_t *s = (const int8_t *)a.w.p2 + blk * 16;
#pragma unroll
                    for (int j = 0; j < 16; j++) scs[j][r] = s[j];
                    dws[r] = h2f(*(const uint16_t *)(a.w.p3 + blk * 2));
                }
            }
        }
        __syncthreads();

        // ---- integer block sums scaled by the integer sub-block scales: I (exact int32)
        int I[16];
#pragma unroll
        for (int r = 0; r < 16; r++) I[r] = 0;
        const int ncol = wn + fr;  // this lane's column (weight row) within the tile
        const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll 2
        for (int j = 0; j < 8; j++) {
            const v4i af = *(const v4i *)(xs + (wm + fr) * KQROW + 32 * j + fk);
            const v4i bf = *(const v4i *)(ws + (wn + fr) * KQROW + 32 * j + fk);
            if (TYPE == MX_TYPE_Q4_K) {
                const v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, zero, 0, 0, 0);
                const int sc = scs[j][ncol];
#pragma unroll
                for (int r = 0; r < 16; r++) I[r] += sc * S[r];
            } else {
                // lanes 0-31 carry codes 0..15 of the 32, lanes 32-63 codes 16..31: each MFMA keeps one half
                const v4i bz = {0, 0, 0, 0};
                const v16i Slo = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, lane < 32 ? bf : bz, zero, 0, 0, 0);
                const v16i Shi = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, lane < 32 ? bz : bf, zero, 0, 0, 0);
                const int slo = scs[2 * j][ncol], shi = scs[2 * j + 1][ncol];
#pragma unroll
                for (int r = 0; r < 16; r++) I[r] += slo * Slo[r] + shi * Shi[r];
            }
        }

        // ---- float scales, once per super-block
        const float dw = dws[ncol];
        if (TYPE == MX_TYPE_Q4_K) {
            // min term: sum_j mn[n][j] * x32[m][j], K = 8 integers, exact in fp32
            v16f Mt = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int j = 2 * p + (lane >> 5);
                Mt = __builtin_amdgcn_mfma_f32_32x32x2f32(x32s[j][wm + fr], mns[j][ncol], Mt, 0, 0, 0);
            }
            const float dmin = dmws[ncol];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float dx = dxs[m];
                acc[r] += (dw * dx) * (float)I[r] - (dmin * dx) * Mt[r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                acc[r] += (dw * dxs[m]) * (float)I[r];
            }
        }
    }

    const int64_t n = n0 + wn + fr;
    if (n < a.N) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int64_t m = m0 + wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m < a.M) a.y[m * a.ldy + n] = acc[r];
        }
    }
}

size_t gemm_kq_act_bytes(int64_t M, int64_t K) {
    const size_t q = (size_t)align_up((uint64_t)(M * K), 256);
    const size_t d = (size_t)align_up((uint64_t)M * (uint64_t)(K / 256) * 4, 256);
    const size_t s = (size_t)align_up((uint64_t)M * (uint64_t)(K / 32) * 4, 256);
    return q + d + s;
}

struct KqScratch {
    int8_t *xq;
    float *xd, *xs32;
};

static KqScratch kq_scratch(void *scratch, int64_t M, int64_t K) {
    KqScratch p;
    p.xq = (int8_t *)scratch;
    p.xd = (float *)((uint8_t *)scratch + align_up((uint64_t)(M * K), 256));
    p.xs32 = (float *)((uint8_t *)p.xd + align_up((uint64_t)M * (uint64_t)(K / 256) * 4, 256));
    return p;
}

hipError_t launch_gemm_kq_quant(const float *x, int64_t x_stride, int64_t M, int64_t K, void *scratch, hipStream_t s) {
    if (K % 256 != 0) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    const KqScratch p = kq_scratch(scratch, M, K);
    hipLaunchKernelGGL(k_gemm_quant_q8k, dim3((unsigned)M, (unsigned)((K / 256 + 3) / 4)), dim3(256), 0, s, x, x_stride,
                       K, p.xq, p.xd, p.xs32);
    return hipGetLastError();
}

hipError_t launch_gemm_kq(int type, const WPlanes &w, int64_t M, int64_t N, int64_t K, const void *scratch, float *y,
                          int64_t ldy, hipStream_t s) {
    if ((type != MX_TYPE_Q4_K && type != MX_TYPE_Q6_K) || K % 256 != 0) return hipErrorInvalidValue;
    const KqScratch p = kq_scratch(const_cast<void *>(scratch), M, K);
    KqArgs a{w, M, N, K, p.xq, p.xd, p.xs32, y, ldy};
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    if (type == MX_TYPE_Q4_K) hipLaunchKernelGGL(k_gemm_kq<MX_TYPE_Q4_K>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(k_gemm_kq<MX_TYPE_Q6_K>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mx
