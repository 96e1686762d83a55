// Host-side weight quantization: ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, imatrix = NULL), the
// path `speech quantize` takes (src/common/quantize.cpp:164-182), which with no importance matrix runs ggml-quants.c's
// reference quantizers quantize_row_q8_0_ref / quantize_row_q4_K_ref / quantize_row_q5_K_ref / quantize_row_q6_K_ref
// (F16 rows are converted, F32 rows copied). Also the seeded synthetic generator used for weights and activations.
//
// Compiled without FMA contraction (see the Makefile) so every product is rounded before it is summed, as in ggml-base,
// which is built for the x86-64 baseline ISA.
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/mx.h"

namespace {

// IEEE binary16 from binary32, round to nearest even, subnormals kept, NaN -> 0x7E00 with its sign.
uint16_t to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int exp = (int)((x >> 23) & 0xFF);
    const uint32_t man = x & 0x7FFFFF;
    if (exp == 0xFF) return (uint16_t)(sign | (man ? 0x7E00u : 0x7C00u));
    if (exp == 0) return (uint16_t)sign;
    const int e = exp - 112;  // binary16 biased exponent of a normal result
    const uint64_t sig = (uint64_t)(man | 0x800000u);
    const int drop = e >= 1 ? 13 : 13 + (1 - e);
    if (drop >= 26) return (uint16_t)sign;
    uint64_t q = sig >> drop;
    const uint64_t r = sig & ((1ull << drop) - 1);
    const uint64_t h = 1ull << (drop - 1);
    q += (r > h || (r == h && (q & 1))) ? 1 : 0;
    if (e < 1) return (uint16_t)(sign | (uint32_t)q);
    int ee = e;
    if (q >> 11) { q >>= 1; ee++; }
    if (ee >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)ee << 10) | ((uint32_t)q & 0x3FF));
}

float from_half(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
    float f;
    if (e == 0) {
        f = std::ldexp((float)m, -24);
        return (h & 0x8000) ? -f : f;
    }
    const uint32_t bits = e == 0x1F ? (sign | 0x7F800000u | (m << 13)) : (sign | ((e + 112) << 23) | (m << 13));
    std::memcpy(&f, &bits, 4);
    return f;
}

inline int rne(float v) { return (int)std::nearbyint(v); }  // ggml-quants.c nearest_int (default rounding mode)

void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)(v & 0xFF); p[1] = (uint8_t)(v >> 8); }

// quantize_row_q8_0_ref over one 32-block: block_q8_0 {fp16 d; int8 qs[32]}.
void q8_0_block(const float *x, uint8_t *out) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(out, to_half(d));
    for (int j = 0; j < 32; j++) out[2 + j] = (uint8_t)(int8_t)std::round(x[j] * id);
}

// make_qkx2_quants(n = 32, nmax, rmin, rdelta = 0.1, nstep, use_mad = false): codes L[] and the (scale, -min) pair of
// the asymmetric fit with the least weighted squared error over nstep + 1 candidate scales. Q4_K fits with nmax = 15,
// rmin = -1, nstep = 20; Q5_K with nmax = 31, rmin = -0.5, nstep = 15.
template <int nmax, int nstep>
float fit_asym(const float *x, const float *w, uint8_t *L, float *neg_min, float rmin) {
    constexpr int n = 32;
    constexpr float rdelta = 0.1f;
    float lo = x[0], hi = x[0], sw = w[0], sx = w[0] * x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sw += w[i];
        sx += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        std::fill(L, L + n, 0);
        *neg_min = -lo;
        return 0.0f;
    }
    float iscale = nmax / (hi - lo);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; i++) {
        const int l = std::clamp(rne(iscale * (x[i] - lo)), 0, nmax);
        L[i] = (uint8_t)l;
        const float diff = scale * L[i] + lo - x[i];
        best += w[i] * (diff * diff);
    }
    std::array<uint8_t, n> cand;
    for (int is = 0; is <= nstep; is++) {
        iscale = (rmin + rdelta * is + nmax) / (hi - lo);
        float sl = 0, sl2 = 0, sxl = 0;
        for (int i = 0; i < n; i++) {
            const int l = std::clamp(rne(iscale * (x[i] - lo)), 0, nmax);
            cand[i] = (uint8_t)l;
            sl += w[i] * l;
            sl2 += w[i] * l * l;
            sxl += w[i] * l * x[i];
        }
        const float D = sw * sl2 - sl * sl;
        if (!(D > 0)) continue;
        float s = (sw * sxl - sx * sl) / D;
        float m = (sl2 * sx - sl * sxl) / D;
        if (m > 0) {
            m = 0;
            s = sxl / sl2;
        }
        float err = 0;
        for (int i = 0; i < n; i++) {
            const float diff = s * cand[i] + m - x[i];
            err += w[i] * (diff * diff);
        }
        if (err < best) {
            std::copy(cand.begin(), cand.end(), L);
            best = err;
            scale = s;
            lo = m;
        }
    }
    *neg_min = -lo;
    return scale;
}

// The 6-bit scale and min of sub-block j from block_q4_K's 12 packed bytes (get_scale_min_k4).
void q4k_unpack(const uint8_t *s, int j, int &sc, int &m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// The shared first half of quantize_row_q4_K_ref / _q5_K_ref on one super-block: per 32-element sub-block an
// asymmetric fit with NMAX + 1 levels, then the eight (scale, min) pairs as 6-bit integers against fp16 d and dmin,
// written to out[0..15] (d, dmin, packed scales); returns the codes of the final rounding in L.
template <int NMAX, int NSTEP>
void k_scales_and_codes(const float *x, uint8_t *out, float rmin, std::array<uint8_t, 256> &L) {
    std::array<float, 8> scales{}, mins{};
    float wts[32];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; j++) {
        const float *xs = x + 32 * j;
        float s2 = 0;
        for (int l = 0; l < 32; l++) s2 += xs[l] * xs[l];
        const float av = std::sqrt(s2 / 32);
        for (int l = 0; l < 32; l++) wts[l] = av + std::fabs(xs[l]);
        scales[j] = fit_asym<NMAX, NSTEP>(xs, wts, L.data() + 32 * j, &mins[j], rmin);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_s = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_m = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t *sb = out + 4;
    for (int j = 0; j < 8; j++) {
        const uint8_t ls = std::min<uint8_t>(63, (uint8_t)rne(inv_s * scales[j]));
        const uint8_t lm = std::min<uint8_t>(63, (uint8_t)rne(inv_m * mins[j]));
        if (j < 4) {
            sb[j] = ls;
            sb[j + 4] = lm;
        } else {
            sb[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sb[j - 4] |= (uint8_t)((ls >> 4) << 6);
            sb[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint16_t hd = to_half(max_scale / 63.f), hm = to_half(max_min / 63.f);
    put16(out, hd);
    put16(out + 2, hm);
    for (int j = 0; j < 8; j++) {
        int sc, m;
        q4k_unpack(sb, j, sc, m);
        const float d = from_half(hd) * sc;
        if (d == 0.0f) continue;
        const float dm = from_half(hm) * m;
        for (int i = 0; i < 32; i++) L[32 * j + i] = (uint8_t)std::clamp(rne((x[32 * j + i] + dm) / d), 0, NMAX);
    }
}

// quantize_row_q4_K_ref over one super-block: block_q4_K {fp16 d, dmin; uint8 scales[12]; uint8 qs[128]}.
void q4_K_block(const float *x, uint8_t *out) {
    std::array<uint8_t, 256> L{};
    k_scales_and_codes<15, 20>(x, out, -1.0f, L);
    uint8_t *qs = out + 16;
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) qs[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
}

// quantize_row_q5_K_ref over one super-block: block_q5_K {fp16 d, dmin; uint8 scales[12]; uint8 qh[32]; qs[128]}.
// The low 4 bits of each code go to qs as in Q4_K; bit 4 of element l of sub-block j goes to bit j of qh[l].
void q5_K_block(const float *x, uint8_t *out) {
    std::array<uint8_t, 256> L{};
    k_scales_and_codes<31, 15>(x, out, -0.5f, L);
    uint8_t *qh = out + 16, *qs = out + 48;
    std::memset(qh, 0, 32);
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            const int lo = L[64 * c + l], hi = L[64 * c + 32 + l];
            qs[32 * c + l] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
            qh[l] |= (uint8_t)(((lo >> 4) << (2 * c)) | ((hi >> 4) << (2 * c + 1)));
        }
}

void f16_block(const float *x, uint8_t *out) { put16(out, to_half(*x)); }
void f32_block(const float *x, uint8_t *out) { std::memcpy(out, x, 4); }

// make_qx_quants(n = 16, nmax = 32, rmse_type = 1, no weights): symmetric 6-bit fit weighted by x^2, searched over
// 19 scales; writes codes l + 32 to L and returns the scale.
float fit_sym32(const float *x, int8_t *L) {
    constexpr int n = 16, nmax = 32;
    float maxv = 0, amax = 0;
    for (int i = 0; i < n; i++) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) { amax = ax; maxv = x[i]; }
    }
    if (amax < 1e-15f) {
        std::fill(L, L + n, 0);
        return 0.f;
    }
    auto code = [](float v) { return std::clamp(rne(v), -nmax, nmax - 1); };
    float iscale = -nmax / maxv;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; i++) {
        const int l = code(iscale * x[i]);
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; is++) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / maxv;
        float slx = 0, sl2 = 0;
        for (int i = 0; i < n; i++) {
            const int l = code(iscale * x[i]);
            const float w = x[i] * x[i];
            slx += w * x[i] * l;
            sl2 += w * l * l;
        }
        if (sl2 > 0 && slx * slx > best * sl2) {
            for (int i = 0; i < n; i++) L[i] = (int8_t)(nmax + code(iscale * x[i]));
            scale = slx / sl2;
            best = scale * slx;
        }
    }
    return scale;
}

// quantize_row_q6_K_ref over one super-block: block_q6_K {uint8 ql[128], qh[64]; int8 scales[16]; fp16 d}.
void q6_K_block(const float *x, uint8_t *out) {
    std::array<int8_t, 256> L{};
    std::array<float, 16> scales{};
    float max_scale = 0, max_abs = 0;
    for (int ib = 0; ib < 16; ib++) {
        scales[ib] = fit_sym32(x + 16 * ib, L.data() + 16 * ib);
        if (std::fabs(scales[ib]) > max_abs) {
            max_abs = std::fabs(scales[ib]);
            max_scale = scales[ib];
        }
    }
    if (max_abs < 1e-15f) {
        std::memset(out, 0, 210);
        return;
    }
    const float iscale = -128.f / max_scale;
    const uint16_t hd = to_half(1 / iscale);
    int8_t *sc = (int8_t *)(out + 192);
    for (int ib = 0; ib < 16; ib++) sc[ib] = (int8_t)std::min(127, rne(iscale * scales[ib]));
    put16(out + 208, hd);
    for (int j = 0; j < 16; j++) {
        const float d = from_half(hd) * sc[j];
        if (d == 0.0f) continue;
        for (int i = 0; i < 16; i++) L[16 * j + i] = (int8_t)(std::clamp(rne(x[16 * j + i] / d), -32, 31) + 32);
    }
    uint8_t *ql = out, *qh = out + 128;
    for (int h = 0; h < 2; h++) {
        const int8_t *Lh = L.data() + 128 * h;
        for (int l = 0; l < 32; l++) {
            ql[64 * h + l] = (uint8_t)((Lh[l] & 0xF) | ((Lh[l + 64] & 0xF) << 4));
            ql[64 * h + l + 32] = (uint8_t)((Lh[l + 32] & 0xF) | ((Lh[l + 96] & 0xF) << 4));
            qh[32 * h + l] = (uint8_t)((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) |
                                       ((Lh[l + 96] >> 4) << 6));
        }
    }
}

struct Geometry {
    int elems, bytes;
    void (*block)(const float *, uint8_t *);
};

bool geometry(int type, Geometry &g) {
    switch (type) {
        case MX_TYPE_Q8_0: g = {32, 34, q8_0_block}; return true;
        case MX_TYPE_Q4_K: g = {256, 144, q4_K_block}; return true;
        case MX_TYPE_Q5_K: g = {256, 176, q5_K_block}; return true;
        case MX_TYPE_Q6_K: g = {256, 210, q6_K_block}; return true;
        case MX_TYPE_F16: g = {1, 2, f16_block}; return true;
        case MX_TYPE_F32: g = {1, 4, f32_block}; return true;
        default: return false;
    }
}

// splitmix64 seeding of xoshiro256**, one stream per row.
struct RowStream {
    uint64_t s[4];
    RowStream(uint64_t seed, int64_t row) {
        uint64_t z0 = seed ^ ((uint64_t)row * 0xD1B54A32D192ED03ull);
        for (auto &v : s) {
            uint64_t z = (z0 += 0x9E3779B97F4A7C15ull);
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            v = z ^ (z >> 31);
        }
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        const uint64_t r = rotl(s[1] * 5, 7) * 9;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
};

void normal_row(uint64_t seed, int64_t row, int64_t n, float mean, float stddev, float *out) {
    RowStream rs(seed, row);
    for (int64_t j = 0; j < n; j += 2) {
        const double u1 = (double)((rs.next() >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(rs.next() >> 11) * 0x1.0p-53;
        const double rad = std::sqrt(-2.0 * std::log(u1));
        const double th = 6.283185307179586476925286766559 * u2;
        out[j] = (float)(mean + stddev * rad * std::cos(th));
        if (j + 1 < n) out[j + 1] = (float)(mean + stddev * rad * std::sin(th));
    }
}

}  // namespace

extern "C" {

MX_API size_t mx_quantize_chunk(int type, const float *src, void *dst, int64_t start, int64_t nrows, int64_t n_per_row) {
    Geometry g;
    if (!geometry(type, g) || !src || !dst || n_per_row <= 0 || nrows < 0) return 0;
    if (n_per_row % g.elems != 0 || start % n_per_row != 0) return 0;
    const size_t row_bytes = (size_t)(n_per_row / g.elems) * g.bytes;
    uint8_t *out = (uint8_t *)dst + (size_t)(start / n_per_row) * row_bytes;
    const float *in = src + start;
    const int64_t nblk = nrows * (n_per_row / g.elems);
    for (int64_t b = 0; b < nblk; b++) g.block(in + b * g.elems, out + b * g.bytes);
    return (size_t)nrows * row_bytes;
}

MX_API void mx_fill_normal_rows(uint64_t seed, int64_t row0, int64_t nrows, int64_t n_per_row, float mean, float stddev,
                                float *out) {
    for (int64_t r = 0; r < nrows; r++) normal_row(seed, row0 + r, n_per_row, mean, stddev, out + r * n_per_row);
}

MX_API size_t mx_quantize_normal_rows(int type, uint64_t seed, int64_t row0, int64_t nrows, int64_t n_per_row,
                                      float mean, float stddev, void *dst, int nthreads) {
    Geometry g;
    if (!geometry(type, g) || !dst || n_per_row <= 0 || n_per_row % g.elems != 0 || nrows < 0) return 0;
    const size_t row_bytes = (size_t)(n_per_row / g.elems) * g.bytes;
    nthreads = std::max(1, std::min<int>(nthreads, 256));
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; t++) {
        pool.emplace_back([=] {
            std::vector<float> row((size_t)n_per_row);
            for (int64_t r = t; r < nrows; r += nthreads) {
                normal_row(seed, row0 + r, n_per_row, mean, stddev, row.data());
                mx_quantize_chunk(type, row.data(), (uint8_t *)dst + (size_t)r * row_bytes, 0, 1, n_per_row);
            }
        });
    }
    for (auto &th : pool) th.join();
    return (size_t)nrows * row_bytes;
}

}  // extern "C"
