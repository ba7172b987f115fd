// Seeded synthetic weights and GGUF quantisers (host only).  See
// include/cima_synth.h.  The block layouts written here are the ones the
// reference decodes (src/quant.rs:599-896); the choice of scales is this
// library's own.
#include "cima_synth.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// normals for element indices [i0, i0 + count) of the stream `seed`;
// pair p = i/2 draws two uniforms from counters 2p and 2p+1
void normals(uint64_t seed, float stddev, size_t i0, size_t count, float* out) {
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = i0, end = i0 + count;
    while (i < end) {
        size_t p = i >> 1;
        uint64_t a = splitmix64(seed ^ (2 * p * 0xD1B54A32D192ED03ull));
        uint64_t b = splitmix64(seed ^ ((2 * p + 1) * 0xD1B54A32D192ED03ull));
        double u1 = ((double)(a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        double v = (i & 1) ? r * sin(two_pi * u2) : r * cos(two_pi * u2);
        out[i - i0] = (float)(v * stddev);
        i++;
    }
}

// IEEE binary16, round to nearest even (used for block scales)
uint16_t to_f16(float v) {
    uint32_t x;
    memcpy(&x, &v, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t ef = (x >> 23) & 0xff, man = x & 0x7fffff;
    if (ef == 0xff) return (uint16_t)(sign | (man ? 0x7e00 : 0x7c00));
    int e = (int)ef - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return sign;
        man |= 0x800000;
        uint32_t sh = (uint32_t)(14 - e);
        uint32_t h = man >> sh, rem = man & ((1u << sh) - 1), tie = 1u << (sh - 1);
        if (rem > tie || (rem == tie && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

float from_f16(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, b;
    if (e == 0) {
        if (m == 0) {
            b = s;
        } else {
            int p = 31 - __builtin_clz(m);
            b = s | ((uint32_t)(103 + p) << 23) | ((m << (23 - p)) & 0x7fffff);
        }
    } else if (e == 0x1f) {
        b = s | 0x7f800000u | (m << 13);
    } else {
        b = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &b, 4);
    return f;
}

void put16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xff);
    p[1] = (uint8_t)(v >> 8);
}

int iround(float v) { return (int)lrintf(v); }

void quant_q8_0(const float* x, uint8_t* blk) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = std::max(amax, fabsf(x[i]));
    uint16_t dh = to_f16(amax / 127.f);
    float d = from_f16(dh);
    put16(blk, dh);
    for (int i = 0; i < 32; i++) {
        int q = d > 0.f ? iround(x[i] / d) : 0;
        blk[2 + i] = (uint8_t)(int8_t)std::min(127, std::max(-127, q));
    }
}

void quant_q4_0(const float* x, uint8_t* blk) {
    float amax = 0.f, vmax = 0.f;
    for (int i = 0; i < 32; i++)
        if (fabsf(x[i]) > amax) {
            amax = fabsf(x[i]);
            vmax = x[i];
        }
    uint16_t dh = to_f16(vmax / -8.f);
    float d = from_f16(dh);
    put16(blk, dh);
    int q[32];
    for (int i = 0; i < 32; i++) q[i] = d != 0.f ? std::min(15, std::max(0, iround(x[i] / d) + 8)) : 8;
    for (int j = 0; j < 16; j++) blk[2 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

void quant_q4_1(const float* x, uint8_t* blk) {
    float mn = x[0], mx = x[0];
    for (int i = 1; i < 32; i++) {
        mn = std::min(mn, x[i]);
        mx = std::max(mx, x[i]);
    }
    uint16_t dh = to_f16((mx - mn) / 15.f), mh = to_f16(mn);
    float d = from_f16(dh), m = from_f16(mh);
    put16(blk, dh);
    put16(blk + 2, mh);
    int q[32];
    for (int i = 0; i < 32; i++) q[i] = d > 0.f ? std::min(15, std::max(0, iround((x[i] - m) / d))) : 0;
    for (int j = 0; j < 16; j++) blk[4 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

// 5-bit quants q[32] -> qh (bit e = q[e] bit 4) and the nibble bytes
void pack_q5(const int* q, uint8_t* qh4, uint8_t* qs) {
    uint32_t qh = 0;
    for (int e = 0; e < 32; e++) qh |= (uint32_t)((q[e] >> 4) & 1) << e;
    for (int i = 0; i < 4; i++) qh4[i] = (uint8_t)(qh >> (8 * i));
    for (int j = 0; j < 16; j++) qs[j] = (uint8_t)((q[j] & 15) | ((q[j + 16] & 15) << 4));
}

void quant_q5_0(const float* x, uint8_t* blk) {
    float amax = 0.f, vmax = 0.f;
    for (int i = 0; i < 32; i++)
        if (fabsf(x[i]) > amax) {
            amax = fabsf(x[i]);
            vmax = x[i];
        }
    uint16_t dh = to_f16(vmax / -16.f);
    float d = from_f16(dh);
    put16(blk, dh);
    int q[32];
    for (int i = 0; i < 32; i++) q[i] = d != 0.f ? std::min(31, std::max(0, iround(x[i] / d) + 16)) : 16;
    pack_q5(q, blk + 2, blk + 6);
}

void quant_q5_1(const float* x, uint8_t* blk) {
    float mn = x[0], mx = x[0];
    for (int i = 1; i < 32; i++) {
        mn = std::min(mn, x[i]);
        mx = std::max(mx, x[i]);
    }
    uint16_t dh = to_f16((mx - mn) / 31.f), mh = to_f16(mn);
    float d = from_f16(dh), m = from_f16(mh);
    put16(blk, dh);
    put16(blk + 2, mh);
    int q[32];
    for (int i = 0; i < 32; i++) q[i] = d > 0.f ? std::min(31, std::max(0, iround((x[i] - m) / d))) : 0;
    pack_q5(q, blk + 4, blk + 8);
}

// Q4_K / Q5_K: per 32-element sub-block a min/max fit to 0..LEVELS, the
// 6-bit scales and mins relative to the super-block's d and dmin; Q5_K adds
// the quants' 5th bits (bit 2c / 2c+1 of qh[l] for chunk c's low / high
// nibbles)
template <int LEVELS>
void quant_kq(const float* x, uint8_t* blk) {
    constexpr bool Q5 = LEVELS == 31;
    constexpr int BB = Q5 ? 176 : 144;
    float scale[8], minv[8];
    float max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; j++) {
        float mn = 0.f, mx = 0.f;
        for (int i = 0; i < 32; i++) {
            mn = std::min(mn, x[32 * j + i]);
            mx = std::max(mx, x[32 * j + i]);
        }
        scale[j] = (mx - mn) / (float)LEVELS;
        minv[j] = -mn;
        max_scale = std::max(max_scale, scale[j]);
        max_min = std::max(max_min, minv[j]);
    }
    uint16_t dh = to_f16(max_scale / 63.f), mh = to_f16(max_min / 63.f);
    float d = from_f16(dh), dmin = from_f16(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0.f ? std::min(63, std::max(0, iround(scale[j] / d))) : 0;
        m[j] = dmin > 0.f ? std::min(63, std::max(0, iround(minv[j] / dmin))) : 0;
    }
    memset(blk, 0, BB);
    put16(blk, dh);
    put16(blk + 2, mh);
    uint8_t* s = blk + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)(sc[j] & 63);
        s[j + 4] = (uint8_t)(m[j] & 63);
    }
    for (int j = 4; j < 8; j++) {
        s[j + 4] = (uint8_t)((sc[j] & 0xF) | ((m[j] & 0xF) << 4));
        s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
        s[j] |= (uint8_t)((m[j] >> 4) << 6);
    }
    int q[256];
    for (int j = 0; j < 8; j++) {
        float ds = d * (float)sc[j], dm = dmin * (float)m[j];
        for (int i = 0; i < 32; i++)
            q[32 * j + i] = ds > 0.f ? std::min(LEVELS, std::max(0, iround((x[32 * j + i] + dm) / ds))) : 0;
    }
    uint8_t* qs = blk + (Q5 ? 48 : 16);
    for (int c = 0; c < 4; c++)
        for (int i = 0; i < 32; i++)
            qs[c * 32 + i] = (uint8_t)((q[c * 64 + i] & 15) | ((q[c * 64 + 32 + i] & 15) << 4));
    if (Q5) {
        uint8_t* qh = blk + 16;
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++)
                qh[l] |= (uint8_t)((((q[c * 64 + l] >> 4) & 1) << (2 * c)) | (((q[c * 64 + 32 + l] >> 4) & 1) << (2 * c + 1)));
    }
}
void quant_q4_k(const float* x, uint8_t* blk) { quant_kq<15>(x, blk); }
void quant_q5_k(const float* x, uint8_t* blk) { quant_kq<31>(x, blk); }

// IQ4_XS: per sub-block the largest-magnitude value maps to the codebook's
// -127 end; the sub-block scales become 6-bit steps (ls - 32) of the
// super-block d, and each value takes the nearest codebook entry
const float kIQ4NL[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                          1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};
void quant_iq4_xs(const float* x, uint8_t* blk) {
    float dl[8], amax_dl = 0.f;
    for (int ib = 0; ib < 8; ib++) {
        float amax = 0.f, vmax = 0.f;
        for (int i = 0; i < 32; i++)
            if (fabsf(x[32 * ib + i]) > amax) {
                amax = fabsf(x[32 * ib + i]);
                vmax = x[32 * ib + i];
            }
        dl[ib] = vmax / -127.f;
        amax_dl = std::max(amax_dl, fabsf(dl[ib]));
    }
    uint16_t dh = to_f16(amax_dl / 31.f);
    float d = from_f16(dh);
    memset(blk, 0, 136);
    put16(blk, dh);
    uint16_t scales_h = 0;
    for (int ib = 0; ib < 8; ib++) {
        int ls = d > 0.f ? std::min(63, std::max(0, iround(dl[ib] / d) + 32)) : 32;
        scales_h |= (uint16_t)(((ls >> 4) & 3) << (2 * ib));
        blk[4 + ib / 2] |= (uint8_t)((ls & 15) << (4 * (ib % 2)));
        float dq = d * (float)(ls - 32);
        int q[32];
        for (int i = 0; i < 32; i++) {
            int best = 0;
            float be = INFINITY;
            for (int j = 0; j < 16; j++) {
                float e = fabsf(dq * kIQ4NL[j] - x[32 * ib + i]);
                if (e < be) {
                    be = e;
                    best = j;
                }
            }
            q[i] = best;
        }
        for (int j = 0; j < 16; j++) blk[8 + 16 * ib + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
    }
    put16(blk + 2, scales_h);
}

// sub-block j (16 elements) of a Q6_K super-block holds elements
// 128h + 32g + 16s + [0,16) with h = j/8, g = (j%8)/2, s = j%2, and uses
// scale byte sc[8h + 2g + s]
void quant_q6_k(const float* x, uint8_t* blk) {
    float sf[16];
    float amax_s = 0.f;
    for (int j = 0; j < 16; j++) {
        int h = j / 8, g = (j % 8) / 2, s = j % 2;
        const float* v = x + 128 * h + 32 * g + 16 * s;
        float a = 0.f;
        for (int i = 0; i < 16; i++) a = std::max(a, fabsf(v[i]));
        sf[j] = a / 31.f;
        amax_s = std::max(amax_s, sf[j]);
    }
    uint16_t dh = to_f16(amax_s / 127.f);
    float d = from_f16(dh);
    memset(blk, 0, 210);
    uint8_t* ql = blk;
    uint8_t* qh = blk + 128;
    int8_t* sc = (int8_t*)(blk + 192);
    for (int j = 0; j < 16; j++) {
        int h = j / 8, g = (j % 8) / 2, s = j % 2;
        int isc = d > 0.f ? std::min(127, std::max(-128, iround(sf[j] / d))) : 0;
        sc[8 * h + 2 * g + s] = (int8_t)isc;
        float ds = d * (float)isc;
        for (int i = 0; i < 16; i++) {
            int l = 16 * s + i;
            float v = x[128 * h + 32 * g + l];
            int q = ds != 0.f ? std::min(31, std::max(-32, iround(v / ds))) : 0;
            int u = q + 32;
            uint8_t& lb = ql[64 * h + l + 32 * (g & 1)];
            lb |= (uint8_t)((g < 2) ? (u & 0xF) : ((u & 0xF) << 4));
            qh[32 * h + l] |= (uint8_t)(((u >> 4) & 3) << (2 * g));
        }
    }
    put16(blk + 208, dh);
}

struct QFmt {
    int be, bb;
    void (*fn)(const float*, uint8_t*);
};

bool qfmt(int t, QFmt* f) {
    switch (t) {
    case 8: *f = {32, 34, quant_q8_0}; return true;
    case 2: *f = {32, 18, quant_q4_0}; return true;
    case 3: *f = {32, 20, quant_q4_1}; return true;
    case 6: *f = {32, 22, quant_q5_0}; return true;
    case 7: *f = {32, 24, quant_q5_1}; return true;
    case 12: *f = {256, 144, quant_q4_k}; return true;
    case 13: *f = {256, 176, quant_q5_k}; return true;
    case 14: *f = {256, 210, quant_q6_k}; return true;
    case 23: *f = {256, 136, quant_iq4_xs}; return true;
    default: return false;
    }
}

}  // namespace

extern "C" {

void cima_synth_normal(uint64_t seed, float stddev, float* out, size_t count, int threads) {
    const size_t chunk = 1 << 16;
    long nchunks = (long)((count + chunk - 1) / chunk);
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
    for (long c = 0; c < nchunks; c++) {
        size_t i0 = (size_t)c * chunk, len = std::min(chunk, count - i0);
        normals(seed, stddev, i0, len, out + i0);
    }
    (void)threads;
}

int cima_synth_quantize(int t, const float* src, size_t rows, size_t k, uint8_t* dst, int threads) {
    QFmt f;
    if (!qfmt(t, &f) || k == 0 || k % (size_t)f.be) return -1;
    size_t bpr = k / (size_t)f.be;
    long total = (long)(rows * bpr);
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
    for (long b = 0; b < total; b++) f.fn(src + (size_t)b * f.be, dst + (size_t)b * f.bb);
    (void)threads;
    return 0;
}

int cima_synth_weights(int t, uint64_t seed, float stddev, size_t rows, size_t k, uint8_t* dst, int threads) {
    QFmt f;
    if (!qfmt(t, &f) || k == 0 || k % (size_t)f.be) return -1;
    size_t row_bytes = k / (size_t)f.be * (size_t)f.bb;
#ifdef _OPENMP
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
#endif
    {
        std::vector<float> buf(k);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (long r = 0; r < (long)rows; r++) {
            normals(seed, stddev, (size_t)r * k, k, buf.data());
            for (size_t b = 0; b < k / (size_t)f.be; b++)
                f.fn(buf.data() + b * f.be, dst + (size_t)r * row_bytes + b * f.bb);
        }
    }
    (void)threads;
    return 0;
}

}  // extern "C"
