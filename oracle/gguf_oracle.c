/*
 * CPU oracle for the GGUF dequant-GEMV hot path.  TEST INFRASTRUCTURE ONLY:
 * the tests, the smoke check and the CPU-baseline leg of the benchmark load
 * this library as the checker.  The product (libcima_hip.so + the gfx950
 * code object) never links, loads or calls it.
 *
 * This is a plain-C restatement of the reference engine's CPU arithmetic
 * (the reference is Rust; no Rust toolchain exists here, so the reference
 * itself cannot be built -- there is no oracle/_ref build).  Every function
 * cites the reference file:line it restates.
 *
 * Pinning (what checks each function against something other than itself):
 *   f16 <-> f32          exhaustive 65536-value round trip + RTNE ties
 *                        (reference test src/quant.rs:1171-1204), and numpy's
 *                        IEEE float16 cast over all f16 values and 1e6 random
 *                        f32 (independent library oracle).
 *   dequant_q8_0/q4_0/q4_1/q5_0/q5_1/q4_k/q5_k/q6_k/iq4_xs
 *                        reference known-answer tests src/quant.rs:1011,1027,
 *                        1075,1101,1140,1220,1245,1261,1281 restated in
 *                        tests/test_oracle.py; an
 *                        independent numpy decoder (tests/golden/make_golden.py)
 *                        that computes each value in float64 and rounds once
 *                        to float16 (closed form: every product is exact);
 *                        committed fixtures from that decoder.
 *   storage sizes        reference test src/quant.rs:1207-1218.
 *   nf4 dequant / fold   the reference has no NF4 test: pinned by an
 *                        independent numpy restatement (tests/test_nf4.py,
 *                        closed form f16(f32(code * absmax))), exact special
 *                        cases (power-of-two codes and scales) and the
 *                        nibble order src/kernels.cu:320-329 states.
 *   gemv / gemm          brute-force float64 dot over the decoded weights
 *                        (numpy einsum in the tests); epilogue semantics
 *                        against their closed forms.
 *   synthetic quantizers are the product's (the reference has none); the
 *                        oracle only decodes what they produce.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stddef.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ggml tensor type ids, src/formats.rs:90-117 */
enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q4_K = 12,
       T_Q5_K = 13, T_Q6_K = 14, T_IQ4_XS = 23 };

/* ---------------------------------------------------------------------- */
/* f16 primitives: src/traits.rs:832-854 (f16_to_f32), :857-896 (f32_to_f16) */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)(h >> 15)) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0 && man == 0) {
        bits = sign;
    } else if (exp == 0) {
        /* subnormal: man * 2^-24, renormalised on its leading one */
        uint32_t p = 31 - (uint32_t)__builtin_clz(man);
        uint32_t e = 103 + p;
        uint32_t frac = (man << (23 - p)) & 0x7fffff;
        bits = sign | (e << 23) | frac;
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13); /* inf, or NaN with payload */
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    return u2f(bits);
}

uint16_t oracle_f32_to_f16(float v) {
    uint32_t x = f2u(v);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t exp_f = (x >> 23) & 0xff;
    uint32_t man = x & 0x7fffff;
    if (exp_f == 0xff) return man ? (uint16_t)(sign | 0x7e00) : (uint16_t)(sign | 0x7c00);
    int exp = (int)exp_f - 127 + 15;
    if (exp >= 31) return (uint16_t)(sign | 0x7c00);
    if (exp <= 0) {
        if (exp < -10) return sign;
        man |= 0x800000;
        uint32_t shift = (uint32_t)(14 - exp);
        uint16_t half = (uint16_t)(man >> shift);
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t tie = 1u << (shift - 1);
        if (rem > tie || (rem == tie && (half & 1))) half++;
        return (uint16_t)(sign | half);
    }
    uint16_t half = (uint16_t)(((uint32_t)exp << 10) | (man >> 13));
    uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (half & 1))) half++;
    return (uint16_t)(sign | half);
}

/* d16: little-endian f16 field -> f32, src/quant.rs:571-573 */
static inline float d16(const uint8_t* b) { return oracle_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

/* ---------------------------------------------------------------------- */
/* format tables: src/formats.rs:119-132 (storage_bytes), src/traits.rs:264-272 */

int oracle_block_elems(int t) {
    switch (t) {
    case T_Q8_0: case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: return 32;
    case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_IQ4_XS: return 256;
    default: return 0;
    }
}

int oracle_block_bytes(int t) {
    switch (t) {
    case T_Q8_0: return 34;
    case T_Q4_0: return 18;
    case T_Q4_1: return 20;
    case T_Q5_0: return 22;
    case T_Q5_1: return 24;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    case T_IQ4_XS: return 136;
    default: return 0;
    }
}

size_t oracle_storage_bytes(int t, size_t numel) {
    int e = oracle_block_elems(t);
    return e ? (numel / (size_t)e) * (size_t)oracle_block_bytes(t) : 0;
}

/* ---------------------------------------------------------------------- */
/* decoders: f16 bits out.  Each returns 0, or -1 on the reference's size
 * mismatch error (numel not a block multiple, or src too short). */

/* src/quant.rs:599-617 */
int oracle_dequant_q8_0(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 32;
    if (src_len < blocks * 34 || numel % 32) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 34;
        float d = d16(blk);
        for (int i = 0; i < 32; i++) out[b * 32 + i] = oracle_f32_to_f16(d * (float)(int8_t)blk[2 + i]);
    }
    return 0;
}

/* src/quant.rs:624-644 */
int oracle_dequant_q4_0(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 32;
    if (src_len < blocks * 18 || numel % 32) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 18;
        float d = d16(blk);
        for (int j = 0; j < 16; j++) {
            uint8_t q = blk[2 + j];
            out[b * 32 + j] = oracle_f32_to_f16(d * (float)((int)(q & 0x0F) - 8));
            out[b * 32 + j + 16] = oracle_f32_to_f16(d * (float)((int)(q >> 4) - 8));
        }
    }
    return 0;
}

/* src/quant.rs:646-669: x = d q + m (the product is exact; the sum is
 * rounded once to fp32) */
int oracle_dequant_q4_1(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 32;
    if (src_len < blocks * 20 || numel % 32) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 20;
        float d = d16(blk), m = d16(blk + 2);
        for (int j = 0; j < 16; j++) {
            uint8_t q = blk[4 + j];
            out[b * 32 + j] = oracle_f32_to_f16(d * (float)(q & 0x0F) + m);
            out[b * 32 + j + 16] = oracle_f32_to_f16(d * (float)(q >> 4) + m);
        }
    }
    return 0;
}

/* src/quant.rs:671-699: bit j of qh is element j's 5th bit, bit j + 16
 * element j + 16's; x = d (q5 - 16) */
int oracle_dequant_q5_0(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 32;
    if (src_len < blocks * 22 || numel % 32) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 22;
        float d = d16(blk);
        uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
        for (int j = 0; j < 16; j++) {
            uint8_t q = blk[6 + j];
            uint32_t hi0 = ((qh >> j) << 4) & 0x10, hi1 = (qh >> (j + 12)) & 0x10;
            int x0 = (int)((q & 0x0F) | hi0) - 16, x1 = (int)((q >> 4) | hi1) - 16;
            out[b * 32 + j] = oracle_f32_to_f16(d * (float)x0);
            out[b * 32 + j + 16] = oracle_f32_to_f16(d * (float)x1);
        }
    }
    return 0;
}

/* src/quant.rs:701-729: Q5_0's bits with a min; x = d q5 + m */
int oracle_dequant_q5_1(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 32;
    if (src_len < blocks * 24 || numel % 32) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 24;
        float d = d16(blk), m = d16(blk + 2);
        uint32_t qh = (uint32_t)blk[4] | ((uint32_t)blk[5] << 8) | ((uint32_t)blk[6] << 16) | ((uint32_t)blk[7] << 24);
        for (int j = 0; j < 16; j++) {
            uint8_t q = blk[8 + j];
            uint32_t hi0 = ((qh >> j) << 4) & 0x10, hi1 = (qh >> (j + 12)) & 0x10;
            out[b * 32 + j] = oracle_f32_to_f16(d * (float)((q & 0x0F) | hi0) + m);
            out[b * 32 + j + 16] = oracle_f32_to_f16(d * (float)((q >> 4) | hi1) + m);
        }
    }
    return 0;
}

/* src/quant.rs:731-740 (get_scale_min_k4) */
static void scale_min_k4(int j, const uint8_t* s, float* sc, float* m) {
    if (j < 4) {
        *sc = (float)(s[j] & 63);
        *m = (float)(s[j + 4] & 63);
    } else {
        *sc = (float)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (float)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

void oracle_scale_min_k4(int j, const uint8_t* s, float* sc, float* m) { scale_min_k4(j, s, sc, m); }

/* src/quant.rs:743-774 */
int oracle_dequant_q4_k(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 256;
    if (src_len < blocks * 144 || numel % 256) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 144;
        float d = d16(blk), dmin = d16(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        for (int c = 0; c < 4; c++) {
            float sc0, m0, sc1, m1;
            scale_min_k4(2 * c, scales, &sc0, &m0);
            scale_min_k4(2 * c + 1, scales, &sc1, &m1);
            float d0 = d * sc0, mm0 = dmin * m0, d1 = d * sc1, mm1 = dmin * m1;
            for (int i = 0; i < 32; i++) {
                uint8_t q = qs[c * 32 + i];
                /* products are exact in f32, so the only f32 rounding is the
                 * subtraction -- same as the reference with or without FMA */
                float lo = d0 * (float)(q & 0x0F);
                float hi = d1 * (float)(q >> 4);
                out[b * 256 + c * 64 + i] = oracle_f32_to_f16(lo - mm0);
                out[b * 256 + c * 64 + 32 + i] = oracle_f32_to_f16(hi - mm1);
            }
        }
    }
    return 0;
}

/* src/quant.rs:776-815: Q4_K's layout plus qh[32]; chunk c's low and high
 * nibbles take bits 2c and 2c + 1 of qh[l] as +16 */
int oracle_dequant_q5_k(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 256;
    if (src_len < blocks * 176 || numel % 256) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 176;
        float d = d16(blk), dmin = d16(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* qh = blk + 16;
        const uint8_t* ql = blk + 48;
        for (int c = 0; c < 4; c++) {
            float sc0, m0, sc1, m1;
            scale_min_k4(2 * c, scales, &sc0, &m0);
            scale_min_k4(2 * c + 1, scales, &sc1, &m1);
            float d1 = d * sc0, mm1 = dmin * m0, d2 = d * sc1, mm2 = dmin * m1;
            uint8_t u1 = (uint8_t)(1u << (2 * c)), u2 = (uint8_t)(2u << (2 * c));
            for (int l = 0; l < 32; l++) {
                float hi1 = (qh[l] & u1) ? 16.0f : 0.0f, hi2 = (qh[l] & u2) ? 16.0f : 0.0f;
                uint8_t q = ql[c * 32 + l];
                float lo = d1 * ((float)(q & 0x0F) + hi1);
                float hi = d2 * ((float)(q >> 4) + hi2);
                out[b * 256 + c * 64 + l] = oracle_f32_to_f16(lo - mm1);
                out[b * 256 + c * 64 + 32 + l] = oracle_f32_to_f16(hi - mm2);
            }
        }
    }
    return 0;
}

/* src/quant.rs:817-822: ggml's kvalues_iq4nl codebook */
static const float IQ4NL[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};

/* src/quant.rs:823-854: 6-bit sub-block scales split over scales_h (2 bits
 * each) and scales_l (4 bits each); x = (d (ls - 32)) codebook[q] */
int oracle_dequant_iq4_xs(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 256;
    if (src_len < blocks * 136 || numel % 256) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 136;
        float d = d16(blk);
        uint32_t scales_h = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8);
        const uint8_t* scales_l = blk + 4;
        const uint8_t* qs = blk + 8;
        for (int ib = 0; ib < 8; ib++) {
            int ls = (int)((scales_l[ib / 2] >> (4 * (ib % 2))) & 0x0F) | ((int)((scales_h >> (2 * ib)) & 3) << 4);
            float dl = d * (float)(ls - 32);
            const uint8_t* q = qs + ib * 16;
            for (int j = 0; j < 16; j++) {
                out[b * 256 + ib * 32 + j] = oracle_f32_to_f16(dl * IQ4NL[q[j] & 0x0F]);
                out[b * 256 + ib * 32 + 16 + j] = oracle_f32_to_f16(dl * IQ4NL[q[j] >> 4]);
            }
        }
    }
    return 0;
}

/* src/quant.rs:857-896 */
int oracle_dequant_q6_k(const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    size_t blocks = numel / 256;
    if (src_len < blocks * 210 || numel % 256) return -1;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t* blk = src + b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const uint8_t* sc = blk + 192;
        float d = d16(blk + 208);
        for (int half = 0; half < 2; half++) {
            const uint8_t* qlh = ql + half * 64;
            const uint8_t* qhh = qh + half * 32;
            const uint8_t* sch = sc + half * 8;
            size_t base = b * 256 + (size_t)half * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)(int8_t)((qlh[l] & 0x0F) | ((qhh[l] & 0x03) << 4)) - 32;
                int q2 = (int)(int8_t)((qlh[l + 32] & 0x0F) | (((qhh[l] >> 2) & 0x03) << 4)) - 32;
                int q3 = (int)(int8_t)((qlh[l] >> 4) | (((qhh[l] >> 4) & 0x03) << 4)) - 32;
                int q4 = (int)(int8_t)((qlh[l + 32] >> 4) | (((qhh[l] >> 6) & 0x03) << 4)) - 32;
                /* left-to-right: (d * sc) * q, both products exact */
                out[base + l] = oracle_f32_to_f16(d * (float)(int8_t)sch[is] * (float)q1);
                out[base + l + 32] = oracle_f32_to_f16(d * (float)(int8_t)sch[is + 2] * (float)q2);
                out[base + l + 64] = oracle_f32_to_f16(d * (float)(int8_t)sch[is + 4] * (float)q3);
                out[base + l + 96] = oracle_f32_to_f16(d * (float)(int8_t)sch[is + 6] * (float)q4);
            }
        }
    }
    return 0;
}

/* ---------------------------------------------------------------------- */
/* bitsandbytes NF4 / FP4 (src/quant.rs:18-437): packed nibbles (element
 * 2j the HIGH nibble of byte j), f32 absmax per blocksize elements, a
 * 16-entry f32 codebook */

/* folded_absmax, src/quant.rs:258-330 (the double-quantised branch):
 * absmax[i] = nested_quant_map[code[i]] * nested_absmax[i / nested_blocksize]
 * + nested_offset, each operation rounded in f32.  -1 when nested_absmax is
 * too short. */
int oracle_nf4_fold_absmax(const uint8_t* codes, size_t nblocks, const float* nested_quant_map,
                           const float* nested_absmax, size_t n_nested, size_t nested_blocksize,
                           float nested_offset, float* out) {
    for (size_t i = 0; i < nblocks; i++) {
        size_t j = i / nested_blocksize;
        if (j >= n_nested) return -1;
        float p = nested_quant_map[codes[i]] * nested_absmax[j];
        out[i] = p + nested_offset;
    }
    return 0;
}

/* dequant_host, src/quant.rs:401-437: w[i] = f16(qmap[nib(i)] * absmax[i / bs]) */
int oracle_nf4_dequant(const uint8_t* packed, const float* absmax, const float* qmap, uint16_t* out, size_t n,
                       size_t blocksize) {
    if (!blocksize || n % 2 || n % blocksize) return -1;
    for (size_t i = 0; i < n; i++) {
        uint8_t b = packed[i / 2];
        int nib = (i % 2 == 0) ? (b >> 4) : (b & 0x0F);
        out[i] = oracle_f32_to_f16(qmap[nib] * absmax[i / blocksize]);
    }
    return 0;
}

/* dequant_host dispatch, src/quant.rs:578-597; -2 = not a supported format */
int oracle_dequant(int t, const uint8_t* src, size_t src_len, size_t numel, uint16_t* out) {
    switch (t) {
    case T_Q8_0: return oracle_dequant_q8_0(src, src_len, numel, out);
    case T_Q4_0: return oracle_dequant_q4_0(src, src_len, numel, out);
    case T_Q4_1: return oracle_dequant_q4_1(src, src_len, numel, out);
    case T_Q5_0: return oracle_dequant_q5_0(src, src_len, numel, out);
    case T_Q5_1: return oracle_dequant_q5_1(src, src_len, numel, out);
    case T_Q4_K: return oracle_dequant_q4_k(src, src_len, numel, out);
    case T_Q5_K: return oracle_dequant_q5_k(src, src_len, numel, out);
    case T_Q6_K: return oracle_dequant_q6_k(src, src_len, numel, out);
    case T_IQ4_XS: return oracle_dequant_iq4_xs(src, src_len, numel, out);
    default: return -2;
    }
}

/* ---------------------------------------------------------------------- */
/* GEMV: the reference CPU path -- host f16 dequant (above), then an fp32
 * dot per row, sequential in k.  Epilogue semantics follow the engine's
 * GEMV contract, src/kernels.cu:1063-1069 (GEMV_TAIL: + bias, mode 1 adds
 * the old y) and src/kernels.cu:493-538 (mode 2: gate|up pair,
 * y = silu(g + bg) * (u + bu)).  Weights of all n (or 2n) rows are decoded
 * once into w16 by the caller. */

static inline float silu(float g) { return g / (1.0f + expf(-g)); }

/* y[r] for r in [0, n); w16 is [rows, k] f16 bits, rows = n (modes 0/1) or
 * 2n (mode 2: rows [0,n) gate, [n,2n) up).  bias has the same row count
 * (NULL = none).  y_old is read for mode 1.  fp32 accumulate. */
void oracle_gemv_f32(const uint16_t* w16, const float* x, const float* bias, const float* y_old,
                     float* y, int n, int k, int mode, int threads) {
#ifdef _OPENMP
    int nt = threads > 0 ? threads : 1;
#pragma omp parallel for num_threads(nt) schedule(static)
#endif
    for (int r = 0; r < n; r++) {
        const uint16_t* wr = w16 + (size_t)r * k;
        float acc = 0.0f;
        for (int e = 0; e < k; e++) acc += oracle_f16_to_f32(wr[e]) * x[e];
        if (mode == 2) {
            const uint16_t* ur = w16 + (size_t)(r + n) * k;
            float acc2 = 0.0f;
            for (int e = 0; e < k; e++) acc2 += oracle_f16_to_f32(ur[e]) * x[e];
            if (bias) { acc += bias[r]; acc2 += bias[r + n]; }
            y[r] = silu(acc) * acc2;
        } else {
            if (bias) acc += bias[r];
            if (mode == 1) acc += y_old[r];
            y[r] = acc;
        }
    }
}

/* float64 dot over the decoded weights, for tolerance tests: y64[r] and the
 * L2 norm of the terms w*x per row (the selftest's noise unit,
 * src/selftest.rs:1078-1089). */
void oracle_gemv_f64(const uint16_t* w16, const float* x, double* y64, double* l2, int n, int k) {
    for (int r = 0; r < n; r++) {
        const uint16_t* wr = w16 + (size_t)r * k;
        double acc = 0.0, sq = 0.0;
        for (int e = 0; e < k; e++) {
            double t = (double)oracle_f16_to_f32(wr[e]) * (double)x[e];
            acc += t;
            sq += t * t;
        }
        y64[r] = acc;
        l2[r] = sqrt(sq);
    }
}

/* The CPU baseline: the reference CPU path end to end on packed bytes --
 * decode row r to f16 (quant::gguf::dequant_*), then the fp32 dot.  One row
 * at a time so the working set is one row of f16.  threads = 1 is the
 * reference's own scalar single-thread loop. */
int oracle_gguf_gemv_packed(int t, const uint8_t* w, const float* x, float* y, int n, int k, int threads) {
    int be = oracle_block_elems(t);
    if (!be || k % be) return -1;
    size_t row_bytes = oracle_storage_bytes(t, (size_t)k);
    int bad = 0;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : 1;
#pragma omp parallel num_threads(nt)
#endif
    {
        uint16_t rowbuf[65536];
        int kk = k <= 65536 ? k : 0;
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int r = 0; r < n; r++) {
            if (!kk || oracle_dequant(t, w + (size_t)r * row_bytes, row_bytes, (size_t)kk, rowbuf)) {
                bad = 1;
                continue;
            }
            float acc = 0.0f;
            for (int e = 0; e < kk; e++) acc += oracle_f16_to_f32(rowbuf[e]) * x[e];
            y[r] = acc;
        }
    }
    return bad ? -1 : 0;
}

/* ---------------------------------------------------------------------- */
/* prefill GEMM: Y[m, n] = X[m, k] . W16[n, k]^T, fp32 accumulate (the
 * reference's lin_gemm: gguf_dequant to f16 then gemm_f16 with f32 compute,
 * src/models/transformer.rs:618-655, src/cuda.rs:2484-2541). */
void oracle_gemm_f32(const float* x, const uint16_t* w16, float* y, int m, int n, int k, int threads) {
#ifdef _OPENMP
    int nt = threads > 0 ? threads : 1;
#pragma omp parallel for num_threads(nt) schedule(static)
#endif
    for (int c = 0; c < n; c++) {
        const uint16_t* wr = w16 + (size_t)c * k;
        for (int r = 0; r < m; r++) {
            const float* xr = x + (size_t)r * k;
            float acc = 0.0f;
            for (int e = 0; e < k; e++) acc += oracle_f16_to_f32(wr[e]) * xr[e];
            y[(size_t)r * n + c] = acc;
        }
    }
}

/* ---------------------------------------------------------------------- */
/* embedding gather from a packed table: out[i, :] = dequant(table[ids[i]]),
 * src/kernels.cu:1381-1401 (device) / the host side of the selftest,
 * src/selftest.rs:1148-1160. */
int oracle_gguf_gather(int t, const uint8_t* table, size_t table_len, const uint32_t* ids,
                       uint16_t* out, int n, int hidden) {
    size_t row_bytes = oracle_storage_bytes(t, (size_t)hidden);
    for (int i = 0; i < n; i++) {
        size_t off = (size_t)ids[i] * row_bytes;
        if (off + row_bytes > table_len) return -1;
        int rc = oracle_dequant(t, table + off, row_bytes, (size_t)hidden, out + (size_t)i * hidden);
        if (rc) return rc;
    }
    return 0;
}

/* array forms of the f16 primitives, for exhaustive / bulk checks */
void oracle_f16_to_f32_array(const uint16_t* h, float* out, size_t count) {
    for (size_t i = 0; i < count; i++) out[i] = oracle_f16_to_f32(h[i]);
}

void oracle_f32_to_f16_array(const float* v, uint16_t* out, size_t count) {
    for (size_t i = 0; i < count; i++) out[i] = oracle_f32_to_f16(v[i]);
}
