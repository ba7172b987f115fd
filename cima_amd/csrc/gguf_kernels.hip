// GGUF block-quant kernels for gfx950 (CDNA4), built into one code object
// (cima_gguf.hsaco) that the host library loads with hipModuleLoad and
// launches with hipModuleLaunchKernel.
//
// Consumers of packed GGUF weights (formats Q8_0, Q4_0, Q4_K, Q6_K, block
// layouts as decoded by the reference's quant::gguf, src/quant.rs:599-896):
//   cima_gemv_*     fused decode GEMV, y = W.x (+bias)(+y)(SwiGLU pair),
//                   counterpart of k_gguf_<fmt>_gemv, src/kernels.cu:1071-1313
//   cima_dequant_*  packed -> f16, bit-exact with the host decoders,
//                   counterpart of k_gguf_<fmt>, src/kernels.cu:963-1009
//   cima_gather_*   packed embedding-row gather -> f16,
//                   counterpart of k_gguf_gather, src/kernels.cu:1381-1401
//
// Work decomposition.  A "unit" is the slice of one block that one lane
// decodes in one step; every format is split into 32- or 64-weight units
// whose bytes are contiguous or nearly so:
//   Q8_0  unit = 1 block   (34 B: f16 d + 32 x i8)              32 weights
//   Q4_0  unit = 1 block   (18 B: f16 d + 16 B of nibble pairs) 32 weights
//   Q4_K  unit = 16 B of qs + the 16 B block header             32 weights
//   Q6_K  unit = 16 B of ql (x2) + 16 B of qh + scales + d      64 weights
// A 256-thread workgroup is split into groups of LPR lanes (LPR = 16..256,
// a power of two); each group owns R consecutive output rows and its lanes
// stride over the units of those rows together, so one x fragment (loaded
// once, from L1/L2) is reused for R rows.  Partial sums are reduced inside
// the wave with DPP row ops + lane swizzles, then across waves through LDS
// when LPR > 64.  No atomics: the reduction order is fixed, so results are
// deterministic run to run.
//
// Numerics.  Activations are fp32 (or f16, widened to fp32).  Weights are
// never rounded: integer quants are converted exactly to fp32, dotted with
// x by fp32 FMA, and each block's scale (and Q4_K's min term, via the sum of
// x over the sub-block) is applied once per block fragment.  There is no
// activation quantisation.
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DEV __device__ __forceinline__

enum { GT_Q4_0 = 2, GT_Q8_0 = 8, GT_Q4_K = 12, GT_Q6_K = 14 };
enum { ACT_F32 = 0, ACT_F16 = 1 };

// ---------------------------------------------------------------- helpers

DEV float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
// v_cvt_f16_f32: round to nearest even, f16 subnormals kept.
DEV uint32_t f2h(float v) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v); }

DEV uint4 ld16a(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
// 2-byte-aligned 16-byte load: gfx950 runs with unaligned global access
// enabled, so this is one global_load_dwordx4 (split by the TA if it crosses
// a cache line), not a byte loop.
DEV uint4 ld16u(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 16);
    return v;
}
DEV uint32_t ld2(const uint8_t* p) {
    uint16_t v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 2);
    return v;
}

// byte b of a dword as an exact fp32 (v_cvt_f32_ubyte{0..3})
DEV float ub(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xffu); }

// 16 activations starting at element e, widened to fp32
template <int ACT>
DEV void load_x16(const void* __restrict__ x, int e, float (&o)[16]) {
    if constexpr (ACT == ACT_F32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + e);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 v = p[i];
            o[4 * i + 0] = v.x; o[4 * i + 1] = v.y; o[4 * i + 2] = v.z; o[4 * i + 3] = v.w;
        }
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + e);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            uint4 v = p[i];
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                o[8 * i + 2 * j] = h2f(w[j] & 0xffffu);
                o[8 * i + 2 * j + 1] = h2f(w[j] >> 16);
            }
        }
    }
}

DEV float sum16(const float (&v)[16]) {
    float a = (v[0] + v[1]) + (v[2] + v[3]), b = (v[4] + v[5]) + (v[6] + v[7]);
    float c = (v[8] + v[9]) + (v[10] + v[11]), d = (v[12] + v[13]) + (v[14] + v[15]);
    return (a + b) + (c + d);
}

// dot of the 4 bytes of each of 4 dwords (16 values, byte order = element
// order) with 16 activations
DEV float dot16_u8(const uint32_t (&w)[4], const float (&x)[16]) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a0 = fmaf(ub(w[i], 0), x[4 * i + 0], a0);
        a1 = fmaf(ub(w[i], 1), x[4 * i + 1], a1);
        a0 = fmaf(ub(w[i], 2), x[4 * i + 2], a0);
        a1 = fmaf(ub(w[i], 3), x[4 * i + 3], a1);
    }
    return a0 + a1;
}

// --------------------------------------------------------- format: Q8_0
// block: f16 d, i8 qs[32]; x[i] = d * qs[i]   (src/quant.rs:599-617)
struct FQ8_0 {
    static constexpr int BE = 32, BB = 34, UE = 32, UPB = 1;
    struct Raw { uint4 a, b; uint32_t d; };
    struct Xf { float v0[16], v1[16]; float s; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 34;
        Raw r;
        r.d = ld2(blk);
        r.a = ld16u(blk + 2);
        r.b = ld16u(blk + 18);
        return r;
    }
    template <int ACT>
    DEV static void loadx(const void* x, int u, Xf& f) {
        load_x16<ACT>(x, u * 32, f.v0);
        load_x16<ACT>(x, u * 32 + 16, f.v1);
        f.s = sum16(f.v0) + sum16(f.v1);
    }
    // signed bytes: (q ^ 0x80) = q + 128 as an unsigned byte, so
    // sum q.x = sum (q+128).x - 128 * sum x
    DEV static float dot(const Raw& r, const Xf& f, int) {
        uint32_t w0[4] = {r.a.x ^ 0x80808080u, r.a.y ^ 0x80808080u, r.a.z ^ 0x80808080u, r.a.w ^ 0x80808080u};
        uint32_t w1[4] = {r.b.x ^ 0x80808080u, r.b.y ^ 0x80808080u, r.b.z ^ 0x80808080u, r.b.w ^ 0x80808080u};
        float acc = dot16_u8(w0, f.v0) + dot16_u8(w1, f.v1);
        return h2f(r.d) * fmaf(-128.f, f.s, acc);
    }
    // dequant of one unit -> 32 f16 at out (element order)
    DEV static void dequant(const Raw& r, int, uint16_t* out) {
        float d = h2f(r.d);
        uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        uint32_t o[16];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float v0 = d * (float)(int8_t)(w[i] & 0xff), v1 = d * (float)(int8_t)((w[i] >> 8) & 0xff);
            float v2 = d * (float)(int8_t)((w[i] >> 16) & 0xff), v3 = d * (float)(int8_t)(w[i] >> 24);
            o[2 * i] = f2h(v0) | (f2h(v1) << 16);
            o[2 * i + 1] = f2h(v2) | (f2h(v3) << 16);
        }
        uint4* p = reinterpret_cast<uint4*>(out);
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
    DEV static int out_elem(int u) { return u * 32; }
};

// --------------------------------------------------------- format: Q4_0
// block: f16 d, u8 qs[16]; byte j = elem j (low nibble), elem j+16 (high);
// x = d * (q - 8)   (src/quant.rs:624-644)
struct FQ4_0 {
    static constexpr int BE = 32, BB = 18, UE = 32, UPB = 1;
    struct Raw { uint4 q; uint32_t d; };
    struct Xf { float lo[16], hi[16]; float s; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 18;
        Raw r;
        r.d = ld2(blk);
        r.q = ld16u(blk + 2);
        return r;
    }
    template <int ACT>
    DEV static void loadx(const void* x, int u, Xf& f) {
        load_x16<ACT>(x, u * 32, f.lo);
        load_x16<ACT>(x, u * 32 + 16, f.hi);
        f.s = sum16(f.lo) + sum16(f.hi);
    }
    DEV static float dot(const Raw& r, const Xf& f, int) {
        uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) { lo[i] = q[i] & 0x0F0F0F0Fu; hi[i] = (q[i] >> 4) & 0x0F0F0F0Fu; }
        float acc = dot16_u8(lo, f.lo) + dot16_u8(hi, f.hi);
        return h2f(r.d) * fmaf(-8.f, f.s, acc);
    }
    DEV static void dequant(const Raw& r, int, uint16_t* out) {
        float d = h2f(r.d);
        uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t o[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                int b0 = (q[i] >> (16 * j)) & 0xff, b1 = (q[i] >> (16 * j + 8)) & 0xff;
                float l0 = d * (float)((b0 & 15) - 8), l1 = d * (float)((b1 & 15) - 8);
                float h0 = d * (float)((b0 >> 4) - 8), h1 = d * (float)((b1 >> 4) - 8);
                o[2 * i + j] = f2h(l0) | (f2h(l1) << 16);
                o[8 + 2 * i + j] = f2h(h0) | (f2h(h1) << 16);
            }
        }
        uint4* p = reinterpret_cast<uint4*>(out);
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
    DEV static int out_elem(int u) { return u * 32; }
};

// --------------------------------------------------------- format: Q4_K
// super-block (144 B): f16 d, f16 dmin, u8 scales[12], u8 qs[128].
// 64-element chunk c uses qs[32c..32c+32): low nibbles are sub-block 2c,
// high nibbles sub-block 2c+1; x = (d*sc)*q - dmin*m  (src/quant.rs:743-774,
// 6-bit scale/min unpack src/quant.rs:731-740).
// Unit u: super-block u/8, qs bytes [16*(u%8), +16) -> chunk c = (u%8)/2,
// elements c*64 + 16*(u%2) + [0,16) (low) and the same +32 (high).
struct FQ4_K {
    static constexpr int BE = 256, BB = 144, UE = 32, UPB = 8;
    struct Raw { uint4 q; uint4 h; };
    struct Xf { float lo[16], hi[16]; float slo, shi; };
    DEV static int elem0(int u) { return (u >> 3) * 256 + ((u & 7) >> 1) * 64 + (u & 1) * 16; }
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 144;
        Raw r;
        r.h = ld16a(blk);
        r.q = ld16a(blk + 16 + (u & 7) * 16);
        return r;
    }
    template <int ACT>
    DEV static void loadx(const void* x, int u, Xf& f) {
        int e = elem0(u);
        load_x16<ACT>(x, e, f.lo);
        load_x16<ACT>(x, e + 32, f.hi);
        f.slo = sum16(f.lo);
        f.shi = sum16(f.hi);
    }
    // (sc, m) of sub-blocks 2c and 2c+1, from the 12 scale bytes held in
    // header dwords y (bytes 0-3), z (4-7), w (8-11)
    DEV static void scales(const uint4& h, int c, uint32_t& sc0, uint32_t& m0, uint32_t& sc1, uint32_t& m1) {
        int t = (c & 1) * 16;
        uint32_t A = h.y >> t, B = h.z >> t, C = h.w >> t;
        if (c < 2) {
            sc0 = A & 63; sc1 = (A >> 8) & 63;
            m0 = B & 63; m1 = (B >> 8) & 63;
        } else {
            sc0 = (C & 0xF) | (((A >> 6) & 3) << 4);
            sc1 = ((C >> 8) & 0xF) | (((A >> 14) & 3) << 4);
            m0 = ((C >> 4) & 0xF) | (((B >> 6) & 3) << 4);
            m1 = ((C >> 12) & 0xF) | (((B >> 14) & 3) << 4);
        }
    }
    DEV static float dot(const Raw& r, const Xf& f, int u) {
        uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) { lo[i] = q[i] & 0x0F0F0F0Fu; hi[i] = (q[i] >> 4) & 0x0F0F0F0Fu; }
        float dl = dot16_u8(lo, f.lo), dh = dot16_u8(hi, f.hi);
        uint32_t sc0, m0, sc1, m1;
        scales(r.h, (u & 7) >> 1, sc0, m0, sc1, m1);
        float d = h2f(r.h.x & 0xffffu), dmin = h2f(r.h.x >> 16);
        float pos = fmaf(d * (float)sc0, dl, (d * (float)sc1) * dh);
        float neg = fmaf(dmin * (float)m0, f.slo, (dmin * (float)m1) * f.shi);
        return pos - neg;
    }
    DEV static void dequant(const Raw& r, int u, uint16_t* out) {
        uint32_t sc0, m0, sc1, m1;
        scales(r.h, (u & 7) >> 1, sc0, m0, sc1, m1);
        float d = h2f(r.h.x & 0xffffu), dmin = h2f(r.h.x >> 16);
        float d0 = d * (float)sc0, mm0 = dmin * (float)m0, d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t ol[8], oh[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                uint32_t b0 = (q[i] >> (16 * j)) & 0xff, b1 = (q[i] >> (16 * j + 8)) & 0xff;
                // (d*sc)*q is exact in fp32, so the subtraction is the only
                // fp32 rounding, fused or not -- identical to the host decoder
                float l0 = d0 * (float)(b0 & 15) - mm0, l1 = d0 * (float)(b1 & 15) - mm0;
                float h0 = d1 * (float)(b0 >> 4) - mm1, h1 = d1 * (float)(b1 >> 4) - mm1;
                ol[2 * i + j] = f2h(l0) | (f2h(l1) << 16);
                oh[2 * i + j] = f2h(h0) | (f2h(h1) << 16);
            }
        }
        uint4* pl = reinterpret_cast<uint4*>(out);
        uint4* ph = reinterpret_cast<uint4*>(out + 32);
        pl[0] = make_uint4(ol[0], ol[1], ol[2], ol[3]);
        pl[1] = make_uint4(ol[4], ol[5], ol[6], ol[7]);
        ph[0] = make_uint4(oh[0], oh[1], oh[2], oh[3]);
        ph[1] = make_uint4(oh[4], oh[5], oh[6], oh[7]);
    }
    DEV static int out_elem(int u) { return elem0(u); }
};

// --------------------------------------------------------- format: Q6_K
// super-block (210 B): u8 ql[128], u8 qh[64], i8 sc[16], f16 d (at 208).
// Half h (128 elements), l in [0,32): elements +l, +l+32, +l+64, +l+96 take
// (low ql[64h+l], low ql[64h+l+32], high ql[64h+l], high ql[64h+l+32]) with
// qh[32h+l] bits (0-1, 2-3, 4-5, 6-7) as bits 4-5, minus 32; scale
// sc[8h + l/16 + 2g]; x = (d*sc)*q   (src/quant.rs:857-896).
// Unit u: super-block u/4, half h = (u/2)%2, l in 16*(u%2) + [0,16): four
// groups g of 16 consecutive elements.
struct FQ6_K {
    static constexpr int BE = 256, BB = 210, UE = 64, UPB = 4;
    struct Raw { uint4 a, b, h, sc; uint32_t d; };
    struct Xf { float v[4][16]; float s[4]; };
    DEV static int elem0(int u) { return (u >> 2) * 256 + ((u >> 1) & 1) * 128 + (u & 1) * 16; }
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 2) * 210;
        int hh = (u >> 1) & 1, is = u & 1;
        Raw r;
        r.a = ld16u(blk + hh * 64 + is * 16);
        r.b = ld16u(blk + hh * 64 + 32 + is * 16);
        r.h = ld16u(blk + 128 + hh * 32 + is * 16);
        r.sc = ld16u(blk + 192);
        r.d = ld2(blk + 208);
        return r;
    }
    template <int ACT>
    DEV static void loadx(const void* x, int u, Xf& f) {
        int e = elem0(u);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            load_x16<ACT>(x, e + 32 * g, f.v[g]);
            f.s[g] = sum16(f.v[g]);
        }
    }
    // 6-bit quants (0..63) of group g packed one per byte
    DEV static void q6(const Raw& r, uint32_t (&q)[4][4]) {
        uint32_t a[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        uint32_t b[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        uint32_t h[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            q[0][i] = (a[i] & 0x0F0F0F0Fu) | ((h[i] << 4) & 0x30303030u);
            q[1][i] = (b[i] & 0x0F0F0F0Fu) | ((h[i] << 2) & 0x30303030u);
            q[2][i] = ((a[i] >> 4) & 0x0F0F0F0Fu) | (h[i] & 0x30303030u);
            q[3][i] = ((b[i] >> 4) & 0x0F0F0F0Fu) | ((h[i] >> 2) & 0x30303030u);
        }
    }
    DEV static void scales(const Raw& r, int u, float (&s)[4]) {
        int hh = (u >> 1) & 1, is = u & 1;
        uint32_t D0 = hh ? r.sc.z : r.sc.x, D1 = hh ? r.sc.w : r.sc.y;
        int sh = 8 * is;
        s[0] = (float)(int8_t)(D0 >> sh);
        s[1] = (float)(int8_t)(D0 >> (sh + 16));
        s[2] = (float)(int8_t)(D1 >> sh);
        s[3] = (float)(int8_t)(D1 >> (sh + 16));
    }
    DEV static float dot(const Raw& r, const Xf& f, int u) {
        uint32_t q[4][4];
        q6(r, q);
        float s[4];
        scales(r, u, s);
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float p = dot16_u8(q[g], f.v[g]);
            acc = fmaf(s[g], fmaf(-32.f, f.s[g], p), acc);
        }
        return h2f(r.d) * acc;
    }
    DEV static void dequant(const Raw& r, int u, uint16_t* out) {
        uint32_t q[4][4];
        q6(r, q);
        float s[4];
        scales(r, u, s);
        float d = h2f(r.d);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float ds = d * s[g];  // exact: 11-bit x 8-bit
            uint32_t o[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v0 = ds * (float)((int)((q[g][i]) & 0xff) - 32);
                float v1 = ds * (float)((int)((q[g][i] >> 8) & 0xff) - 32);
                float v2 = ds * (float)((int)((q[g][i] >> 16) & 0xff) - 32);
                float v3 = ds * (float)((int)((q[g][i] >> 24) & 0xff) - 32);
                o[2 * i] = f2h(v0) | (f2h(v1) << 16);
                o[2 * i + 1] = f2h(v2) | (f2h(v3) << 16);
            }
            uint4* p = reinterpret_cast<uint4*>(out + 32 * g);
            p[0] = make_uint4(o[0], o[1], o[2], o[3]);
            p[1] = make_uint4(o[4], o[5], o[6], o[7]);
        }
    }
    DEV static int out_elem(int u) { return elem0(u); }
};

// ------------------------------------------------------ reductions (wave64)

// sum over aligned groups of `width` lanes (width a power of two <= 64);
// every lane of the group ends with the group total
DEV float group_sum(float v, int width) {
    // within rows of 16 lanes: DPP quad/row permutes
    if (width >= 2) v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
    if (width >= 4) v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));  // quad_perm [2,3,0,1]
    if (width >= 8) v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false)); // row_half_mirror
    if (width >= 16) v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false)); // row_mirror
    if (width >= 32) v += __shfl_xor(v, 16, 64);
    if (width >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// ------------------------------------------------------------ GEMV kernel
//
// y[row] = epilogue( sum_k W[row,k] x[k] ), rows in [0, n).
// PAIR = 0: mode 0 -> y = dot (+bias); mode 1 -> y = y + dot (+bias).
// PAIR = 1: SwiGLU pair, wa = gate rows, wb = up rows (same shape),
//           y = silu(g + bias_a) * (u + bias_b)    (src/kernels.cu:516-537).
// Group g of the workgroup (LPR lanes) owns rows [row0, row0 + R).
template <typename F, int R, int ACT, int PAIR>
__device__ void gemv_body(const void* __restrict__ x, const uint8_t* __restrict__ wa,
                          const uint8_t* __restrict__ wb, const void* __restrict__ bias_a,
                          const void* __restrict__ bias_b, void* __restrict__ y, int n, int k,
                          int mode, int lpr_shift) {
    constexpr int S = PAIR ? 2 * R : R;  // weight row streams per lane
    __shared__ float red[4][S * 4];       // cross-wave partials (LPR > 64)
    const int tid = threadIdx.x;
    const int lpr = 1 << lpr_shift;
    const int g = tid >> lpr_shift, li = tid & (lpr - 1);
    const int groups = 256 >> lpr_shift;
    const int row0 = (blockIdx.x * groups + g) * R;
    const int U = k / F::UE;
    const size_t row_bytes = (size_t)(k / F::BE) * F::BB;

    const uint8_t* rp[S];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int rr = min(row0 + r, n - 1);  // tail rows re-read the last row; not written
        rp[r] = wa + (size_t)rr * row_bytes;
        if constexpr (PAIR) rp[R + r] = wb + (size_t)rr * row_bytes;
    }
    float acc[S];
#pragma unroll
    for (int s = 0; s < S; s++) acc[s] = 0.f;

    for (int u = li; u < U; u += lpr) {
        typename F::Raw raw[S];
#pragma unroll
        for (int s = 0; s < S; s++) raw[s] = F::load(rp[s], u);
        typename F::Xf xf;
        F::template loadx<ACT>(x, u, xf);
#pragma unroll
        for (int s = 0; s < S; s++) acc[s] += F::dot(raw[s], xf, u);
    }

    // reduce over the LPR lanes of the group
    const int width = lpr < 64 ? lpr : 64;
#pragma unroll
    for (int s = 0; s < S; s++) acc[s] = group_sum(acc[s], width);
    if (lpr > 64) {
        const int wave = tid >> 6, lane = tid & 63;
        if (lane < S) {
            float v = 0.f;
#pragma unroll
            for (int s = 0; s < S; s++) v = (lane == s) ? acc[s] : v;
            red[wave][lane] = v;
        }
        __syncthreads();
        const int waves_per_group = lpr >> 6;
        const int w0 = (tid >> lpr_shift) * waves_per_group;
#pragma unroll
        for (int s = 0; s < S; s++) {
            float v = 0.f;
            for (int i = 0; i < waves_per_group; i++) v += red[w0 + i][s];
            acc[s] = v;
        }
    }

    // epilogue: lane r of the group writes row row0 + r
    if (li < R) {
        const int row = row0 + li;
        if (row < n) {
            float v = 0.f, v2 = 0.f;
#pragma unroll
            for (int r = 0; r < R; r++) {
                v = (li == r) ? acc[r] : v;
                if constexpr (PAIR) v2 = (li == r) ? acc[R + r] : v2;
            }
            if constexpr (ACT == ACT_F32) {
                float* yo = static_cast<float*>(y);
                if constexpr (PAIR) {
                    if (bias_a) v += static_cast<const float*>(bias_a)[row];
                    if (bias_b) v2 += static_cast<const float*>(bias_b)[row];
                    yo[row] = (v / (1.0f + __expf(-v))) * v2;
                } else {
                    if (bias_a) v += static_cast<const float*>(bias_a)[row];
                    if (mode == 1) v += yo[row];
                    yo[row] = v;
                }
            } else {
                uint16_t* yo = static_cast<uint16_t*>(y);
                if constexpr (PAIR) {
                    if (bias_a) v += h2f(static_cast<const uint16_t*>(bias_a)[row]);
                    if (bias_b) v2 += h2f(static_cast<const uint16_t*>(bias_b)[row]);
                    yo[row] = (uint16_t)f2h((v / (1.0f + __expf(-v))) * v2);
                } else {
                    if (bias_a) v += h2f(static_cast<const uint16_t*>(bias_a)[row]);
                    if (mode == 1) v += h2f(yo[row]);
                    yo[row] = (uint16_t)f2h(v);
                }
            }
        }
    }
}

#define GEMV_KERNEL(NAME, F, R, ACT, PAIR)                                                       \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                      \
        const void* x, const uint8_t* wa, const uint8_t* wb, const void* bias_a,                 \
        const void* bias_b, void* y, int n, int k, int mode, int lpr_shift) {                    \
        gemv_body<F, R, ACT, PAIR>(x, wa, wb, bias_a, bias_b, y, n, k, mode, lpr_shift);         \
    }

#define GEMV_ACT(FN, F, R)                                  \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_f32, F, R, ACT_F32, 0) \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_f16, F, R, ACT_F16, 0) \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_f32_pair, F, R, ACT_F32, 1) \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_f16_pair, F, R, ACT_F16, 1)

#define GEMV_FMT(FN, F) GEMV_ACT(FN, F, 1) GEMV_ACT(FN, F, 2) GEMV_ACT(FN, F, 4) GEMV_ACT(FN, F, 8)

GEMV_FMT(q8_0, FQ8_0)
GEMV_FMT(q4_0, FQ4_0)
GEMV_FMT(q4_k, FQ4_K)
GEMV_FMT(q6_k, FQ6_K)

// --------------------------------------------------------- dequant / gather
// One thread per unit.  dequant: units of a flat run of nblocks blocks,
// f16 out in element order.  gather: out[i, :] = dequant(table[ids[i]]).

template <typename F>
__device__ void dequant_body(const uint8_t* __restrict__ src, uint16_t* __restrict__ out, long long nblocks) {
    long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long units = nblocks * F::UPB;
    if (t >= units) return;
    long long blk = t / F::UPB;
    int u = (int)(t % F::UPB);
    typename F::Raw r = F::load(src + blk * F::BB, u);
    F::dequant(r, u, out + blk * F::BE + F::out_elem(u));
}

template <typename F>
__device__ void gather_body(const uint8_t* __restrict__ table, const uint32_t* __restrict__ ids,
                            uint16_t* __restrict__ out, int n, int hidden) {
    long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int upr = hidden / F::UE;  // units per row
    if (t >= (long long)n * upr) return;
    int i = (int)(t / upr), u = (int)(t % upr);
    const size_t row_bytes = (size_t)(hidden / F::BE) * F::BB;
    typename F::Raw r = F::load(table + (size_t)ids[i] * row_bytes, u);
    F::dequant(r, u, out + (size_t)i * hidden + F::out_elem(u));
}

#define DQ_KERNELS(FN, F)                                                                         \
    extern "C" __global__ __launch_bounds__(256) void cima_dequant_##FN(                          \
        const uint8_t* src, uint16_t* out, long long nblocks) {                                   \
        dequant_body<F>(src, out, nblocks);                                                       \
    }                                                                                             \
    extern "C" __global__ __launch_bounds__(256) void cima_gather_##FN(                           \
        const uint8_t* table, const uint32_t* ids, uint16_t* out, int n, int hidden) {            \
        gather_body<F>(table, ids, out, n, hidden);                                               \
    }

DQ_KERNELS(q8_0, FQ8_0)
DQ_KERNELS(q4_0, FQ4_0)
DQ_KERNELS(q4_k, FQ4_K)
DQ_KERNELS(q6_k, FQ6_K)
