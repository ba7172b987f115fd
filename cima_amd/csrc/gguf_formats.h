// Shared device code of the GGUF kernels for gfx950 (CDNA4): f16 helpers,
// unaligned loads and the per-format block decoders.  Included by
// gguf_gemv.hip, gguf_gemm.hip and gguf_dequant.hip, each compiled to its
// own code object.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DEV __device__ __forceinline__

enum { GT_Q4_0 = 2, GT_Q4_1 = 3, GT_Q5_0 = 6, GT_Q5_1 = 7, GT_Q8_0 = 8, GT_Q4_K = 12, GT_Q5_K = 13, GT_Q6_K = 14,
       GT_IQ4_XS = 23 };
enum { ACT_F32 = 0, ACT_F16 = 1 };

// ---------------------------------------------------------------- helpers

DEV float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
// fp32 -> f16 bits with v_cvt_f16_f32 (round to nearest even, f16
// subnormals kept).  The empty asm makes `v` opaque: without it LLVM folds
// f16(a * b) into v_fma_mix(a, b, +0), which returns +0 where a * b is -0
// and, for a * b - c, skips the fp32 rounding the host decoders perform.
DEV uint32_t f2h(float v) {
    __asm__("" : "+v"(v));
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
}

// two fp32 -> packed f16 bits (lo in bits 0-15) with one v_cvt_pk_f16_f32
// (round to nearest even, like f2h); the empty asm has f2h's purpose
DEV uint32_t f2h2(float lo, float hi) {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    __asm__("" : "+v"(lo), "+v"(hi));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){lo, hi}, h2_t));
}

// ------------------------------------------------------ reductions (wave64)

// Sum over aligned groups of `width` lanes (16, 32 or 64); the total lands in
// the LAST lane of each group.  Rows of 16 lanes reduce with DPP quad
// permutes and half-row / row mirrors (every lane of the row then holds the
// row sum); row_bcast:15 / row_bcast:31 then fold rows 0->1, 2->3 and 1->3.
template <int CTRL, int ROW_MASK>
DEV float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                     0xf, false));
}
DEV float group_sum_last(float v, int width) {
    v = dpp_add<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
    v = dpp_add<0x140, 0xf>(v);  // row_mirror
    if (width >= 32) v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    if (width >= 64) v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

// DPP lane exchanges inside a quad (lane ^ 1, lane ^ 2)
DEV float dpp_xor1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
}
DEV float dpp_xor2(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
}
// the four 16-lane row values of a wave read into scalars and combined:
// after a row reduction (quad permutes + mirrors) every lane of a row holds
// its row's value, so four readlanes finish a wave reduction without any
// LDS round trip (ds_bpermute)
DEV float rows_sum(float v) {
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}
DEV float rows_max(float v) {
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
template <int CTRL>
DEV float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// wave-uniform sum / max of v over all 64 lanes
DEV float wave_sum_u(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    return rows_sum(v);
}
DEV float wave_max_u(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    return rows_max(v);
}

DEV uint4 ld16a(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
// 2-byte-aligned 16-byte load: gfx950 runs with unaligned global access
// enabled, so this is one global_load_dwordx4 (measured at full streaming
// bandwidth on MI355X), not a byte loop.
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

DEV uint32_t ld4u(const uint8_t* p) {
    uint32_t v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 4);
    return v;
}

// byte B of v as fp32 (v_cvt_f32_ubyte<B>: one instruction, where the
// compiler would extract the byte first)
template <int B>
DEV float ubyte_f32(uint32_t v) {
    float r;
    if constexpr (B == 0) __asm__("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (B == 1) __asm__("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (B == 2) __asm__("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else __asm__("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}
// the four bytes u of v as f16 pairs of s * u + t, each rounded once: with
// s * u exact in fp32 (every format here) this is the host decoders'
// s * u + t -- rounded once to fp32, then to f16 -- where they add a term
// (t: a min or an offset product), signs of zero included
DEV void bytes_affine(uint32_t v, float s, float t, uint32_t& lo, uint32_t& hi) {
    lo = f2h2(__builtin_fmaf(s, ubyte_f32<0>(v), t), __builtin_fmaf(s, ubyte_f32<1>(v), t));
    hi = f2h2(__builtin_fmaf(s, ubyte_f32<2>(v), t), __builtin_fmaf(s, ubyte_f32<3>(v), t));
}

// the four bytes u of v as f16 pairs of s * (u - c): c and u - c exact
// small integers, so this is the host decoders' d * q with its sign of zero
// (an fma of s u - s c would give +0 where d * 0 is -0)
DEV void bytes_scaled(uint32_t v, float s, float c, uint32_t& lo, uint32_t& hi) {
    lo = f2h2(s * (ubyte_f32<0>(v) - c), s * (ubyte_f32<1>(v) - c));
    hi = f2h2(s * (ubyte_f32<2>(v) - c), s * (ubyte_f32<3>(v) - c));
}

// bits 0..3 of b -> bit 4 of bytes 0..3 (the 5th bits of four elements):
// the four shifted copies of b in the product never overlap
DEV uint32_t spread4(uint32_t b) { return ((b * 0x00204081u) & 0x01010101u) << 4; }

// IQ4_XS: the four nibbles (one per byte, 0..15) of n -> their codebook
// values (ggml kvalues_iq4nl, src/quant.rs:817-822) as int8 bytes: two
// byte permutes over the 16-entry table, then a per-byte select on bit 3
DEV uint32_t iq4nl_bytes(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(0xF6EADDCFu, 0xBFAD9881u, sel);  // entries 0..7
    const uint32_t hi = __builtin_amdgcn_perm(0x71594535u, 0x26190D01u, sel);  // entries 8..15
    const uint32_t m = ((n >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}

DEV void store32h(uint16_t* out, const uint32_t (&o)[16]) {
    uint4* p = reinterpret_cast<uint4*>(out);
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

// Decoders of one unit to f16 (dequant and gather).  Each value is computed
// exactly as the host decoder does -- (d*sc)*q [- dmin*m] in fp32, then one
// RTNE conversion to f16 -- so the bits match.

// --------------------------------------------------------- format: Q8_0
// block: f16 d, i8 qs[32]; x[i] = d * qs[i]   (src/quant.rs:599-617)
struct FQ8_0 {
    static constexpr int BE = 32, BB = 34, UE = 32, UPB = 1;
    struct Raw { uint4 a, b; uint32_t d; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 34;
        Raw r;
        r.d = ld2(blk);
        r.a = ld16u(blk + 2);
        r.b = ld16u(blk + 18);
        return r;
    }
    DEV static void dequant(const Raw& r, int, uint16_t* out) {
        float d = h2f(r.d);
        uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        uint32_t o[16];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float v0 = d * (float)(int8_t)(w[i] & 0xff), v1 = d * (float)(int8_t)((w[i] >> 8) & 0xff);
            float v2 = d * (float)(int8_t)((w[i] >> 16) & 0xff), v3 = d * (float)(int8_t)(w[i] >> 24);
            o[2 * i] = f2h2(v0, v1);
            o[2 * i + 1] = f2h2(v2, v3);
        }
        store32h(out, o);
    }
    DEV static int out_elem(int u) { return u * 32; }
};

// --------------------------------------------------------- format: Q4_0
// block: f16 d, u8 qs[16]; byte j = elem j (low nibble), elem j+16 (high);
// x = d * (q - 8)   (src/quant.rs:624-644)
struct FQ4_0 {
    static constexpr int BE = 32, BB = 18, UE = 32, UPB = 1;
    struct Raw { uint4 q; uint32_t d; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 18;
        Raw r;
        r.d = ld2(blk);
        r.q = ld16u(blk + 2);
        return r;
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
                o[2 * i + j] = f2h2(l0, l1);
                o[8 + 2 * i + j] = f2h2(h0, h1);
            }
        }
        store32h(out, o);
    }
    DEV static int out_elem(int u) { return u * 32; }
};

// --------------------------------------------------------- format: Q4_1
// block (20 B): f16 d, f16 m, u8 qs[16]; byte j = elem j (low nibble),
// elem j+16 (high); x = d * q + m   (src/quant.rs:646-669)
struct FQ4_1 {
    static constexpr int BE = 32, BB = 20, UE = 32, UPB = 1;
    struct Raw { uint4 q; uint32_t dm; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 20;
        Raw r;
        r.dm = ld4u(blk);
        r.q = ld16u(blk + 4);
        return r;
    }
    DEV static void dequant(const Raw& r, int, uint16_t* out) {
        const float d = h2f(r.dm & 0xffffu), m = h2f(r.dm >> 16);
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t o[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            bytes_affine(q[i] & 0x0F0F0F0Fu, d, m, o[2 * i], o[2 * i + 1]);
            bytes_affine((q[i] >> 4) & 0x0F0F0F0Fu, d, m, o[8 + 2 * i], o[8 + 2 * i + 1]);
        }
        store32h(out, o);
    }
    DEV static int out_elem(int u) { return u * 32; }
};

// --------------------------------------------------------- format: Q5_0
// block (22 B): f16 d, u32 qh (bit e = element e's 5th bit), u8 qs[16];
// x = d * (q5 - 16)   (src/quant.rs:671-699)
struct FQ5_0 {
    static constexpr int BE = 32, BB = 22, UE = 32, UPB = 1;
    struct Raw { uint4 q; uint32_t d, qh; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 22;
        Raw r;
        r.d = ld2(blk);
        r.qh = ld4u(blk + 2);
        r.q = ld16u(blk + 6);
        return r;
    }
    // the 32 5-bit quants, one per byte in element order (q5[0..3] =
    // elements 0..15, q5[4..7] = 16..31)
    DEV static void q5(uint4 qv, uint32_t qh, uint32_t (&o)[8]) {
        const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[i] = (q[i] & 0x0F0F0F0Fu) | spread4((qh >> (4 * i)) & 15u);
            o[4 + i] = ((q[i] >> 4) & 0x0F0F0F0Fu) | spread4((qh >> (16 + 4 * i)) & 15u);
        }
    }
    DEV static void dequant(const Raw& r, int, uint16_t* out) {
        const float d = h2f(r.d);
        uint32_t v[8], o[16];
        q5(r.q, r.qh, v);
#pragma unroll
        for (int i = 0; i < 8; i++) bytes_scaled(v[i], d, 16.f, o[2 * i], o[2 * i + 1]);
        store32h(out, o);
    }
    DEV static int out_elem(int u) { return u * 32; }
};

// --------------------------------------------------------- format: Q5_1
// block (24 B): f16 d, f16 m, u32 qh, u8 qs[16]; x = d * q5 + m
// (src/quant.rs:701-729)
struct FQ5_1 {
    static constexpr int BE = 32, BB = 24, UE = 32, UPB = 1;
    struct Raw { uint4 q; uint32_t dm, qh; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 24;
        Raw r;
        r.dm = ld4u(blk);
        r.qh = ld4u(blk + 4);
        r.q = ld16u(blk + 8);
        return r;
    }
    DEV static void dequant(const Raw& r, int, uint16_t* out) {
        const float d = h2f(r.dm & 0xffffu), m = h2f(r.dm >> 16);
        uint32_t v[8], o[16];
        FQ5_0::q5(r.q, r.qh, v);
#pragma unroll
        for (int i = 0; i < 8; i++) bytes_affine(v[i], d, m, o[2 * i], o[2 * i + 1]);
        store32h(out, o);
    }
    DEV static int out_elem(int u) { return u * 32; }
};

// (sc, m) of sub-blocks 2c and 2c+1 of a Q4_K super-block from its header
// (dwords y, z, w hold the 12 packed scale bytes), without branches:
//   j < 4 : sc = s[j] & 63,                        m = s[j+4] & 63
//   j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4, m = (s[j+4] >> 4) | (s[j] >> 6) << 4
// (src/quant.rs:731-740)
DEV void q4k_scales(const uint4& h, int c, uint32_t& sc0, uint32_t& m0, uint32_t& sc1, uint32_t& m1) {
    const int t = (c & 1) * 16;
    const uint32_t A = h.y >> t, B = h.z >> t, C = h.w >> t;
    const bool lo = c < 2;
    const uint32_t L = lo ? A : C, M = lo ? B : (C >> 4);
    const uint32_t s6 = lo ? 4 : 6;
    sc0 = (L & 0xF) | (((A >> s6) & 3) << 4);
    sc1 = ((L >> 8) & 0xF) | (((A >> (s6 + 8)) & 3) << 4);
    m0 = (M & 0xF) | (((B >> s6) & 3) << 4);
    m1 = ((M >> 8) & 0xF) | (((B >> (s6 + 8)) & 3) << 4);
}

// The same eight (sc, m) pairs decoded all at once, one per byte, then the
// pair of chunk c picked with one byte permute each (sel = q4k_sel(c)):
// bytes 0,1 of *sc are sc[2c], sc[2c+1]; of *m, m[2c], m[2c+1].
DEV uint32_t q4k_sel(int c) { return (uint32_t)(2 * c) | ((uint32_t)(2 * c + 1) << 8) | 0x0c0c0000u; }
DEV void q4k_scale_pair(const uint4& h, uint32_t sel, uint32_t& sc, uint32_t& m) {
    const uint32_t sclo = h.y & 0x3F3F3F3Fu;
    const uint32_t mlo = h.z & 0x3F3F3F3Fu;
    const uint32_t schi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t mhi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    sc = __builtin_amdgcn_perm(schi, sclo, sel);
    m = __builtin_amdgcn_perm(mhi, mlo, sel);
}

// --------------------------------------------------------- format: Q4_K
// super-block (144 B): f16 d, f16 dmin, u8 scales[12], u8 qs[128].
// 64-element chunk c uses qs[32c..32c+32): low nibbles are sub-block 2c,
// high nibbles sub-block 2c+1; x = (d*sc)*q - dmin*m  (src/quant.rs:743-774).
// Unit u: super-block u/8, qs bytes [16*(u%8), +16) -> chunk c = (u%8)/2,
// elements c*64 + 16*(u%2) + [0,16) (low) and the same +32 (high).
struct FQ4_K {
    static constexpr int BE = 256, BB = 144, UE = 32, UPB = 8;
    struct Raw { uint4 q; uint4 h; };
    DEV static int elem0(int u) { return (u >> 3) * 256 + ((u & 7) >> 1) * 64 + (u & 1) * 16; }
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 144;
        Raw r;
        r.h = ld16a(blk);
        r.q = ld16a(blk + 16 + (u & 7) * 16);
        return r;
    }
    DEV static void dequant(const Raw& r, int u, uint16_t* out) {
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(r.h, (u & 7) >> 1, sc0, m0, sc1, m1);
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
                // fp32 rounding -- identical to the host decoder
                float l0 = d0 * (float)(b0 & 15) - mm0, l1 = d0 * (float)(b1 & 15) - mm0;
                float h0 = d1 * (float)(b0 >> 4) - mm1, h1 = d1 * (float)(b1 >> 4) - mm1;
                ol[2 * i + j] = f2h2(l0, l1);
                oh[2 * i + j] = f2h2(h0, h1);
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

// --------------------------------------------------------- format: Q5_K
// super-block (176 B): f16 d, f16 dmin, u8 scales[12] (as Q4_K), u8 qh[32],
// u8 qs[128] (Q4_K's nibble layout); chunk c's low / high nibbles take bit
// 2c / 2c+1 of qh[l] as +16; x = (d*sc)*q5 - dmin*m  (src/quant.rs:776-815).
// Unit u as FQ4_K's, plus qh bytes [16*(u%2), +16).
struct FQ5_K {
    static constexpr int BE = 256, BB = 176, UE = 32, UPB = 8;
    struct Raw { uint4 h, q, qh; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 176;
        Raw r;
        r.h = ld16a(blk);
        r.qh = ld16a(blk + 16 + (u & 1) * 16);
        r.q = ld16a(blk + 48 + (u & 7) * 16);
        return r;
    }
    DEV static void dequant(const Raw& r, int u, uint16_t* out) {
        const int c = (u & 7) >> 1;
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(r.h, c, sc0, m0, sc1, m1);
        const float d = h2f(r.h.x & 0xffffu), dmin = h2f(r.h.x >> 16);
        const float d0 = d * (float)sc0, mm0 = dmin * (float)m0, d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        const uint32_t h[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        uint32_t ol[8], oh[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (((h[i] >> (2 * c)) & 0x01010101u) << 4);
            const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            // (d*sc)*q5 is exact, so the subtraction is the one fp32 rounding
            bytes_affine(lo, d0, -mm0, ol[2 * i], ol[2 * i + 1]);
            bytes_affine(hi, d1, -mm1, oh[2 * i], oh[2 * i + 1]);
        }
        uint4* pl = reinterpret_cast<uint4*>(out);
        uint4* ph = reinterpret_cast<uint4*>(out + 32);
        pl[0] = make_uint4(ol[0], ol[1], ol[2], ol[3]);
        pl[1] = make_uint4(ol[4], ol[5], ol[6], ol[7]);
        ph[0] = make_uint4(oh[0], oh[1], oh[2], oh[3]);
        ph[1] = make_uint4(oh[4], oh[5], oh[6], oh[7]);
    }
    DEV static int out_elem(int u) { return FQ4_K::elem0(u); }
};

// ------------------------------------------------------- format: IQ4_XS
// super-block (136 B): f16 d, u16 scales_h (2 bits per sub-block), u8
// scales_l[4] (4 bits per sub-block), u8 qs[128]; sub-block ib (32
// elements) = qs[16 ib, +16): low nibbles elements 0..15, high 16..31;
// x = (d (ls - 32)) * codebook[q]   (src/quant.rs:823-854).  Unit u =
// sub-block u % 8 of super-block u / 8.
DEV float iq4xs_dl(uint2 hdr, int ib) {
    const uint32_t ls = ((hdr.y >> (4 * ib)) & 15u) | (((hdr.x >> (16 + 2 * ib)) & 3u) << 4);
    return h2f(hdr.x & 0xffffu) * (float)((int)ls - 32);  // exact: 11-bit x 6-bit
}
struct FIQ4_XS {
    static constexpr int BE = 256, BB = 136, UE = 32, UPB = 8;
    struct Raw { uint4 q; uint2 hdr; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 136;
        Raw r;
        r.hdr = *reinterpret_cast<const uint2*>(blk);
        r.q = ld16u(blk + 8 + (u & 7) * 16);
        return r;
    }
    DEV static void dequant(const Raw& r, int u, uint16_t* out) {
        const float dl = iq4xs_dl(r.hdr, u & 7);
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t o[16];
        // codebook values are int8: v = (v ^ 0x80) - 128 as unsigned bytes
        // (dl v is exact: a 17-bit by 7-bit product)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            bytes_scaled(iq4nl_bytes(q[i] & 0x0F0F0F0Fu) ^ 0x80808080u, dl, 128.f, o[2 * i], o[2 * i + 1]);
            bytes_scaled(iq4nl_bytes((q[i] >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u, dl, 128.f, o[8 + 2 * i],
                         o[8 + 2 * i + 1]);
        }
        store32h(out, o);
    }
    DEV static int out_elem(int u) { return u * 32; }
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
    struct Raw { uint4 a, b, h; uint2 sc; uint32_t d; };
    DEV static int elem0(int u) { return (u >> 2) * 256 + ((u >> 1) & 1) * 128 + (u & 1) * 16; }
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 2) * 210;
        const int hh = (u >> 1) & 1, is = u & 1;
        Raw r;
        r.a = ld16u(blk + hh * 64 + is * 16);
        r.b = ld16u(blk + hh * 64 + 32 + is * 16);
        r.h = ld16u(blk + 128 + hh * 32 + is * 16);
        __builtin_memcpy(&r.sc, __builtin_assume_aligned(blk + 192 + hh * 8, 2), 8);
        r.d = ld2(blk + 208);
        return r;
    }
    // 6-bit quants (0..63) of group g, one per byte in element order
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
    // int8 scales of the unit's four groups: sc[8hh + is + 2g]
    DEV static void scales(const Raw& r, int u, float (&s)[4]) {
        const int sh = 8 * (u & 1);
        s[0] = (float)(int8_t)(r.sc.x >> sh);
        s[1] = (float)(int8_t)(r.sc.x >> (sh + 16));
        s[2] = (float)(int8_t)(r.sc.y >> sh);
        s[3] = (float)(int8_t)(r.sc.y >> (sh + 16));
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
                o[2 * i] = f2h2(v0, v1);
                o[2 * i + 1] = f2h2(v2, v3);
            }
            uint4* p = reinterpret_cast<uint4*>(out + 32 * g);
            p[0] = make_uint4(o[0], o[1], o[2], o[3]);
            p[1] = make_uint4(o[4], o[5], o[6], o[7]);
        }
    }
    DEV static int out_elem(int u) { return elem0(u); }
};

