// Fused GGUF dequant-GEMV for gfx950 (CDNA4), compiled once per format set
// into the code objects cima_gemv_a/b/c.hsaco, loaded by the host library
// with hipModuleLoad and launched with hipModuleLaunchKernel.  Counterpart
// of the reference's k_gguf_<fmt>_gemv + GEMV_TAIL (src/kernels.cu:
// 1057-1313) and of the f16 GEMV's epilogue modes (src/kernels.cu:493-538),
// for the nine GGUF block formats, weights kept in their block layout.
//
// Kernel names: cima_gemv_<fmt>_r<R>_i<ITERS>_<f32|f16>[_ring|_ringl][_pair|_att|_amax][_epi]
//   R      rows per lane group, ITERS unit steps per row and lane
//   f32/16 activation, bias and output type
//   _pair  SwiGLU over a gate and an up weight
//   _att   x merged from split-attention partials (o projection)
//   _amax  outputs also reduced into a greedy argmax (head)
//   _ring  item-ring main loop (deeper prefetch; tall one-unit-row matrices)
//   _ringl stepped item ring (long rows: several steps of ITERS units per row)
//   _epi   bias and/or residual (mode 1) operands present
// Every variant can take an RMSNorm prologue (GemvExt::norm_w).
#include <type_traits>

#include "gguf_formats.h"

// ------------------------------------------------------------------ GEMV
//
// Activations.  Every workgroup stages x once in LDS as 16-bit fixed point
// per 32-element block b:  x ~= s_b * (256*hi + lo),  hi, lo in int8,
// s_b = amax_b / 32639 (so |hi| <= 127).  The per-element error is at most
// s_b/2 = amax_b/65278 -- about 1.5e-5 of the block's largest |x|, against
// the 1e-3 output tolerance -- and it replaces nothing the weights carry:
// weight quants are used exactly, so the kernel computes W . x^ for the
// staged x^ up to fp32 rounding.  (The reference's device GEMV quantises x
// to 8 bits, src/kernels.cu:1039-1055.)  Per-16-element sums of x^ are
// staged alongside for the formats' offset / min terms.
//
// Weights.  Quants are unpacked to bytes in the dword order of the elements
// and dotted four at a time with v_dot4_i32_i8 against the hi and lo planes:
// integer sums are exact, then scaled once per block in fp32.  This is ~1.3
// VALU ops per weight for Q4_K, low enough that the kernel stays HBM-bound.
//
// LDS layout of the x planes: 16-element chunks of 32 bytes (16 hi bytes,
// then 16 lo bytes), with 16 bytes of padding after every 2^PADSH elements
// so lanes reading consecutive units fall in different banks.

DEV int dot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

template <int PADSH>
DEV int chunk_off(int c) { return c * 32 + 16 * (c >> (PADSH - 4)); }

// hi and lo dwords of 16-element chunk c
template <int PADSH>
DEV void lds_chunk(const uint8_t* xq, int c, uint32_t* h, uint32_t* l) {
    const uint4* p = reinterpret_cast<const uint4*>(xq + chunk_off<PADSH>(c));
    uint4 a = p[0], b = p[1];
    h[0] = a.x; h[1] = a.y; h[2] = a.z; h[3] = a.w;
    l[0] = b.x; l[1] = b.y; l[2] = b.z; l[3] = b.w;
}

// 256 * hi-plane sum + lo-plane sum, converted once
DEV float fix16(int sh, int sl) { return (float)((sh << 8) + sl); }

// Q8_0 unit = 1 block (32 weights): signed quants dot signed planes.
struct IQ8_0 {
    static constexpr int BE = 32, BB = 34, UE = 32, PADSH = 5;
    using Raw = FQ8_0::Raw;
    struct Xf { uint32_t h[8], l[8]; float s; };
    DEV static Raw load(const uint8_t* row, int u) { return FQ8_0::load(row, u); }
    DEV static void loadx(const uint8_t* xq, const float* xs, const float*, int u, Xf& f) {
        lds_chunk<PADSH>(xq, 2 * u, f.h, f.l);
        lds_chunk<PADSH>(xq, 2 * u + 1, f.h + 4, f.l + 4);
        f.s = xs[u];
    }
    DEV static float dot(const Raw& r, const Xf& f, int) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        int sh = 0, sl = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sh = dot4(w[i], f.h[i], sh);
            sl = dot4(w[i], f.l[i], sl);
        }
        return (h2f(r.d) * f.s) * fix16(sh, sl);
    }
};

// Q4_0 unit = 1 block: byte j -> element j (low nibble), j+16 (high);
// sum (n-8) x = sum n x - 8 sum x.
struct IQ4_0 {
    static constexpr int BE = 32, BB = 18, UE = 32, PADSH = 5;
    using Raw = FQ4_0::Raw;
    struct Xf { uint32_t h[8], l[8]; float s, sum; };
    DEV static Raw load(const uint8_t* row, int u) { return FQ4_0::load(row, u); }
    DEV static void loadx(const uint8_t* xq, const float* xs, const float* xsum, int u, Xf& f) {
        lds_chunk<PADSH>(xq, 2 * u, f.h, f.l);
        lds_chunk<PADSH>(xq, 2 * u + 1, f.h + 4, f.l + 4);
        f.s = xs[u];
        f.sum = xsum[2 * u] + xsum[2 * u + 1];
    }
    DEV static float dot(const Raw& r, const Xf& f, int) {
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        int sh = 0, sl = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
            sh = dot4(lo, f.h[i], sh);
            sl = dot4(lo, f.l[i], sl);
            sh = dot4(hi, f.h[4 + i], sh);
            sl = dot4(hi, f.l[4 + i], sl);
        }
        return h2f(r.d) * fmaf(f.s, fix16(sh, sl), -8.f * f.sum);
    }
};

// Q4_1 unit = 1 block: sum (d q + m) x = d sum q x + m sum x.
struct IQ4_1 {
    static constexpr int BE = 32, BB = 20, UE = 32, PADSH = 5;
    using Raw = FQ4_1::Raw;
    using Xf = IQ4_0::Xf;
    DEV static Raw load(const uint8_t* row, int u) { return FQ4_1::load(row, u); }
    DEV static void loadx(const uint8_t* xq, const float* xs, const float* xsum, int u, Xf& f) {
        IQ4_0::loadx(xq, xs, xsum, u, f);
    }
    DEV static float dot(const Raw& r, const Xf& f, int) {
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        int sh = 0, sl = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
            sh = dot4(lo, f.h[i], sh);
            sl = dot4(lo, f.l[i], sl);
            sh = dot4(hi, f.h[4 + i], sh);
            sl = dot4(hi, f.l[4 + i], sl);
        }
        return fmaf(h2f(r.dm & 0xffffu) * f.s, fix16(sh, sl), h2f(r.dm >> 16) * f.sum);
    }
};

// Q5_0 / Q5_1 unit = 1 block: the 5-bit quants (0..31) dot x;
// Q5_0: d (sum q5 x - 16 sum x), Q5_1: d sum q5 x + m sum x.
template <bool MIN>
struct IQ5_01 {
    static constexpr int BE = 32, BB = MIN ? 24 : 22, UE = 32, PADSH = 5;
    using FQ = typename std::conditional<MIN, FQ5_1, FQ5_0>::type;
    using Raw = typename FQ::Raw;
    using Xf = IQ4_0::Xf;
    DEV static Raw load(const uint8_t* row, int u) { return FQ::load(row, u); }
    DEV static void loadx(const uint8_t* xq, const float* xs, const float* xsum, int u, Xf& f) {
        IQ4_0::loadx(xq, xs, xsum, u, f);
    }
    DEV static float dot(const Raw& r, const Xf& f, int) {
        uint32_t v[8];
        FQ5_0::q5(r.q, r.qh, v);
        int sh = 0, sl = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sh = dot4(v[i], f.h[i], sh);
            sl = dot4(v[i], f.l[i], sl);
        }
        if constexpr (MIN) {
            return fmaf(h2f(r.dm & 0xffffu) * f.s, fix16(sh, sl), h2f(r.dm >> 16) * f.sum);
        } else {
            return h2f(r.d) * fmaf(f.s, fix16(sh, sl), -16.f * f.sum);
        }
    }
};
using IQ5_0 = IQ5_01<false>;
using IQ5_1 = IQ5_01<true>;

// Q4_K unit = one 64-element chunk c of a super-block: 32 qs bytes whose low
// nibbles are sub-block 2c and high nibbles sub-block 2c+1, plus the header.
struct IQ4_K {
    static constexpr int BE = 256, BB = 144, UE = 64, PADSH = 6;
    struct Raw { uint4 h, q0, q1; };
    struct Xf { uint32_t h[16], l[16]; float s0, s1, sum0, sum1; };
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 2) * 144;
        Raw r;
        r.h = ld16a(blk);
        r.q0 = ld16a(blk + 16 + (u & 3) * 32);
        r.q1 = ld16a(blk + 32 + (u & 3) * 32);
        return r;
    }
    DEV static void loadx(const uint8_t* xq, const float* xs, const float* xsum, int u, Xf& f) {
#pragma unroll
        for (int i = 0; i < 4; i++) lds_chunk<PADSH>(xq, 4 * u + i, f.h + 4 * i, f.l + 4 * i);
        f.s0 = xs[2 * u];
        f.s1 = xs[2 * u + 1];
        f.sum0 = xsum[4 * u] + xsum[4 * u + 1];
        f.sum1 = xsum[4 * u + 2] + xsum[4 * u + 3];
    }
    DEV static float dot(const Raw& r, const Xf& f, int u) {
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        int h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
            h0 = dot4(lo, f.h[i], h0);
            l0 = dot4(lo, f.l[i], l0);
            h1 = dot4(hi, f.h[8 + i], h1);
            l1 = dot4(hi, f.l[8 + i], l1);
        }
        uint32_t sc, m;
        q4k_scale_pair(r.h, q4k_sel(u & 3), sc, m);
        const float d = h2f(r.h.x & 0xffffu), dmin = h2f(r.h.x >> 16);
        const float pos = fmaf((float)(sc & 0xff) * f.s0, fix16(h0, l0), ((float)((sc >> 8) & 0xff) * f.s1) * fix16(h1, l1));
        const float neg = fmaf((float)(m & 0xff), f.sum0, (float)((m >> 8) & 0xff) * f.sum1);
        return fmaf(d, pos, -dmin * neg);
    }
};

// Q5_K unit = IQ4_K's 64-element chunk, each quant lifted by its 5th bit
// (bits 2c / 2c+1 of the 32 qh bytes).
struct IQ5_K {
    static constexpr int BE = 256, BB = 176, UE = 64, PADSH = 6;
    struct Raw { uint4 h, q0, q1, qh0, qh1; };
    using Xf = IQ4_K::Xf;
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 2) * 176;
        Raw r;
        r.h = ld16a(blk);
        r.qh0 = ld16a(blk + 16);
        r.qh1 = ld16a(blk + 32);
        r.q0 = ld16a(blk + 48 + (u & 3) * 32);
        r.q1 = ld16a(blk + 64 + (u & 3) * 32);
        return r;
    }
    DEV static void loadx(const uint8_t* xq, const float* xs, const float* xsum, int u, Xf& f) {
        IQ4_K::loadx(xq, xs, xsum, u, f);
    }
    DEV static float dot(const Raw& r, const Xf& f, int u) {
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t qh[8] = {r.qh0.x, r.qh0.y, r.qh0.z, r.qh0.w, r.qh1.x, r.qh1.y, r.qh1.z, r.qh1.w};
        const int c = u & 3;
        int h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (((qh[i] >> (2 * c)) & 0x01010101u) << 4);
            const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            h0 = dot4(lo, f.h[i], h0);
            l0 = dot4(lo, f.l[i], l0);
            h1 = dot4(hi, f.h[8 + i], h1);
            l1 = dot4(hi, f.l[8 + i], l1);
        }
        uint32_t sc, m;
        q4k_scale_pair(r.h, q4k_sel(c), sc, m);
        const float d = h2f(r.h.x & 0xffffu), dmin = h2f(r.h.x >> 16);
        const float pos = fmaf((float)(sc & 0xff) * f.s0, fix16(h0, l0), ((float)((sc >> 8) & 0xff) * f.s1) * fix16(h1, l1));
        const float neg = fmaf((float)(m & 0xff), f.sum0, (float)((m >> 8) & 0xff) * f.sum1);
        return fmaf(d, pos, -dmin * neg);
    }
};

// IQ4_XS unit = 64 elements = sub-blocks 2(u%4), 2(u%4)+1: 32 qs bytes
// (each sub-block's low nibbles then high nibbles in element order) as
// codebook int8 values dot x, times the sub-block scales d (ls - 32).
struct IIQ4_XS {
    static constexpr int BE = 256, BB = 136, UE = 64, PADSH = 6;
    struct Raw { uint4 q0, q1; uint2 hdr; };
    using Xf = IQ4_K::Xf;
    DEV static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 2) * 136;
        Raw r;
        r.hdr = *reinterpret_cast<const uint2*>(blk);
        r.q0 = ld16u(blk + 8 + (u & 3) * 32);
        r.q1 = ld16u(blk + 24 + (u & 3) * 32);
        return r;
    }
    DEV static void loadx(const uint8_t* xq, const float* xs, const float* xsum, int u, Xf& f) {
        IQ4_K::loadx(xq, xs, xsum, u, f);
    }
    DEV static float dot(const Raw& r, const Xf& f, int u) {
        // x chunks 4u..4u+3 = sub-block A low, A high, B low, B high
        const uint32_t a[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w}, b[4] = {r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        int h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t al = iq4nl_bytes(a[i] & 0x0F0F0F0Fu), ah = iq4nl_bytes((a[i] >> 4) & 0x0F0F0F0Fu);
            const uint32_t bl = iq4nl_bytes(b[i] & 0x0F0F0F0Fu), bh = iq4nl_bytes((b[i] >> 4) & 0x0F0F0F0Fu);
            h0 = dot4(al, f.h[i], h0);
            l0 = dot4(al, f.l[i], l0);
            h0 = dot4(ah, f.h[4 + i], h0);
            l0 = dot4(ah, f.l[4 + i], l0);
            h1 = dot4(bl, f.h[8 + i], h1);
            l1 = dot4(bl, f.l[8 + i], l1);
            h1 = dot4(bh, f.h[12 + i], h1);
            l1 = dot4(bh, f.l[12 + i], l1);
        }
        const int ib = 2 * (u & 3);
        return fmaf(iq4xs_dl(r.hdr, ib) * f.s0, fix16(h0, l0), (iq4xs_dl(r.hdr, ib + 1) * f.s1) * fix16(h1, l1));
    }
};

// Q6_K unit = (super-block, half, 16-element l range): four 16-element
// groups, each exactly one x chunk; sum (q6-32) x = sum q6 x - 32 sum x.
struct IQ6_K {
    static constexpr int BE = 256, BB = 210, UE = 64, PADSH = 6;
    using Raw = FQ6_K::Raw;
    struct Xf { uint32_t h[16], l[16]; float s[4], sum[4]; };
    DEV static Raw load(const uint8_t* row, int u) { return FQ6_K::load(row, u); }
    DEV static void loadx(const uint8_t* xq, const float* xs, const float* xsum, int u, Xf& f) {
        const int c0 = FQ6_K::elem0(u) >> 4;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            lds_chunk<PADSH>(xq, c0 + 2 * g, f.h + 4 * g, f.l + 4 * g);
            f.s[g] = xs[(c0 + 2 * g) >> 1];
            f.sum[g] = xsum[c0 + 2 * g];
        }
    }
    DEV static float dot(const Raw& r, const Xf& f, int u) {
        uint32_t q[4][4];
        FQ6_K::q6(r, q);
        float sc[4];
        FQ6_K::scales(r, u, sc);
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int sh = 0, sl = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sh = dot4(q[g][i], f.h[4 * g + i], sh);
                sl = dot4(q[g][i], f.l[4 * g + i], sl);
            }
            acc = fmaf(sc[g], fmaf(f.s[g], fix16(sh, sl), -32.f * f.sum[g]), acc);
        }
        return h2f(r.d) * acc;
    }
};

// ------------------------------------------------- direct-to-LDS copies
//
// dma16: every lane copies the 16 bytes at its global address g into LDS at
// byte lds + 16 * lane (global_load_lds_dwordx4, gfx950; m0 holds the
// wave-uniform LDS address).  Written in asm so that the compiler's wait
// counting leaves these copies alone; their waits are explicit (wait_vm).
DEV void dma16(const void* g, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
// wait until at most N vector memory operations of this wave are in flight
template <int N>
DEV void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// plain loads in asm, for the same reason: 16 bytes, 4 bytes, 2 bytes
// (zero-extended); their registers must pass through tie16 / tie32 after
// the wait_vm that covers them and before any use
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
DEV uint4 ld16_asm(const void* p) {
    v4u32 r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return __builtin_bit_cast(uint4, r);
}
DEV uint32_t ld32_asm(const void* p) {
    uint32_t r;
    asm volatile("global_load_dword %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}
DEV uint32_t ld16b_asm(const void* p) {
    uint32_t r;
    asm volatile("global_load_ushort %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}
DEV void tie16(uint4& v) {
    v4u32 r = __builtin_bit_cast(v4u32, v);
    asm volatile("" : "+v"(r));
    v = __builtin_bit_cast(uint4, r);
}
DEV void tie32(uint32_t& v) { asm volatile("" : "+v"(v)); }
// the 32-bit LDS address of a generic pointer into LDS (the low half of
// its flat address: the shared aperture is 4 GiB aligned)
DEV uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)p; }


// Workgroup shape: one persistent workgroup of GNW waves per CU (a single
// dispatch wave of workgroups across the chip; x is staged once per CU).
#ifndef CIMA_GEMV_WAVES
#define CIMA_GEMV_WAVES 4
#endif
constexpr int GNW = CIMA_GEMV_WAVES;
constexpr int GNT = 64 * GNW;

// Item-ring depth: row groups in flight per lane for items of one unit of
// one weight stream, and for items of two (two units, or the gate|up pair).
// The one-unit item ring (RING 1) keeps three: measured on MI355X, cold,
// one workgroup per CU, depth 4 -> 3: Q4_K 14336x4096 8.21 -> 7.96 us,
// 4096x4096 5.04 -> 4.61, 6144x4096 5.60 -> 5.27, Q5_K 14336x4096 10.12 ->
// 9.19, Q6_K 11.82 -> 10.78 (2: 10.41), IQ4_XS 10.79 -> 9.83; the Q6_K
// head unchanged.  More bytes in flight per CU only queue behind HBM and
// leave more items to compute after the last one lands.  The stepped ring
// keeps three (at two workgroups per CU, measured on MI355X, 4096x14336,
// cold, against four at one: Q8_0 17.05 -> 16.72 us, Q4_0 11.45 -> 11.07,
// Q4_1 10.74 -> 10.26, Q5_0 12.89 -> 12.40, Q5_1 12.02 -> 11.49); the wave
// k-split keeps four.
#ifndef CIMA_RING_DEPTH
#define CIMA_RING_DEPTH 4
#endif
#ifndef CIMA_RING_DEPTH_STEP
#define CIMA_RING_DEPTH_STEP 3
#endif
#ifndef CIMA_RING_DEPTH_ITEM
#define CIMA_RING_DEPTH_ITEM 3
#endif
#ifndef CIMA_RING_DEPTH_PAIR
#define CIMA_RING_DEPTH_PAIR 2
#endif
// Extra items of the item ring's first issue, in flight while x is fetched
// and staged (see RING 1).  Measured on MI355X, cold, bit-identical
// results, one extra against none: Q4_K 14336x4096 7.99 -> 7.80 us,
// 4096x4096 4.58 -> 4.39, 6144x4096 5.28 -> 5.06, Q8_0 4096x4096 6.51 ->
// 6.24, the Q4_K gate+up pair and Q6_K unchanged; two or three extra were
// slower than none (Q4_K 14336x4096 8.25 / 8.39).
#ifndef CIMA_RING_BURST
#define CIMA_RING_BURST 1
#endif

// sum over the workgroup (every thread calls it; all get the total)
DEV float block_sum(float v) {
    __shared__ float red[GNW];
    v = wave_sum_u(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < GNW; w++) t += red[w];
    return t;
}

// LDS bytes the GEMV stages for a row length k (x planes + padding, the
// per-32 scales, the per-16 sums)
template <int PADSH>
constexpr int xstage_bytes(int k) { return 2 * k + 16 * (k >> PADSH) + 4 * (k >> 5) + 4 * (k >> 4); }

template <int ACT>
DEV void load16(const void* __restrict__ x, int c, float v[16]) {
    if constexpr (ACT == ACT_F32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + 16 * c);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 t = p[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + 16 * c);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            uint4 t = p[i];
            const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[8 * i + 2 * j] = h2f(w[j] & 0xffffu);
                v[8 * i + 2 * j + 1] = h2f(w[j] >> 16);
            }
        }
    }
}

// |v| clamped to 65000 (k_rmsnorm's g_sat16, src/kernels.cu:30-35); NaN
// becomes a finite value as with CUDA's fminf/fmaxf
DEV float sat16(float v) { return fmaxf(fminf(v, 65000.f), -65000.f); }

// Optional RMSNorm prologue (k_rmsnorm, src/kernels.cu:37-50): with norm_w
// set, the GEMV multiplies W by h = f16(sat(x) * rsqrt(mean(sat(x)^2) + eps)
// * norm_w) instead of x -- h is rounded to f16 (f32 activations: kept in
// fp32) as the reference's separate rmsnorm launch writes it (stage_x).

// x staging.  Thread t owns 16-element chunks t + GNT j (j < XB); their raw
// loads are issued together before the GEMV's first weight rows, so x and
// weights arrive in one round trip, and held in registers through the
// RMSNorm reduction.  XB is
// sized to the row length the kernel variant is built for (ITERS units of
// every one of up to 64 lanes), so one batch covers x.
template <int ACT, int XB>
struct XBatch {
    static constexpr int U = ACT == ACT_F32 ? 4 : 2;  // uint4 per chunk
    // f16 rows of up to 2 x 4096 elements also hold the RMSNorm weights, so
    // they too are loaded ahead of the weight rows (longer or f32 rows load
    // them while staging, after the weight rows are issued)
    static constexpr bool G = ACT == ACT_F16 && XB <= 2;
    uint4 u[XB][U];
    uint4 g[G ? XB : 1][U];
    DEV void load(const void* __restrict__ x, int nck, const void* __restrict__ nw = nullptr, int c0 = 0) {
#pragma unroll
        for (int j = 0; j < XB; j++) {
            const int c = min(c0 + (int)threadIdx.x + GNT * j, nck - 1);
            const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(x) + (size_t)c * 16 * U);
#pragma unroll
            for (int i = 0; i < U; i++) u[j][i] = p[i];
        }
        if constexpr (G) {
            if (nw) {
#pragma unroll
                for (int j = 0; j < XB; j++) {
                    const int c = min((int)threadIdx.x + GNT * j, nck - 1);
                    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(nw) + (size_t)c * 16 * U);
#pragma unroll
                    for (int i = 0; i < U; i++) g[j][i] = p[i];
                }
            }
        }
    }
    // The same loads issued in asm, for the direct-to-LDS loop: the
    // compiler neither counts nor waits for them, so its own waits cannot
    // drain the weight copies issued after them; wait_asm<N> waits for
    // them explicitly (N = vector memory operations issued since) and hands
    // the registers back to the compiler as defined at that point.
    DEV void load_asm(const void* __restrict__ x, int nck, const void* __restrict__ nw) {
#pragma unroll
        for (int j = 0; j < XB; j++) {
            const int c = min((int)threadIdx.x + GNT * j, nck - 1);
            const uint8_t* p = static_cast<const uint8_t*>(x) + (size_t)c * 16 * U;
#pragma unroll
            for (int i = 0; i < U; i++) u[j][i] = ld16_asm(p + 16 * i);
        }
        if constexpr (G) {
            if (nw) {
#pragma unroll
                for (int j = 0; j < XB; j++) {
                    const int c = min((int)threadIdx.x + GNT * j, nck - 1);
                    const uint8_t* p = static_cast<const uint8_t*>(nw) + (size_t)c * 16 * U;
#pragma unroll
                    for (int i = 0; i < U; i++) g[j][i] = ld16_asm(p + 16 * i);
                }
            }
        }
    }
    template <int N>
    DEV void wait_asm() {
        wait_vm<N>();
#pragma unroll
        for (int j = 0; j < XB; j++)
#pragma unroll
            for (int i = 0; i < U; i++) {
                tie16(u[j][i]);
                if constexpr (G) tie16(g[j][i]);
            }
    }
    // norm weights of chunk j (c = threadIdx.x + GNT j)
    DEV void get_norm(const void* __restrict__ nw, int j, int c, float v[16]) const {
        if constexpr (G) {
#pragma unroll
            for (int i = 0; i < U; i++) unpack(g[j][i], v + 8 * i);
        } else {
            load16<ACT>(nw, c, v);
        }
    }
    DEV void get(int j, float v[16]) const {
#pragma unroll
        for (int i = 0; i < U; i++) unpack(u[j][i], v + (16 / U) * i);
    }
    // one uint4 -> 4 fp32 or 8 f16 values
    DEV static void unpack(uint4 q, float* v) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if constexpr (ACT == ACT_F32) {
                v[e] = __builtin_bit_cast(float, w[e]);
            } else {
                v[2 * e] = h2f(w[e] & 0xffffu);
                v[2 * e + 1] = h2f(w[e] >> 16);
            }
        }
    }
};

// one chunk -> LDS: 16-bit fixed point split into hi / lo byte planes with
// the 32-element block's scale; the two chunks of a block sit in
// neighbouring lanes, which exchange their |x| maxima with one DPP quad
// permute (both lanes run this, `ok` only gates the stores)
template <int PADSH>
DEV void quant_chunk(const float v[16], int c, bool ok, uint8_t* xq, float* xs, float* xsum) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, amax), 0xB1, 0xf, 0xf, false)));
    // qinv by the hardware reciprocal (1 ulp): any qinv with |v| qinv <=
    // 32767 quantises correctly against `scale`; a correctly rounded
    // division costs ten instructions more per chunk
    const float qinv = amax > 0.f ? 32639.f * __builtin_amdgcn_rcpf(amax) : 0.f;
    const float scale = amax * (1.0f / 32639.f);
    // q = rint(v * qinv) by the float rounding of v * qinv + 1.5 * 2^23 in
    // one fused multiply-add (|v qinv| < 2^15, so the sum rounds to an
    // integer, to nearest even); the extra +128 makes the two low bytes of
    // the sum's bits those of q' = q + 128.  With q = 256 hi + lo, lo in
    // [-128, 127]: lo = byte0(q') ^ 0x80 and hi = byte1(q') (two's
    // complement).
    constexpr float kMagic = 12582912.0f + 128.0f;
    constexpr uint32_t kMagicBits = 0x4B400080u;
    uint32_t b[16];
    uint32_t bsum = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        b[i] = __builtin_bit_cast(uint32_t, __builtin_fmaf(v[i], qinv, kMagic));
        bsum += b[i];
    }
    const int qsum = (int)(bsum - 16u * kMagicBits);
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // byte 1 of b[4i..4i+3] -> hw[i]; byte 0 -> lw[i]
        const uint32_t h01 = __builtin_amdgcn_perm(b[4 * i + 1], b[4 * i], 0x0c0c0501u);
        const uint32_t h23 = __builtin_amdgcn_perm(b[4 * i + 3], b[4 * i + 2], 0x05010c0cu);
        const uint32_t l01 = __builtin_amdgcn_perm(b[4 * i + 1], b[4 * i], 0x0c0c0400u);
        const uint32_t l23 = __builtin_amdgcn_perm(b[4 * i + 3], b[4 * i + 2], 0x04000c0cu);
        hw[i] = h01 | h23;
        lw[i] = (l01 | l23) ^ 0x80808080u;
    }
    if (ok) {
        uint4* dst = reinterpret_cast<uint4*>(xq + chunk_off<PADSH>(c));
        dst[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        dst[1] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        // the sum of the staged (quantised) x, so offset and min terms act
        // on exactly the activations the dot products see
        xsum[c] = scale * (float)qsum;
        if ((c & 1) == 0) xs[c >> 1] = scale;
    }
}

// x -> LDS from the batch already in flight in `xb`, which covers the
// whole row: the variant serves rows of at most 64 lanes x ITERS units, and
// XB is sized for that, so staging is one straight pass (no loop-carried
// registers, which would make the compiler copy the weight registers still
// in flight and wait for them).  With norm_w, x is first replaced by its
// RMSNorm (sum of squares from the registers).
template <int ACT, int XB, int PADSH>
DEV void stage_x(const void* __restrict__ x, int k, XBatch<ACT, XB>& xb, uint8_t* xq, float* xs, float* xsum,
                 const void* __restrict__ norm_w, float eps) {
    const int nck = k >> 4;  // <= GNT * XB
    const int t = threadIdx.x;
    float inv = 1.f;
    if (norm_w) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < XB; j++) {
            float v[16];
            xb.get(j, v);
            float sj = 0.f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float sv = sat16(v[i]);
                sj += sv * sv;
            }
            ss += t + GNT * j < nck ? sj : 0.f;
        }
        inv = 1.0f / sqrtf(block_sum(ss) / (float)k + eps);
    }
#pragma unroll
    for (int j = 0; j < XB; j++) {
        const int c = t + GNT * j;
        float v[16];
        xb.get(j, v);
        if (norm_w) {
            float g[16];
            xb.get_norm(norm_w, j, min(c, nck - 1), g);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float h = sat16(v[i]) * inv * g[i];
                if constexpr (ACT == ACT_F32) v[i] = h;
                else v[i] = h2f(f2h(h));
            }
        }
        quant_chunk<PADSH>(v, c, c < nck, xq, xs, xsum);
    }
    __syncthreads();
}

// x -> LDS for rows of any length in batches of XB chunks per thread (the
// direct-to-LDS loop, whose row length is not fixed at compile time).  The
// first batch is already in flight in `xb`; a row of one batch is staged
// by stage_x.  Longer rows load batch after batch (x is a few KB, read by
// every workgroup, so the later batches come from L2); with norm_w the
// first pass sums the squares and the second re-reads x.
template <int ACT, int XB, int PADSH>
DEV void stage_x_loop(const void* __restrict__ x, int k, XBatch<ACT, XB>& xb, uint8_t* xq, float* xs, float* xsum,
                      const void* __restrict__ norm_w, float eps) {
    const int nck = k >> 4;
    constexpr int PER = GNT * XB;  // chunks per batch
    const int nb = (nck + PER - 1) / PER;
    if (nb == 1) {
        stage_x<ACT, XB, PADSH>(x, k, xb, xq, xs, xsum, norm_w, eps);
        return;
    }
    const int t = threadIdx.x;
    float inv = 1.f;
    if (norm_w) {
        float ss = 0.f;
        for (int b = 0; b < nb; b++) {
            if (b > 0) xb.load(x, nck, nullptr, b * PER);
#pragma unroll
            for (int j = 0; j < XB; j++) {
                float v[16];
                xb.get(j, v);
                float sj = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float sv = sat16(v[i]);
                    sj += sv * sv;
                }
                ss += b * PER + t + GNT * j < nck ? sj : 0.f;
            }
        }
        inv = 1.0f / sqrtf(block_sum(ss) / (float)k + eps);
    }
    for (int b = 0; b < nb; b++) {
        if (b > 0 || norm_w) xb.load(x, nck, nullptr, b * PER);
#pragma unroll
        for (int j = 0; j < XB; j++) {
            const int c = b * PER + t + GNT * j;
            float v[16];
            xb.get(j, v);
            if (norm_w) {
                float g[16];
                load16<ACT>(norm_w, min(c, nck - 1), g);
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float h = sat16(v[i]) * inv * g[i];
                    if constexpr (ACT == ACT_F32) v[i] = h;
                    else v[i] = h2f(f2h(h));
                }
            }
            quant_chunk<PADSH>(v, c, c < nck, xq, xs, xsum);
        }
    }
    __syncthreads();
}


// Optional operands of the fused prologues and epilogues, passed by value.
struct GemvExt {
    const void* norm_w;        // RMSNorm prologue weight, or null
    float eps;
    int att_chunks;            // attention-merge x source: chunks per head,
    int att_csz;               //   positions per chunk,
    int att_dim;               //   head dim,
    int max_seq;               //   cache length,
    const int* pos_dev;        //   current position (live length *pos_dev + 1)
    unsigned long long* slot;  // argmax epilogue target
    int att_window;            //   sliding window (> 0: the last att_window positions)
};

// Attention-merge x source: x[h*D + d] = f16(sum_c e^(m_c - M) acc_c[d] /
// sum_c e^(m_c - M) l_c) over the live chunks c of head h, M = max_c m_c,
// from split attention partials part[(h * chunks + c) * (D + 2)] = {m, l,
// acc[D]} -- the two passes of k_attn_reduce (src/kernels.cu:614-639), done
// by every workgroup of the o-projection that consumes it, into LDS `xt`
// (fp32).  Four neighbouring lanes share a 16-element x chunk, each taking
// every fourth partial: the maximum is combined across the four first, then
// each lane's weighted sums, which are independent per chunk, and the four
// lanes' sums add up (DPP).
//
// Each lane's first ATT_ML (m, l) pairs and ATT_PRE partial rows (chunks
// sub, sub + 4, ...) are loaded before the position is read -- their
// addresses do not depend on it -- so the merge costs one memory round trip
// up to 4 ATT_PRE live chunks; further chunks are walked after.  Chunks
// past the live length or wholly before the window are skipped, never
// multiplied (they may hold anything).  ATT_PRE = 4 covers the 16 chunks of
// 128 positions at context 2048 in that one round trip (measured on MI355X,
// config 5: 1535 / 1542 -> 1548 / 1560 tok/s against 3 rows, 1543 with 5).
constexpr int ATT_PRE = 4;
constexpr int ATT_ML = 8;

DEV void stage_attn(const float* __restrict__ part, int k, const GemvExt& ext, float* xt) {
    const int D = ext.att_dim, nch = ext.att_chunks, csz = ext.att_csz;
    for (int idx = threadIdx.x; idx < (k >> 2); idx += GNT) {
        const int e0 = (idx >> 2) * 16, sub = idx & 3;
        const int h = e0 / D, d0 = e0 - h * D;
        const float* ph = part + (size_t)h * nch * (D + 2);
        float2 pml[ATT_ML];
#pragma unroll
        for (int j = 0; j < ATT_ML; j++)
            pml[j] = *reinterpret_cast<const float2*>(ph + (size_t)min(sub + 4 * j, nch - 1) * (D + 2));
        float pb[ATT_PRE][16];
#pragma unroll
        for (int j = 0; j < ATT_PRE; j++) {
            const float* pc = ph + (size_t)min(sub + 4 * j, nch - 1) * (D + 2);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float2 v = reinterpret_cast<const float2*>(pc + 2 + d0)[i];
                pb[j][2 * i] = v.x;
                pb[j][2 * i + 1] = v.y;
            }
        }
        const int seq = min(*ext.pos_dev + 1, ext.max_seq);
        const int wlo = (ext.att_window > 0 && seq > ext.att_window) ? seq - ext.att_window : 0;
        const int active = min((seq + csz - 1) / csz, nch), c0 = wlo / csz;
        const int first = c0 + ((sub - c0) & 3);  // this lane's first live-range chunk
        // pass 1: the head's maximum
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < ATT_ML; j++) {
            const int c = sub + 4 * j;
            if (c >= c0 && c < active) M = fmaxf(M, pml[j].x);
        }
        for (int c = max(sub + 4 * ATT_ML, first); c < active; c += 4) M = fmaxf(M, ph[(size_t)c * (D + 2)]);
        M = fmaxf(M, dpp_xor1(M));
        M = fmaxf(M, dpp_xor2(M));
        // pass 2: the weighted sums
        float L = 0.f, a[16];
#pragma unroll
        for (int i = 0; i < 16; i++) a[i] = 0.f;
#pragma unroll
        for (int j = 0; j < ATT_PRE; j++) {
            const int c = sub + 4 * j;
            if (c >= c0 && c < active) {
                const float w = __expf(pml[j].x - M);
                L += w * pml[j].y;
#pragma unroll
                for (int i = 0; i < 16; i++) a[i] += w * pb[j][i];
            }
        }
        for (int c = max(sub + 4 * ATT_PRE, first); c < active; c += 4) {
            const float* pc = ph + (size_t)c * (D + 2);
            const float2 ml = *reinterpret_cast<const float2*>(pc);
            const float w = __expf(ml.x - M);
            L += w * ml.y;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float2 v = reinterpret_cast<const float2*>(pc + 2 + d0)[i];
                a[2 * i] += w * v.x;
                a[2 * i + 1] += w * v.y;
            }
        }
        L += dpp_xor1(L);
        L += dpp_xor2(L);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            a[i] += dpp_xor1(a[i]);
            a[i] += dpp_xor2(a[i]);
        }
        if (sub == 0) {
#pragma unroll
            for (int i = 0; i < 16; i++) xt[e0 + i] = h2f(f2h(a[i] / L));
        }
    }
    __syncthreads();
}

// packed argmax key of an f16 value at index i: orderable f32 bits << 32 | i
// (k_argmax_softcap without softcap, src/kernels.cu:244-262)
DEV unsigned long long argmax_key(uint32_t h16, int i) {
    uint32_t b = __builtin_bit_cast(uint32_t, h2f(h16));
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (uint32_t)i;
}
DEV unsigned long long umax64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

// y[row] = epilogue(W[row,:] . x), rows in [0, n).
// PAIR = 0: mode 0 -> y = dot (+bias); mode 1 -> y += dot (+bias).
// PAIR = 1: wa = gate rows, wb = up rows; y = silu(g + bias_a) * (u + bias_b)
//           (the semantics of k_gemv_f16 mode 2, src/kernels.cu:516-537).
//
// Lanes are split into groups of LPR (16..64, within one wave).  A group
// owns R consecutive rows at a time (a "row group"); lane li of the group
// takes units li + j*LPR, j < ITERS, of every row (ITERS = ceil(units /
// LPR), a compile-time constant, so a row's loads are one straight block).
// Row groups are interleaved over the groups so the grid sweeps the weight
// front to back; each group loads its next row group's weights before
// computing the current one.  Loads are never predicated (a group's extra
// step re-loads its own last row group, a cache hit), so the compiler can
// wait for exactly one row group's loads at a time.  With ITERS == 1 a lane's x
// fragment never changes and stays in registers for the whole kernel.
template <int ACT>
DEV float load_act(const void* p, int i) {
    if constexpr (ACT == ACT_F32) return static_cast<const float*>(p)[i];
    else return h2f(static_cast<const uint16_t*>(p)[i]);
}

// XS = 1: x is split-attention partials (stage_attn); AMAX = 1: the f16
// outputs also feed a greedy argmax into *ext.slot (one u64 atomic max per
// workgroup).
template <typename F, int R, int ITERS, int ACT, int PAIR, int EPI, int XS, int AMAX, int RING, int LPRS = 6,
          int DD = 1>
__device__ void gemv_body(const void* __restrict__ x, const uint8_t* __restrict__ wa,
                          const uint8_t* __restrict__ wb, const void* __restrict__ bias_a,
                          const void* __restrict__ bias_b, void* __restrict__ y, int n, int k,
                          int mode, int lpr_shift, const GemvExt& ext) {
    extern __shared__ __align__(16) uint8_t lds[];
    // every kernel argument into SGPRs up front: one wait on the kernarg
    // segment instead of one per first use, ahead of the first loads
    asm volatile("" ::"s"(x), "s"(wa), "s"(wb), "s"(bias_a), "s"(bias_b), "s"(y), "s"(n), "s"(k), "s"(mode),
                 "s"(lpr_shift), "s"(ext.norm_w), "s"(ext.pos_dev));
    constexpr int S = PAIR ? 2 * R : R;  // weight row streams per lane
    uint8_t* xq = lds;
    float* xs = reinterpret_cast<float*>(lds + 2 * k + 16 * (k >> F::PADSH));
    float* xsum = xs + (k >> 5);

    // the wave index as a scalar, so row and address arithmetic that only
    // depends on it stays on the scalar unit
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & ((1 << lpr_shift) - 1);
    const int gpw = 64 >> lpr_shift;  // groups per wave
    const int U = k / F::UE;
    const int nrg = (n + R - 1) / R;
    // row groups are interleaved over the groups (group gid takes gid,
    // gid + ngroups, ...), so at any moment the whole grid streams one
    // contiguous window of the weight; every wave runs `per` steps (the
    // count of its first group) and a group's extra step re-loads (and does
    // not write) its own last row group
    const int ngroups = gridDim.x * GNW * gpw;
    const int gid = (blockIdx.x * GNW + wave) * gpw + (lane >> lpr_shift);
    const int gid0 = (blockIdx.x * GNW + wave) * gpw;
    // row groups of this wave's first group (the loop count) and of this
    // lane's group (which rows it writes): two integer divisions, computed
    // only once the first loads are in flight (past a row group's last
    // step a group re-loads a clamped row, which it never uses)
    int per = 0, cnt = 0;
    auto counts = [&]() {
        per = gid0 < nrg ? (nrg - 1 - gid0) / ngroups + 1 : 0;
        cnt = gid < nrg ? (nrg - 1 - gid) / ngroups + 1 : 0;
    };
    const size_t row_bytes = (size_t)(k / F::BE) * F::BB;

    // this lane's units (clamped; `uok` masks the tail lanes)
    int uu[ITERS];
    bool uok[ITERS];
#pragma unroll
    for (int j = 0; j < ITERS; j++) {
        const int u = li + (j << lpr_shift);
        uok[j] = u < U;
        uu[j] = min(u, U - 1);
    }

    // epilogue operands (EPI variants only): e1 = bias_a[row]; e2 =
    // bias_b[row] (pair) or the old y[row] (mode 1).  Absent ones read x[0]
    // and are ignored.
    const bool has1 = EPI && bias_a != nullptr;
    const bool has2 = EPI && (PAIR ? (bias_b != nullptr) : (mode == 1));
    const void* p1 = has1 ? bias_a : x;
    const void* p2 = has2 ? (PAIR ? bias_b : static_cast<const void*>(y)) : x;

    // x chunks per thread for the longest row this variant serves (ITERS
    // units of 64 lanes; 8 for the stepped item ring): k / 16 / GNT
    constexpr int XB = RING >= 3 ? 2 : ((RING == 2 ? 8 : ITERS) * F::UE * 4 + GNT - 1) / GNT;
    // x -> LDS; the caller has the first weights in flight (and, for plain
    // x, x's first batch ahead of them in `xb`)
    auto stage = [&](XBatch<ACT, XB>& xb) {
        if constexpr (XS == 1) {
            float* xt = reinterpret_cast<float*>(lds + ((xstage_bytes<F::PADSH>(k) + 15) & ~15));
            stage_attn(static_cast<const float*>(x), k, ext, xt);
            XBatch<ACT_F32, XB> xa;
            xa.load(xt, k >> 4);
            if constexpr (RING == 3) stage_x_loop<ACT_F32, XB, F::PADSH>(xt, k, xa, xq, xs, xsum, nullptr, 0.f);
            else stage_x<ACT_F32, XB, F::PADSH>(xt, k, xa, xq, xs, xsum, nullptr, 0.f);
        } else if constexpr (RING >= 3) {
            stage_x_loop<ACT, XB, F::PADSH>(x, k, xb, xq, xs, xsum, ext.norm_w, ext.eps);
        } else {
            stage_x<ACT, XB, F::PADSH>(x, k, xb, xq, xs, xsum, ext.norm_w, ext.eps);
        }
    };
    unsigned long long best = 0ull;
    typename F::Xf xreg;

    // reduce a row group's per-lane partial sums over the lane group; its
    // last lane applies the epilogue and writes the R rows of group i
    auto finish = [&](float (&acc)[S], const float* e1, const float* e2, int i) {
#pragma unroll
        for (int s = 0; s < S; s++) acc[s] = group_sum_last(acc[s], 1 << lpr_shift);
        const int rg = gid + i * ngroups;
        if (li == (1 << lpr_shift) - 1 && i < cnt) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = rg * R + r;
                float v = acc[r];
                float out;
                if constexpr (EPI) {
                    if (has1) v += e1[r];
                }
                if constexpr (PAIR) {
                    float v2 = acc[R + r];
                    if constexpr (EPI) {
                        if (has2) v2 += e2[r];
                    }
                    out = (v / (1.0f + __expf(-v))) * v2;
                } else {
                    out = v;
                    if constexpr (EPI) {
                        if (has2) out += e2[r];
                    }
                }
                if (row < n) {
                    if constexpr (ACT == ACT_F32) {
                        static_cast<float*>(y)[row] = out;
                    } else {
                        const uint32_t hb = f2h(out);
                        static_cast<uint16_t*>(y)[row] = (uint16_t)hb;
                        if constexpr (AMAX) best = umax64(best, argmax_key(hb, row));
                    }
                }
            }
        }
    };
    auto epi_load = [&](float* e1, float* e2, int g) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int erow = min(g * R + r, n - 1);
            e1[r] = load_act<ACT>(p1, has1 ? erow : 0);
            e2[r] = load_act<ACT>(p2, has2 ? erow : 0);
        }
    };
    auto wdot = [&](const typename F::Raw& w, const typename F::Xf& xf, int u) -> float {
        return F::dot(w, xf, u);
    };

    if constexpr (RING == 1) {
        // Item ring (single-row rows of one or two units per lane): item q
        // is the lane's q-th row group (its gate and up rows for the pair);
        // DEPTH items are in flight in a ring of slots and the loop body is
        // unrolled over the slots so slot indices are compile-time constants.  Items past the lane's last
        // row group re-load that row group (a cache hit) and write nothing.
        static_assert(ITERS <= 2 && R == 1, "the item ring serves one-row groups of one or two units");
        constexpr int DEPTH = S * ITERS >= 2 ? CIMA_RING_DEPTH_PAIR : CIMA_RING_DEPTH_ITEM;
        struct Item {
            typename F::Raw w[S][ITERS];
            float e1[R], e2[R];
        };
        auto issue = [&](Item& dst, int q) {
            const int g = min(gid + q * ngroups, nrg - 1);
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int row = min(g * R + (s % R), n - 1);
                const uint8_t* rp = ((PAIR && s >= R) ? wb : wa) + (size_t)row * row_bytes;
#pragma unroll
                for (int j = 0; j < ITERS; j++) dst.w[s][j] = F::load(rp, uu[j]);
            }
            if constexpr (EPI) epi_load(dst.e1, dst.e2, g);
        };
        // DEPTH + 1 slots: item q + DEPTH is issued into the slot freed by
        // item q - 1 before item q is computed, so DEPTH items stay in flight
        // while a wave computes (issuing after the compute left DEPTH - 1).
        // With BURST > 0, BURST more items go out with the first ones (while
        // x is fetched and staged) and the first BURST items are computed
        // without issuing, after which DEPTH stay in flight as before.
        constexpr int BURST = CIMA_RING_BURST;
        constexpr int NS = DEPTH + 1 + BURST;
        Item ring[NS];
        XBatch<ACT, XB> xb;
        if constexpr (XS == 0) xb.load(x, k >> 4, ext.norm_w);
#pragma unroll
        for (int d = 0; d < DEPTH + BURST; d++) issue(ring[d], d);
        __builtin_amdgcn_sched_barrier(0);
        counts();
        stage(xb);
        typename F::Xf xr[ITERS];
#pragma unroll
        for (int j = 0; j < ITERS; j++) F::loadx(xq, xs, xsum, uu[j], xr[j]);
        auto compute = [&](const Item& it, int q) {
            float acc[S];
#pragma unroll
            for (int s = 0; s < S; s++) {
                acc[s] = 0.f;
#pragma unroll
                for (int j = 0; j < ITERS; j++) acc[s] += uok[j] ? wdot(it.w[s][j], xr[j], uu[j]) : 0.f;
            }
            finish(acc, it.e1, it.e2, q);
        };
        // the burst's first items (a padding item past the wave's count
        // computes a re-loaded row and writes nothing)
#pragma unroll
        for (int b = 0; b < BURST; b++) compute(ring[b], b);
        // whole rounds of NS items with no condition in the body, then the
        // wave's remaining items
        int base = BURST;
        for (; base + NS <= per; base += NS) {
#pragma unroll
            for (int b = 0; b < NS; b++) {
                issue(ring[(BURST + b + DEPTH) % NS], base + b + DEPTH);
                __builtin_amdgcn_sched_barrier(0);
                compute(ring[(BURST + b) % NS], base + b);
            }
        }
        if constexpr (BURST == 0) {
            // all in flight already; no padding item is waited for
#pragma unroll
            for (int b = 0; b < DEPTH; b++)
                if (base + b < per) compute(ring[b], base + b);
        } else {
            // up to NS - 1 items remain, not all issued yet: issue ahead as
            // in the rounds (padding items past the count re-load a row)
#pragma unroll
            for (int b = 0; b < NS - 1; b++) {
                issue(ring[(BURST + b + DEPTH) % NS], base + b + DEPTH);
                __builtin_amdgcn_sched_barrier(0);
                if (base + b < per) compute(ring[(BURST + b) % NS], base + b);
            }
        }
    } else if constexpr (RING == 2) {
        // Stepped item ring (long rows): a row group takes T steps of ITERS
        // units per lane, and an item is one step of one row group -- the
        // lane's q-th item is step q % T of its (q / T)-th row group.  Items
        // flow through the same ring of DEPTH slots across row-group
        // boundaries; x is read from LDS per item (the units differ per
        // step), the partial sums carry over the steps, and the last step
        // of a row group reduces and writes it.  Items past the lane's last
        // row group re-load it and write nothing.
        static_assert(ITERS <= 2 && R == 1, "the stepped item ring serves one-row groups");
        constexpr int DEPTH = S * ITERS >= 2 ? CIMA_RING_DEPTH_PAIR : CIMA_RING_DEPTH_STEP;
        const int T = (U + (ITERS << lpr_shift) - 1) / (ITERS << lpr_shift);
        int items = 0;  // per * T, once the counts are known
        struct Item {
            typename F::Raw w[S][ITERS];
            float e1[R], e2[R];
        };
        int ii = 0, is = 0;  // next item to load: row group, step
        auto issue = [&](Item& dst) {
            const int g = min(gid + ii * ngroups, nrg - 1);
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int row = min(g * R + (s % R), n - 1);
                const uint8_t* rp = ((PAIR && s >= R) ? wb : wa) + (size_t)row * row_bytes;
#pragma unroll
                for (int j = 0; j < ITERS; j++)
                    dst.w[s][j] = F::load(rp, min(li + ((is * ITERS + j) << lpr_shift), U - 1));
            }
            if constexpr (EPI) epi_load(dst.e1, dst.e2, g);
            if (++is == T) {
                is = 0;
                ++ii;
            }
        };
        int ci = 0, cs = 0;  // next item to compute
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; s++) acc[s] = 0.f;
        auto consume = [&](const Item& src) {
#pragma unroll
            for (int j = 0; j < ITERS; j++) {
                const int u = li + ((cs * ITERS + j) << lpr_shift);
                typename F::Xf xf;
                F::loadx(xq, xs, xsum, min(u, U - 1), xf);
#pragma unroll
                for (int s = 0; s < S; s++) {
                    const float p = wdot(src.w[s][j], xf, min(u, U - 1));
                    acc[s] += u < U ? p : 0.f;
                }
            }
            if (++cs == T) {
                finish(acc, src.e1, src.e2, ci);
#pragma unroll
                for (int s = 0; s < S; s++) acc[s] = 0.f;
                cs = 0;
                ++ci;
            }
        };
        // DEPTH + 1 slots, the next item issued before the current one is
        // consumed (as in the item ring above)
        constexpr int NS = DEPTH + 1;
        Item ring[NS];
        XBatch<ACT, XB> xb;
        if constexpr (XS == 0) xb.load(x, k >> 4, ext.norm_w);
#pragma unroll
        for (int d = 0; d < DEPTH; d++) issue(ring[d]);
        __builtin_amdgcn_sched_barrier(0);
        counts();
        items = per * T;
        stage(xb);
        int base = 0;
        for (; base + NS <= items; base += NS) {
#pragma unroll
            for (int b = 0; b < NS; b++) {
                issue(ring[(b + DEPTH) % NS]);
                __builtin_amdgcn_sched_barrier(0);
                consume(ring[b]);
            }
        }
#pragma unroll
        for (int b = 0; b < DEPTH; b++)
            if (base + b < items) consume(ring[b]);
    } else if constexpr (RING == 4) {
        // k split over the waves of the workgroup, for long rows: the
        // workgroup takes rows blockIdx.x, blockIdx.x + gridDim.x, ...; wave
        // w takes the w-th quarter of every row's units (lane l: units
        // w UQ + l + 64 j, j < ITERS), so each lane's x fragment is fixed
        // for the whole kernel and held in registers, and the four waves
        // stream four neighbouring runs of the same row.  Each wave's
        // partial sum goes to LDS; after every KB rows (one barrier) the
        // first KB threads add the four partials in wave order, apply the
        // epilogue and store -- the partials are double-buffered, so one
        // barrier per batch suffices.  Weights come through an item ring of
        // DEPTH rows as in RING 1.  The epilogue operands of the
        // workgroup's first 64 rows are loaded with x, one per lane.
        static_assert(R == 1 && !PAIR && !AMAX && XS == 0, "k-split rows serve plain and epilogue GEMVs");
        constexpr int DEPTH = CIMA_RING_DEPTH;
        constexpr int KB = 16;  // rows per batch
        const int UQ = (U + GNW - 1) / GNW;
        const int u0 = wave * UQ, u1 = min(u0 + UQ, U);
        int qu[ITERS];
        bool qok[ITERS];
#pragma unroll
        for (int j = 0; j < ITERS; j++) {
            const int u = u0 + lane + 64 * j;
            qok[j] = u < u1;
            qu[j] = min(u, U - 1);
        }
        const int nrow = (int)blockIdx.x < n ? (n - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
        __shared__ float kred[2][KB][GNW];
        struct Item {
            typename F::Raw w[ITERS];
        };
        auto issue = [&](Item& dst, int q) {
            const int row = min((int)blockIdx.x + q * (int)gridDim.x, n - 1);
            const uint8_t* rp = wa + (size_t)row * row_bytes;
#pragma unroll
            for (int j = 0; j < ITERS; j++) dst.w[j] = F::load(rp, qu[j]);
        };
        constexpr int NS = DEPTH + 1;
        Item ring[NS];
        XBatch<ACT, XB> xb;
        xb.load(x, k >> 4, ext.norm_w);
        float ep1 = 0.f, ep2 = 0.f;
        auto epi_load = [&](int b) {  // rows q = 64 b + lane
            const int row = min((int)blockIdx.x + (64 * b + lane) * (int)gridDim.x, n - 1);
            ep1 = load_act<ACT>(p1, has1 ? row : 0);
            ep2 = load_act<ACT>(p2, has2 ? row : 0);
        };
        if constexpr (EPI) epi_load(0);
#pragma unroll
        for (int d = 0; d < DEPTH; d++) issue(ring[d], d);
        __builtin_amdgcn_sched_barrier(0);
        stage(xb);
        typename F::Xf xr[ITERS];
#pragma unroll
        for (int j = 0; j < ITERS; j++) F::loadx(xq, xs, xsum, qu[j], xr[j]);
        // rows [KB bt, KB bt + KB) of batch bt: sum, epilogue, store
        auto finalize = [&](int bt) {
            const int q0 = KB * bt;
            if constexpr (EPI) {
                if ((q0 & 63) == 0 && q0 > 0 && wave == 0) epi_load(q0 >> 6);
            }
            float e1 = 0.f, e2 = 0.f;
            if constexpr (EPI) {
                e1 = __shfl(ep1, (q0 + lane) & 63);
                e2 = __shfl(ep2, (q0 + lane) & 63);
            }
            const int q = q0 + (int)threadIdx.x;
            if (wave == 0 && threadIdx.x < KB && q < nrow) {
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < GNW; w++) v += kred[bt & 1][threadIdx.x][w];
                if constexpr (EPI) {
                    if (has1) v += e1;
                    if (has2) v += e2;
                }
                const int row = (int)blockIdx.x + q * (int)gridDim.x;
                if constexpr (ACT == ACT_F32) static_cast<float*>(y)[row] = v;
                else static_cast<uint16_t*>(y)[row] = (uint16_t)f2h(v);
            }
        };
        auto compute = [&](const Item& it, int q) {
            float p = 0.f;
#pragma unroll
            for (int j = 0; j < ITERS; j++) p += qok[j] ? wdot(it.w[j], xr[j], qu[j]) : 0.f;
            p = group_sum_last(p, 64);
            if (lane == 63) kred[(q / KB) & 1][q % KB][wave] = p;
            if (q % KB == KB - 1 || q == nrow - 1) {
                __syncthreads();
                finalize(q / KB);
            }
        };
        int base = 0;
        for (; base + NS <= nrow; base += NS) {
#pragma unroll
            for (int b = 0; b < NS; b++) {
                issue(ring[(b + DEPTH) % NS], base + b + DEPTH);
                __builtin_amdgcn_sched_barrier(0);
                compute(ring[b], base + b);
            }
        }
#pragma unroll
        for (int b = 0; b < DEPTH; b++)
            if (base + b < nrow) compute(ring[b], base + b);
    } else if constexpr (RING == 3) {
        // Direct-to-LDS row streaming.  An item is one segment of SEGU =
        // LPR * ITERS consecutive units of each of the wave's GPW rows (one
        // row per lane group), for each weight stream.  It is copied from
        // HBM into this wave's slot of LDS with global_load_lds_dwordx4:
        // every instruction moves 64 lanes x 16 B = 1 KB of contiguous
        // weight bytes (the 16-byte lines that hold the segment; lanes past
        // its end repeat its last line, which costs no HBM traffic), so the
        // whole grid reads the weight as fully coalesced 1 KB runs and no
        // VGPRs hold weights in flight.  Lanes then decode their units from
        // LDS (unaligned ds_read_b128 is supported on gfx950) exactly as the
        // register paths decode them from global memory.
        //
        // The copies are issued in inline asm, which the compiler's wait
        // counting does not see: each item waits for its own copies with an
        // explicit vmcnt of the copies issued after it (loads and stores the
        // compiler adds only make that wait stricter).  Every compiler-
        // visible load is therefore issued before the main loop -- x, and
        // the epilogue operands of the wave's first 64 rows, held one row
        // per lane -- so no wait inside the loop drains the copies.
        //
        // Measured on MI355X against the register item ring (Q8_0 14336 x
        // 4096, cold): one item in flight per wave with three workgroups per
        // CU streams the weight at 0.87 of the plain read ceiling.
        static_assert(R == 1, "direct-to-LDS streaming serves one-row groups");
        constexpr int LPR = 1 << LPRS, GPW = 64 / LPR;
        constexpr int SEGU = LPR * ITERS;
        static_assert((SEGU * F::UE) % F::BE == 0, "a segment holds whole blocks");
        constexpr int SEGB = SEGU * F::UE / F::BE * F::BB;   // segment bytes
        constexpr int NPC = (SEGB + 15 + 15) / 16;            // 16-B lines, any start alignment
        constexpr int NCH = (NPC + 63) / 64;                  // copy instructions per row segment
        constexpr int SUB = NCH * 1024;                       // LDS bytes per row segment
        constexpr int SLOT = S * GPW * SUB;                   // LDS bytes per item
        constexpr int NI = S * GPW * NCH;                     // copies per item
        constexpr int D = DD;                                 // items in flight per wave
        const int nseg = (U + SEGU - 1) / SEGU;
        const int g = lane >> LPRS;  // this lane's group in the wave
        // LDS: x staging (and the merge's fp32 x for XS == 1), then one
        // region of D slots per wave
        const unsigned xbytes = XS == 1 ? (((xstage_bytes<F::PADSH>(k) + 15) & ~15) + 4 * k)
                                        : ((xstage_bytes<F::PADSH>(k) + 15) & ~15);
        const unsigned wofs = xbytes + (unsigned)wave * D * SLOT;
        const uint32_t lds_base = lds_addr(lds);
        const uint8_t* wptr[2] = {wa, PAIR ? wb : wa};
        // copies of item q (row group q / nseg, segment q % nseg) into slot d
        int qi = 0, qs = 0;  // next item to issue: row group, segment
        auto issue = [&](int d) {
            const int rg = min(gid0 + qi * ngroups, nrg - 1);
#pragma unroll
            for (int st = 0; st < S; st++) {
#pragma unroll
                for (int gg = 0; gg < GPW; gg++) {
                    const int row = min(rg + gg, n - 1);
                    const size_t seg0 = (size_t)row * row_bytes + (size_t)qs * SEGB;
                    const int len = (int)min((size_t)SEGB, row_bytes - (size_t)qs * SEGB);
                    const uintptr_t start = (uintptr_t)(wptr[st] + seg0);
                    const uintptr_t al = start & ~(uintptr_t)15;
                    const int last = (int)((start - al + len - 1) >> 4);  // last line index
#pragma unroll
                    for (int c = 0; c < NCH; c++) {
                        const int line = min(c * 64 + lane, last);
                        dma16(reinterpret_cast<const void*>(al + 16 * (uintptr_t)line),
                              lds_base + wofs + d * SLOT + (st * GPW + gg) * SUB + c * 1024);
                    }
                }
            }
            if (++qs == nseg) {
                qs = 0;
                ++qi;
            }
        };
        // x (and the RMSNorm weights) and the epilogue operands of the
        // wave's rows j < 64 (row group j / GPW, group j % GPW; one per lane)
        // are loaded first, in asm, then the first items' copies; one
        // explicit wait then covers the former only
        XBatch<ACT, XB> xb;
        if constexpr (XS == 0) xb.load_asm(x, k >> 4, ext.norm_w);
        float ep1 = 0.f, ep2 = 0.f;
        constexpr int IPB = 64 / GPW;  // row groups per epilogue block
        auto epi_row = [&](int b) {
            const int j = b * 64 + lane;
            return min(gid0 + (j % GPW) + (j / GPW) * ngroups, n - 1);
        };
        auto epi_block = [&](int b) {
            const int row = epi_row(b);
            ep1 = load_act<ACT>(p1, has1 ? row : 0);
            ep2 = load_act<ACT>(p2, has2 ? row : 0);
        };
        uint32_t eb1 = 0, eb2 = 0;
        if constexpr (EPI) {
            const int row = epi_row(0);
            constexpr int ES = ACT == ACT_F32 ? 4 : 2;
            const uint8_t* a1 = static_cast<const uint8_t*>(p1) + (size_t)(has1 ? row : 0) * ES;
            const uint8_t* a2 = static_cast<const uint8_t*>(p2) + (size_t)(has2 ? row : 0) * ES;
            if constexpr (ACT == ACT_F32) {
                eb1 = ld32_asm(a1);
                eb2 = ld32_asm(a2);
            } else {
                eb1 = ld16b_asm(a1);
                eb2 = ld16b_asm(a2);
            }
        }
#pragma unroll
        for (int d = 0; d < D; d++) issue(d);
        if constexpr (XS == 0) xb.template wait_asm<D * NI>();
        else wait_vm<D * NI>();
        if constexpr (EPI) {
            tie32(eb1);
            tie32(eb2);
            ep1 = ACT == ACT_F32 ? __builtin_bit_cast(float, eb1) : h2f(eb1);
            ep2 = ACT == ACT_F32 ? __builtin_bit_cast(float, eb2) : h2f(eb2);
        }
        counts();
        stage(xb);
        // x fragments held in registers when a row is one segment
        typename F::Xf xr[ITERS];
        if (nseg == 1) {
#pragma unroll
            for (int j = 0; j < ITERS; j++) F::loadx(xq, xs, xsum, uu[j], xr[j]);
        }
        const int items = per * nseg;
        int ci = 0, cs = 0;  // next item to compute
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; s++) acc[s] = 0.f;
        auto consume = [&](int d, bool xreg_ok) {
            const int rg = gid + ci * ngroups;
            const int row = min(rg, n - 1);
#pragma unroll
            for (int st = 0; st < S; st++) {
                const size_t seg0 = (size_t)row * row_bytes + (size_t)cs * SEGB;
                const int shift = (int)((uintptr_t)(wptr[st] + seg0) & 15);
                const uint8_t* sp = lds + wofs + d * SLOT + (st * GPW + g) * SUB + shift;
#pragma unroll
                for (int j = 0; j < ITERS; j++) {
                    const int ul = li + j * LPR;
                    const int u = cs * SEGU + ul;
                    const bool ok = u < U;
                    const typename F::Raw w = F::load(sp, ok ? ul : 0);
                    float p;
                    if (xreg_ok) {
                        p = wdot(w, xr[j], uu[j]);
                    } else {
                        typename F::Xf xf;
                        F::loadx(xq, xs, xsum, min(u, U - 1), xf);
                        p = wdot(w, xf, min(u, U - 1));
                    }
                    acc[st] += ok ? p : 0.f;
                }
            }
            if (++cs == nseg) {
                float e1[1], e2[1];
                if constexpr (EPI) {
                    const int j = ci * GPW + g;
                    if (ci > 0 && ci % IPB == 0) epi_block(ci / IPB);
                    e1[0] = __shfl(ep1, j & 63);
                    e2[0] = __shfl(ep2, j & 63);
                }
                finish(acc, e1, e2, ci);
#pragma unroll
                for (int s = 0; s < S; s++) acc[s] = 0.f;
                cs = 0;
                ++ci;
            }
        };
        auto run = [&](auto xreg_tag) {
            constexpr bool XR = decltype(xreg_tag)::value;
            int base = 0;
            for (; base + D <= items; base += D) {
#pragma unroll
                for (int d = 0; d < D; d++) {
                    wait_vm<(D - 1) * NI>();
                    consume(d, XR);
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    issue(d);
                }
            }
            wait_vm<0>();
#pragma unroll
            for (int d = 0; d < D; d++)
                if (base + d < items) consume(d, XR);
        };
        if (nseg == 1) run(std::true_type{});
        else run(std::false_type{});
    } else {
        // Row-group double buffer: a lane holds all ITERS units of a row
        // group; the next row group is loaded while the current one is
        // computed.  Loads are never predicated (a group's extra step
        // re-loads its own last row group, a cache hit) and issue/compute
        // alternate unconditionally within whole pairs, so every loop
        // iteration leaves exactly one row group in flight and the loop head
        // needs no drain; an odd count ends with one more compute.
        struct Slot {
            typename F::Raw w[S][ITERS];
            float e1[R], e2[R];
        };
        auto issue = [&](Slot& dst, int i) {
            const int g = min(gid + i * ngroups, nrg - 1);
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int row = min(g * R + (s % R), n - 1);
                const uint8_t* rp = ((PAIR && s >= R) ? wb : wa) + (size_t)row * row_bytes;
#pragma unroll
                for (int j = 0; j < ITERS; j++) dst.w[s][j] = F::load(rp, uu[j]);
            }
            if constexpr (EPI) epi_load(dst.e1, dst.e2, g);
        };
        auto compute = [&](const Slot& cur, int i) {
            float acc[S];
#pragma unroll
            for (int s = 0; s < S; s++) acc[s] = 0.f;
#pragma unroll
            for (int j = 0; j < ITERS; j++) {
                typename F::Xf xl;
                if constexpr (ITERS != 1) F::loadx(xq, xs, xsum, uu[j], xl);
                const typename F::Xf& xf = (ITERS == 1) ? xreg : xl;
#pragma unroll
                for (int s = 0; s < S; s++) {
                    const float p = wdot(cur.w[s][j], xf, uu[j]);
                    acc[s] += uok[j] ? p : 0.f;
                }
            }
            finish(acc, cur.e1, cur.e2, i);
        };
        Slot bufA, bufB;
        XBatch<ACT, XB> xb;
        if constexpr (XS == 0) xb.load(x, k >> 4, ext.norm_w);
        issue(bufA, 0);
        __builtin_amdgcn_sched_barrier(0);
        counts();
        stage(xb);
        if constexpr (ITERS == 1) F::loadx(xq, xs, xsum, uu[0], xreg);
        // whole pairs of row groups, then an odd wave's last one (a padding
        // row group is loaded at most, never waited for)
        int i = 0;
        for (; i + 2 <= per; i += 2) {
            issue(bufB, i + 1);
            compute(bufA, i);
            issue(bufA, i + 2);
            compute(bufB, i + 1);
        }
        if (i < per) compute(bufA, i);
    }
    if constexpr (AMAX) {
        __shared__ unsigned long long red[GNW];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)best, o), hi = __shfl_xor((uint32_t)(best >> 32), o);
            best = umax64(best, ((unsigned long long)hi << 32) | lo);
        }
        if (lane == 0) red[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long m = 0ull;
#pragma unroll
            for (int w = 0; w < GNW; w++) m = umax64(m, red[w]);
            // every workgroup's atomic lands on one word: skip it where the
            // slot already holds a larger key (the slot only grows, so a
            // stale read can only let through an atomic that was not
            // needed, never skip one that was)
            const unsigned long long cur = __hip_atomic_load(ext.slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (m > cur) atomicMax(ext.slot, m);
        }
    }
}

#define GEMV_KERNEL(NAME, F, R, IT, ACT, PAIR, EPI, XS, AMAX, RING)                              \
    extern "C" __global__ __launch_bounds__(GNT) void NAME(                                       \
        const void* x, const uint8_t* wa, const uint8_t* wb, const void* bias_a,                  \
        const void* bias_b, void* y, int n, int k, int mode, int lpr_shift, GemvExt ext) {       \
        gemv_body<F, R, IT, ACT, PAIR, EPI, XS, AMAX, RING>(x, wa, wb, bias_a, bias_b, y, n, k,   \
                                                            mode, lpr_shift, ext);                \
    }

// name: cima_gemv_<fmt>_r<R>_i<ITERS>_<f32|f16>[_pair][_epi]
#define GEMV_EPI(FN, F, R, IT, ACT, AN)                                                               \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_i##IT##_##AN, F, R, IT, ACT, 0, 0, 0, 0, 0)                    \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_i##IT##_##AN##_epi, F, R, IT, ACT, 0, 1, 0, 0, 0)              \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_i##IT##_##AN##_pair, F, R, IT, ACT, 1, 0, 0, 0, 0)             \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_i##IT##_##AN##_pair_epi, F, R, IT, ACT, 1, 1, 0, 0, 0)

// decode-step variants (f16 activations): _att_epi = attention partials as
// x with bias/residual epilogue (the o projection); _amax = outputs also
// reduced into a greedy argmax (the head)
#define GEMV_DECODE(FN, F, R, IT)                                                                     \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_i##IT##_f16_att_epi, F, R, IT, ACT_F16, 0, 1, 1, 0, 0)         \
    GEMV_KERNEL(cima_gemv_##FN##_r##R##_i##IT##_f16_amax, F, R, IT, ACT_F16, 0, 0, 0, 1, 0)

#define GEMV_ACT(FN, F, R, IT) GEMV_EPI(FN, F, R, IT, ACT_F32, f32) GEMV_EPI(FN, F, R, IT, ACT_F16, f16) \
    GEMV_DECODE(FN, F, R, IT)

// item-ring variants (one row, one or two units per lane; large matrices):
// cima_gemv_<fmt>_r1_i<1|2>_<f32|f16>_ring[_pair][_epi], cima_gemv_<fmt>_r1_i<1|2>_f16_ring_amax
// (_pair: an item is one gate row and one up row)
#define GEMV_RING_IT(FN, F, IT)                                                                        \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f32_ring, F, 1, IT, ACT_F32, 0, 0, 0, 0, 1)                  \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f32_ring_epi, F, 1, IT, ACT_F32, 0, 1, 0, 0, 1)              \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ring, F, 1, IT, ACT_F16, 0, 0, 0, 0, 1)                  \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ring_epi, F, 1, IT, ACT_F16, 0, 1, 0, 0, 1)              \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ring_amax, F, 1, IT, ACT_F16, 0, 0, 0, 1, 1)              \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f32_ring_pair, F, 1, IT, ACT_F32, 1, 0, 0, 0, 1)             \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f32_ring_pair_epi, F, 1, IT, ACT_F32, 1, 1, 0, 0, 1)         \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ring_pair, F, 1, IT, ACT_F16, 1, 0, 0, 0, 1)             \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ring_pair_epi, F, 1, IT, ACT_F16, 1, 1, 0, 0, 1)
// stepped item-ring variants (long rows, k up to the i8 kernels'):
// cima_gemv_<fmt>_r1_i<1|2>_<f32|f16>_ringl[_epi]
#define GEMV_RINGL_IT(FN, F, IT)                                                                       \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f32_ringl, F, 1, IT, ACT_F32, 0, 0, 0, 0, 2)                 \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f32_ringl_epi, F, 1, IT, ACT_F32, 0, 1, 0, 0, 2)             \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ringl, F, 1, IT, ACT_F16, 0, 0, 0, 0, 2)                 \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ringl_epi, F, 1, IT, ACT_F16, 0, 1, 0, 0, 2)
#define GEMV_RING(FN, F) GEMV_RING_IT(FN, F, 1) GEMV_RING_IT(FN, F, 2) GEMV_RINGL_IT(FN, F, 1)

// direct-to-LDS streaming variants, lanes per row L = 2^LS fixed at compile time:
// cima_gemv_<fmt>_l<L>_i<IT>_<f32|f16>_dma<D>[_pair][_epi], ..._f16_dma<D>_att_epi, ..._f16_dma<D>_amax
#define GEMV_KERNEL_D(NAME, F, IT, ACT, PAIR, EPI, XS, AMAX, LS, DD)                               \
    extern "C" __global__ __launch_bounds__(GNT) void NAME(                                       \
        const void* x, const uint8_t* wa, const uint8_t* wb, const void* bias_a,                  \
        const void* bias_b, void* y, int n, int k, int mode, int lpr_shift, GemvExt ext) {       \
        gemv_body<F, 1, IT, ACT, PAIR, EPI, XS, AMAX, 3, LS, DD>(x, wa, wb, bias_a, bias_b, y, n, \
                                                                 k, mode, lpr_shift, ext);       \
    }
// name: cima_gemv_<fmt>_l<L>_i<IT>_<act>_dma<D>[...], D items in flight per wave
#define GEMV_DMA_ACT(FN, F, L, LS, IT, ACT, AN, D)                                                             \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_##AN##_dma##D, F, IT, ACT, 0, 0, 0, 0, LS, D)                 \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_##AN##_dma##D##_epi, F, IT, ACT, 0, 1, 0, 0, LS, D)           \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_##AN##_dma##D##_pair, F, IT, ACT, 1, 0, 0, 0, LS, D)          \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_##AN##_dma##D##_pair_epi, F, IT, ACT, 1, 1, 0, 0, LS, D)
#define GEMV_DMA_SHAPE_D(FN, F, L, LS, IT, D)                                                                  \
    GEMV_DMA_ACT(FN, F, L, LS, IT, ACT_F32, f32, D) GEMV_DMA_ACT(FN, F, L, LS, IT, ACT_F16, f16, D)             \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_f16_dma##D##_att_epi, F, IT, ACT_F16, 0, 1, 1, 0, LS, D)      \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_f16_dma##D##_amax, F, IT, ACT_F16, 0, 0, 0, 1, LS, D)
// two items in flight: built for the gate+up pair at every shape and for
// the short-row shapes (16 and 32 lanes, one unit), the cases the host
// picks them for
#define GEMV_DMA_PAIR2(FN, F, L, LS, IT)                                                                       \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_f32_dma2_pair, F, IT, ACT_F32, 1, 0, 0, 0, LS, 2)             \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_f32_dma2_pair_epi, F, IT, ACT_F32, 1, 1, 0, 0, LS, 2)         \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_f16_dma2_pair, F, IT, ACT_F16, 1, 0, 0, 0, LS, 2)             \
    GEMV_KERNEL_D(cima_gemv_##FN##_l##L##_i##IT##_f16_dma2_pair_epi, F, IT, ACT_F16, 1, 1, 0, 0, LS, 2)
// k split over the waves (long rows): cima_gemv_<fmt>_r1_i<1|2>_<f32|f16>_ksplit[_epi]
#define GEMV_KSPLIT_IT(FN, F, IT)                                                                      \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f32_ksplit, F, 1, IT, ACT_F32, 0, 0, 0, 0, 4)               \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f32_ksplit_epi, F, 1, IT, ACT_F32, 0, 1, 0, 0, 4)           \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ksplit, F, 1, IT, ACT_F16, 0, 0, 0, 0, 4)               \
    GEMV_KERNEL(cima_gemv_##FN##_r1_i##IT##_f16_ksplit_epi, F, 1, IT, ACT_F16, 0, 1, 0, 0, 4)
#define GEMV_KSPLIT(FN, F) GEMV_KSPLIT_IT(FN, F, 1) GEMV_KSPLIT_IT(FN, F, 2)

#define GEMV_DMA(FN, F)                                                                                 \
    GEMV_DMA_SHAPE_D(FN, F, 64, 6, 1, 1) GEMV_DMA_SHAPE_D(FN, F, 64, 6, 2, 1) GEMV_DMA_SHAPE_D(FN, F, 32, 5, 1, 1) \
    GEMV_DMA_SHAPE_D(FN, F, 32, 5, 2, 1) GEMV_DMA_SHAPE_D(FN, F, 16, 4, 1, 1)                          \
    GEMV_DMA_SHAPE_D(FN, F, 32, 5, 1, 2) GEMV_DMA_SHAPE_D(FN, F, 16, 4, 1, 2)                          \
    GEMV_DMA_PAIR2(FN, F, 64, 6, 1) GEMV_DMA_PAIR2(FN, F, 64, 6, 2) GEMV_DMA_PAIR2(FN, F, 32, 5, 2)

// (rows, unit steps) shapes: R * ITERS <= 8, R <= 2
#define GEMV_FMT(FN, F)                                                                         \
    GEMV_ACT(FN, F, 1, 1) GEMV_ACT(FN, F, 1, 2) GEMV_ACT(FN, F, 1, 4) GEMV_ACT(FN, F, 1, 8)   \
    GEMV_ACT(FN, F, 2, 1) GEMV_ACT(FN, F, 2, 2) GEMV_ACT(FN, F, 2, 4) GEMV_RING(FN, F) GEMV_DMA(FN, F) \
    GEMV_KSPLIT(FN, F)

// the formats of this code object: the file is compiled once per set (in
// parallel), each set to its own code object
#if !defined(CIMA_GEMV_SET)
#error "CIMA_GEMV_SET (0, 1 or 2) selects the formats of this code object"
#elif CIMA_GEMV_SET == 0
GEMV_FMT(q8_0, IQ8_0)
GEMV_FMT(q4_0, IQ4_0)
GEMV_FMT(q4_k, IQ4_K)
#elif CIMA_GEMV_SET == 1
GEMV_FMT(q6_k, IQ6_K)
GEMV_FMT(q5_k, IQ5_K)
#elif CIMA_GEMV_SET == 3
// no kernels: a translation unit that includes this file instantiates its own
#else
GEMV_FMT(q4_1, IQ4_1)
GEMV_FMT(q5_0, IQ5_0)
GEMV_FMT(q5_1, IQ5_1)
GEMV_FMT(iq4_xs, IIQ4_XS)
#endif

