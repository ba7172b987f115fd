#include <type_traits>

#include "gguf_formats.h"

// ------------------------------------------------------- prefill GEMM (MFMA)
//
// Y[m, n] (row stride ldy) = X[m, k] . W[n, k]^T: X holds m tokens, W is the
// packed GGUF weight (the engine's lin_gemm, src/models/transformer.rs:
// 618-655, which dequantises W to an f16 slab and runs an f16 GEMM).
// Each stage a workgroup dequantises its weight tile to f16 -- bit-exact
// with the host decoders, so the operand equals the reference's
// dequantised weight -- stages the X tile as f16 in LDS (bf16 -> f16 is
// exact for 2^-14 <= |x| < 65520), and multiplies with f16 MFMA, fp32
// accumulation.  LDS is double-buffered; the global loads of the next PF
// stages are in flight in registers while a stage is multiplied.  Three
// kernels: gemm_body_sk16 (16 tokens, four k-splits, weights dequantised
// into the A operand registers, 16x16x32 MFMA), gemm_body_ra (32 or 64 tokens,
// weights into the A operand registers, 32x32x16 MFMA) and
// gemm_body_pipe (128 or 256 tokens, weights through LDS, 32x32x16 MFMA).

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
enum { XT_F32 = 0, XT_F16 = 1, XT_BF16 = 2 };

// 32 contiguous elements [32j, 32j+32) of a row -> f16 bits, 2 per dword,
// the values of the host decoders (formats whose decoders multiply only,
// d * (q - c), use fma(d, q, -c d) here: the same value, though a zero
// weight may come out +0 where the decoder gives -0 -- a difference no
// product sum shows)
struct DQ8_0 {
    static constexpr int BE = 32, BB = 34;
    using Raw = FQ8_0::Raw;
    DEV static Raw load(const uint8_t* row, int j) { return FQ8_0::load(row, j); }
    DEV static void deq(const Raw& r, int, uint32_t (&o)[16]) {
        // q = (q ^ 0x80) - 128 as unsigned bytes: d q = d u - 128 d exactly
        const float d = h2f(r.d);
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) bytes_affine(w[i] ^ 0x80808080u, d, -128.f * d, o[2 * i], o[2 * i + 1]);
    }
};
struct DQ4_0 {
    static constexpr int BE = 32, BB = 18;
    using Raw = FQ4_0::Raw;
    DEV static Raw load(const uint8_t* row, int j) { return FQ4_0::load(row, j); }
    DEV static void deq(const Raw& r, int, uint32_t (&o)[16]) {
        // byte j -> element j (low nibble), j + 16 (high); d (n - 8) exact
        const float d = h2f(r.d);
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            bytes_affine(q[i] & 0x0F0F0F0Fu, d, -8.f * d, o[2 * i], o[2 * i + 1]);
            bytes_affine((q[i] >> 4) & 0x0F0F0F0Fu, d, -8.f * d, o[8 + 2 * i], o[8 + 2 * i + 1]);
        }
    }
};
struct DQ4_1 {
    static constexpr int BE = 32, BB = 20;
    using Raw = FQ4_1::Raw;
    DEV static Raw load(const uint8_t* row, int j) { return FQ4_1::load(row, j); }
    DEV static void deq(const Raw& r, int, uint32_t (&o)[16]) {
        // d q + m: the product is exact, the sum rounded once
        const float d = h2f(r.dm & 0xffffu), m = h2f(r.dm >> 16);
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            bytes_affine(q[i] & 0x0F0F0F0Fu, d, m, o[2 * i], o[2 * i + 1]);
            bytes_affine((q[i] >> 4) & 0x0F0F0F0Fu, d, m, o[8 + 2 * i], o[8 + 2 * i + 1]);
        }
    }
};
template <bool MIN>
struct DQ5_01 {
    static constexpr int BE = 32, BB = MIN ? 24 : 22;
    using FQ = typename std::conditional<MIN, FQ5_1, FQ5_0>::type;
    using Raw = typename FQ::Raw;
    DEV static Raw load(const uint8_t* row, int j) { return FQ::load(row, j); }
    DEV static void deq(const Raw& r, int, uint32_t (&o)[16]) {
        uint32_t v[8];
        FQ5_0::q5(r.q, r.qh, v);
        float d, t;
        if constexpr (MIN) {
            d = h2f(r.dm & 0xffffu);
            t = h2f(r.dm >> 16);   // d q5 + m
        } else {
            d = h2f(r.d);
            t = -16.f * d;         // d (q5 - 16), exact
        }
#pragma unroll
        for (int i = 0; i < 8; i++) bytes_affine(v[i], d, t, o[2 * i], o[2 * i + 1]);
    }
};
// sub-block j: super-block j/8, s = j%8 -> chunk c = s/2 of Q4_K's nibble
// layout (low nibbles if s is even) with 5th bits = bit s of qh[l]
struct DQ5_K {
    static constexpr int BE = 256, BB = 176;
    struct Raw { uint4 h, q0, q1, qh0, qh1; };
    DEV static Raw load(const uint8_t* row, int j) {
        const uint8_t* blk = row + (size_t)(j >> 3) * 176;
        const int c = (j & 7) >> 1;
        Raw r;
        r.h = ld16a(blk);
        r.qh0 = ld16a(blk + 16);
        r.qh1 = ld16a(blk + 32);
        r.q0 = ld16a(blk + 48 + 32 * c);
        r.q1 = ld16a(blk + 64 + 32 * c);
        return r;
    }
    DEV static void deq(const Raw& r, int j, uint32_t (&o)[16]) {
        const int s = j & 7, c = s >> 1;
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(r.h, c, sc0, m0, sc1, m1);
        const bool hi = s & 1;
        const float d = h2f(r.h.x & 0xffffu), dmin = h2f(r.h.x >> 16);
        const float ds = d * (float)(hi ? sc1 : sc0), mm = dmin * (float)(hi ? m1 : m0);
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t h[8] = {r.qh0.x, r.qh0.y, r.qh0.z, r.qh0.w, r.qh1.x, r.qh1.y, r.qh1.z, r.qh1.w};
        const int sh = hi ? 4 : 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t n = ((q[i] >> sh) & 0x0F0F0F0Fu) | (((h[i] >> s) & 0x01010101u) << 4);
            bytes_affine(n, ds, -mm, o[2 * i], o[2 * i + 1]);  // (d sc) q5 exact; one rounding
        }
    }
};
// sub-block j: super-block j/8, ib = j%8: codebook values of qs[16 ib, +16)
struct DIQ4_XS {
    static constexpr int BE = 256, BB = 136;
    using Raw = FIQ4_XS::Raw;
    DEV static Raw load(const uint8_t* row, int j) { return FIQ4_XS::load(row, j); }
    DEV static void deq(const Raw& r, int j, uint32_t (&o)[16]) {
        const float dl = iq4xs_dl(r.hdr, j & 7);
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            bytes_affine(iq4nl_bytes(q[i] & 0x0F0F0F0Fu) ^ 0x80808080u, dl, -128.f * dl, o[2 * i], o[2 * i + 1]);
            bytes_affine(iq4nl_bytes((q[i] >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u, dl, -128.f * dl, o[8 + 2 * i],
                         o[8 + 2 * i + 1]);
        }
    }
};
// sub-block j: super-block j/8, sub s = j%8 -> qs bytes 32*(s/2) + [0,32),
// low nibbles if s is even, high if odd
struct DQ4_K {
    static constexpr int BE = 256, BB = 144;
    struct Raw { uint4 h, q0, q1; };
    DEV static Raw load(const uint8_t* row, int j) {
        const uint8_t* blk = row + (size_t)(j >> 3) * 144;
        const int c = (j & 7) >> 1;
        Raw r;
        r.h = ld16a(blk);
        r.q0 = ld16a(blk + 16 + 32 * c);
        r.q1 = ld16a(blk + 32 + 32 * c);
        return r;
    }
    DEV static void deq(const Raw& r, int j, uint32_t (&o)[16]) {
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(r.h, (j & 7) >> 1, sc0, m0, sc1, m1);
        const bool hi = j & 1;
        const float d = h2f(r.h.x & 0xffffu), dmin = h2f(r.h.x >> 16);
        const float ds = d * (float)(hi ? sc1 : sc0), mm = dmin * (float)(hi ? m1 : m0);
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const int sh = hi ? 4 : 0;
        // (d*sc)*q is exact, so the subtraction is the only fp32 rounding --
        // and a fused multiply-add rounds exactly there too
#pragma unroll
        for (int i = 0; i < 8; i++) bytes_affine((q[i] >> sh) & 0x0F0F0F0Fu, ds, -mm, o[2 * i], o[2 * i + 1]);
    }
};
// sub-block j: super-block j/8, r = j%8 -> half h = r/4, group g = r%4:
// l in [0,32) takes nibble (g<2 low, else high) of ql[64h + 32(g&1) + l],
// bits 2g..2g+1 of qh[32h + l], scale sc[8h + l/16 + 2g]
struct DQ6_K {
    static constexpr int BE = 256, BB = 210;
    struct Raw { uint4 a0, a1, h0, h1; uint32_t sc, d; };
    DEV static Raw load(const uint8_t* row, int j) {
        const uint8_t* blk = row + (size_t)(j >> 3) * 210;
        const int hh = (j & 7) >> 2, g = j & 3;
        Raw r;
        r.a0 = ld16u(blk + 64 * hh + 32 * (g & 1));
        r.a1 = ld16u(blk + 64 * hh + 32 * (g & 1) + 16);
        r.h0 = ld16u(blk + 128 + 32 * hh);
        r.h1 = ld16u(blk + 128 + 32 * hh + 16);
        r.sc = ld2(blk + 192 + 8 * hh + 2 * g);  // sc[8h + 2g], sc[8h + 2g + 1]
        r.d = ld2(blk + 208);
        return r;
    }
    DEV static void deq(const Raw& r, int j, uint32_t (&o)[16]) {
        const int g = j & 3;
        const int nsh = g < 2 ? 0 : 4, hsh = 2 * g;
        const float d = h2f(r.d);
        const float ds0 = d * (float)(int8_t)(r.sc & 0xff), ds1 = d * (float)(int8_t)(r.sc >> 8);
        const uint32_t a[8] = {r.a0.x, r.a0.y, r.a0.z, r.a0.w, r.a1.x, r.a1.y, r.a1.z, r.a1.w};
        const uint32_t h[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
        // ds (u - 32) rounded once, as fma(ds, u, -32 ds) rounds it
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float ds = i < 4 ? ds0 : ds1;
            const uint32_t q = ((a[i] >> nsh) & 0x0F0F0F0Fu) | (((h[i] >> hsh) & 0x03030303u) << 4);
            bytes_affine(q, ds, -32.f * ds, o[2 * i], o[2 * i + 1]);
        }
    }
};

// Per-call operands of formats that need more than the packed weight:
// bitsandbytes 4-bit (absmax per `bsz` elements, the 16-entry codebook).
// The GGUF formats ignore them.
struct GemmExt {
    const float* absmax;
    const float* qmap;
    long long bsz;   // elements per absmax entry
    int bs_shift;    // log2(bsz) when bsz is a power of two, else -1
    unsigned* status;  // X range flags (cima_gemm_status), OR-ed in
    float* part;       // k-split partial tiles, [ksplit][m][n] fp32 (16-token tiles only)
    int ksplit;        // workgroups along k (blockIdx.z); 1 = Y written directly
};

// X range report.  The tiles round X to f16.  That is exact for bf16 values
// of 2^-17 <= |x| < 65536 (and zero); larger ones become +-inf, and smaller
// nonzero ones may lose bits (f16 subnormals step by 2^-24).  f32 X is
// rounded anyway (the 1e-3 bar), but |x| >= 65520 becomes inf too.  Every
// workgroup checks its own 1/(grid size) share of X once (XScan: a few
// 16-byte words per thread, loaded ahead of the first weight stage) and ORs
// flags into a word of this code object, which the host reads back on
// request (cima_hip_gemm_status): bit 0 = values beyond f16's range, or not
// finite; bit 1 = nonzero bf16 values below 2^-17.  The loads go out after
// the main loop, beside the output stores, and are checked last.  Measured
// on MI355X (Q4_K 14336x4096, bf16 X), against no check: +0.8-1.2 / +0.9 /
// +0.5 / +0.5 / +1-2 us at 16 / 32 / 64 / 128 / 512 tokens (1-6 %);
// checked before the main loop instead it cost 1.3-2.6 us at 16-32
// tokens, and inside the tiles' own conversions every stage (+1170 VALU
// instructions in the 256-token tile, 102 -> 150 us at 512 tokens).
__device__ unsigned cima_gemm_status;
struct XRange {
    // one word of flags, two bf16 halves at a time (magnitudes h <= 0x7fff,
    // so the additions below never carry out of a half): bit 15 of a half
    // <- h >= 0x4780 (65536: beyond f16, or inf / NaN); bit 14 <- 0 < h <
    // 0x3700 (below 2^-17); f32: bit 31 <- |x| >= 65520
    uint32_t acc = 0;
    DEV void bf16(uint32_t w) {
        const uint32_t a = w & 0x7fff7fffu;
        acc |= ((a + 0x38803880u) & 0x80008000u) | ((~(a + 0x49004900u) & (a + 0x7fff7fffu) & 0x80008000u) >> 1);
    }
    DEV void f32(uint32_t w) { acc |= ((w & 0x7fffffffu) + 0x38801000u) & 0x80000000u; }
    template <int XT>
    DEV void add(uint4 v) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if constexpr (XT == XT_BF16) bf16(w[i]);
            else f32(w[i]);
        }
    }
    DEV void report(unsigned* st) const {
        const unsigned long long bo = __ballot((acc & 0x80008000u) != 0), bt = __ballot((acc & 0x40004000u) != 0);
        if ((bo | bt) && (threadIdx.x & 63) == 0 && st) atomicOr(st, (bo ? 1u : 0u) | (bt ? 2u : 0u));
    }
};

// This workgroup's share of X for the range check: words [w0, we) of X's
// 16-byte words, thread t taking w0 + t + T j.  issue() loads the first NB
// per thread; finish() checks them (and, for large X, the rest, batch by
// batch) and reports.  Nothing for f16 X.
typedef uint32_t v4u32_t __attribute__((ext_vector_type(4)));
template <int XT, int T>  // T: threads per workgroup (a constant: reading blockDim is a load, and a wait)
struct XScan {
    static constexpr int NB = 4;
    v4u32_t v[XT == XT_F16 ? 1 : NB];
    long long w0 = 0, we = 0;
    bool on = false;
    DEV void issue(const void* x, int m, int k, const unsigned* st) {
        on = st != nullptr;  // uniform: a null status word switches the check off
        if constexpr (XT != XT_F16) {
            if (!on) return;
            const long long nw = (long long)m * k * (XT == XT_F32 ? 4 : 2) / 16;
            const long long nwg = (long long)gridDim.x * gridDim.y * gridDim.z;
            const long long per = (nw + nwg - 1) / nwg;
            w0 = (((long long)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * per;
            we = min(w0 + per, nw);
            const uint4* p = static_cast<const uint4*>(x);
            // Loads in asm: compiled as plain loads, predicated per lane,
            // they are joined with the lanes that load nothing and waited
            // for on the spot; in asm they stay in flight beside the output
            // stores until finish().  Batches the share does not reach
            // are skipped (a uniform branch); lanes past the share repeat
            // the share's last word, which their wave's request coalesces
            // (clamping to one word of X for every workgroup made 448
            // workgroups queue on one L2 line: +2 us at 16 tokens).
            const long long last = max(min(we, nw) - 1, 0LL);
            v[0] = v4u32_t{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < NB; j++) {
                if (w0 + (long long)T * j >= we) break;
                const long long i = min(w0 + threadIdx.x + (long long)T * j, last);
                asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v[j]) : "v"(p + i) : "memory");
            }
        }
    }
    DEV void finish(const void* x, unsigned* st) {
        if constexpr (XT != XT_F16) {
            if (!on) return;
            XRange rg;
            const uint4* p = static_cast<const uint4*>(x);
            // the asm loads above are not counted by the compiler: wait for
            // everything in flight (the tile's first stage, which comes next
            // anyway) and hand the registers back as defined here
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
            for (int j = 0; j < NB; j++) {
                asm volatile("" : "+v"(v[j]));
                if (w0 + threadIdx.x + (long long)T * j < we) rg.add<XT>(__builtin_bit_cast(uint4, v[j]));
            }
            for (long long i = w0 + threadIdx.x + (long long)T * NB; i < we; i += T) rg.add<XT>(p[i]);
            rg.report(st);
        }
    }
};

// The tile bodies call D::ctx / init / load / deq with a per-call context;
// GG adapts the context-free GGUF decoders above.
template <typename DQ>
struct GG {
    static constexpr int BE = DQ::BE, BB = DQ::BB;
    using Raw = typename DQ::Raw;
    struct Ctx {};
    DEV static Ctx ctx(const uint8_t*, const GemmExt&) { return Ctx{}; }
    DEV static void init(const Ctx&) {}
    DEV static Raw load(const Ctx&, const uint8_t* row, int j) { return DQ::load(row, j); }
    DEV static void deq(const Ctx&, const Raw& r, int j, uint32_t (&o)[16]) { DQ::deq(r, j, o); }
};

// bitsandbytes NF4 / FP4 (src/quant.rs:18-70): a row is k/2 packed bytes,
// element 2i in the HIGH nibble of byte i; sub-block j of a row is 16
// bytes, and its 32 elements share one absmax (bsz % 32 == 0, k % 32 ==
// 0, checked on the host).  The value is f16(code[nib] * absmax): one fp32
// product rounded once to nearest even, the decode of dequant_host
// (src/quant.rs:401-437) and k_nf4_dequant (src/kernels.cu:320-329), so the
// MFMA operand equals the reference's decoded f16 weight.  The codebook
// sits in LDS (16 words in 16 banks: lanes never conflict).
struct DNF4 {
    static constexpr int BE = 32, BB = 16;
    struct Raw { uint4 q; float a; };
    struct Ctx {
        const uint8_t* base;
        const float* absmax;
        const float* code;
        long long bsz;
        int bs_shift;
    };
    DEV static Ctx ctx(const uint8_t* w, const GemmExt& e) {
        __shared__ float code[16];
        return Ctx{w, e.absmax, code, e.bsz, e.bs_shift};
    }
    // every thread of the workgroup calls it before its first deq
    DEV static void init(const Ctx& c, const float* qmap) {
        if (threadIdx.x < 16) const_cast<float*>(c.code)[threadIdx.x] = qmap[threadIdx.x];
        __syncthreads();
    }
    DEV static Raw load(const Ctx& c, const uint8_t* row, int j) {
        Raw r;
        r.q = *reinterpret_cast<const uint4*>(row + 16 * j);
        const long long e = (long long)(row - c.base) * 2 + 32 * j;  // flat index of the first element
        r.a = c.absmax[c.bs_shift >= 0 ? (e >> c.bs_shift) : (e / c.bsz)];
        return r;
    }
    DEV static void deq(const Ctx& c, const Raw& r, int, uint32_t (&o)[16]) {
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t byte = (w[i] >> (8 * b)) & 0xFFu;
                o[4 * i + b] = f2h2(c.code[byte >> 4] * r.a, c.code[byte & 0xFu] * r.a);
            }
    }
};

// f16 weights as they stand (a row is k f16 values): the tile bodies as a
// plain f16 GEMM, for bitsandbytes shapes the fused decoder does not take,
// decoded into the caller's slab first
struct DF16 {
    static constexpr int BE = 32, BB = 64;
    struct Raw { uint4 a[4]; };
    struct Ctx {};
    DEV static Ctx ctx(const uint8_t*, const GemmExt&) { return Ctx{}; }
    DEV static void init(const Ctx&) {}
    DEV static Raw load(const Ctx&, const uint8_t* row, int j) {
        Raw r;
        const uint4* p = reinterpret_cast<const uint4*>(row + 64 * j);
#pragma unroll
        for (int i = 0; i < 4; i++) r.a[i] = p[i];
        return r;
    }
    DEV static void deq(const Ctx&, const Raw& r, int, uint32_t (&o)[16]) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[4 * i] = r.a[i].x;
            o[4 * i + 1] = r.a[i].y;
            o[4 * i + 2] = r.a[i].z;
            o[4 * i + 3] = r.a[i].w;
        }
    }
};

// D::init with the codebook for DNF4, nothing for the others
template <typename D>
DEV void fmt_init(const typename D::Ctx& c, const GemmExt& e) {
    if constexpr (std::is_same<D, DNF4>::value) D::init(c, e.qmap);
    else D::init(c);
}

// x tile loads: BN tokens x BK k per stage, as 16-byte words (V elements);
// LR = BK / V lanes cover one token's row, so each load instruction reads
// whole rows, and load i of thread t takes token t / LR + i * 256 / LR at
// k offset (t % LR) V (tokens past m re-read the last one; never stored
// out).  Offsets are 32-bit bytes from the uniform base (the host keeps X
// under 4 GiB).  Words are converted to f16 only when the stage is
// consumed, so the loads stay in flight.
template <int XT, int BN, int BK>
struct XTile {
    static constexpr int ES = XT == XT_F32 ? 4 : 2;   // bytes per element
    static constexpr int V = 16 / ES;                 // elements per load
    static constexpr int LR = BK / V;                 // lanes per token row
    static constexpr int RPI = 256 / LR;              // token rows per load
    static constexpr int NL = BN / RPI;               // loads per thread
    static_assert(NL >= 1 && BN % RPI == 0, "tile too small for 256 threads");
    uint4 r[NL];
    // byte offsets of this thread's words at stage 0 and LDS slots
    struct Map {
        uint32_t off[NL];
        int lds[NL];
    };
    DEV static Map map(int t0, int m, int k, int kp) {
        Map mp;
        const int tid = threadIdx.x, kk = (tid % LR) * V;
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int tok = tid / LR + i * RPI;
            mp.off[i] = (uint32_t)(min(t0 + tok, m - 1) * k + kk) * ES;
            mp.lds[i] = tok * kp + kk;
        }
        return mp;
    }
    DEV void load(const void* x, const Map& mp, uint32_t stage_off) {
        const uint8_t* b = static_cast<const uint8_t*>(x) + stage_off;
#pragma unroll
        for (int i = 0; i < NL; i++) r[i] = *reinterpret_cast<const uint4*>(b + mp.off[i]);
    }
    DEV void store(uint16_t* xl, const Map& mp) const {
#pragma unroll
        for (int i = 0; i < NL; i++) {
            uint16_t* dst = xl + mp.lds[i];
            const uint32_t w[4] = {r[i].x, r[i].y, r[i].z, r[i].w};
            if constexpr (XT == XT_F16) {
                // component-wise: a whole-struct copy here leaves the load
                // ring in scratch memory (the aggregate is not promoted)
                *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
            } else if constexpr (XT == XT_BF16) {
                // bf16 -> f16 is exact for 2^-17 <= |x| < 65536
                uint32_t o[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    o[j] = f2h2(__builtin_bit_cast(float, w[j] << 16), __builtin_bit_cast(float, w[j] & 0xffff0000u));
                }
                *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
            } else {
                *reinterpret_cast<uint2*>(dst) =
                    make_uint2(f2h2(__builtin_bit_cast(float, w[0]), __builtin_bit_cast(float, w[1])),
                               f2h2(__builtin_bit_cast(float, w[2]), __builtin_bit_cast(float, w[3])));
            }
        }
    }
};

// Tile shapes.  BN = 16 (up to 16 tokens): gemm_body_sk16, 32 rows per
// 512-thread workgroup (RT = 2 row tiles x 4 k-splits, one stage in
// flight), so a 14336-row weight spreads over 448 workgroups of 8 waves,
// two per CU (measured on MI355X, Q4_K, bf16 X, m = 16, cold weights:
// 18.4 / 42.7 / 12.7 us for 14336x4096 / 4096x14336 / 4096x4096 against
// 19.8 / 47.8 / 16.6 us for 64-row tiles of 16 waves with two stages in
// flight, 25 us with 16-row tiles; 64-row tiles of 4 waves staging the
// weights through LDS took 23.0 us on 14336x4096).  BN = 64: gemm_body_ra,
// 128 rows (32 per wave) x 64 k per stage, weights dequantised straight
// into the MFMA operand registers.  BN = 128: gemm_body_pipe, 128 x 64
// stages through LDS on a 2 x 2 wave grid.  PF stages of weights and
// activations are in flight in registers, in the order they are consumed
// (the memory counter retires loads in issue order).  Measured on MI355X
// (14336x4096 Q4_K, bf16 X, the two kernels in one process): register-A
// tiles 40 / 43 / 44 us at m = 32 / 64 / 128 against 44 / 47 / 48 us
// through LDS; at m = 256 / 512 the LDS-staged 2 x 2 grid is faster (68 /
// 105 us against 72 / 112).
template <int BN> struct GemmTile;
template <> struct GemmTile<32> { static constexpr int BM = 128, PF = 4; };
template <> struct GemmTile<64> { static constexpr int BM = 128, PF = 4; };
template <> struct GemmTile<128> { static constexpr int BM = 128, PF = 2; };
// BN = 256: the same pipelined body with 128 tokens per wave (a 64 x 128
// wave tile), 110 KB of LDS, one workgroup per CU.
template <> struct GemmTile<256> { static constexpr int BM = 128, PF = 2; };

// Wide token tiles (BN = 128): v_mfma_f32_32x32x16_f16 on a 2 x 2 grid
// of waves -- wave (wr, wc) owns weight rows [64 wr, 64 wr + 64) of the
// 128-row tile and tokens [wc BN/2, (wc+1) BN/2) -- so every A fragment
// read from LDS feeds BN/64 MFMAs and every B fragment two.  Stages of 64 k;
// GemmTile<BN>::PF stages are in flight per workgroup, and two workgroups
// share a CU.  Software-pipelined: within one barrier interval the MFMAs
// of the stage in LDS run in four k-step chunks, and between them the next
// stage is dequantised into the other LDS buffer (chunk 0: the weights,
// chunks 1-2: the activation words, chunk 3: the weight rows written);
// fragments are read one k-step ahead, and sched_barrier keeps each chunk's
// instructions together so the matrix core runs under the VALU work.
// Measured on MI355X (Q4_K, bf16 X, 512 tokens): 116 -> 107 us on
// 14336x4096 against dequantising a stage only after the previous one's
// MFMAs, bit-identical results.
template <typename D, int BN, int XT, int YT, int PF>
__device__ void gemm_body_pipe(const void* __restrict__ x, const uint8_t* __restrict__ w, void* __restrict__ y,
                               int m, int n, int k, int ldy, const GemmExt& ext) {
    constexpr int BM = 128, BK = 64, KP = BK + 8;
    constexpr int TB = BN / 64;
    __shared__ __align__(16) uint16_t wl[2][BM * KP];
    __shared__ __align__(16) uint16_t xl[2][BN * KP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;
    const int r0 = blockIdx.x * BM, t0 = blockIdx.y * BN;
    const size_t row_bytes = (size_t)(k / D::BE) * D::BB;
    const auto dc = D::ctx(w, ext);
    fmt_init<D>(dc, ext);
    XScan<XT, 256> xscan;
    const int nk = k / BK;
    const int wrow = tid >> 1, wsub = tid & 1;
    const uint8_t* wp = w + (size_t)min(r0 + wrow, n - 1) * row_bytes;
    using XS = XTile<XT, BN, BK>;
    static_assert(XS::NL % 2 == 0, "x words split over two chunks");
    const typename XS::Map xm = XS::map(t0, m, k, KP);
    struct Stage {
        typename D::Raw wr;
        XS xr;
    };
    auto issue = [&](Stage& st, int s) {
        const int sc = min(s, nk - 1);
        st.wr = D::load(dc, wp, 2 * sc + wsub);
        st.xr.load(x, xm, (uint32_t)(sc * BK * XS::ES));
    };
    // activation words [i0, i1) of a raw stage -> f16 in LDS buffer buf
    auto xstore = [&](const XS& xr, int buf, int i0, int i1) {
#pragma unroll
        for (int i = 0; i < XS::NL; i++) {
            if (i < i0 || i >= i1) continue;
            uint16_t* dst = &xl[buf][xm.lds[i]];
            const uint32_t wv[4] = {xr.r[i].x, xr.r[i].y, xr.r[i].z, xr.r[i].w};
            if constexpr (XT == XT_F16) {
                *reinterpret_cast<uint4*>(dst) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
            } else if constexpr (XT == XT_BF16) {
                uint32_t o[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    o[j] = f2h2(__builtin_bit_cast(float, wv[j] << 16), __builtin_bit_cast(float, wv[j] & 0xffff0000u));
                }
                *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
            } else {
                *reinterpret_cast<uint2*>(dst) =
                    make_uint2(f2h2(__builtin_bit_cast(float, wv[0]), __builtin_bit_cast(float, wv[1])),
                               f2h2(__builtin_bit_cast(float, wv[2]), __builtin_bit_cast(float, wv[3])));
            }
        }
    };
    float16_t acc[2][TB];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < TB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][b][i] = 0.f;
    auto rd = [&](int buf, int ks, half8_t (&a_)[2], half8_t (&b_)[TB]) {
        const int kof = 16 * ks + 8 * (lane >> 5);
#pragma unroll
        for (int a = 0; a < 2; a++)
            a_[a] = *reinterpret_cast<const half8_t*>(&wl[buf][(64 * wr + 32 * a + (lane & 31)) * KP + kof]);
#pragma unroll
        for (int b = 0; b < TB; b++)
            b_[b] = *reinterpret_cast<const half8_t*>(&xl[buf][((BN / 2) * wc + 32 * b + (lane & 31)) * KP + kof]);
    };
    auto mfma4 = [&](const half8_t (&a_)[2], const half8_t (&b_)[TB]) {
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < TB; b++)
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_[a], b_[b], acc[a][b], 0, 0, 0);
    };
    Stage ring[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) issue(ring[i], i);
    {
        uint32_t o[16];
        D::deq(dc, ring[0].wr, wsub, o);
        uint4* dst = reinterpret_cast<uint4*>(&wl[0][wrow * KP + 32 * wsub]);
#pragma unroll
        for (int i = 0; i < 4; i++) dst[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
        xstore(ring[0].xr, 0, 0, XS::NL);
        issue(ring[0], PF);
    }
    __syncthreads();
    // step s: multiply stage s (buffer s & 1) while stage s + 1 (ring
    // slot nxt) is decoded into buffer (s + 1) & 1; `more`: stage s + 1
    // exists
    auto step = [&](Stage& nxt, int s, bool more) {
        const int buf = s & 1, nb = buf ^ 1;
        half8_t fa[2][2], fb[2][TB];
        uint32_t o[16];
        rd(buf, 0, fa[0], fb[0]);
        rd(buf, 1, fa[1], fb[1]);
        if (more) D::deq(dc, nxt.wr, 2 * (s + 1) + wsub, o);
        mfma4(fa[0], fb[0]);
        __builtin_amdgcn_sched_barrier(0);
        rd(buf, 2, fa[0], fb[0]);
        if (more) xstore(nxt.xr, nb, 0, XS::NL / 2);
        mfma4(fa[1], fb[1]);
        __builtin_amdgcn_sched_barrier(0);
        rd(buf, 3, fa[1], fb[1]);
        if (more) xstore(nxt.xr, nb, XS::NL / 2, XS::NL);
        mfma4(fa[0], fb[0]);
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
            uint4* dst = reinterpret_cast<uint4*>(&wl[nb][wrow * KP + 32 * wsub]);
#pragma unroll
            for (int i = 0; i < 4; i++) dst[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
            issue(nxt, s + 1 + PF);
        }
        mfma4(fa[1], fb[1]);
        __syncthreads();
    };
    int base = 0;
    for (; base + PF <= nk - 1; base += PF) {
#pragma unroll
        for (int b0 = 0; b0 < PF; b0++) step(ring[(b0 + 1) % PF], base + b0, true);
    }
#pragma unroll
    for (int b0 = 0; b0 < PF - 1; b0++)
        if (base + b0 < nk - 1) step(ring[(b0 + 1) % PF], base + b0, true);
    step(ring[0], nk - 1, false);
    xscan.issue(x, m, k, ext.status);  // the range check's loads overlap the output stores

#pragma unroll
    for (int a = 0; a < 2; a++) {
#pragma unroll
        for (int b = 0; b < TB; b++) {
            const int tok = t0 + (BN / 2) * wc + 32 * b + (lane & 31);
            if (tok >= m) continue;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = r0 + 64 * wr + 32 * a + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (row < n) {
                    const size_t off = (size_t)tok * ldy + row;
                    if constexpr (YT == XT_F32) static_cast<float*>(y)[off] = acc[a][b][i];
                    else static_cast<uint16_t*>(y)[off] = (uint16_t)f2h(acc[a][b][i]);
                }
            }
        }
    }

    xscan.finish(x, ext.status);
}

// Split-k tiles for up to 16 tokens: a workgroup of 4 RT waves owns 16 RT
// weight rows x 16 tokens; wave w takes the 16-row tile w % RT and the
// k-split w / RT, whose 128-k stages are s = w / RT, w / RT + 4, ...  Lane l
// takes row l % 16 of its tile and dequantises sub-block g = l / 16 of the
// stage straight into its A operand registers; v_mfma_f32_16x16x32_f16
// step q uses elements [8q, 8q+8) of it, so its B fragment is x[32g + 8q,
// +8) of token l % 16, read from the split's activation tile in LDS (the
// split's RT waves stage it together).  The four splits' partial tiles are
// summed through LDS at the end.
template <typename D, int XT, int YT, int PF, int RT>
__device__ void gemm_body_sk16(const void* __restrict__ x, const uint8_t* __restrict__ w, void* __restrict__ y,
                               int m, int n, int k, int ldy, const GemmExt& ext) {
    constexpr int ES = XT == XT_F32 ? 4 : 2, KP = 136;  // tile pitch in halves (pads away bank conflicts)
    constexpr int NW = 4 * RT;                           // waves: RT row tiles x 4 k-splits
    constexpr int E = 32 / RT;                           // x elements per lane and stage
    constexpr int XW = E * ES / 16;                      // 16-byte x loads per lane and stage
    __shared__ __align__(16) uint16_t xl[2][4][16 * KP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rt = wave % RT, ks = wave / RT, g = lane >> 4;
    const int r0 = blockIdx.x * (16 * RT), t0 = blockIdx.y * 16;
    const size_t row_bytes = (size_t)(k / D::BE) * D::BB;
    const auto dc = D::ctx(w, ext);
    fmt_init<D>(dc, ext);
    XScan<XT, 64 * NW> xscan;
    // k-split over workgroups (blockIdx.z of ext.ksplit; the host makes the
    // 128-k stages divide evenly): this workgroup's stages [s0, s0 + nk)
    const int ksp = ext.ksplit > 1 ? ext.ksplit : 1;
    const int nk = k / 128 / ksp, s0 = (int)blockIdx.z * nk;
    const int cnt = (nk + 3) >> 2;  // every wave runs cnt steps (a uniform barrier count)
    const uint8_t* wp = w + (size_t)min(r0 + 16 * rt + (lane & 15), n - 1) * row_bytes;
    // this lane's share of the split's x tile: E elements of one token
    const int lt = 64 * rt + lane, xtok = (lt * E) >> 7, xk = (lt * E) & 127;
    const uint8_t* xp = static_cast<const uint8_t*>(x) + ((size_t)min(t0 + xtok, m - 1) * k + xk) * ES;
    struct Stage {
        typename D::Raw wr;
        uint4 xr[XW];
    };
    auto issue = [&](Stage& st, int i) {
        const int s = s0 + min(ks + 4 * i, nk - 1);  // past the split's last stage: re-load the last one
        st.wr = D::load(dc, wp, 4 * s + g);
#pragma unroll
        for (int j = 0; j < XW; j++) st.xr[j] = reinterpret_cast<const uint4*>(xp + (size_t)s * 128 * ES)[j];
    };
    float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
    Stage ring[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) issue(ring[i], i);
    auto step = [&](Stage& st, int i, bool next) {
        const int buf = i & 1;
        // the lane's activations -> f16 in the split's tile
        uint4* dst = reinterpret_cast<uint4*>(&xl[buf][ks][xtok * KP + xk]);
        if constexpr (XT == XT_F32) {
#pragma unroll
            for (int j = 0; j < XW / 2; j++) {
                const uint4 a = st.xr[2 * j], b = st.xr[2 * j + 1];
                dst[j] = make_uint4(f2h2(__builtin_bit_cast(float, a.x), __builtin_bit_cast(float, a.y)),
                                    f2h2(__builtin_bit_cast(float, a.z), __builtin_bit_cast(float, a.w)),
                                    f2h2(__builtin_bit_cast(float, b.x), __builtin_bit_cast(float, b.y)),
                                    f2h2(__builtin_bit_cast(float, b.z), __builtin_bit_cast(float, b.w)));
            }
        } else {
#pragma unroll
            for (int j = 0; j < XW; j++) {
                const uint32_t v[4] = {st.xr[j].x, st.xr[j].y, st.xr[j].z, st.xr[j].w};
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    o[e] = XT == XT_F16 ? v[e]
                                        : f2h2(__builtin_bit_cast(float, v[e] << 16),
                                               __builtin_bit_cast(float, v[e] & 0xffff0000u));
                }
                dst[j] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
        uint32_t o[16];
        D::deq(dc, st.wr, 4 * (s0 + min(ks + 4 * i, nk - 1)) + g, o);
        __syncthreads();
        if (next) issue(st, i + PF);
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 4 * i < nk) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const half8_t bv =
                    *reinterpret_cast<const half8_t*>(&xl[buf][ks][(lane & 15) * KP + 32 * g + 8 * q]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(half8_t, make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3])), bv,
                    acc, 0, 0, 0);
            }
        }
    };
    int base = 0;
    for (; base + PF <= cnt; base += PF) {
#pragma unroll
        for (int b0 = 0; b0 < PF; b0++) step(ring[b0], base + b0, true);
    }
#pragma unroll
    for (int b0 = 0; b0 < PF - 1; b0++)
        if (base + b0 < cnt) step(ring[b0], base + b0, false);

    xscan.issue(x, m, k, ext.status);  // the range check's loads overlap the split reduction
    // lane l holds D[row 4(l/16) + i][token l%16] of its tile; sum the splits
    __syncthreads();
    float* red = reinterpret_cast<float*>(&xl[0][0][0]);  // [NW waves][256]
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave * 256 + (4 * g + i) * 16 + (lane & 15)] = acc[i];
    __syncthreads();
    for (int o = tid; o < 256 * RT; o += 64 * NW) {
        const int orow = o >> 4, otok = o & 15, ot = orow >> 4, oi = (orow & 15) * 16 + otok;
        const float v = (red[ot * 256 + oi] + red[(RT + ot) * 256 + oi]) +
                        (red[(2 * RT + ot) * 256 + oi] + red[(3 * RT + ot) * 256 + oi]);
        const int row = r0 + orow, tok = t0 + otok;
        if (row < n && tok < m) {
            if (ksp > 1) {
                ext.part[((size_t)blockIdx.z * m + tok) * n + row] = v;  // summed by cima_gemm_ksum_*
            } else {
                const size_t off = (size_t)tok * ldy + row;
                if constexpr (YT == XT_F32) static_cast<float*>(y)[off] = v;
                else static_cast<uint16_t*>(y)[off] = (uint16_t)f2h(v);
            }
        }
    }

    xscan.finish(x, ext.status);
}


// Register-A tiles: each wave owns RW weight rows (RW / 32 tiles of 32
// rows) and all BN tokens of the workgroup's tile, and dequantises its own
// A operand straight into registers -- no LDS round trip for the weights.
// Lane l of a 32-row tile takes row l % 32 and dequantises sub-block
// h = l / 32 of the stage's two (64 k): its 32 values are the A fragments of
// the four k-steps, step q holding elements [8q, 8q+8).  The MFMA sums over
// k in any order as long as A and B agree, so the B fragment of lane l, step
// q, is x[32h + 8q, +8) of its token.  Only the activation tile goes through
// LDS; per 64-k stage a wave issues 4 (RW/32) (BN/32) v_mfma_f32_32x32x16_f16.
template <typename D, int BN, int RW, int PF, int XT, int YT>
__device__ void gemm_body_ra(const void* __restrict__ x, const uint8_t* __restrict__ w, void* __restrict__ y,
                             int m, int n, int k, int ldy, const GemmExt& ext) {
    constexpr int BM = 4 * RW, BK = 64, KP = BK + 8;
    constexpr int RA = RW / 32, TB = BN / 32;
    __shared__ __align__(16) uint16_t xl[2][BN * KP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * BM + RW * wave, t0 = blockIdx.y * BN;
    const size_t row_bytes = (size_t)(k / D::BE) * D::BB;
    const auto dc = D::ctx(w, ext);
    fmt_init<D>(dc, ext);
    XScan<XT, 256> xscan;
    const int nk = k / BK;
    const int h = lane >> 5;

    const uint8_t* wp[RA];
#pragma unroll
    for (int a = 0; a < RA; a++) wp[a] = w + (size_t)min(r0 + 32 * a + (lane & 31), n - 1) * row_bytes;
    using XS = XTile<XT, BN, BK>;
    const typename XS::Map xm = XS::map(t0, m, k, KP);
    struct Stage {
        typename D::Raw wr[RA];
        XS xr;
    };
    auto issue = [&](Stage& st, int s) {
        const int sc = min(s, nk - 1);  // stages past the end re-load the last one
#pragma unroll
        for (int a = 0; a < RA; a++) st.wr[a] = D::load(dc, wp[a], 2 * sc + h);
        st.xr.load(x, xm, (uint32_t)(sc * BK * XS::ES));
    };

    float16_t acc[RA][TB];
#pragma unroll
    for (int a = 0; a < RA; a++)
#pragma unroll
        for (int b = 0; b < TB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][b][i] = 0.f;

    Stage ring[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) issue(ring[i], i);

    auto step = [&](Stage& st, int s, bool next) {
        const int buf = s & 1;
        st.xr.store(xl[buf], xm);
        uint32_t o[RA][16];
#pragma unroll
        for (int a = 0; a < RA; a++) D::deq(dc, st.wr[a], 2 * s + h, o[a]);
        __syncthreads();
        if (next) issue(st, s + PF);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            half8_t av[RA], bv[TB];
#pragma unroll
            for (int a = 0; a < RA; a++)
                av[a] = __builtin_bit_cast(half8_t, make_uint4(o[a][4 * q], o[a][4 * q + 1], o[a][4 * q + 2],
                                                               o[a][4 * q + 3]));
#pragma unroll
            for (int b = 0; b < TB; b++)
                bv[b] = *reinterpret_cast<const half8_t*>(&xl[buf][(32 * b + (lane & 31)) * KP + 32 * h + 8 * q]);
#pragma unroll
            for (int a = 0; a < RA; a++)
#pragma unroll
                for (int b = 0; b < TB; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
    };
    int base = 0;
    for (; base + PF <= nk; base += PF) {
#pragma unroll
        for (int b0 = 0; b0 < PF; b0++) step(ring[b0], base + b0, true);
    }
#pragma unroll
    for (int b0 = 0; b0 < PF - 1; b0++)
        if (base + b0 < nk) step(ring[b0], base + b0, false);

    xscan.issue(x, m, k, ext.status);  // the range check's loads overlap the output stores
    // lane l, element i of a 32x32 tile: row 8(i/4) + 4(l/32) + i%4, column l%32
#pragma unroll
    for (int a = 0; a < RA; a++) {
#pragma unroll
        for (int b = 0; b < TB; b++) {
            const int tok = t0 + 32 * b + (lane & 31);
            if (tok >= m) continue;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = r0 + 32 * a + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (row < n) {
                    const size_t off = (size_t)tok * ldy + row;
                    if constexpr (YT == XT_F32) static_cast<float*>(y)[off] = acc[a][b][i];
                    else static_cast<uint16_t*>(y)[off] = (uint16_t)f2h(acc[a][b][i]);
                }
            }
        }
    }

    xscan.finish(x, ext.status);
}


// Stages in flight for gemm_body_ra: GemmTile<BN>::PF, fewer where a stage
// (the raw weight sub-block plus the thread's activation words) is so large
// that the ring would spill to scratch memory.
template <typename D, int BN, int XT>
constexpr int ra_pf() {
    if constexpr (BN < 32) {
        return 1;  // not a register-A tile
    } else {
        constexpr int stage = (int)(sizeof(typename D::Raw) / 4) + 4 * XTile<XT, BN, 64>::NL;
        constexpr int fit = (BN == 64 ? 84 : 60) / stage;
        return fit < 1 ? 1 : (fit < GemmTile<BN>::PF ? fit : GemmTile<BN>::PF);
    }
}

// name: cima_gemm_<fmt>_b<BN>_<x type>_<y type>
// (HIP's second bound is the minimum waves per SIMD: the 16-token tiles
// ask for 4, two 512-thread workgroups per CU, which the compiler then
// schedules for -- measured on MI355X, Q4_K, bf16 X, bit-identical:
// 14336x4096 18.4 -> 17.6 us at 16 tokens and 33.8 -> 31.0 at 32 in a
// sweep, 18.7 -> 18.6 at 16 in bench.py's run; the wider tiles ask for 1,
// which left the 64-token tile at 232 VGPRs (two workgroups per CU still
// fit) and ran 1-3% faster than asking for 2: 14336x4096 at 48 / 64 / 128
// tokens 35.0 -> 34.1, 35.2 -> 34.6, 44.0 -> 43.7 us)
#define GEMM_KERNEL(FN, D, BN, XT, XN, YT, YN)                                                       \
    extern "C" __global__ __launch_bounds__(BN == 16 ? 512 : 256, BN == 16 ? 4 : 1) void         \
    cima_gemm_##FN##_b##BN##_##XN##_##YN(                                                             \
        const void* x, const uint8_t* w, void* y, int m, int n, int k, int ldy, GemmExt ext) {      \
        if constexpr (BN == 16) gemm_body_sk16<D, XT, YT, 1, 2>(x, w, y, m, n, k, ldy, ext);         \
        else if constexpr (BN <= 64)                                                                  \
            gemm_body_ra<D, BN, 32, ra_pf<D, BN, XT>(), XT, YT>(x, w, y, m, n, k, ldy, ext);          \
        else gemm_body_pipe<D, BN, XT, YT, GemmTile<128>::PF>(x, w, y, m, n, k, ldy, ext);         \
    }
#define GEMM_XY(FN, D, BN)                                                    \
    GEMM_KERNEL(FN, D, BN, XT_F32, f32, XT_F32, f32)                          \
    GEMM_KERNEL(FN, D, BN, XT_F16, f16, XT_F32, f32)                          \
    GEMM_KERNEL(FN, D, BN, XT_BF16, bf16, XT_F32, f32)                        \
    GEMM_KERNEL(FN, D, BN, XT_F32, f32, XT_F16, f16)                          \
    GEMM_KERNEL(FN, D, BN, XT_F16, f16, XT_F16, f16)                          \
    GEMM_KERNEL(FN, D, BN, XT_BF16, bf16, XT_F16, f16)
// 16-row split-k tiles (four waves) for weights too narrow to fill the CUs
// with 32-row tiles: the _b16n_ kernels.  Two stages in flight at three
// workgroups per CU where a stage's registers allow it without spilling
// (not for f32 X, eight load words per stage, nor Q6_K, Q5_K and f16
// weights, whose stages are the largest), else one at four
// (measured on MI355X, Q4_K, bf16 X, 16 tokens: 38.8 -> 25.0 us on
// 4096x14336, 12.9 -> 9.2 on 4096x4096).
template <typename D, int XT>
constexpr int sk16n_pf() {
    return (XT != XT_F32 && !std::is_same<D, GG<DQ6_K>>::value && !std::is_same<D, GG<DQ5_K>>::value &&
            !std::is_same<D, DF16>::value)
               ? 2
               : 1;
}
#define GEMM_KERNEL_NARROW(FN, D, XT, XN, YT, YN)                                                   \
    extern "C" __global__ __launch_bounds__(256, (sk16n_pf<D, XT>() == 2 ? 3 : 4)) void            \
    cima_gemm_##FN##_b16n_##XN##_##YN(const void* x, const uint8_t* w, void* y, int m, int n, int k, \
                                      int ldy, GemmExt ext) {                                       \
        gemm_body_sk16<D, XT, YT, sk16n_pf<D, XT>(), 1>(x, w, y, m, n, k, ldy, ext);                \
    }
#define GEMM_XY_NARROW(FN, D)                                                 \
    GEMM_KERNEL_NARROW(FN, D, XT_F32, f32, XT_F32, f32)                       \
    GEMM_KERNEL_NARROW(FN, D, XT_F16, f16, XT_F32, f32)                       \
    GEMM_KERNEL_NARROW(FN, D, XT_BF16, bf16, XT_F32, f32)                     \
    GEMM_KERNEL_NARROW(FN, D, XT_F32, f32, XT_F16, f16)                       \
    GEMM_KERNEL_NARROW(FN, D, XT_F16, f16, XT_F16, f16)                       \
    GEMM_KERNEL_NARROW(FN, D, XT_BF16, bf16, XT_F16, f16)
#define GEMM_FMT(FN, D) \
    GEMM_XY(FN, D, 16) GEMM_XY_NARROW(FN, D) GEMM_XY(FN, D, 32) GEMM_XY(FN, D, 64) GEMM_XY(FN, D, 128) GEMM_XY(FN, D, 256)

GEMM_FMT(q8_0, GG<DQ8_0>)
GEMM_FMT(q4_0, GG<DQ4_0>)
GEMM_FMT(q4_1, GG<DQ4_1>)
GEMM_FMT(q5_0, GG<DQ5_01<false>>)
GEMM_FMT(q5_1, GG<DQ5_01<true>>)
GEMM_FMT(q4_k, GG<DQ4_K>)
GEMM_FMT(q5_k, GG<DQ5_K>)
GEMM_FMT(q6_k, GG<DQ6_K>)
GEMM_FMT(iq4_xs, GG<DIQ4_XS>)
// bitsandbytes 4-bit weights decoded in the tiles, and plain f16 weights
GEMM_FMT(nf4, DNF4)
GEMM_FMT(f16w, DF16)

// f16 weights of any k (the slab route for k % 64 != 0): one thread per
// output, X rounded to f16 as the tiles round it, fp32 accumulation in k
// order.  Not a fast kernel: it serves shapes no real checkpoint has.
template <int XT, int YT>
__device__ void gemm_small_body(const void* __restrict__ x, const uint16_t* __restrict__ w, void* __restrict__ y,
                                int m, int n, int k, int ldy) {
    const long long o = (long long)blockIdx.x * 256 + threadIdx.x;
    if (o >= (long long)m * n) return;
    const int tok = (int)(o / n), row = (int)(o % n);
    const uint16_t* wr = w + (size_t)row * k;
    float acc = 0.f;
    for (int i = 0; i < k; i++) {
        float xv;
        if constexpr (XT == XT_F32) xv = h2f(f2h(static_cast<const float*>(x)[(size_t)tok * k + i]));
        else if constexpr (XT == XT_F16) xv = h2f(static_cast<const uint16_t*>(x)[(size_t)tok * k + i]);
        else xv = h2f(f2h(__builtin_bit_cast(float, (uint32_t)static_cast<const uint16_t*>(x)[(size_t)tok * k + i] << 16)));
        acc = fmaf(xv, h2f(wr[i]), acc);
    }
    const size_t off = (size_t)tok * ldy + row;
    if constexpr (YT == XT_F32) static_cast<float*>(y)[off] = acc;
    else static_cast<uint16_t*>(y)[off] = (uint16_t)f2h(acc);
}
#define GEMM_SMALL(XT, XN, YT, YN)                                                                      \
    extern "C" __global__ __launch_bounds__(256) void cima_gemm_f16w_small_##XN##_##YN(                 \
        const void* x, const uint16_t* w, void* y, int m, int n, int k, int ldy) {                      \
        gemm_small_body<XT, YT>(x, w, y, m, n, k, ldy);                                                 \
    }
GEMM_SMALL(XT_F32, f32, XT_F32, f32)
GEMM_SMALL(XT_F16, f16, XT_F32, f32)
GEMM_SMALL(XT_BF16, bf16, XT_F32, f32)
GEMM_SMALL(XT_F32, f32, XT_F16, f16)
GEMM_SMALL(XT_F16, f16, XT_F16, f16)
GEMM_SMALL(XT_BF16, bf16, XT_F16, f16)


// Y[tok, row] (row stride ldy) = sum over z < S of part[z][tok][row], z in
// order: the k-split partial tiles of the 16-token kernels, added in one
// fixed order (results do not depend on the launch)
template <int YT>
__device__ void ksum_body(const float* __restrict__ part, void* __restrict__ y, int m, int n, int ldy, int S) {
    const long long o = (long long)blockIdx.x * 256 + threadIdx.x;
    if (o >= (long long)m * n) return;
    const int tok = (int)(o / n), row = (int)(o % n);
    float v = part[o];
    for (int z = 1; z < S; z++) v += part[(size_t)z * m * n + o];
    const size_t off = (size_t)tok * ldy + row;
    if constexpr (YT == XT_F32) static_cast<float*>(y)[off] = v;
    else static_cast<uint16_t*>(y)[off] = (uint16_t)f2h(v);
}
extern "C" __global__ __launch_bounds__(256) void cima_gemm_ksum_f32(const float* part, void* y, int m, int n, int ldy,
                                                                     int S) {
    ksum_body<XT_F32>(part, y, m, n, ldy, S);
}
extern "C" __global__ __launch_bounds__(256) void cima_gemm_ksum_f16(const float* part, void* y, int m, int n, int ldy,
                                                                     int S) {
    ksum_body<XT_F16>(part, y, m, n, ldy, S);
}
