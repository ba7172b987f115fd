// bitsandbytes 4-bit (NF4 / FP4) weights on gfx950 (code object
// cima_bnb4.hsaco): dequantisation to f16 and the fused decode GEMV.
//
// Layout (src/quant.rs:18-70): a row-major [n, k] weight is n*k/2 packed
// bytes, element 2j in the HIGH nibble of byte j; absmax holds one f32 per
// `blocksize` consecutive elements (the double quantisation already folded
// on the host); qmap is the 16-entry f32 codebook.  Weight element i is
// qmap[nibble(i)] * absmax[i / blocksize].
#include "gguf_formats.h"

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- dequant
// out[i] = f16(qmap[nib(i)] * absmax[i / blocksize]): one fp32 product,
// rounded once to nearest even -- bit-exact with dequant_host
// (src/quant.rs:401-437) and k_nf4_dequant (src/kernels.cu:320-329).

// one thread per 32 elements (16 packed bytes in, 64 bytes out): n % 32 == 0,
// blocksize % 32 == 0, packed and out 16-byte aligned
extern "C" __global__ __launch_bounds__(256) void cima_nf4_dequant_v(const uint4* __restrict__ packed,
                                                                     const float* __restrict__ absmax,
                                                                     const float* __restrict__ qmap,
                                                                     uint4* __restrict__ out, long long nseg,
                                                                     int seg_per_block) {
    __shared__ float code[16];
    if (threadIdx.x < 16) code[threadIdx.x] = qmap[threadIdx.x];
    __syncthreads();
    const long long s = (long long)blockIdx.x * 256 + threadIdx.x;
    if (s >= nseg) return;
    const uint4 w = packed[s];
    const float a = absmax[s / seg_per_block];
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {  // 8 elements per packed dword
        const uint32_t v = wd[q];
        uint4 o;
        uint32_t* op = &o.x;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t byte = (v >> (8 * b)) & 0xFFu;
            op[b] = f2h2(code[byte >> 4] * a, code[byte & 0xFu] * a);
        }
        out[s * 4 + q] = o;
    }
}

// general shape: one thread per element (any n, any blocksize >= 1)
extern "C" __global__ __launch_bounds__(256) void cima_nf4_dequant_e(const uint8_t* __restrict__ packed,
                                                                     const float* __restrict__ absmax,
                                                                     const float* __restrict__ qmap,
                                                                     uint16_t* __restrict__ out, long long n,
                                                                     int blocksize) {
    __shared__ float code[16];
    if (threadIdx.x < 16) code[threadIdx.x] = qmap[threadIdx.x];
    __syncthreads();
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint32_t b = packed[i >> 1];
    const uint32_t nib = (i & 1) ? (b & 0xFu) : (b >> 4);
    out[i] = (uint16_t)f2h(code[nib] * absmax[i / blocksize]);
}

// ------------------------------------------------------------------- GEMV
//
// y[r] = sum_c x[c] * qmap[nib(r*k + c)] * absmax[(r*k + c) / blocksize]
// (k_nf4_gemv, src/kernels.cu:331-387: the decode-path fused GEMV).
//
// Fast path (k % 32 == 0, blocksize a power of two >= 32): one lane takes
// 16 packed bytes = 32 elements of a row, which all share one absmax; the
// 32-element dot runs in v_dot2_f32_f16 on f16 codes and f16 x, fp32
// accumulation, and is scaled by absmax once.  The only rounding beyond the
// fp32 accumulation is the codebook value's rounding to f16 (relative error
// <= 2^-11 per code); x is f16 (f32 x is rounded to f16 on staging, like
// the reference's f16 activations).  Two ways to turn packed bytes into f16
// code pairs:
//
//  * pair table (PairTab): a byte b names the pair (code[b >> 4],
//    code[b & 15]) of elements 2j, 2j+1 -- a 256-entry table of f16 pairs in
//    LDS, with 64 copies of each entry side by side (row b = 256 bytes), so
//    that lane L reads column L: one v_perm_b32 forms the address
//    (b << 8 | 4L) from the packed dword, one ds_read_b32 fetches the pair,
//    no two lanes ever share a bank.  About 1 VALU operation per element;
//    64 KB of LDS per workgroup besides x;
//  * codebook in registers (RegCode): the codebook as two byte planes (low
//    and high byte of each f16 code) of 16 entries in eight wave-uniform
//    registers; a nibble dword is looked up with two v_perm_b32 per plane
//    (entries 0-7 and 8-15) and a bit-3 select, and the plane bytes are
//    paired into f16 code pairs with one more v_perm_b32 (about 3.5 VALU
//    operations per element).  x is staged with each group of 8 in the
//    order [x0 x2 x4 x6 x1 x3 x5 x7], so that the pairs of codes a packed
//    dword yields (even elements from the high nibbles, odd from the low)
//    meet their x pair in one v_dot2_f32_f16.  For k too large for the
//    pair table next to x in LDS.
//
// x in LDS: group g of 8 elements (segment g / 4, quarter g % 4) at index
// (g % 4) * (k / 32) + g / 4, so that the 64 lanes of a wave, on 64
// consecutive segments, read one quarter as 1 KB of consecutive LDS (no bank
// conflicts).
//
// Each wave owns R consecutive rows at a time and walks them together
// (R 16-byte loads, plus their absmax, per lane and step), so one LDS read
// of x serves R rows; loads run ahead of the compute in a ring of steps that
// crosses row groups.  The grid is persistent: workgroups stride over row
// groups after staging x (and the table) once.

DEV float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}

template <typename XT>
DEV uint32_t xh(const XT* x, int i);
template <>
DEV uint32_t xh<uint16_t>(const uint16_t* x, int i) {
    return x[i];
}
template <>
DEV uint32_t xh<float>(const float* x, int i) {
    return f2h(x[i]);
}

// x[8g .. 8g+7] as four f16 pairs (x0,x1) (x2,x3) (x4,x5) (x6,x7); x is
// 16-byte aligned
DEV uint4 load8(const uint16_t* __restrict__ x, int g) {
    return reinterpret_cast<const uint4*>(x)[g];
}
DEV uint4 load8(const float* __restrict__ x, int g) {
    const float4 a = reinterpret_cast<const float4*>(x)[2 * g], b = reinterpret_cast<const float4*>(x)[2 * g + 1];
    return make_uint4(f2h2(a.x, a.y), f2h2(a.z, a.w), f2h2(b.x, b.y), f2h2(b.z, b.w));
}

template <typename YT>
DEV void store_y(YT* y, int r, float v);
template <>
DEV void store_y<float>(float* y, int r, float v) {
    y[r] = v;
}
template <>
DEV void store_y<uint16_t>(uint16_t* y, int r, float v) {
    y[r] = (uint16_t)f2h(v);
}

struct RegCode {
    uint32_t lb[4], hb[4];  // byte i of the planes: low / high byte of f16(qmap[i])
    const uint4* xs;        // x, permuted groups of 8 (see the staging)
    int segs;               // k / 32

    template <typename XT>
    DEV void stage(uint8_t* smem, const XT* __restrict__ x, const float* __restrict__ qmap, int k, int nthreads) {
        uint4* xw = reinterpret_cast<uint4*>(smem);
        for (int g = threadIdx.x; g < (k >> 3); g += nthreads) {
            const uint4 h = load8(x, g);
            xw[(g & 3) * (k >> 5) + (g >> 2)] = make_uint4(__builtin_amdgcn_perm(h.y, h.x, 0x05040100u), __builtin_amdgcn_perm(h.w, h.z, 0x05040100u),
                               __builtin_amdgcn_perm(h.y, h.x, 0x07060302u), __builtin_amdgcn_perm(h.w, h.z, 0x07060302u));
        }
        planes(qmap);
        xs = xw;
        segs = k >> 5;
    }

    DEV void planes(const float* __restrict__ qmap) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            uint32_t l = 0, h = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t c = f2h(qmap[p * 4 + b]);
                l |= (c & 0xFFu) << (8 * b);
                h |= (c >> 8) << (8 * b);
            }
            lb[p] = __builtin_amdgcn_readfirstlane(l);
            hb[p] = __builtin_amdgcn_readfirstlane(h);
        }
    }

    // f16 bits of code[i] for one lane-varying index i < 16
    DEV uint32_t at(uint32_t i) const {
        const uint32_t m = i & 8 ? 0xFFu : 0u;
        return (plane16(lb, i & 7, m) & 0xFFu) | ((plane16(hb, i & 7, m) & 0xFFu) << 8);
    }

    static DEV uint32_t plane16(const uint32_t (&t)[4], uint32_t i7, uint32_t m) {
        // __builtin_amdgcn_perm(s0, s1, sel): selector 0-3 -> byte of s1, 4-7 -> byte of s0
        const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], i7);  // entries 0-7
        const uint32_t hi = __builtin_amdgcn_perm(t[3], t[2], i7);  // entries 8-15
        return (hi & m) | (lo & ~m);
    }

    // the 8 elements of one packed dword w (byte j: element 2j high nibble,
    // 2j+1 low) -> f16 code pairs h01 = (c[e0], c[e2]), h23 = (c[e4], c[e6]),
    // l01 = (c[e1], c[e3]), l23 = (c[e5], c[e7]).  The bit-3 select masks
    // come from v_perm_b32's sign-replicating selectors (8-11: 0xFF if bit 7
    // of byte 1 / 3 of s1, byte 1 / 3 of s0 is set, else 0x00): with
    // s1 = v << 8 and s0 = v, selector 0x0B090A08 spreads bit 7 of every
    // byte of v over it.
    DEV void lookup8(uint32_t w, uint32_t& h01, uint32_t& h23, uint32_t& l01, uint32_t& l23) const {
        const uint32_t i7h = (w >> 4) & 0x07070707u, i7l = w & 0x07070707u;
        const uint32_t mh = __builtin_amdgcn_perm(w, w << 8, 0x0B090A08u);
        const uint32_t w4 = w << 4;  // bit 3 of every byte -> bit 7
        const uint32_t ml = __builtin_amdgcn_perm(w4, w4 << 8, 0x0B090A08u);
        const uint32_t lbh = plane16(lb, i7h, mh), hbh = plane16(hb, i7h, mh);
        const uint32_t lbl = plane16(lb, i7l, ml), hbl = plane16(hb, i7l, ml);
        h01 = __builtin_amdgcn_perm(hbh, lbh, 0x05010400u);
        h23 = __builtin_amdgcn_perm(hbh, lbh, 0x07030602u);
        l01 = __builtin_amdgcn_perm(hbl, lbl, 0x05010400u);
        l23 = __builtin_amdgcn_perm(hbl, lbl, 0x07030602u);
    }

    DEV float dot32(const uint4 w, int j) const {
        const uint4* xg = xs + j;
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 xv = xg[q * segs];  // (x0,x2) (x4,x6) (x1,x3) (x5,x7)
            uint32_t h01, h23, l01, l23;
            lookup8(wd[q], h01, h23, l01, l23);
            s0 = dot2(h01, xv.x, s0);
            s1 = dot2(h23, xv.y, s1);
            s0 = dot2(l01, xv.z, s0);
            s1 = dot2(l23, xv.w, s1);
        }
        return s0 + s1;
    }
};

struct PairTab {
    static constexpr unsigned TAB_BYTES = 65536;  // 256 rows x 64 lanes x 4 bytes
    const uint8_t* lds;  // table at 0, x (natural order, f16) at TAB_BYTES
    uint32_t lane4;      // 4 * lane
    int segs;            // k / 32

    template <typename XT>
    DEV void stage(uint8_t* smem, const XT* __restrict__ x, const float* __restrict__ qmap, int k, int nthreads) {
        uint4* xs = reinterpret_cast<uint4*>(smem + TAB_BYTES);
        for (int g = threadIdx.x; g < (k >> 3); g += nthreads) xs[(g & 3) * (k >> 5) + (g >> 2)] = load8(x, g);
        RegCode c;
        c.planes(qmap);
        uint4* tab = reinterpret_cast<uint4*>(smem);
        for (int i = threadIdx.x; i < (int)(TAB_BYTES / 16); i += nthreads) {
            const uint32_t b = (uint32_t)i >> 4;  // 16 uint4 per row
            const uint32_t pr = c.at(b >> 4) | (c.at(b & 15) << 16);
            tab[i] = make_uint4(pr, pr, pr, pr);
        }
        lds = smem;
        lane4 = (threadIdx.x & 63) * 4;
        segs = k >> 5;
    }

    DEV uint32_t pair(uint32_t v, uint32_t sel) const {
        // sel picks byte j of v into bits 8-15 and lane4 into bits 0-7
        const uint32_t addr = __builtin_amdgcn_perm(v, lane4, sel);
        return *reinterpret_cast<const uint32_t*>(lds + addr);
    }

    // 32 elements: 16 packed bytes against x of segment j
    DEV float dot32(const uint4 w, int j) const {
        const uint4* xg = reinterpret_cast<const uint4*>(lds + TAB_BYTES) + j;
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 xv = xg[q * segs];  // (x0,x1) (x2,x3) (x4,x5) (x6,x7)
            s0 = dot2(pair(wd[q], 0x0C0C0400u), xv.x, s0);
            s1 = dot2(pair(wd[q], 0x0C0C0500u), xv.y, s1);
            s0 = dot2(pair(wd[q], 0x0C0C0600u), xv.z, s0);
            s1 = dot2(pair(wd[q], 0x0C0C0700u), xv.w, s1);
        }
        return s0 + s1;
    }
};

template <class Dec, int NT, int R, int D, typename XT, typename YT>
DEV void nf4_gemv_body(const XT* __restrict__ x, const uint8_t* __restrict__ packed,
                       const float* __restrict__ absmax, const float* __restrict__ qmap, YT* __restrict__ y,
                       int n, int k, int bshift) {
    extern __shared__ uint4 smem_[];
    Dec dec;

    // Work of one wave: its row groups g = wave, wave + nwaves, ..., each
    // walked in T steps of 64 segments (one per lane).  An item is one step
    // of one group: R 16-byte weight loads and R absmax loads per lane.  The
    // items form one sequence across groups, and a ring of D items keeps
    // D - 1 of them in flight while one is computed, also over the boundary
    // between groups.
    constexpr int WPG = NT / 64;  // waves per workgroup
    const int lane = threadIdx.x & 63;
    const int segs = k >> 5;
    const int T = (segs + 63) >> 6;
    const int groups = (n + R - 1) / R;
    const int nwaves = gridDim.x * WPG;
    const int wave = blockIdx.x * WPG + (threadIdx.x >> 6);
    // a wave past the last row group loads the last one's rows (its loads
    // are never used) rather than branching around the loads, so the first
    // items can go out before x and the table are staged
    const int wv = min(wave, groups - 1);
    const int items = ((groups - 1 - wv) / nwaves + 1) * T;
    const size_t rowb = (size_t)(k >> 1);

    struct Item {
        uint4 w[R];
        float a[R];
    };
    int ig = wv, it = 0;  // next item to load: group, step
    auto issue = [&](Item& s) {
        const int j = min(it * 64 + lane, segs - 1);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(ig * R + r, n - 1);
            s.w[r] = *reinterpret_cast<const uint4*>(packed + (size_t)row * rowb + (size_t)j * 16);
            s.a[r] = absmax[((uint32_t)row * (uint32_t)segs + (uint32_t)j) >> bshift];
        }
        if (++it == T) {
            it = 0;
            ig += nwaves;
        }
    };
    // finished rows wait in lane `slot` of res / rowv and are written once
    // after the loop, so that no store sits between the weight loads (the
    // host sizes the grid so that no wave owns more than 64 rows)
    int cg = wv, ct = 0, slot = 0;
    float acc[R], res = 0.f;
    int rowv = n;
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    auto consume = [&](const Item& s) {
        const int jr = ct * 64 + lane;
        const int j = min(jr, segs - 1);
        const float keep = jr < segs ? 1.f : 0.f;  // lanes past the row end (clamped loads) add 0
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = __builtin_fmaf(s.a[r] * keep, dec.dot32(s.w[r], j), acc[r]);
        if (++ct == T) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float v = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, group_sum_last(acc[r], 64)), 63));
                res = lane == slot + r ? v : res;
                rowv = lane == slot + r ? cg * R + r : rowv;
                acc[r] = 0.f;
            }
            slot += R;
            ct = 0;
            cg += nwaves;
        }
    };
    // Loads are issued unconditionally, also past the wave's last item
    // (clamped to the last row: in bounds, and their values never used): a
    // load under a condition makes the compiler's wait counting assume the
    // worst and drain the ring.
    Item ring[D];
    issue(ring[0]);
    // x (and the pair table) while the first item is in flight; the rest of
    // the ring after (measured on MI355X, cold, against issuing after the
    // staging: 4096x4096 5.59 -> 5.03 us, 128256x4096 57.7 -> 55.6-56.3,
    // 4096x14336 10.2-10.9 -> 10.1-10.2, 14336x4096 9.7-10.1 -> 10.25; the
    // whole ring up front flooded HBM at 32 waves per CU: 14336x4096 11.35)
    dec.stage(reinterpret_cast<uint8_t*>(smem_), x, qmap, k, NT);
    __syncthreads();
    if (wave >= groups) return;
#pragma unroll
    for (int d = 1; d < D; d++) issue(ring[d]);
    int i = 0;
    for (; i + D <= items; i += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            consume(ring[d]);
            issue(ring[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < D - 1; d++)
        if (i + d < items) consume(ring[d]);
    if (lane < slot && rowv < n) store_y(y, rowv, res);
}

// general shape (any k, any blocksize >= 1): one wave per row, one element
// per lane and step, each weight decoded exactly like the dequant kernel
template <typename XT, typename YT>
DEV void nf4_gemv_e_body(const XT* __restrict__ x, const uint8_t* __restrict__ packed,
                         const float* __restrict__ absmax, const float* __restrict__ qmap, YT* __restrict__ y,
                         int n, int k, int blocksize) {
    __shared__ float code[16];
    if (threadIdx.x < 16) code[threadIdx.x] = qmap[threadIdx.x];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const long long base = (long long)row * k;
    float acc = 0.f;
    for (int cix = lane; cix < k; cix += 64) {
        const long long i = base + cix;
        const uint32_t b = packed[i >> 1];
        const uint32_t nib = (i & 1) ? (b & 0xFu) : (b >> 4);
        const float w = h2f(f2h(code[nib] * absmax[i / blocksize]));
        acc = __builtin_fmaf(h2f(xh(x, cix)), w, acc);
    }
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) store_y(y, row, acc);
}

#ifndef CIMA_NF4_RING
#define CIMA_NF4_RING 3
#endif
// pair table: 1024-thread workgroups (one per CU: the table and x fill most
// of the LDS); register codebook: 256-thread workgroups
#define NF4_GEMV(R, XN, XT, YN, YT)                                                                              \
    extern "C" __global__ __launch_bounds__(1024) void cima_nf4_gemv_t_r##R##_##XN##_##YN(                      \
        const XT* x, const uint8_t* packed, const float* absmax, const float* qmap, YT* y, int n, int k,         \
        int bshift) {                                                                                            \
        nf4_gemv_body<PairTab, 1024, R, CIMA_NF4_RING, XT, YT>(x, packed, absmax, qmap, y, n, k, bshift);        \
    }                                                                                                            \
    extern "C" __global__ __launch_bounds__(256) void cima_nf4_gemv_c_r##R##_##XN##_##YN(                       \
        const XT* x, const uint8_t* packed, const float* absmax, const float* qmap, YT* y, int n, int k,         \
        int bshift) {                                                                                            \
        nf4_gemv_body<RegCode, 256, R, CIMA_NF4_RING, XT, YT>(x, packed, absmax, qmap, y, n, k, bshift);         \
    }
#define NF4_GEMV_ACTS(R)                        \
    NF4_GEMV(R, f16, uint16_t, f16, uint16_t)   \
    NF4_GEMV(R, f32, float, f32, float)

NF4_GEMV_ACTS(1)
NF4_GEMV_ACTS(2)
NF4_GEMV_ACTS(4)

#define NF4_GEMV_E(XN, XT, YN, YT)                                                                           \
    extern "C" __global__ __launch_bounds__(256) void cima_nf4_gemv_e_##XN##_##YN(                          \
        const XT* x, const uint8_t* packed, const float* absmax, const float* qmap, YT* y, int n, int k,     \
        int blocksize) {                                                                                     \
        nf4_gemv_e_body<XT, YT>(x, packed, absmax, qmap, y, n, k, blocksize);                                \
    }
NF4_GEMV_E(f16, uint16_t, f16, uint16_t)
NF4_GEMV_E(f32, float, f32, float)
