// Dequantisation to f16 and packed embedding gather (gfx950 code object
// cima_dequant.hsaco): one thread per unit of a block, bit-exact with the
// host decoders (src/quant.rs:599-896).
#include <type_traits>

#include "gguf_formats.h"

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
DQ_KERNELS(q4_1, FQ4_1)
DQ_KERNELS(q5_0, FQ5_0)
DQ_KERNELS(q5_1, FQ5_1)
DQ_KERNELS(q4_k, FQ4_K)
DQ_KERNELS(q5_k, FQ5_K)
DQ_KERNELS(q6_k, FQ6_K)
DQ_KERNELS(iq4_xs, FIQ4_XS)



// ------------------------------------------------------ bandwidth reference
// Streaming reads that fold the data into a value stored only if it
// matches an improbable pattern: the plain HBM read ceiling the GEMVs are
// measured against, in a family swept over the three things that set a
// read's pace on gfx950 -- loads in flight per lane, load width and the
// destination (registers, or LDS through global_load_lds_dwordx4) -- the
// host choosing workgroups per CU (cima_hip_stream_read_cfg).
//
// Register reads: grid-stride over W-byte words, NL independent loads per
// thread in flight.
typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));
typedef uint32_t v2u_t __attribute__((ext_vector_type(2)));
template <int NL, int W>
DEV void stream_read_reg(const uint8_t* __restrict__ src, long long nbytes, uint32_t* __restrict__ sink) {
    using V = typename std::conditional<W == 16, v4u_t, v2u_t>::type;
    const V* p = reinterpret_cast<const V*>(src);
    const long long nw = nbytes / W;
    const long long nt = (long long)gridDim.x * 256;
    long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (NL - 1) * nt < nw; i += NL * nt) {
        V a[NL];
#pragma unroll
        for (int j = 0; j < NL; j++) a[j] = __builtin_nontemporal_load(p + i + j * nt);
#pragma unroll
        for (int j = 0; j < NL; j++) acc ^= a[j].x + a[j].y;
    }
    for (; i < nw; i += nt) {
        const V a = __builtin_nontemporal_load(p + i);
        acc ^= a.x ^ a.y;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// Direct-to-LDS reads: each wave streams 1 KB runs (64 lanes x 16 B,
// grid-stride over waves) through a ring of D 1 KB slots in LDS, D copies in
// flight, each slot read back once (the GEMV's _dma loop without the dot).
DEV void dma16_rd(const void* g, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
template <int N>
DEV void wait_vm_rd() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
template <int D>
DEV void stream_read_lds(const uint8_t* __restrict__ src, long long nbytes, uint32_t* __restrict__ sink) {
    __shared__ __align__(16) uint8_t ring[4][D * 1024];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const long long nch = nbytes >> 10;  // whole 1 KB runs (the tail < 1 KB is not read)
    const long long W = (long long)gridDim.x * 4, g = (long long)blockIdx.x * 4 + wave;
    const long long per = g < nch ? (nch - 1 - g) / W + 1 : 0;
    const uint32_t base = (uint32_t)(uintptr_t)&ring[wave][0];
    auto at = [&](long long q) { return src + (min(g + q * W, nch - 1) << 10) + 16 * lane; };
    uint32_t acc = 0;
    if (per > 0) {
#pragma unroll
        for (int d = 0; d < D; d++) dma16_rd(at(d), base + d * 1024);
        long long i = 0;
        for (; i + D <= per; i += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                wait_vm_rd<D - 1>();
                const uint2 v = *reinterpret_cast<const uint2*>(&ring[wave][d * 1024 + 16 * lane]);
                acc ^= v.x + v.y;
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                dma16_rd(at(i + d + D), base + d * 1024);
            }
        }
        wait_vm_rd<0>();
        for (int d = 0; i + d < per; d++) {
            const uint2 v = *reinterpret_cast<const uint2*>(&ring[wave][d * 1024 + 16 * lane]);
            acc ^= v.x + v.y;
        }
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// cima_stream_read: four 16-byte loads in flight per thread (the default
// of cima_hip_stream_read: of the patterns measured on MI355X, cold, the
// fastest or within 2% of it at 33, 62 and 431 MB with two workgroups per
// CU: 6.5 / 10.6 / 63.0 us, against 7.0-9.2 / 11.1-13.7 / 66 us for 8 or 16
// loads in flight or one workgroup per CU, and 6.9-8.2 / 10.9-12.4 /
// 68-78 us for direct-to-LDS rings of 8-32 KB per wave)
extern "C" __global__ __launch_bounds__(256) void cima_stream_read(const uint8_t* __restrict__ src, long long nbytes,
                                                                   uint32_t* __restrict__ sink) {
    stream_read_reg<4, 16>(src, nbytes, sink);
}
#define STREAM_READ_REG(NL, W)                                                                              \
    extern "C" __global__ __launch_bounds__(256) void cima_stream_read_r##NL##_w##W(                      \
        const uint8_t* __restrict__ src, long long nbytes, uint32_t* __restrict__ sink) {                  \
        stream_read_reg<NL, W>(src, nbytes, sink);                                                          \
    }
STREAM_READ_REG(1, 16)
STREAM_READ_REG(2, 16)
STREAM_READ_REG(4, 16)
STREAM_READ_REG(8, 16)
STREAM_READ_REG(16, 16)
STREAM_READ_REG(4, 8)
STREAM_READ_REG(8, 8)
STREAM_READ_REG(16, 8)
#define STREAM_READ_LDS(D)                                                                                   \
    extern "C" __global__ __launch_bounds__(256) void cima_stream_read_l##D(                               \
        const uint8_t* __restrict__ src, long long nbytes, uint32_t* __restrict__ sink) {                  \
        stream_read_lds<D>(src, nbytes, sink);                                                               \
    }
STREAM_READ_LDS(2)
STREAM_READ_LDS(4)
STREAM_READ_LDS(8)
STREAM_READ_LDS(16)
