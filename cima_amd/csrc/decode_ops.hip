// Decode-step support kernels for gfx950 (CDNA4): the code object
// cima_decode.hsaco.  These are the non-GEMV launches of one batch-1 decode
// step of the reference's transformer family (forward_chunk_at,
// src/models/transformer.rs:1012-1300, and enqueue_decode_device,
// :1440-1461): RMSNorm, RoPE, the KV-cache append, split ("flash-decode")
// attention with its log-sum-exp merge, and the greedy argmax feedback.
//
// Every kernel reads and writes f16 activations (the engine's activation
// type) and computes in fp32.  The standalone kernels keep the reference's
// argument meaning (src/kernels.cu:37-50, 244-262, 397-454, 547-639) so they
// are drop-ins one by one; cima_attn_decode_* fuses RoPE, the KV append and
// the per-chunk attention of one layer into a single launch.
#include "gguf_formats.h"

// |v| clamped to 65000 (g_sat16, src/kernels.cu:30-35)
DEV float sat16(float v) { return fmaxf(fminf(v, 65000.f), -65000.f); }

DEV float wave_sum(float v) { return wave_sum_u(v); }
DEV float wave_max(float v) { return wave_max_u(v); }

// ------------------------------------------------------------------ RMSNorm

// y[row] = f16(sat(x) * rsqrt(mean(sat(x)^2) + eps) * w); w may be null
// (unit weight).  One 256-thread workgroup per row (k_rmsnorm,
// src/kernels.cu:37-50).
extern "C" __global__ __launch_bounds__(256) void cima_rmsnorm_f16(const uint16_t* __restrict__ x,
                                                                   const uint16_t* __restrict__ w,
                                                                   uint16_t* __restrict__ y, int n, float eps) {
    __shared__ float red[4];
    const uint16_t* xr = x + (size_t)blockIdx.x * n;
    uint16_t* yr = y + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = sat16(h2f(xr[i]));
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float g = w ? h2f(w[i]) : 1.0f;
        yr[i] = (uint16_t)f2h(sat16(h2f(xr[i])) * inv * g);
    }
}

// --------------------------------------------------------------------- RoPE

// NeoX half-split rotation of pair i (elements i and i + dim/2) at position
// p: frequency theta^(-2i/dim) (k_rope, src/kernels.cu:397-414).
DEV float rope_freq(int i, int dim, float theta) { return powf(theta, -2.0f * (float)i / (float)dim); }
DEV void rope_rot_f(float a, float b, float p, float freq, float& oa, float& ob) {
    float s, c;
    sincosf(p * freq, &s, &c);
    oa = a * c - b * s;
    ob = a * s + b * c;
}
DEV void rope_rot(float a, float b, float p, int i, int dim, float theta, float& oa, float& ob) {
    rope_rot_f(a, b, p, rope_freq(i, dim, theta), oa, ob);
}

// In place over x [rows, heads, dim]: row r sits at position pos0 + r, or
// *pos_dev + r when pos_dev is set (graph replay).  Pairs i >= nfreqs pass
// through.  Grid rows * heads, 64 threads striding the dim/2 pairs.
extern "C" __global__ __launch_bounds__(64) void cima_rope_f16(uint16_t* __restrict__ x, int heads, int dim,
                                                               int pos0, float theta, int nfreqs,
                                                               const int* __restrict__ pos_dev) {
    const int row = blockIdx.x / heads, h = blockIdx.x % heads;
    if (pos_dev) pos0 = *pos_dev;
    uint16_t* v = x + ((size_t)row * heads + h) * dim;
    const float p = (float)(pos0 + row);
    const int half = dim >> 1;
    for (int i = threadIdx.x; i < half && i < nfreqs; i += 64) {
        float oa, ob;
        rope_rot(h2f(v[i]), h2f(v[i + half]), p, i, dim, theta, oa, ob);
        v[i] = (uint16_t)f2h(oa);
        v[i + half] = (uint16_t)f2h(ob);
    }
}

// ---------------------------------------------------------------- KV append

// Rows r of k, v [rows, kv_heads*dim] go to cache [kv_heads, max_seq, dim]
// at position pos + r (or *pos_dev + r); positions >= max_seq are dropped
// rather than written out of bounds (k_kv_append, src/kernels.cu:440-454).
extern "C" __global__ __launch_bounds__(256) void cima_kv_append_f16(const uint16_t* __restrict__ k,
                                                                     const uint16_t* __restrict__ v,
                                                                     uint16_t* __restrict__ kc,
                                                                     uint16_t* __restrict__ vc, int kv_heads,
                                                                     int dim, int pos, int max_seq,
                                                                     const int* __restrict__ pos_dev) {
    const int row = blockIdx.x;
    if (pos_dev) pos = *pos_dev;
    const int at = pos + row;
    if (at < 0 || at >= max_seq) return;
    const int n = kv_heads * dim;
    for (int i = threadIdx.x; i < n; i += 256) {
        const int h = i / dim, d = i % dim;
        const size_t idx = ((size_t)h * max_seq + at) * dim + d;
        kc[idx] = k[(size_t)row * n + i];
        vc[idx] = v[(size_t)row * n + i];
    }
}

// ---------------------------------------------------------------- attention
//
// Partials: part[(head * n_chunks + chunk) * (D + 2)] = {m, l, acc[D]} with m
// the chunk's maximum score, l = sum exp(score - m), acc = sum exp(score -
// m) * v -- the reference's layout (src/kernels.cu:547-610), so the split
// and merge kernels below interoperate with it.
//
// A workgroup of 256 threads takes one chunk of at most 256 positions of
// one query head.  Every load of the chunk is issued before any of them is
// used -- thread t's key row (position s0 + t) and a 1/256 slice of the
// chunk's value rows -- so a chunk costs one memory round trip even when
// the cache is cold in HBM; the weighted value sum runs on the slices in
// registers and reduces across lanes, with no sequential loop over the
// chunk's positions.

constexpr int ATT_MAX_CSZ = 256;

// Device scratch of cima_hip_attn_decode_noalloc (the split partials of one
// call, at most 4 MiB): one copy per device that loads this code object,
// its address taken once per context with hipModuleGetGlobal.  Every call
// on a device shares it.
__device__ __align__(256) float scratch[(4 << 20) / 4];

template <int D>
struct AttnLds {
    float q[D];
    float kn[D];
    float vn[D];
    float p[ATT_MAX_CSZ];
    float red[8];
    float acc[4][D];  // one accumulator row per wave
};

// The chunk's loads, held in registers until used: thread t's key row
// (position s0 + t, clamped into the chunk) and value slice t + 256 j of the
// chunk's contiguous value rows (clamped likewise).
template <int D>
struct AttnRegs {
    uint4 k[D / 8];
    uint4 v[D / 8];
};

template <int D>
DEV void attn_issue(AttnRegs<D>& R, const uint16_t* __restrict__ kh, const uint16_t* __restrict__ vh, int s0,
                    int s1) {
    constexpr int RV = D / 8;
    const int t = threadIdx.x, len = s1 - s0;
    const uint4* kp = reinterpret_cast<const uint4*>(kh + (size_t)(s0 + min(t, len - 1)) * D);
#pragma unroll
    for (int c = 0; c < RV; c++) R.k[c] = kp[c];
    const uint4* vp = reinterpret_cast<const uint4*>(vh + (size_t)s0 * D);
#pragma unroll
    for (int j = 0; j < RV; j++) R.v[j] = vp[min(t + 256 * j, len * RV - 1)];
}

// Chunk [s0, s1) of one query head (q in L.q, fp32) from the loads in R;
// position `snew` (if in the chunk) takes its key and value from L.kn /
// L.vn.  Writes {m, l, acc} to dst.
template <int D>
DEV void attn_chunk(AttnLds<D>& L, const AttnRegs<D>& R, int s0, int s1, int snew, float scale,
                    float* __restrict__ dst) {
    constexpr int RV = D / 8;
    const int t = threadIdx.x, len = s1 - s0;
    // score of position s0 + t
    float d = 0.f;
    if (s0 + t == snew) {
#pragma unroll
        for (int e = 0; e < D; e++) d += L.q[e] * L.kn[e];
    } else {
#pragma unroll
        for (int c = 0; c < RV; c++) {
            const uint32_t w[4] = {R.k[c].x, R.k[c].y, R.k[c].z, R.k[c].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                d += L.q[8 * c + 2 * e] * h2f(w[e] & 0xffffu);
                d += L.q[8 * c + 2 * e + 1] * h2f(w[e] >> 16);
            }
        }
    }
    const bool live = t < len;
    const float sc = live ? d * scale : -INFINITY;
    const float mw = wave_max(sc);
    if ((t & 63) == 0) L.red[t >> 6] = mw;
    __syncthreads();
    const float M = fmaxf(fmaxf(L.red[0], L.red[1]), fmaxf(L.red[2], L.red[3]));
    const float e = live ? __expf(sc - M) : 0.f;
    L.p[t] = e;
    const float lw = wave_sum(e);
    if ((t & 63) == 0) L.red[4 + (t >> 6)] = lw;
    __syncthreads();
    // weighted value sum from the registers: thread t holds dims
    // [8 (t % RV), +8) of rows t / RV + (256 / RV) j; rows past the chunk
    // have p = 0, and the new position's row comes from L.vn
    const int pc = t % RV, rnew = snew - s0;
    float a[8];
#pragma unroll
    for (int i = 0; i < 8; i++) a[i] = 0.f;
#pragma unroll
    for (int j = 0; j < RV; j++) {
        const int row = t / RV + (256 / RV) * j;
        const float pr = L.p[row];
        const uint32_t w[4] = {R.v[j].x, R.v[j].y, R.v[j].z, R.v[j].w};
        if (row == rnew) {
#pragma unroll
            for (int i = 0; i < 8; i++) a[i] += pr * L.vn[8 * pc + i];
        } else {
            // rows past the chunk's live length hold clamped copies of
            // another row (possibly the new position's stale cache row,
            // which may hold anything): selected away, not multiplied by 0
            const bool live_row = row < len;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a[2 * i] += live_row ? pr * h2f(w[i] & 0xffffu) : 0.f;
                a[2 * i + 1] += live_row ? pr * h2f(w[i] >> 16) : 0.f;
            }
        }
    }
    // sum over the lanes of a wave holding the same dims (lane % RV), then
    // over the four waves
#pragma unroll
    for (int o = RV; o < 64; o <<= 1)
#pragma unroll
        for (int i = 0; i < 8; i++) a[i] += __shfl_xor(a[i], o);
    if ((t & 63) < RV) {
#pragma unroll
        for (int i = 0; i < 8; i++) L.acc[t >> 6][8 * pc + i] = a[i];
    }
    __syncthreads();
    if (t < D) dst[2 + t] = (L.acc[0][t] + L.acc[1][t]) + (L.acc[2][t] + L.acc[3][t]);
    if (t == 0) {
        dst[0] = M;
        dst[1] = (L.red[4] + L.red[5]) + (L.red[6] + L.red[7]);
    }
}

// Merge chunks [c0, active) of one head: out = sum_c e^(m_c - M) acc_c /
// sum_c e^(m_c - M) l_c (k_attn_reduce, src/kernels.cu:614-639), with a
// running maximum so every chunk is read once.  Threads t < D each produce
// one output element.
template <int D>
DEV void attn_merge(const float* __restrict__ ph, int c0, int active, uint16_t* __restrict__ oh) {
    const int t = threadIdx.x;
    if (t >= D) return;
    float M = -INFINITY, Ls = 0.f, a = 0.f;
#pragma unroll 4
    for (int c = c0; c < active; c++) {
        const float* pc = ph + (size_t)c * (D + 2);
        const float m = pc[0], l = pc[1], v = pc[2 + t];
        const float Mn = fmaxf(M, m);
        const float so = __expf(M - Mn), sn = __expf(m - Mn);
        Ls = Ls * so + l * sn;
        a = a * so + v * sn;
        M = Mn;
    }
    oh[t] = (uint16_t)f2h(a / Ls);
}

// Live length and first position of the attention window: seq = *pos_dev +
// 1 when pos_dev is set, capped at max_seq; window > 0 keeps the last
// `window` positions.
DEV void attn_range(int& seq, int max_seq, int window, const int* pos_dev, int& wlo) {
    if (pos_dev) seq = *pos_dev + 1;
    seq = min(seq, max_seq);
    wlo = (window > 0 && seq > window) ? seq - window : 0;
}

// Split decode attention (k_attn_decode_split, src/kernels.cu:547-610): one
// workgroup per (query head, chunk of csz <= 256 positions); q [q_heads, D]
// f16 already rotated; GQA maps head h to kv head h / (q_heads / kv_heads).
// Chunks past the live length write nothing.
template <int D>
DEV void attn_split_body(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
                         const uint16_t* __restrict__ vc, float* __restrict__ part, int q_heads, int kv_heads,
                         int seq, int max_seq, int csz, int n_chunks, float scale, int window,
                         const int* __restrict__ pos_dev) {
    __shared__ AttnLds<D> L;
    int wlo;
    attn_range(seq, max_seq, window, pos_dev, wlo);
    const int h = blockIdx.x / n_chunks, ci = blockIdx.x % n_chunks;
    const int s0 = max(ci * csz, wlo), s1 = min(ci * csz + csz, seq);
    if (s0 >= s1) return;
    const int kvh = h / (q_heads / kv_heads);
    AttnRegs<D> R;
    attn_issue<D>(R, kc + (size_t)kvh * max_seq * D, vc + (size_t)kvh * max_seq * D, s0, s1);
    if (threadIdx.x < D) L.q[threadIdx.x] = h2f(q[(size_t)h * D + threadIdx.x]);
    __syncthreads();
    attn_chunk<D>(L, R, s0, s1, -1, scale, part + ((size_t)h * n_chunks + ci) * (D + 2));
}

template <int D>
DEV void attn_reduce_body(const float* __restrict__ part, uint16_t* __restrict__ out, int csz, int n_chunks,
                          int seq, int max_seq, int window, const int* __restrict__ pos_dev) {
    int wlo;
    attn_range(seq, max_seq, window, pos_dev, wlo);
    const int h = blockIdx.x;
    const int active = min((seq + csz - 1) / csz, n_chunks);
    attn_merge<D>(part + (size_t)h * n_chunks * (D + 2), wlo / csz, active, out + (size_t)h * D);
}

// Decode attention partials of one layer at position pos = *pos_dev, with
// RoPE and the KV append folded in (replaces k_rope x2 + k_kv_append +
// k_attn_decode_split, src/models/transformer.rs:1100-1160):
//   qkv = [q (q_heads*D) | k (kv_heads*D) | v (kv_heads*D)] f16, the output
//   of the fused q/k/v GEMV (biases applied, RoPE not yet).
//
// One workgroup of CP / 16 waves per (kv head, group of up to AT_GMAX of
// its query heads, chunk of csz <= CP positions): the chunk's keys and
// values are read once for every query head that shares them (GQA).
// Everything the workgroup reads is addressed without the position -- the
// chunk's cache rows, the group's q, the new k and v -- so those loads go
// out together with the load of *pos_dev and the kernel pays one memory
// round trip; rows past the live length are selected away (never
// multiplied: they may hold anything).  The chunk holding pos takes the new
// position's key and value from LDS and, in the first head group, appends
// them to the cache.  window > 0 keeps the last `window` positions (the
// split kernel's wlo, src/kernels.cu:557-559).
//
// Both contractions run on the matrix cores.  Scores: wave w takes
// positions [16 w, 16 w + 16) and computes S^T = K Q^T with f16 MFMA
// (16x16x16, fp32 accumulate; K and the f16-rounded rotated q are exact
// f16 operands, so this is the fp32 dot of the reference up to summation
// order); its key rows go straight from HBM into the A operand (lane l:
// row l % 16, a contiguous D/4-dim slice, the k order permuted alike in A
// and B).  Softmax: wave h < g, head h, over the chunk, with DPP
// reductions.  Value sum: O^T = V^T P^T with fp32 MFMA (16x16x4): the
// probabilities stay fp32, V^T is read from the LDS copy of the value rows;
// waves split dims into 16-wide tiles and, where waves outnumber tiles,
// positions into ranges whose partial sums add through LDS in a fixed
// order.
constexpr int AT_GMAX = 8;                      // query heads per workgroup

typedef _Float16 at_half4 __attribute__((ext_vector_type(4)));
typedef float at_float4 __attribute__((ext_vector_type(4)));

template <int D, int CP>
struct AttnLds2 {
    static constexpr int NW = CP / 16;          // waves
    static constexpr int TT = D / 16;           // 16-dim tiles of the value sum
    static constexpr int NS = NW >= TT ? NW / TT : 1;  // position ranges of the value sum
    static constexpr int VS = D + 16;           // f16 stride of a value row (padded: no bank conflicts)
    static constexpr int QS = D + 8;            // f16 stride of a query row
    static constexpr int PS = 17;               // fp32 stride of a probability row
    uint16_t q[16][QS];                         // rotated queries, f16; rows >= g zero
    uint16_t kn[D];                             // the new position's rotated key, f16
    float vn[D];                                // the new position's value
    float p[CP][PS];                            // per position: scores, then e^(s - m), per head
    float ml[AT_GMAX][2];                       // per head: m, l
    uint16_t v[CP][VS];                         // the chunk's value rows (dead rows zero)
    float red[NS][D][16];                       // value-sum partials per position range
};

template <int D, int CP>
DEV void attn_fused_body(const uint16_t* __restrict__ qkv, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                         float* __restrict__ part, int q_heads, int kv_heads, int max_seq, int csz, int n_chunks,
                         float theta, float scale, int window, const int* __restrict__ pos_dev) {
    extern __shared__ __align__(16) uint8_t at_lds[];
    using Lds = AttnLds2<D, CP>;
    Lds& L = *reinterpret_cast<Lds*>(at_lds);
    constexpr int NW = Lds::NW, TT = Lds::TT, NS = Lds::NS;
    constexpr int TPW = NW >= TT ? 1 : TT / NW;  // value-sum tiles per wave
    constexpr int PR = CP / NS;                  // positions per value-sum range
    constexpr int KD = D / 4;                    // key dims per lane (A operand)
    constexpr int NK = KD / 8;                   // uint4 per lane
    constexpr int NT = 4 * CP;                   // threads
    static_assert(NW * 64 == NT && TT % (NW >= TT ? 1 : NW) == 0 && PR % 4 == 0, "attention tile shape");
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int lr = lane & 15, lg = lane >> 4;    // MFMA row / column (lr), lane group (lg)
    const int grp = q_heads / kv_heads;
    const int hgs = (grp + AT_GMAX - 1) / AT_GMAX;
    const int ci = blockIdx.x % n_chunks;
    const int hg = (blockIdx.x / n_chunks) % hgs;
    const int kvh = blockIdx.x / n_chunks / hgs;
    const int qh0 = kvh * grp + hg * AT_GMAX;
    const int g = min(AT_GMAX, grp - hg * AT_GMAX);
    const int s0 = ci * csz;
    uint16_t* kh = kc + (size_t)kvh * max_seq * D;
    uint16_t* vh = vc + (size_t)kvh * max_seq * D;

    // ---- loads that do not depend on the position
    // key rows in the A layout: lane l of wave w holds dims [KD lg, +KD) of
    // position s0 + 16 w + lr
    const int kp = 16 * wave + lr;
    uint4 kr[NK];
    {
        const int row = min(s0 + min(kp, csz - 1), max_seq - 1);
        const uint4* src = reinterpret_cast<const uint4*>(kh + (size_t)row * D + KD * lg);
#pragma unroll
        for (int j = 0; j < NK; j++) kr[j] = src[j];
    }
    // value rows, contiguous: thread t holds 16 bytes (8 dims) of row
    // t / (D / 8), for CP * D / 8 / NT row slices per thread
    constexpr int VPT = CP * (D / 8) / NT;       // = D / 32
    uint4 vr[VPT];
#pragma unroll
    for (int j = 0; j < VPT; j++) {
        const int e = t + NT * j, r = e / (D / 8), c8 = e % (D / 8);
        const int row = min(s0 + min(r, csz - 1), max_seq - 1);
        vr[j] = reinterpret_cast<const uint4*>(vh + (size_t)row * D)[c8];
    }
    // rotation operands: item e < g*D/2 is pair e % (D/2) of query head
    // e / (D/2); the next D/2 items the new key's pairs; the next D the new
    // value (thread t takes items t, t + NT, ...)
    const int nq = g * (D / 2);
    constexpr int RI = (AT_GMAX * (D / 2) + D / 2 + D + NT - 1) / NT;  // items per thread
    uint32_t ra[RI], rb[RI];
#pragma unroll
    for (int j = 0; j < RI; j++) {
        const int e = t + NT * j;
        ra[j] = rb[j] = 0;
        if (e < nq) {
            const uint16_t* qh = qkv + (size_t)(qh0 + e / (D / 2)) * D;
            ra[j] = qh[e % (D / 2)];
            rb[j] = qh[e % (D / 2) + D / 2];
        } else if (e < nq + D / 2) {
            const uint16_t* kn = qkv + (size_t)q_heads * D + (size_t)kvh * D;
            ra[j] = kn[e - nq];
            rb[j] = kn[e - nq + D / 2];
        } else if (e < nq + D / 2 + D) {
            ra[j] = qkv[(size_t)(q_heads + kv_heads) * D + (size_t)kvh * D + (e - nq - D / 2)];
        }
    }
    // the rotation frequencies do not depend on the position either
    float fq[RI];
#pragma unroll
    for (int j = 0; j < RI; j++) {
        const int e = t + NT * j;
        fq[j] = e < nq + D / 2 ? rope_freq(e < nq ? e % (D / 2) : e - nq, D, theta) : 0.f;
    }
    const int pos = *pos_dev;
    const int seq = min(pos + 1, max_seq);
    const int wlo = (window > 0 && seq > window) ? seq - window : 0;
    const int lo = max(s0, wlo), hi = min(s0 + csz, seq);
    if (lo >= hi) return;
    const bool has_new = pos < max_seq && s0 <= pos && pos < s0 + csz;
    auto live = [&](int r) { return r < csz && s0 + r >= lo && s0 + r < hi; };

    // ---- RoPE of the group's queries and the new key; the append; rows
    // g..15 of the query block are zero
    const float fp = (float)pos;
#pragma unroll
    for (int j = 0; j < RI; j++) {
        const int e = t + NT * j;
        if (e < nq) {
            const int h = e / (D / 2), i = e % (D / 2);
            float oa, ob;
            rope_rot_f(h2f(ra[j]), h2f(rb[j]), fp, fq[j], oa, ob);
            L.q[h][i] = (uint16_t)f2h(oa);
            L.q[h][i + D / 2] = (uint16_t)f2h(ob);
        } else if (has_new && e < nq + D / 2) {
            const int i = e - nq;
            float oa, ob;
            rope_rot_f(h2f(ra[j]), h2f(rb[j]), fp, fq[j], oa, ob);
            const uint32_t ha = f2h(oa), hb = f2h(ob);
            L.kn[i] = (uint16_t)ha;
            L.kn[i + D / 2] = (uint16_t)hb;
            if (hg == 0) {
                kh[(size_t)pos * D + i] = (uint16_t)ha;
                kh[(size_t)pos * D + i + D / 2] = (uint16_t)hb;
            }
        } else if (has_new && e < nq + D / 2 + D) {
            const int i = e - nq - D / 2;
            L.vn[i] = h2f(ra[j]);
            if (hg == 0) vh[(size_t)pos * D + i] = (uint16_t)ra[j];
        }
    }
    for (int e = t; e < (16 - g) * D; e += NT) L.q[g + e / D][e % D] = 0;
    __syncthreads();

    // ---- value rows -> LDS (dead rows as zeros; the new position from vn)
#pragma unroll
    for (int j = 0; j < VPT; j++) {
        const int e = t + NT * j, r = e / (D / 8), c8 = e % (D / 8);
        uint4 w = vr[j];
        if (has_new && s0 + r == pos) {
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; k++) o[k] = f2h2(L.vn[8 * c8 + 2 * k], L.vn[8 * c8 + 2 * k + 1]);
            w = make_uint4(o[0], o[1], o[2], o[3]);
        }
        if (!live(r)) w = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(&L.v[r][8 * c8]) = w;
    }

    // ---- scores S^T (positions x heads) of wave `wave`'s 16 positions
    if (has_new && s0 + kp == pos) {
#pragma unroll
        for (int j = 0; j < NK; j++) kr[j] = reinterpret_cast<const uint4*>(&L.kn[KD * lg])[j];
    }
    at_float4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NK; j++) {
        const uint4 qv = *reinterpret_cast<const uint4*>(&L.q[lr][KD * lg + 8 * j]);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(at_half4, make_uint2(kr[j].x, kr[j].y)),
                                                     __builtin_bit_cast(at_half4, make_uint2(qv.x, qv.y)), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(at_half4, make_uint2(kr[j].z, kr[j].w)),
                                                     __builtin_bit_cast(at_half4, make_uint2(qv.z, qv.w)), acc, 0, 0, 0);
    }
    // lane l holds S[position 16 wave + 4 lg + i][head lr]
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 16 * wave + 4 * lg + i;
        L.p[r][lr] = live(r) ? acc[i] * scale : -INFINITY;
    }
    __syncthreads();

    // ---- softmax of heads wave, wave + NW, ... over the chunk
    for (int h = wave; h < g; h += NW) {
        constexpr int SP = CP / 64;      // scores per lane
        float sc[SP];
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < SP; i++) {
            sc[i] = L.p[lane + 64 * i][h];
            m = fmaxf(m, sc[i]);
        }
        m = wave_max_u(m);
        float l = 0.f;
#pragma unroll
        for (int i = 0; i < SP; i++) {
            const float e = sc[i] == -INFINITY ? 0.f : __expf(sc[i] - m);
            L.p[lane + 64 * i][h] = e;
            l += e;
        }
        l = wave_sum_u(l);
        if (lane == 0) {
            L.ml[h][0] = m;
            L.ml[h][1] = l;
        }
    }
    __syncthreads();

    // ---- value sum O^T (dims x heads): tile(s) of 16 dims over a range of
    // PR positions, 4 positions per fp32 MFMA step
    {
        const int split = NW >= TT ? wave / TT : 0;
        const int tile0 = NW >= TT ? wave % TT : wave * TPW;
        // the range's operands read first, then four independent MFMA
        // chains (steps st % 4) summed in a fixed order
        constexpr int NST = PR / 4;
        const int pb = split * PR;
        float pv[NST], vv[TPW][NST];
#pragma unroll
        for (int st = 0; st < NST; st++) {
            const int r = pb + 4 * st + lg;
            pv[st] = L.p[r][lr];
#pragma unroll
            for (int u = 0; u < TPW; u++) vv[u][st] = h2f(L.v[r][16 * (tile0 + u) + lr]);
        }
        at_float4 o[TPW];
#pragma unroll
        for (int u = 0; u < TPW; u++) {
            at_float4 oc[4];
#pragma unroll
            for (int c = 0; c < 4; c++) oc[c] = (at_float4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < NST; st++)
                oc[st & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[u][st], pv[st], oc[st & 3], 0, 0, 0);
            o[u] = (oc[0] + oc[1]) + (oc[2] + oc[3]);
        }
        // lane l holds O[dim 16 tile + 4 lg + i][head lr]
#pragma unroll
        for (int u = 0; u < TPW; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) L.red[split][16 * (tile0 + u) + 4 * lg + i][lr] = o[u][i];
    }
    __syncthreads();
    for (int e = t; e < g * D; e += NT) {
        const int h = e / D, d = e % D;
        float s = 0.f;
#pragma unroll
        for (int sp = 0; sp < NS; sp++) s += L.red[sp][d][h];
        float* dst = part + ((size_t)(qh0 + h) * n_chunks + ci) * (D + 2);
        dst[2 + d] = s;
        if (d == 0) {
            dst[0] = L.ml[h][0];
            dst[1] = L.ml[h][1];
        }
    }
}

// cima_attn_decode_d<D>_c<CP>: 4 CP threads, chunks of up to CP positions
#define ATTN_FUSED(D, CP)                                                                                        \
    extern "C" __global__ __launch_bounds__(4 * CP) void cima_attn_decode_d##D##_c##CP(                          \
        const uint16_t* qkv, uint16_t* kc, uint16_t* vc, float* part, int q_heads, int kv_heads, int max_seq,    \
        int csz, int n_chunks, float theta, float scale, int window, const int* pos_dev) {                       \
        attn_fused_body<D, CP>(qkv, kc, vc, part, q_heads, kv_heads, max_seq, csz, n_chunks, theta, scale,       \
                               window, pos_dev);                                                                 \
    }

#define ATTN_KERNELS(D)                                                                                          \
    extern "C" __global__ __launch_bounds__(256) void cima_attn_split_d##D(                                      \
        const uint16_t* q, const uint16_t* kc, const uint16_t* vc, float* part, int q_heads, int kv_heads,       \
        int seq, int max_seq, int csz, int n_chunks, float scale, int window, const int* pos_dev) {              \
        attn_split_body<D>(q, kc, vc, part, q_heads, kv_heads, seq, max_seq, csz, n_chunks, scale, window,       \
                           pos_dev);                                                                             \
    }                                                                                                            \
    extern "C" __global__ __launch_bounds__(256) void cima_attn_reduce_d##D(                                     \
        const float* part, uint16_t* out, int csz, int n_chunks, int seq, int max_seq, int window,               \
        const int* pos_dev) {                                                                                    \
        attn_reduce_body<D>(part, out, csz, n_chunks, seq, max_seq, window, pos_dev);                            \
    }                                                                                                            \
    ATTN_FUSED(D, 64) ATTN_FUSED(D, 128) ATTN_FUSED(D, 256)

ATTN_KERNELS(64)
ATTN_KERNELS(128)

// ------------------------------------------------------------ greedy argmax

// slot = max over i of (orderable(f32 bits of v_i) << 32 | i), v_i = x_i or
// cap * tanh(x_i / cap) when cap > 0: one u64 atomic max per workgroup
// resolves value and index together, ties going to the higher index
// (k_argmax_softcap, src/kernels.cu:244-262).  slot must hold 0 on entry.
DEV unsigned long long umax64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

extern "C" __global__ __launch_bounds__(256) void cima_argmax_f16(const uint16_t* __restrict__ x,
                                                                  unsigned long long* __restrict__ slot, int n,
                                                                  float cap) {
    __shared__ unsigned long long red[4];
    unsigned long long best = 0ull;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        float v = h2f(x[i]);
        if (cap > 0.f) v = cap * tanhf(v / cap);
        uint32_t b = __builtin_bit_cast(uint32_t, v);
        b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
        best = umax64(best, ((unsigned long long)b << 32) | (uint32_t)i);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)best, o), hi = __shfl_xor((uint32_t)(best >> 32), o);
        best = umax64(best, ((unsigned long long)hi << 32) | lo);
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) atomicMax(slot, umax64(umax64(red[0], red[1]), umax64(red[2], red[3])));
}

// ids[0] = index held in slot; slot back to 0 for the next argmax; and, if
// pos_dev is set, *pos_dev += 1 (k_argmax_extract + k_pos_bump,
// src/kernels.cu:309-318).
extern "C" __global__ void cima_argmax_to_ids(unsigned long long* __restrict__ slot, unsigned* __restrict__ ids,
                                              int* __restrict__ pos_dev) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    if (ids) ids[0] = (unsigned)(*slot);
    *slot = 0ull;
    if (pos_dev) *pos_dev += 1;
}

extern "C" __global__ void cima_pos_bump(int* __restrict__ pos_dev) {
    if (blockIdx.x == 0 && threadIdx.x == 0) *pos_dev += 1;
}
