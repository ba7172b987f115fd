// Host side of the C ABI declared in include/cima_hip.h.
//
// The library loads seven gfx950 code objects (kModuleFiles, built from the
// .hip sources with hipcc --genco) through hipModuleLoad and launches their
// kernels with hipModuleLaunchKernel -- the HIP counterpart of the
// reference's CudaCtx (src/cuda.rs), which JIT-compiles kernels.cu with
// NVRTC and launches through cuLaunchKernel (src/cuda.rs:1112-1151).  No
// call allocates device memory, and no library kernel runs: every GEMV and
// GEMM, the bitsandbytes prefill included, is this project's own.
#include "cima_hip.h"

#include <hip/hip_runtime.h>

#include <dlfcn.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdint.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <unordered_map>

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail((int)e, "hip: %s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

struct Fmt {
    const char* name;
    int block_elems;  // elements per block
    int block_bytes;  // bytes per block
    int unit_elems;   // elements one lane decodes per dequant/gather step
    int w_align;      // required alignment of the weight base pointer
    int gemv_unit;    // elements one lane decodes per GEMV step
    int pad_shift;    // GEMV x staging: 16 B of LDS padding per 2^pad_shift elements
    int gemv_module;  // code object holding the format's GEMVs (kModuleFiles)
};

const Fmt* fmt_of(int t) {
    static const Fmt q8_0 = {"q8_0", 32, 34, 32, 2, 32, 5, 0};
    static const Fmt q4_0 = {"q4_0", 32, 18, 32, 2, 32, 5, 0};
    static const Fmt q4_1 = {"q4_1", 32, 20, 32, 4, 32, 5, 2};
    static const Fmt q5_0 = {"q5_0", 32, 22, 32, 2, 32, 5, 2};
    static const Fmt q5_1 = {"q5_1", 32, 24, 32, 8, 32, 5, 2};
    static const Fmt q4_k = {"q4_k", 256, 144, 32, 16, 64, 6, 0};
    static const Fmt q5_k = {"q5_k", 256, 176, 32, 16, 64, 6, 1};
    static const Fmt q6_k = {"q6_k", 256, 210, 64, 2, 64, 6, 1};
    static const Fmt iq4_xs = {"iq4_xs", 256, 136, 32, 8, 64, 6, 2};
    switch (t) {
    case CIMA_GGML_Q8_0: return &q8_0;
    case CIMA_GGML_Q4_0: return &q4_0;
    case CIMA_GGML_Q4_1: return &q4_1;
    case CIMA_GGML_Q5_0: return &q5_0;
    case CIMA_GGML_Q5_1: return &q5_1;
    case CIMA_GGML_Q4_K: return &q4_k;
    case CIMA_GGML_Q5_K: return &q5_k;
    case CIMA_GGML_Q6_K: return &q6_k;
    case CIMA_GGML_IQ4_XS: return &iq4_xs;
    default: return nullptr;
    }
}

const int kFormats[] = {CIMA_GGML_Q8_0, CIMA_GGML_Q4_0, CIMA_GGML_Q4_1, CIMA_GGML_Q5_0, CIMA_GGML_Q5_1,
                        CIMA_GGML_Q4_K, CIMA_GGML_Q5_K, CIMA_GGML_Q6_K, CIMA_GGML_IQ4_XS};
// prefill GEMM token-tile widths the code object is built for
const int kGemmBN[] = {16, 32, 64, 128, 256};

// (lanes per row, unit steps) of the direct-to-LDS streaming GEMVs built
const int kDmaShapes[][2] = {{64, 1}, {64, 2}, {32, 1}, {32, 2}, {16, 1}};
// which depths are built: one item in flight everywhere; two for the
// gate+up pair and for the short-row shapes (one unit at 16 or 32 lanes)
bool dma_built(int lpr, int iters, int depth, bool pair) {
    return depth == 1 || pair || (iters == 1 && lpr <= 32);
}

// (rows, unit steps) pairs the code object is built for (R * ITERS <= 8)
const int kShapes[][2] = {{1, 1}, {1, 2}, {1, 4}, {1, 8}, {2, 1}, {2, 2}, {2, 4}};

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int pow2_ceil(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}
int log2i(int v) {
    int s = 0;
    while ((1 << s) < v) s++;
    return s;
}

}  // namespace

struct cima_hip_ctx {
    int device = 0;
    int num_cu = 0;
    int max_lds = 0;  // bytes of LDS one workgroup may use
    hipModule_t modules[7] = {};  // kModuleFiles
    bool loaded = false;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::unordered_map<std::string, hipFunction_t> fns;
    // tuning overrides (0 = heuristic): rows per lane group, lanes per group
    int tune_rows = 0;
    int tune_lpr = 0;
    int tune_wgs = 0;  // workgroups per CU of the persistent grid (0 = built-in default)
    int tune_gemm_bn = 0;  // prefill GEMM token tile (0 = smallest built one covering m)
    int tune_ring = 0;     // GEMV main loop: 0 = heuristic, 1 = item ring where built, 2 = never
    int tune_ringl = 0;    // stepped ring: 0 = heuristic (8 units per lane), 1 = from 2 units per lane, 2 = never
    int tune_dma = 0;      // direct-to-LDS streaming GEMV: 0 = heuristic, 1 = wherever built, 2 = never
    int tune_ksplit = 0;   // 16-token GEMM k-split with a slab: 0 = heuristic, 1 = never, 2/4/8 = that many
    int tune_wsplit = 0;   // GEMV rows split over the workgroup's waves: 0 = heuristic, 1 = always, 2 = never
    int tune_nf4_rows = 0;  // NF4 GEMV rows per wave (0 = heuristic, else 1, 2 or 4)
    int tune_nf4_kernel = 0;  // NF4 GEMV: 0 = heuristic, 1 = LDS pair table, 2 = register codebook
    // this device's copy of the decode code object's `scratch` array
    // (cima_hip_attn_decode_noalloc), found by name at init
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // this context's copy of the GEMM code object's X range flags
    // (cima_gemm_status, read by cima_hip_gemm_status)
    unsigned* gemm_status = nullptr;
    bool gemm_xcheck = true;  // CIMA_GEMM_XCHECK=0 at init switches the X range check off
};

namespace {

int get_fn(cima_hip_ctx* ctx, const std::string& name, hipFunction_t* f) {
    auto it = ctx->fns.find(name);
    if (it == ctx->fns.end()) return fail(CIMA_E_NO_KERNEL, "kernel %s is not in the code object", name.c_str());
    *f = it->second;
    return 0;
}

int launch(cima_hip_ctx* ctx, hipFunction_t f, unsigned grid, unsigned block, void** args, const char* what,
           unsigned lds = 0) {
    hipError_t e = hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, lds, ctx->stream, args, nullptr);
    if (e != hipSuccess) return hip_fail(e, what);
    return 0;
}

// code objects: the GEMVs in three (format sets compiled in parallel),
// the prefill GEMMs, dequant / gather, the decode-step kernels
enum { MOD_GEMM = 3, MOD_DEQUANT = 4, MOD_DECODE = 5, MOD_BNB4 = 6, NUM_MODULES = 7 };
const char* const kModuleFiles[NUM_MODULES] = {"cima_gemv_a.hsaco", "cima_gemv_b.hsaco", "cima_gemv_c.hsaco",
                                               "cima_gemm.hsaco",   "cima_dequant.hsaco", "cima_decode.hsaco",
                                               "cima_bnb4.hsaco"};

// decode-step kernels (cima_decode.hsaco)
const char* const kDecodeKernels[] = {
    "cima_rmsnorm_f16",     "cima_rope_f16",        "cima_kv_append_f16",    "cima_attn_split_d64",
    "cima_attn_reduce_d64", "cima_attn_split_d128", "cima_attn_reduce_d128", "cima_attn_decode_d64_c64",
    "cima_attn_decode_d64_c128", "cima_attn_decode_d64_c256", "cima_attn_decode_d128_c64",
    "cima_attn_decode_d128_c128", "cima_attn_decode_d128_c256", "cima_argmax_f16", "cima_argmax_to_ids",
    "cima_pos_bump"};

std::string default_code_dir() {
    Dl_info info;
    if (dladdr((void*)&cima_hip_init, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t s = p.rfind('/');
        return s == std::string::npos ? std::string(".") : p.substr(0, s);
    }
    return ".";
}

void unload(cima_hip_ctx* ctx) {
    for (auto& m : ctx->modules) {
        if (m) (void)hipModuleUnload(m);
        m = nullptr;
    }
    ctx->loaded = false;
}

// kernel-argument mirror of GemvExt in gguf_gemv.hip (same member order)
struct GemvExt {
    const void* norm_w;
    float eps;
    int att_chunks;
    int att_csz;
    int att_dim;
    int max_seq;
    const int* pos_dev;
    unsigned long long* slot;
    int att_window;
};

// extra x source / epilogue of a decode-step GEMV
enum GemvKind { GK_PLAIN = 0, GK_ATT = 1, GK_AMAX = 2 };

// threads per GEMV workgroup when a kernel does not state it (GNT in
// gguf_gemv.hip; the launch uses each kernel's own __launch_bounds__)
const int kGemvThreads = 256;

struct GemvPlan {
    int rows;        // R: rows per lane group
    int iters;       // unit steps per row and lane
    int lpr_shift;   // log2 of lanes per group (16..64, inside one wave)
    unsigned grid;   // workgroups (of `threads` threads)
    unsigned lds;    // dynamic LDS bytes: x as two int8 planes + padding, scales, sums
    bool ring;       // item-ring main loop (_ring kernels)
    bool ringl;      // stepped item ring for long rows (_ringl kernels, launched with one unit per step)
};

// matches xstage_bytes() in gguf_gemv.hip
size_t gemv_lds_bytes(const Fmt* F, int k) {
    size_t kk = (size_t)k;
    return 2 * kk + 16 * (kk >> F->pad_shift) + 4 * (kk >> 5) + 4 * (kk >> 4);
}

bool have_shape(int r, int it) {
    for (const auto& sh : kShapes)
        if (sh[0] == r && sh[1] == it) return true;
    return false;
}

// Lanes per group: a power of two in [16, 64] such that a row takes at most
// 8 unit steps; rows per group: as many as the built shapes allow (up to 4,
// 2 for the SwiGLU pair, which streams two weights per output row) while
// every CU still gets >= 8 groups.  The grid covers every row group once
// with groups dealt out evenly, capped at what fits on the device at once.
GemvPlan plan_gemv(const cima_hip_ctx* ctx, const Fmt* F, int n, int k, bool pair) {
    int units = k / F->gemv_unit;
    int lpr = pow2_ceil(units);
    if (lpr < 16) lpr = 16;
    if (lpr > 64) lpr = 64;
    if (ctx->tune_lpr) lpr = ctx->tune_lpr > 64 ? 64 : ctx->tune_lpr;
    int iters = (units + lpr - 1) / lpr;
    int it = 1;
    while (it < iters) it <<= 1;
    int rows = 1;  // measured fastest for every decode shape; 2 is kept for tuning
    if (ctx->tune_rows && have_shape(ctx->tune_rows, it)) rows = ctx->tune_rows;
    long row_groups = ((long)n + rows - 1) / rows;
    // the item-ring loop for large matrices of one- or two-unit rows (measured
    // faster from about 8 MB of weights up; smaller ones are latency-bound
    // and finish sooner with the plain double buffer)
    const double wbytes = (double)n * (double)(k / F->block_elems) * F->block_bytes;
    const bool big = ctx->tune_ring == 1 || (ctx->tune_ring == 0 && wbytes >= 8e6);
    // the longest rows of large matrices (8 units per lane): the stepped
    // ring, one unit per lane and step.  Measured on MI355X at 4096x14336:
    // Q8_0 18.3 -> 16.8 us, Q6_K 17.7 -> 15.5, Q4_0 13.7 -> 12.4; at 4
    // units per lane the double buffer stays faster (Q4_K 9.6 against
    // 11.6, Q5_K 12.9 against 13.9, Q8_0 14336x8192 28.5 against 29.4).
    const bool ringl = !pair && rows == 1 && big && ctx->tune_ringl != 2 &&
                       (it == 8 || (ctx->tune_ringl == 1 && it >= 2));
    // (the gate+up pair too: measured on MI355X, same process, Q4_K
    // 2x14336x4096 14.5 -> 13.8 us cold, Q8_0 27.9 -> 27.5, against the
    // row-group double buffer; bit-identical)
    const bool ring = rows == 1 && it <= 2 && big && !ringl;
    return GemvPlan{rows, it, log2i(lpr), (unsigned)row_groups, (unsigned)gemv_lds_bytes(F, k), ring, ringl};
}

// Direct-to-LDS streaming GEMV (the _dma kernels, RING == 3 in
// gguf_gemv.hip).  Built for lanes per row 64 or 32 with 1 or 2 units per
// lane and step, and 16 with 1.  An item is a segment of lpr * iters units of
// each of the wave's 64 / lpr rows and each weight stream; its LDS slot
// holds, per row segment, the 16-byte lines that cover it, in whole 1 KB
// copies.  These sizes match the kernel's SEGB / NPC / NCH / SLOT.
struct DmaPlan {
    int lpr, iters;
    int segb;       // bytes of one row segment
    unsigned slot;  // LDS bytes per item
};
DmaPlan plan_dma(const Fmt* F, int k, bool pair, int lpr_override) {
    const int units = k / F->gemv_unit;
    int lpr = pow2_ceil(units);
    if (lpr < 16) lpr = 16;
    if (lpr > 64) lpr = 64;
    if (lpr_override == 16 || lpr_override == 32 || lpr_override == 64) lpr = lpr_override;
    const int iters = (lpr >= 32 && units > lpr) ? 2 : 1;
    const int segb = lpr * iters * F->gemv_unit / F->block_elems * F->block_bytes;
    const int npc = (segb + 30) / 16;
    const int nch = (npc + 63) / 64;
    const unsigned slot = (unsigned)((pair ? 2 : 1) * (64 / lpr) * nch * 1024);
    return DmaPlan{lpr, iters, segb, slot};
}

int gemv_common(cima_hip_ctx* ctx, int t, const void* x, const void* wa, const void* wb,
                const void* ba, const void* bb, void* y, int n, int k, int mode, int act, bool pair,
                const char* api, const void* norm_w = nullptr, float eps = 0.f, GemvKind kind = GK_PLAIN,
                const GemvExt* kext = nullptr) {
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "%s: context is not initialised", api);
    const Fmt* F = fmt_of(t);
    if (!F) return fail(CIMA_E_FORMAT, "%s: ggml type %d is not a supported GGUF block format", api, t);
    if (n < 0 || k <= 0 || k % F->block_elems)
        return fail(CIMA_E_INVALID, "%s: shape n=%d k=%d: k must be a positive multiple of %d for %s", api, n,
                    k, F->block_elems, F->name);
    if (act != CIMA_DT_F32 && act != CIMA_DT_F16)
        return fail(CIMA_E_INVALID, "%s: act_dtype %d is not f32 or f16", api, act);
    if (!pair && mode != 0 && mode != 1) return fail(CIMA_E_INVALID, "%s: mode %d is not 0, 1 or 2", api, mode);
    if (n == 0) return 0;
    if (!x || !wa || !y || (pair && !wb)) return fail(CIMA_E_INVALID, "%s: null x, w or y", api);
    if (norm_w && (!aligned(norm_w, 16) || !(eps >= 0.f)))
        return fail(CIMA_E_INVALID, "%s: norm weight must be 16-byte aligned and eps >= 0", api);
    // x and y need only their element alignment, as the reference's f16
    // pointers do (src/cuda.rs:2161): x is read with 16-byte loads that
    // gfx950 serves at any 2-byte alignment (its unaligned-access mode, the
    // same the Q8_0 / Q6_K block loads rely on)
    const uintptr_t es = act == CIMA_DT_F32 ? 4 : 2;
    if (!aligned(x, es) || !aligned(y, es) || !aligned(wa, F->w_align) || (pair && !aligned(wb, F->w_align)))
        return fail(CIMA_E_INVALID, "%s: misaligned pointer (x and y need %d B, %s weights %d B)", api, (int)es,
                    F->name, F->w_align);
    if ((long long)n * (long long)(k / F->block_elems) * F->block_bytes > (1LL << 40))
        return fail(CIMA_E_INVALID, "%s: weight of %d x %d is beyond the supported size", api, n, k);
    GemvPlan p = plan_gemv(ctx, F, n, k, pair);
    if ((long)p.lds > ctx->max_lds)
        return fail(CIMA_E_INVALID, "%s: k=%d needs %u B of LDS for x, the device allows %d", api, k, p.lds,
                    ctx->max_lds);
    char name[96];
    if (p.iters > 8)
        return fail(CIMA_E_INVALID, "%s: k=%d is longer than the GEMV supports (%d units per lane group)", api, k,
                    p.iters);
    bool epi = ba != nullptr || bb != nullptr || mode == 1;
    const char* kind_sfx = pair ? "_pair" : "";
    if (kind != GK_PLAIN) p.ringl = false;  // built for plain and _epi only
    if (p.ringl) p.iters = 1;
    if (kind == GK_ATT) p.ring = false;
    if (kind == GK_ATT) {
        kind_sfx = "_att";
        epi = true;  // built with the epilogue only
        p.lds = (unsigned)(((p.lds + 15u) & ~15u) + 4u * (unsigned)k);
        if ((long)p.lds > ctx->max_lds)
            return fail(CIMA_E_INVALID, "%s: k=%d needs %u B of LDS, the device allows %d", api, k, p.lds,
                        ctx->max_lds);
    } else if (kind == GK_AMAX) {
        kind_sfx = "_amax";
        if (epi) return fail(CIMA_E_INVALID, "%s: the argmax GEMV takes no bias or residual", api);
    }
    // Direct-to-LDS streaming.  Measured on MI355X (cold weights, us):
    // Q8_0 14336x4096 15.4 -> 13.3 (one item in flight per wave, three
    // workgroups per CU), the Q8_0 gate+up pair 29.8 -> 23.4 (two items in
    // flight), the Q8_0 151936x896 head 35.0 -> 27.0 (items of two 952-byte
    // rows: two in flight, four workgroups per CU); slower than the
    // register loops for Q4_K (14336x4096 8.2 -> 9.4), for rows of several
    // segments (4096x14336: Q8_0 17.2 -> 19.1, Q4_K 9.9 -> 12.3) and for
    // matrices of a few MB (about 1 us more), so the heuristic takes it for
    // large Q8_0 matrices of one-segment rows.
    bool dma = false;
    int depth = 1, dma_wgs = 3;
    const DmaPlan dplan = plan_dma(F, k, pair, ctx->tune_dma != 0 ? ctx->tune_lpr : 0);
    const bool one_seg = k / F->gemv_unit <= dplan.lpr * dplan.iters;
    const double wbytes_all = (pair ? 2.0 : 1.0) * (double)n * (double)(k / F->block_elems) * F->block_bytes;
    const bool dma_auto = t == CIMA_GGML_Q8_0 && one_seg && wbytes_all >= 24e6 && kind != GK_ATT;
    if (ctx->tune_dma != 2 && !(ctx->tune_rows > 1) && (!ctx->tune_lpr || ctx->tune_dma != 0) &&
        (ctx->tune_dma != 0 || dma_auto)) {
        const DmaPlan d = dplan;
        const bool small_items = d.segb <= 1536;  // rows of at most ~1.5 KB (k = 896 at Q8_0: 952 B)
        depth = ctx->tune_dma == 3 || (ctx->tune_dma == 0 && (pair || small_items)) ? 2 : 1;
        if (!dma_built(d.lpr, d.iters, depth, pair)) depth = 1;
        dma_wgs = small_items ? 4 : 3;
        const unsigned xb = (unsigned)((gemv_lds_bytes(F, k) + 15) & ~(size_t)15) + (kind == GK_ATT ? 4u * (unsigned)k : 0u);
        const unsigned lds = xb + (unsigned)(kGemvThreads / 64) * depth * d.slot;
        if ((long)lds <= ctx->max_lds) {
            dma = true;
            p.rows = 1;
            p.iters = d.iters;
            p.lpr_shift = log2i(d.lpr);
            p.lds = lds;
            p.grid = (unsigned)n;
            p.ring = p.ringl = false;
        }
    }
    // Rows split over the workgroup's four waves (the _ksplit kernels):
    // long rows, each wave a quarter of every row with its x fragment in
    // registers, for plain and epilogue GEMVs
    const int units_all = k / F->gemv_unit;
    const int wq = (units_all + 3) / 4;  // units per wave
    const bool wsplit_ok = !dma && !pair && kind == GK_PLAIN && wq <= 128 && units_all > 128 && !(ctx->tune_rows > 1);
    // measured on MI355X (cold, us, 4096x14336, fp32 x): Q6_K 16.9 -> 15.1;
    // slower for Q4_K (9.9 -> 11.5), Q8_0 (18.5 -> 19.3), Q4_0 (12.7 ->
    // 13.6) and the decode step's Q8_0 896x4864 (3.7 -> 5.0), whose
    // register loops keep x in LDS at no visible cost
    const bool wsplit = wsplit_ok && ctx->tune_wsplit != 2 && (ctx->tune_wsplit == 1 || t == CIMA_GGML_Q6_K);
    if (wsplit) {
        p.rows = 1;
        p.iters = wq <= 64 ? 1 : 2;
        p.lpr_shift = 6;
        p.ring = p.ringl = false;
        p.grid = (unsigned)n * (unsigned)(kGemvThreads / 64);  // row groups: one row per workgroup
    }
    if (dma)
        snprintf(name, sizeof name, "cima_gemv_%s_l%d_i%d_%s_dma%d%s%s", F->name, 1 << p.lpr_shift, p.iters,
                 act == CIMA_DT_F32 ? "f32" : "f16", depth, kind_sfx, epi ? "_epi" : "");
    else if (wsplit)
        snprintf(name, sizeof name, "cima_gemv_%s_r1_i%d_%s_ksplit%s", F->name, p.iters,
                 act == CIMA_DT_F32 ? "f32" : "f16", epi ? "_epi" : "");
    else
        snprintf(name, sizeof name, "cima_gemv_%s_r%d_i%d_%s%s%s%s", F->name, p.rows, p.iters,
                 act == CIMA_DT_F32 ? "f32" : "f16", p.ring ? "_ring" : (p.ringl ? "_ringl" : ""), kind_sfx,
                 epi ? "_epi" : "");
    hipFunction_t f;
    if (int rc = get_fn(ctx, name, &f)) return rc;
    int threads = kGemvThreads;
    if (hipFuncGetAttribute(&threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f) != hipSuccess || threads < 64)
        threads = kGemvThreads;
    {
        const long groups_per_wg = (long)(threads / 64) * (64 >> p.lpr_shift);
        p.grid = (unsigned)(((long)p.grid + groups_per_wg - 1) / groups_per_wg);  // row groups -> workgroups
    }
    int resident = 0;
    hipError_t oe = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&resident, f, threads, p.lds);
    if (oe != hipSuccess) return hip_fail(oe, "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
    if (resident < 1) resident = 1;
    // persistent grid: one workgroup per CU for the item ring, the wave
    // split and Q8_0's other loops, two otherwise, the stepped ring included
    // (measured on MI355X; the wave split of Q6_K 4096x14336, cold: 14.5 us
    // at two workgroups per CU, 13.5 at one)
    const int want = ctx->tune_wgs > 0 ? ctx->tune_wgs
                                       : (dma ? dma_wgs
                                              : (p.ringl ? 2
                                                         : ((p.ring || wsplit || t == CIMA_GGML_Q8_0) ? 1 : 2)));
    if (want < resident) resident = want;
    unsigned cap = (unsigned)(resident * ctx->num_cu);
    if (p.grid > cap) p.grid = cap;
    const void* xa = x;
    const void* w0 = wa;
    const void* w1 = wb;
    const void* b0 = ba;
    const void* b1 = bb;
    void* yy = y;
    GemvExt ext = kext ? *kext : GemvExt{};
    ext.norm_w = norm_w;
    ext.eps = eps;
    int nn = n, kk = k, mm = mode, ls = p.lpr_shift;
    void* args[] = {&xa, &w0, &w1, &b0, &b1, &yy, &nn, &kk, &mm, &ls, &ext};
    return launch(ctx, f, p.grid, (unsigned)threads, args, api, p.lds);
}

}  // namespace

extern "C" {

int cima_hip_init(int device, const char* code_dir, cima_hip_ctx** out) {
    if (!out) return fail(CIMA_E_INVALID, "cima_hip_init: null out pointer");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return fail(CIMA_E_INVALID, "cima_hip_init: device %d out of range (%d devices)", device, count);
    if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    auto* ctx = new cima_hip_ctx();
    ctx->device = device;
    if ((e = hipDeviceGetAttribute(&ctx->num_cu, hipDeviceAttributeMultiprocessorCount, device)) != hipSuccess) {
        delete ctx;
        return hip_fail(e, "hipDeviceGetAttribute(CU count)");
    }
    if ((e = hipDeviceGetAttribute(&ctx->max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device)) !=
        hipSuccess) {
        delete ctx;
        return hip_fail(e, "hipDeviceGetAttribute(LDS per block)");
    }
    const std::string dir = code_dir ? std::string(code_dir) : default_code_dir();
    for (int i = 0; i < NUM_MODULES; i++) {
        const std::string path = dir + "/" + kModuleFiles[i];
        if ((e = hipModuleLoad(&ctx->modules[i], path.c_str())) != hipSuccess) {
            unload(ctx);
            delete ctx;
            return fail((int)e, "hipModuleLoad(%s) failed: %s", path.c_str(), hipGetErrorString(e));
        }
    }
    ctx->loaded = true;
    {
        // the device address of the decode module's scratch array: taken
        // once here, with this context's device current; the array's name
        // is not an address the host may pass to a kernel
        hipDeviceptr_t sp = nullptr;
        size_t sb = 0;
        if ((e = hipModuleGetGlobal(&sp, &sb, ctx->modules[MOD_DECODE], "scratch")) != hipSuccess) {
            unload(ctx);
            delete ctx;
            return fail((int)e, "hipModuleGetGlobal(scratch) failed: %s", hipGetErrorString(e));
        }
        ctx->scratch = (void*)sp;
        ctx->scratch_bytes = sb;
        if ((e = hipModuleGetGlobal(&sp, &sb, ctx->modules[MOD_GEMM], "cima_gemm_status")) != hipSuccess ||
            sb != sizeof(unsigned)) {
            unload(ctx);
            delete ctx;
            return fail(e != hipSuccess ? (int)e : CIMA_E_NO_KERNEL, "hipModuleGetGlobal(cima_gemm_status) failed");
        }
        ctx->gemm_status = (unsigned*)sp;
    }
    // resolve every kernel up front (the reference's KernelSet)
    auto add = [&](int mod, const std::string& name) -> int {
        hipFunction_t f;
        hipError_t r = hipModuleGetFunction(&f, ctx->modules[mod], name.c_str());
        if (r != hipSuccess) return fail((int)r, "hipModuleGetFunction(%s): %s", name.c_str(), hipGetErrorString(r));
        ctx->fns[name] = f;
        return 0;
    };
    int rc = 0;
    for (int t : kFormats) {
        const Fmt* F = fmt_of(t);
        for (const auto& sh : kShapes)
            for (const char* act : {"f32", "f16"})
                for (const char* sfx : {"", "_epi", "_pair", "_pair_epi", "_att_epi", "_amax"}) {
                    if (!strcmp(act, "f32") && (!strcmp(sfx, "_att_epi") || !strcmp(sfx, "_amax")))
                        continue;  // attention / argmax variants are f16 only
                    char name[96];
                    snprintf(name, sizeof name, "cima_gemv_%s_r%d_i%d_%s%s", F->name, sh[0], sh[1], act, sfx);
                    if (!rc) rc = add(F->gemv_module, name);
                }
        for (int it = 1; it <= 2; it++)
            for (const char* rk : {"_f32_ring", "_f32_ring_epi", "_f16_ring", "_f16_ring_epi", "_f16_ring_amax",
                                   "_f32_ring_pair", "_f32_ring_pair_epi", "_f16_ring_pair", "_f16_ring_pair_epi"}) {
                char name[96];
                snprintf(name, sizeof name, "cima_gemv_%s_r1_i%d%s", F->name, it, rk);
                if (!rc) rc = add(F->gemv_module, name);
            }
        for (const auto& li : kDmaShapes)
            for (int dd = 1; dd <= 2; dd++)
                for (const char* dk : {"f32_dma%d", "f32_dma%d_epi", "f32_dma%d_pair", "f32_dma%d_pair_epi", "f16_dma%d",
                                       "f16_dma%d_epi", "f16_dma%d_pair", "f16_dma%d_pair_epi", "f16_dma%d_att_epi",
                                       "f16_dma%d_amax"}) {
                    if (!dma_built(li[0], li[1], dd, strstr(dk, "pair") != nullptr)) continue;
                    char sfx[48], name[96];
                    snprintf(sfx, sizeof sfx, dk, dd);
                    snprintf(name, sizeof name, "cima_gemv_%s_l%d_i%d_%s", F->name, li[0], li[1], sfx);
                    if (!rc) rc = add(F->gemv_module, name);
                }
        for (int it = 1; it <= 2; it++)
            for (const char* rk : {"_f32_ksplit", "_f32_ksplit_epi", "_f16_ksplit", "_f16_ksplit_epi"}) {
                char name[96];
                snprintf(name, sizeof name, "cima_gemv_%s_r1_i%d%s", F->name, it, rk);
                if (!rc) rc = add(F->gemv_module, name);
            }
        for (const char* rk : {"_f32_ringl", "_f32_ringl_epi", "_f16_ringl", "_f16_ringl_epi"}) {
            char name[96];
            snprintf(name, sizeof name, "cima_gemv_%s_r1_i1%s", F->name, rk);
            if (!rc) rc = add(F->gemv_module, name);
        }
        for (int bn : kGemmBN)
            for (const char* xt : {"f32", "f16", "bf16"})
                for (const char* yt : {"f32", "f16"}) {
                    char name[96];
                    snprintf(name, sizeof name, "cima_gemm_%s_b%d_%s_%s", F->name, bn, xt, yt);
                    if (!rc) rc = add(MOD_GEMM, name);
                    if (bn == 16) {
                        snprintf(name, sizeof name, "cima_gemm_%s_b16n_%s_%s", F->name, xt, yt);
                        if (!rc) rc = add(MOD_GEMM, name);
                    }
                }
        if (!rc) rc = add(MOD_DEQUANT, std::string("cima_dequant_") + F->name);
        if (!rc) rc = add(MOD_DEQUANT, std::string("cima_gather_") + F->name);
    }
    // bitsandbytes weights decoded in the GEMM tiles, f16 weights, and the
    // plain kernel for f16 weights of k % 64 != 0
    for (const char* wn : {"nf4", "f16w"})
        for (int bn : kGemmBN)
            for (const char* xt : {"f32", "f16", "bf16"})
                for (const char* yt : {"f32", "f16"}) {
                    char name[96];
                    snprintf(name, sizeof name, "cima_gemm_%s_b%d_%s_%s", wn, bn, xt, yt);
                    if (!rc) rc = add(MOD_GEMM, name);
                    if (bn == 16) {
                        snprintf(name, sizeof name, "cima_gemm_%s_b16n_%s_%s", wn, xt, yt);
                        if (!rc) rc = add(MOD_GEMM, name);
                    }
                    if (bn == 16 && !strcmp(wn, "f16w")) {
                        snprintf(name, sizeof name, "cima_gemm_f16w_small_%s_%s", xt, yt);
                        if (!rc) rc = add(MOD_GEMM, name);
                    }
                }
    if (!rc) rc = add(MOD_GEMM, "cima_gemm_ksum_f32");
    if (!rc) rc = add(MOD_GEMM, "cima_gemm_ksum_f16");
    if (!rc) rc = add(MOD_DEQUANT, "cima_stream_read");
    for (const char* kn : {"cima_stream_read_r1_w16", "cima_stream_read_r2_w16", "cima_stream_read_r4_w16",
                           "cima_stream_read_r8_w16", "cima_stream_read_r16_w16", "cima_stream_read_r4_w8",
                           "cima_stream_read_r8_w8", "cima_stream_read_r16_w8", "cima_stream_read_l2",
                           "cima_stream_read_l4", "cima_stream_read_l8", "cima_stream_read_l16"})
        if (!rc) rc = add(MOD_DEQUANT, kn);
    for (const char* kn : {"cima_nf4_dequant_v", "cima_nf4_dequant_e", "cima_nf4_gemv_e_f16_f16",
                           "cima_nf4_gemv_e_f32_f32"})
        if (!rc) rc = add(MOD_BNB4, kn);
    for (const char* var : {"t", "c"})
        for (int r : {1, 2, 4})
            for (const char* a : {"f16", "f32"}) {
                char name[64];
                snprintf(name, sizeof name, "cima_nf4_gemv_%s_r%d_%s_%s", var, r, a, a);
                if (!rc) rc = add(MOD_BNB4, name);
            }
    for (const char* kn : kDecodeKernels)
        if (!rc) rc = add(MOD_DECODE, kn);
    if (rc) {
        unload(ctx);
        delete ctx;
        return rc;
    }
    if ((e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking)) != hipSuccess) {
        unload(ctx);
        delete ctx;
        return hip_fail(e, "hipStreamCreateWithFlags");
    }
    ctx->stream = ctx->own_stream;
    int er = 0, el = 0;
    if (const char* s = getenv("CIMA_GEMV_ROWS")) er = atoi(s);
    if (const char* s = getenv("CIMA_GEMV_LPR")) el = atoi(s);
    if (const char* s = getenv("CIMA_GEMV_WGS")) ctx->tune_wgs = atoi(s);
    if (const char* s = getenv("CIMA_GEMV_RING")) ctx->tune_ring = atoi(s);
    if (const char* s = getenv("CIMA_GEMV_RINGL")) ctx->tune_ringl = atoi(s);
    if (const char* s = getenv("CIMA_GEMV_DMA")) ctx->tune_dma = atoi(s);
    if (const char* s = getenv("CIMA_GEMM_XCHECK")) ctx->gemm_xcheck = atoi(s) != 0;
    if (const char* s = getenv("CIMA_GEMM_KSPLIT")) ctx->tune_ksplit = atoi(s);
    if (const char* s = getenv("CIMA_GEMV_WSPLIT")) ctx->tune_wsplit = atoi(s);
    if (er || el) {
        if (int r = cima_hip_set_gemv_tuning(ctx, er, el)) {
            cima_hip_destroy(ctx);
            return r;
        }
    }
    *out = ctx;
    return 0;
}

int cima_hip_destroy(cima_hip_ctx* ctx) {
    if (!ctx) return 0;
    (void)hipSetDevice(ctx->device);
    if (ctx->own_stream) {
        (void)hipStreamSynchronize(ctx->own_stream);
        (void)hipStreamDestroy(ctx->own_stream);
    }
    unload(ctx);
    delete ctx;
    return 0;
}

int cima_hip_bind(cima_hip_ctx* ctx) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_bind: null context");
    hipError_t e = hipSetDevice(ctx->device);
    return e == hipSuccess ? 0 : hip_fail(e, "hipSetDevice");
}

int cima_hip_set_stream(cima_hip_ctx* ctx, void* s) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_set_stream: null context");
    ctx->stream = (hipStream_t)s;
    return 0;
}

int cima_hip_use_own_stream(cima_hip_ctx* ctx) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_use_own_stream: null context");
    ctx->stream = ctx->own_stream;
    return 0;
}

void* cima_hip_get_stream(cima_hip_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int cima_hip_sync(cima_hip_ctx* ctx) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_sync: null context");
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? 0 : hip_fail(e, "hipStreamSynchronize");
}

const char* cima_hip_last_error(void) { return g_err; }

int cima_hip_is_fatal(int code) {
    // Sticky codes after which the device context cannot be used; the same
    // numeric set as the reference's cu_fatal (src/cuda.rs:122-127) --
    // hipError_t keeps CUDA's numbering for these (700 illegal address,
    // 702 launch timeout, 710 device assert, 719 launch failure, ...).
    // 701 (launch out of resources) is not sticky.
    switch (code) {
    case 700: case 702: case 710: case 713: case 714: case 715:
    case 716: case 717: case 718: case 719:
        return 1;
    default:
        return 0;
    }
}

int cima_hip_num_cu(cima_hip_ctx* ctx) { return ctx ? ctx->num_cu : 0; }

int cima_hip_set_gemv_grid(cima_hip_ctx* ctx, int wgs_per_cu) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_set_gemv_grid: null context");
    if (wgs_per_cu < 0 || wgs_per_cu > 64)
        return fail(CIMA_E_INVALID, "cima_hip_set_gemv_grid: %d workgroups per CU is out of range", wgs_per_cu);
    ctx->tune_wgs = wgs_per_cu;
    return 0;
}

int cima_hip_set_gemm_tile(cima_hip_ctx* ctx, int tokens) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_set_gemm_tile: null context");
    bool ok = tokens == 0;
    for (int b : kGemmBN) ok = ok || tokens == b;
    if (!ok) return fail(CIMA_E_INVALID, "cima_hip_set_gemm_tile: %d is not 0, 16, 32, 64, 128 or 256", tokens);
    ctx->tune_gemm_bn = tokens;
    return 0;
}

int cima_hip_gemm_status(cima_hip_ctx* ctx, unsigned int* flags, int clear) {
    const char* api = "cima_hip_gemm_status";
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "%s: context is not initialised", api);
    if (!flags) return fail(CIMA_E_INVALID, "%s: null flags", api);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, api);
    if ((e = hipMemcpy(flags, ctx->gemm_status, sizeof(unsigned), hipMemcpyDeviceToHost)) != hipSuccess)
        return hip_fail(e, api);
    if (clear) {
        const unsigned zero = 0;
        if ((e = hipMemcpy(ctx->gemm_status, &zero, sizeof zero, hipMemcpyHostToDevice)) != hipSuccess)
            return hip_fail(e, api);
    }
    return 0;
}

int cima_hip_set_gemv_wsplit(cima_hip_ctx* ctx, int mode) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_set_gemv_wsplit: null context");
    if (mode < 0 || mode > 2) return fail(CIMA_E_INVALID, "cima_hip_set_gemv_wsplit: mode %d is not 0, 1 or 2", mode);
    ctx->tune_wsplit = mode;
    return 0;
}

int cima_hip_set_gemv_dma(cima_hip_ctx* ctx, int mode) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_set_gemv_dma: null context");
    if (mode < 0 || mode > 3) return fail(CIMA_E_INVALID, "cima_hip_set_gemv_dma: mode %d is not 0, 1, 2 or 3", mode);
    ctx->tune_dma = mode;
    return 0;
}

int cima_hip_set_gemv_tuning(cima_hip_ctx* ctx, int rows, int lpr) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_set_gemv_tuning: null context");
    if (rows != 0 && rows != 1 && rows != 2)
        return fail(CIMA_E_INVALID, "cima_hip_set_gemv_tuning: rows %d is not 0, 1 or 2", rows);
    if (lpr != 0 && (lpr < 16 || lpr > 256 || (lpr & (lpr - 1))))
        return fail(CIMA_E_INVALID, "cima_hip_set_gemv_tuning: lanes %d is not 0 or a power of two in [16, 256]", lpr);
    ctx->tune_rows = rows;
    ctx->tune_lpr = lpr;
    return 0;
}

namespace {
int gemv_entry(cima_hip_ctx* ctx, int t, const void* x, const void* norm_w, float eps, const void* w,
               const void* bias, void* y, int n, int k, int mode, int act, const char* api) {
    if (mode == 2) {
        // gate|up pair stored as one [2n, k] weight; bias has 2n entries
        const Fmt* F = fmt_of(t);
        if (!F) return fail(CIMA_E_FORMAT, "%s: ggml type %d is not a supported GGUF block format", api, t);
        if (k <= 0 || k % F->block_elems)
            return fail(CIMA_E_INVALID, "%s: k=%d must be a positive multiple of %d", api, k, F->block_elems);
        size_t row_bytes = (size_t)(k / F->block_elems) * F->block_bytes;
        size_t esz = act == CIMA_DT_F32 ? 4 : 2;
        const char* wu = w ? (const char*)w + (size_t)(n > 0 ? n : 0) * row_bytes : nullptr;
        const char* bu = bias ? (const char*)bias + (size_t)(n > 0 ? n : 0) * esz : nullptr;
        return gemv_common(ctx, t, x, w, wu, bias, bu, y, n, k, 2, act, true, api, norm_w, eps);
    }
    return gemv_common(ctx, t, x, w, nullptr, bias, nullptr, y, n, k, mode, act, false, api, norm_w, eps);
}
}  // namespace

int cima_hip_gguf_gemv(cima_hip_ctx* ctx, int t, const void* x, const void* w, const void* bias, void* y, int n,
                       int k, int mode, int act) {
    return gemv_entry(ctx, t, x, nullptr, 0.f, w, bias, y, n, k, mode, act, "cima_hip_gguf_gemv");
}

int cima_hip_rmsnorm_gguf_gemv(cima_hip_ctx* ctx, int t, const void* x, const void* norm_w, float eps,
                               const void* w, const void* bias, void* y, int n, int k, int mode, int act) {
    if (!norm_w) return fail(CIMA_E_INVALID, "cima_hip_rmsnorm_gguf_gemv: null norm weight");
    return gemv_entry(ctx, t, x, norm_w, eps, w, bias, y, n, k, mode, act, "cima_hip_rmsnorm_gguf_gemv");
}

int cima_hip_gguf_gemv_swiglu(cima_hip_ctx* ctx, int t, const void* x, const void* wg, const void* wu,
                              const void* bg, const void* bu, void* y, int n, int k, int act) {
    return gemv_common(ctx, t, x, wg, wu, bg, bu, y, n, k, 2, act, true, "cima_hip_gguf_gemv_swiglu");
}

namespace {

// argument checks shared by the two prefill GEMM entry points; on 0, *Fo is
// the format, or null for an empty (m or n == 0) call
int gemm_check(cima_hip_ctx* ctx, int t, const void* x, const void* w, void* y, int m, int n, int k, int ldy,
               int x_dtype, int y_dtype, const char* api, const Fmt** Fo) {
    *Fo = nullptr;
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "%s: context is not initialised", api);
    const Fmt* F = fmt_of(t);
    if (!F) return fail(CIMA_E_FORMAT, "%s: ggml type %d is not a supported GGUF block format", api, t);
    if (m < 0 || n < 0 || k <= 0 || k % 64 || k % F->block_elems)
        return fail(CIMA_E_INVALID, "%s: shape m=%d n=%d k=%d: k must be a positive multiple of %d", api, m, n, k,
                    F->block_elems > 64 ? F->block_elems : 64);
    if (ldy < n) return fail(CIMA_E_INVALID, "%s: ldy=%d < n=%d", api, ldy, n);
    if ((long long)m * k * (x_dtype == CIMA_DT_F32 ? 4 : 2) > 0xffffffffLL)
        return fail(CIMA_E_INVALID, "%s: X of %d x %d is 4 GiB or more", api, m, k);
    if (x_dtype < CIMA_DT_F32 || x_dtype > CIMA_DT_BF16 || (y_dtype != CIMA_DT_F32 && y_dtype != CIMA_DT_F16))
        return fail(CIMA_E_INVALID, "%s: x_dtype %d / y_dtype %d not supported", api, x_dtype, y_dtype);
    if (m == 0 || n == 0) return 0;
    if (!x || !w || !y) return fail(CIMA_E_INVALID, "%s: null x, w or y", api);
    if (!aligned(x, 16) || !aligned(w, F->w_align) || !aligned(y, 4))
        return fail(CIMA_E_INVALID, "%s: misaligned pointer (x 16 B, %s weights %d B, y 4 B)", api, F->name,
                    F->w_align);
    *Fo = F;
    return 0;
}

// Token tile of the fused GEMM (measured on MI355X, Q4_K, bf16 X, cold
// weights): 16 up to 32 tokens (two 16-token tiles at 33.6 us against 40.2
// us for one 64-token tile on 14336x4096); 33-128 tokens 32 while that grid
// fits one workgroup per CU, else 64 (48 tokens: 35.9 against 42.4 us on
// 14336x4096, 33.6 against 40.0 on 6144x4096; 128 tokens on 14336x4096,
// 448 workgroups: 61.0 against 44.0); 128 beyond.
int fused_bn(int m, int n, int num_cu) {
    if (m <= 32) return 16;
    if (m <= 128) return (long long)((n + 127) / 128) * ((m + 31) / 32) <= num_cu ? 32 : 64;
    // 256-token tiles (one workgroup per CU, the weight tile dequantised
    // once per 256 tokens) where 128-token tiles would need more than 1.5
    // workgroups per CU and the 256-token grid still fits one round
    // (measured on MI355X, Q4_K, bf16 X, 14336x4096: 102.2 against 108.8 us
    // at 512 tokens, 195 against 206 at 1024; a second round of 256-token
    // workgroups loses: 193 against 165 at 768, and so does a grid that
    // leaves most CUs idle: 98 against 69 on 6144x4096 at 512)
    const long long rt = (n + 127) / 128;
    if (rt * ((m + 255) / 256) <= num_cu && 2 * rt * ((m + 127) / 128) > 3LL * num_cu) return 256;
    // a weight too narrow for the 128-token grid to fill the CUs takes the
    // widest register-A tile whose grid still fits one round (measured on
    // MI355X, Q4_K, bf16 X: 4096x4096 at 256 / 512 tokens 63.0 / 63.6 us
    // with 128-token tiles, 41.1 / 44.2 with 64-token tiles)
    if (rt * ((m + 127) / 128) < num_cu && rt * ((m + 63) / 64) <= num_cu)
        return rt * ((m + 31) / 32) <= num_cu ? 32 : 64;
    return 128;
}

// the fused MFMA dequant-GEMM (gguf_gemm.hip) on checked arguments
// kernel-argument mirror of GemmExt in gguf_gemm.hip (same member order):
// the bitsandbytes operands; zero for the GGUF formats
struct GemmExt {
    const float* absmax;
    const float* qmap;
    long long bsz;
    int bs_shift;
    unsigned* status;
    float* part;
    int ksplit;
};

// Launches cima_gemm_<fname>_b<BN>[n]_<x>_<y> over Y[m, n] (row stride ldy):
// the token tile from fused_bn (or the tuning override), 16-token tiles
// only for k % 128 == 0.
// Workgroups along k for the 16-token tiles (1 = none), when the caller's
// slab can hold the partial tiles (S x m x n fp32) and the 128-k stages
// divide evenly (at least four per split, one per k-split wave).  A grid
// of 32-row tiles of at most one workgroup per CU is split two ways, a grid
// of 16-row tiles (the narrow kernels, three or four per CU) four ways at
// most a quarter workgroup per CU and two ways at most a half.  Measured
// on MI355X (Q4_K unless noted, bf16 X, cold, us, unsplit -> split): 32
// tokens: 4096x14336 43.6 -> 30.1 (Q8_0 64.5 -> 48.5), 1024x4096 9.6 ->
// 8.9, 4096x4096 13.2 -> 13.3; 16 tokens: 6144x4096 15.5 -> 13.9,
// 1024x4096 9.5 -> 7.9; splitting fuller grids loses (16 tokens:
// 4096x14336 26.4 -> 27.7, 4096x4096 9.8 -> 12.2, 14336x4096 19.0 -> 23.4).
int pick_ksplit(const cima_hip_ctx* ctx, int wgs, bool narrow, int m, int n, int k, size_t part_bytes) {
    const int stages = k / 128;
    auto fits = [&](int s) { return stages % s == 0 && stages / s >= 4 && (size_t)s * m * n * 4 <= part_bytes; };
    if (ctx->tune_ksplit == 1) return 1;
    if (ctx->tune_ksplit > 1) return fits(ctx->tune_ksplit) ? ctx->tune_ksplit : 1;
    int s = 1;
    if (!narrow) s = wgs <= ctx->num_cu ? 2 : 1;
    else s = 4 * wgs <= ctx->num_cu ? 4 : (2 * wgs <= ctx->num_cu ? 2 : 1);
    while (s > 1 && !fits(s)) s /= 2;
    return s;
}

int gemm_launch(cima_hip_ctx* ctx, const char* fname, const void* x, const void* w, void* y, int m, int n, int k,
                int ldy, int x_dtype, int y_dtype, const GemmExt& gext, const char* api, float* part = nullptr,
                size_t part_bytes = 0) {
    // the 16-token tile stages 128 k at a time (32-row weight tiles in
    // 512-thread workgroups), so it needs k % 128 == 0
    int bn = fused_bn(m, n, ctx->num_cu);
    if (ctx->tune_gemm_bn) bn = ctx->tune_gemm_bn;
    if (bn == 16 && k % 128) bn = 32;
    // 16-token tiles: 32 rows per 512-thread workgroup, or 16 rows per
    // 256-thread workgroup (_b16n_) where the 32-row grid, counted over both
    // of its dimensions, would fill at most half the CUs (measured on MI355X,
    // Q4_K, bf16 X, 16-row against 32-row tiles, us: m = 16: 1024x4096 9.0 /
    // 12.9, 4096x4096 9.5 / 13.2, 4096x14336 26.6 / 43.8, 6144x4096 14.8 /
    // 13.4, 14336x4096 28.9 / 18.7; m = 24-32: 1024x4096 9.2 / 12.8,
    // 4096x4096 14.7 / 13.5, 4096x14336 44.5 / 43.5)
    const bool narrow = bn == 16 && 2LL * ((n + 31) / 32) * ((m + 15) / 16) <= ctx->num_cu;
    const int bm = narrow ? 16 : (bn == 16 ? 32 : 128);  // weight rows per workgroup
    static const char* const xn[] = {"f32", "f16", "bf16"};
    char name[96];
    snprintf(name, sizeof name, "cima_gemm_%s_b%d%s_%s_%s", fname, bn, narrow ? "n" : "", xn[x_dtype],
             y_dtype == CIMA_DT_F32 ? "f32" : "f16");
    hipFunction_t f;
    if (int rc = get_fn(ctx, name, &f)) return rc;
    const void* xa = x;
    const void* wa = w;
    void* ya = y;
    int mm = m, nn = n, kk = k, ld = ldy;
    GemmExt ge = gext;
    ge.status = ctx->gemm_xcheck ? ctx->gemm_status : nullptr;
    const unsigned gx = (unsigned)((n + bm - 1) / bm), gy = (unsigned)((m + bn - 1) / bn);
    const int ks = bn == 16 && part ? pick_ksplit(ctx, (int)(gx * gy), narrow, m, n, k, part_bytes) : 1;
    ge.part = ks > 1 ? part : nullptr;
    ge.ksplit = ks;
    void* args[] = {&xa, &wa, &ya, &mm, &nn, &kk, &ld, &ge};
    const unsigned threads = bn == 16 && !narrow ? 512 : 256;
    hipError_t e = hipModuleLaunchKernel(f, gx, gy, (unsigned)ks, threads, 1, 1, 0, ctx->stream, args, nullptr);
    if (e != hipSuccess) return hip_fail(e, api);
    if (ks == 1) return 0;
    // the partial tiles, summed in a fixed order into Y
    hipFunction_t fs;
    if (int rc = get_fn(ctx, y_dtype == CIMA_DT_F32 ? "cima_gemm_ksum_f32" : "cima_gemm_ksum_f16", &fs)) return rc;
    const float* pa = part;
    int S = ks;
    void* sargs[] = {&pa, &ya, &mm, &nn, &ld, &S};
    const long long outs = (long long)m * n;
    return launch(ctx, fs, (unsigned)((outs + 255) / 256), 256, sargs, api);
}
int gemm_fused(cima_hip_ctx* ctx, const Fmt* F, const void* x, const void* w, void* y, int m, int n, int k, int ldy,
               int x_dtype, int y_dtype, const char* api) {
    return gemm_launch(ctx, F->name, x, w, y, m, n, k, ldy, x_dtype, y_dtype, GemmExt{}, api);
}

}  // namespace

int cima_hip_gguf_gemm(cima_hip_ctx* ctx, int t, const void* x, const void* w, void* y, int m, int n, int k,
                       int ldy, int x_dtype, int y_dtype) {
    const char* api = "cima_hip_gguf_gemm";
    const Fmt* F = nullptr;
    int rc = gemm_check(ctx, t, x, w, y, m, n, k, ldy, x_dtype, y_dtype, api, &F);
    if (rc || !F) return rc;
    return gemm_fused(ctx, F, x, w, y, m, n, k, ldy, x_dtype, y_dtype, api);
}

namespace {

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }


}  // namespace

int cima_hip_gguf_gemm_slab(cima_hip_ctx* ctx, int t, const void* x, const void* w, void* y, int m, int n, int k,
                            int ldy, int x_dtype, int y_dtype, void* slab, unsigned long long slab_bytes) {
    const char* api = "cima_hip_gguf_gemm_slab";
    const Fmt* F = nullptr;
    int rc = gemm_check(ctx, t, x, w, y, m, n, k, ldy, x_dtype, y_dtype, api, &F);
    if (rc || !F) return rc;
    if (slab_bytes && (!slab || !aligned(slab, 256)))
        return fail(CIMA_E_INVALID, "%s: slab must be a non-null 256-byte aligned device pointer", api);
    // the fused kernels dequantise W tile by tile; the slab holds the
    // partial tiles when a narrow weight is split along k at 16 tokens
    return gemm_launch(ctx, F->name, x, w, y, m, n, k, ldy, x_dtype, y_dtype, GemmExt{}, api,
                       slab_bytes ? static_cast<float*>(slab) : nullptr, (size_t)slab_bytes);
}


int cima_hip_gguf_dequant(cima_hip_ctx* ctx, int t, const void* src, void* out, long long nblocks) {
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "cima_hip_gguf_dequant: context is not initialised");
    const Fmt* F = fmt_of(t);
    if (!F) return fail(CIMA_E_FORMAT, "cima_hip_gguf_dequant: ggml type %d is not a supported GGUF block format", t);
    if (nblocks < 0) return fail(CIMA_E_INVALID, "cima_hip_gguf_dequant: nblocks %lld < 0", nblocks);
    if (nblocks == 0) return 0;
    if (!src || !out) return fail(CIMA_E_INVALID, "cima_hip_gguf_dequant: null pointer");
    if (!aligned(src, F->w_align) || !aligned(out, 16))
        return fail(CIMA_E_INVALID, "cima_hip_gguf_dequant: misaligned src (%d B) or out (16 B)", F->w_align);
    long long units = nblocks * (F->block_elems / F->unit_elems);
    long long grid = (units + 255) / 256;
    if (grid > 0x7fffffffLL) return fail(CIMA_E_INVALID, "cima_hip_gguf_dequant: %lld blocks is too many", nblocks);
    hipFunction_t f;
    if (int rc = get_fn(ctx, std::string("cima_dequant_") + F->name, &f)) return rc;
    const void* s = src;
    void* o = out;
    long long nb = nblocks;
    void* args[] = {&s, &o, &nb};
    return launch(ctx, f, (unsigned)grid, 256, args, "cima_hip_gguf_dequant");
}

int cima_hip_gguf_gather(cima_hip_ctx* ctx, int t, const void* table, const unsigned int* ids, void* out, int n,
                         int hidden) {
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "cima_hip_gguf_gather: context is not initialised");
    const Fmt* F = fmt_of(t);
    if (!F) return fail(CIMA_E_FORMAT, "cima_hip_gguf_gather: ggml type %d is not a supported GGUF block format", t);
    if (n < 0 || hidden <= 0 || hidden % F->block_elems)
        return fail(CIMA_E_INVALID, "cima_hip_gguf_gather: n=%d hidden=%d (hidden must be a multiple of %d)", n,
                    hidden, F->block_elems);
    if (n == 0) return 0;
    if (!table || !ids || !out) return fail(CIMA_E_INVALID, "cima_hip_gguf_gather: null pointer");
    if (!aligned(table, F->w_align) || !aligned(out, 16))
        return fail(CIMA_E_INVALID, "cima_hip_gguf_gather: misaligned table (%d B) or out (16 B)", F->w_align);
    long long units = (long long)n * (hidden / F->unit_elems);
    long long grid = (units + 255) / 256;
    if (grid > 0x7fffffffLL) return fail(CIMA_E_INVALID, "cima_hip_gguf_gather: too many rows");
    hipFunction_t f;
    if (int rc = get_fn(ctx, std::string("cima_gather_") + F->name, &f)) return rc;
    const void* tb = table;
    const void* id = ids;
    void* o = out;
    int nn = n, hh = hidden;
    void* args[] = {&tb, &id, &o, &nn, &hh};
    return launch(ctx, f, (unsigned)grid, 256, args, "cima_hip_gguf_gather");
}


// ------------------------------------------------------------ decode step

namespace {

const char* const kApiRms = "cima_hip_rmsnorm";

int ready(cima_hip_ctx* ctx, const char* api) {
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "%s: context is not initialised", api);
    return 0;
}

int launch_named(cima_hip_ctx* ctx, const char* name, unsigned grid, unsigned block, void** args, const char* api) {
    hipFunction_t f;
    if (int rc = get_fn(ctx, name, &f)) return rc;
    return launch(ctx, f, grid, block, args, api);
}

int attn_dim_ok(int dim) { return dim == 64 || dim == 128; }

// positions per attention chunk the kernels stage at most (ATT_MAX_CSZ)
const int kAttMaxChunk = 256;

// query heads per workgroup of cima_attn_decode_d<dim>_c<cp> (AT_GMAX in
// decode_ops.hip; 4 cp threads, chunks of up to cp positions) and its LDS
// bytes (sizeof AttnLds2<dim, cp>)
const int kAttGroup = 8;
unsigned attn_fused_lds(int dim, int cp) {
    const int nw = cp / 16, tt = dim / 16, ns = nw >= tt ? nw / tt : 1;
    return (unsigned)(16 * (dim + 8) * 2 + dim * 2 + dim * 4 + cp * 17 * 4 + kAttGroup * 2 * 4 +
                      cp * (dim + 16) * 2 + ns * dim * 16 * 4);
}

int attn_fused(cima_hip_ctx* ctx, const void* qkv, void* kc, void* vc, float* part, int q_heads, int kv_heads,
               int dim, int max_seq, int csz, int n_chunks, float theta, float scale, int window, const int* pos_dev,
               const char* api) {
    if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || !attn_dim_ok(dim) || max_seq <= 0 || csz <= 0 ||
        csz > kAttMaxChunk || n_chunks <= 0 || (long long)n_chunks * csz < max_seq || window < 0)
        return fail(CIMA_E_INVALID,
                    "%s: q_heads=%d kv_heads=%d dim=%d max_seq=%d csz=%d n_chunks=%d (dim 64 or 128, q_heads a "
                    "multiple of kv_heads, csz <= 256, n_chunks * csz >= max_seq)",
                    api, q_heads, kv_heads, dim, max_seq, csz, n_chunks);
    if (!qkv || !kc || !vc || !part || !pos_dev) return fail(CIMA_E_INVALID, "%s: null pointer", api);
    if (!aligned(kc, 16) || !aligned(vc, 16) || !aligned(qkv, 4))
        return fail(CIMA_E_INVALID, "%s: misaligned cache (16 B) or qkv (4 B)", api);
    // the narrowest workgroup whose chunk covers csz positions
    const int cp = csz <= 64 ? 64 : (csz <= 128 ? 128 : 256);
    char name[48];
    snprintf(name, sizeof name, "cima_attn_decode_d%d_c%d", dim, cp);
    void* args[] = {&qkv, &kc, &vc, &part, &q_heads, &kv_heads, &max_seq, &csz, &n_chunks, &theta, &scale,
                    &window, &pos_dev};
    const int grp = q_heads / kv_heads, hgs = (grp + kAttGroup - 1) / kAttGroup;
    hipFunction_t f;
    if (int rc = get_fn(ctx, name, &f)) return rc;
    return launch(ctx, f, (unsigned)(kv_heads * hgs * n_chunks), 4 * cp, args, api, attn_fused_lds(dim, cp));
}

}  // namespace

int cima_hip_rmsnorm(cima_hip_ctx* ctx, const void* x, const void* w, void* y, int rows, int n, float eps) {
    if (int rc = ready(ctx, kApiRms)) return rc;
    if (rows < 0 || n <= 0 || !(eps >= 0.f)) return fail(CIMA_E_INVALID, "%s: rows=%d n=%d eps=%g", kApiRms, rows, n, eps);
    if (rows == 0) return 0;
    if (!x || !y) return fail(CIMA_E_INVALID, "%s: null x or y", kApiRms);
    void* args[] = {&x, &w, &y, &n, &eps};
    return launch_named(ctx, "cima_rmsnorm_f16", (unsigned)rows, 256, args, kApiRms);
}

int cima_hip_rope(cima_hip_ctx* ctx, void* x, int rows, int heads, int dim, int pos0, float theta, int nfreqs,
                  const int* pos_dev) {
    const char* api = "cima_hip_rope";
    if (int rc = ready(ctx, api)) return rc;
    if (rows < 0 || heads <= 0 || dim <= 0 || dim % 2 || nfreqs < 0 || (long long)rows * heads > 0x7fffffffLL)
        return fail(CIMA_E_INVALID, "%s: rows=%d heads=%d dim=%d nfreqs=%d", api, rows, heads, dim, nfreqs);
    if (rows == 0) return 0;
    if (!x) return fail(CIMA_E_INVALID, "%s: null x", api);
    void* args[] = {&x, &heads, &dim, &pos0, &theta, &nfreqs, &pos_dev};
    return launch_named(ctx, "cima_rope_f16", (unsigned)(rows * heads), 64, args, api);
}

int cima_hip_kv_append(cima_hip_ctx* ctx, const void* k, const void* v, void* kc, void* vc, int rows, int kv_heads,
                       int dim, int pos, int max_seq, const int* pos_dev) {
    const char* api = "cima_hip_kv_append";
    if (int rc = ready(ctx, api)) return rc;
    if (rows < 0 || kv_heads <= 0 || dim <= 0 || max_seq <= 0)
        return fail(CIMA_E_INVALID, "%s: rows=%d kv_heads=%d dim=%d max_seq=%d", api, rows, kv_heads, dim, max_seq);
    if (rows == 0) return 0;
    if (!k || !v || !kc || !vc) return fail(CIMA_E_INVALID, "%s: null pointer", api);
    void* args[] = {&k, &v, &kc, &vc, &kv_heads, &dim, &pos, &max_seq, &pos_dev};
    return launch_named(ctx, "cima_kv_append_f16", (unsigned)rows, 256, args, api);
}

int cima_hip_attn_decode_split(cima_hip_ctx* ctx, const void* q, const void* kc, const void* vc, float* part,
                               int q_heads, int kv_heads, int dim, int seq, int max_seq, int csz, int n_chunks,
                               float scale, int window, const int* pos_dev) {
    const char* api = "cima_hip_attn_decode_split";
    if (int rc = ready(ctx, api)) return rc;
    if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || !attn_dim_ok(dim) || max_seq <= 0 || csz <= 0 ||
        csz > kAttMaxChunk || n_chunks <= 0 || (long long)n_chunks * csz < max_seq || seq < 0 || window < 0)
        return fail(CIMA_E_INVALID, "%s: q_heads=%d kv_heads=%d dim=%d seq=%d max_seq=%d csz=%d n_chunks=%d", api,
                    q_heads, kv_heads, dim, seq, max_seq, csz, n_chunks);
    if (!q || !kc || !vc || !part) return fail(CIMA_E_INVALID, "%s: null pointer", api);
    if (!aligned(kc, 16) || !aligned(vc, 16)) return fail(CIMA_E_INVALID, "%s: cache must be 16-byte aligned", api);
    char name[48];
    snprintf(name, sizeof name, "cima_attn_split_d%d", dim);
    void* args[] = {&q, &kc, &vc, &part, &q_heads, &kv_heads, &seq, &max_seq, &csz, &n_chunks, &scale, &window, &pos_dev};
    return launch_named(ctx, name, (unsigned)(q_heads * n_chunks), 256, args, api);
}

int cima_hip_attn_reduce(cima_hip_ctx* ctx, const float* part, void* out, int q_heads, int dim, int csz, int n_chunks,
                         int seq, int max_seq, int window, const int* pos_dev) {
    const char* api = "cima_hip_attn_reduce";
    if (int rc = ready(ctx, api)) return rc;
    if (q_heads <= 0 || !attn_dim_ok(dim) || csz <= 0 || n_chunks <= 0 || seq < 0 || max_seq <= 0 || window < 0)
        return fail(CIMA_E_INVALID, "%s: q_heads=%d dim=%d csz=%d n_chunks=%d seq=%d", api, q_heads, dim, csz,
                    n_chunks, seq);
    if (!part || !out) return fail(CIMA_E_INVALID, "%s: null pointer", api);
    char name[48];
    snprintf(name, sizeof name, "cima_attn_reduce_d%d", dim);
    void* args[] = {&part, &out, &csz, &n_chunks, &seq, &max_seq, &window, &pos_dev};
    return launch_named(ctx, name, (unsigned)q_heads, 256, args, api);
}

int cima_hip_attn_decode_noalloc(cima_hip_ctx* ctx, const void* q, const void* kc, const void* vc, void* out,
                                 int q_heads, int kv_heads, int dim, int seq, int max_seq, int csz, int n_chunks,
                                 float scale, int window, const int* pos_dev) {
    const char* api = "cima_hip_attn_decode_noalloc";
    if (int rc = ready(ctx, api)) return rc;
    if (!ctx->scratch) return fail(CIMA_E_NOT_INIT, "%s: the decode code object has no scratch array", api);
    if (q_heads <= 0 || dim <= 0 || n_chunks <= 0 ||
        (unsigned long long)q_heads * (unsigned long long)n_chunks * (unsigned long long)(dim + 2) * 4ULL >
            (unsigned long long)ctx->scratch_bytes)
        return fail(CIMA_E_INVALID, "%s: q_heads=%d x n_chunks=%d x (dim=%d + 2) fp32 partials exceed the %zu-byte "
                    "device scratch", api, q_heads, n_chunks, dim, ctx->scratch_bytes);
    float* part = static_cast<float*>(ctx->scratch);
    if (int rc = cima_hip_attn_decode_split(ctx, q, kc, vc, part, q_heads, kv_heads, dim, seq, max_seq, csz, n_chunks,
                                            scale, window, pos_dev))
        return rc;
    return cima_hip_attn_reduce(ctx, part, out, q_heads, dim, csz, n_chunks, seq, max_seq, window, pos_dev);
}

int cima_hip_attn_decode(cima_hip_ctx* ctx, const void* qkv, void* kc, void* vc, float* part, int q_heads,
                         int kv_heads, int dim, int max_seq, int csz, int n_chunks, float theta, float scale,
                         int window, const int* pos_dev) {
    const char* api = "cima_hip_attn_decode";
    if (int rc = ready(ctx, api)) return rc;
    return attn_fused(ctx, qkv, kc, vc, part, q_heads, kv_heads, dim, max_seq, csz, n_chunks, theta, scale, window,
                      pos_dev, api);
}

int cima_hip_attn_gguf_gemv(cima_hip_ctx* ctx, int t, const float* part, int q_heads, int dim, int csz, int n_chunks,
                            int max_seq, int window, const int* pos_dev, const void* w, const void* bias, void* y,
                            int n, int mode) {
    const char* api = "cima_hip_attn_gguf_gemv";
    if (int rc = ready(ctx, api)) return rc;
    if (q_heads <= 0 || !attn_dim_ok(dim) || csz <= 0 || n_chunks <= 0 || max_seq <= 0 || window < 0 ||
        (mode != 0 && mode != 1))
        return fail(CIMA_E_INVALID, "%s: q_heads=%d dim=%d csz=%d n_chunks=%d max_seq=%d mode=%d", api, q_heads, dim,
                    csz, n_chunks, max_seq, mode);
    if (!part || !pos_dev) return fail(CIMA_E_INVALID, "%s: null partials or position", api);
    if (!aligned(part, 8)) return fail(CIMA_E_INVALID, "%s: partials must be 8-byte aligned", api);
    GemvExt ext{};
    ext.att_chunks = n_chunks;
    ext.att_csz = csz;
    ext.att_dim = dim;
    ext.max_seq = max_seq;
    ext.pos_dev = pos_dev;
    ext.att_window = window;
    return gemv_common(ctx, t, part, w, nullptr, bias, nullptr, y, n, q_heads * dim, mode, CIMA_DT_F16, false, api,
                       nullptr, 0.f, GK_ATT, &ext);
}

int cima_hip_gguf_gemv_argmax(cima_hip_ctx* ctx, int t, const void* x, const void* norm_w, float eps, const void* w,
                              void* y, int n, int k, unsigned long long* slot) {
    const char* api = "cima_hip_gguf_gemv_argmax";
    if (int rc = ready(ctx, api)) return rc;
    if (!slot || !aligned(slot, 8)) return fail(CIMA_E_INVALID, "%s: null or misaligned slot", api);
    GemvExt ext{};
    ext.slot = slot;
    return gemv_common(ctx, t, x, w, nullptr, nullptr, nullptr, y, n, k, 0, CIMA_DT_F16, false, api, norm_w, eps,
                       GK_AMAX, &ext);
}

int cima_hip_argmax(cima_hip_ctx* ctx, const void* x, unsigned long long* slot, int n, float cap) {
    const char* api = "cima_hip_argmax";
    if (int rc = ready(ctx, api)) return rc;
    if (n <= 0 || !x || !slot || !aligned(slot, 8)) return fail(CIMA_E_INVALID, "%s: n=%d or null/misaligned pointer", api, n);
    unsigned grid = (unsigned)((n + 255) / 256);
    if (grid > 1024) grid = 1024;
    void* args[] = {&x, &slot, &n, &cap};
    return launch_named(ctx, "cima_argmax_f16", grid, 256, args, api);
}

int cima_hip_argmax_to_ids(cima_hip_ctx* ctx, unsigned long long* slot, unsigned int* ids, int* pos_dev) {
    const char* api = "cima_hip_argmax_to_ids";
    if (int rc = ready(ctx, api)) return rc;
    if (!slot) return fail(CIMA_E_INVALID, "%s: null slot", api);
    void* args[] = {&slot, &ids, &pos_dev};
    return launch_named(ctx, "cima_argmax_to_ids", 1, 64, args, api);
}

int cima_hip_pos_bump(cima_hip_ctx* ctx, int* pos_dev) {
    const char* api = "cima_hip_pos_bump";
    if (int rc = ready(ctx, api)) return rc;
    if (!pos_dev) return fail(CIMA_E_INVALID, "%s: null counter", api);
    void* args[] = {&pos_dev};
    return launch_named(ctx, "cima_pos_bump", 1, 64, args, api);
}

int cima_hip_decode_step(cima_hip_ctx* ctx, const cima_decoder* d) {
    const char* api = "cima_hip_decode_step";
    if (int rc = ready(ctx, api)) return rc;
    if (!d || !d->layers) return fail(CIMA_E_INVALID, "%s: null decoder or layer table", api);
    const int hd = d->head_dim, qd = d->q_heads * hd, kvd = d->kv_heads * hd;
    if (d->n_layers <= 0 || d->hidden <= 0 || d->ffn <= 0 || d->vocab <= 0 || d->q_heads <= 0 || d->kv_heads <= 0)
        return fail(CIMA_E_INVALID, "%s: layers=%d hidden=%d ffn=%d vocab=%d heads=%d/%d", api, d->n_layers,
                    d->hidden, d->ffn, d->vocab, d->q_heads, d->kv_heads);
    if (!d->x || !d->qkv || !d->act || !d->logits || !d->part || !d->slot || !d->ids || !d->pos || !d->embed ||
        !d->final_norm)
        return fail(CIMA_E_INVALID, "%s: null workspace, embedding or final norm pointer", api);
    const int csz = d->attn_chunk > 0 ? d->attn_chunk : kAttMaxChunk;
    if (csz > kAttMaxChunk) return fail(CIMA_E_INVALID, "%s: attn_chunk %d > %d", api, csz, kAttMaxChunk);
    const int nch = (d->max_seq + csz - 1) / csz;
    const float scale = 1.0f / sqrtf((float)hd);
    const void* head = d->head ? d->head : d->embed;
    const int head_type = d->head ? d->head_type : d->embed_type;
    // enqueue_decode_device (src/models/transformer.rs:1440-1461)
    if (int rc = cima_hip_gguf_gather(ctx, d->embed_type, d->embed, d->ids, d->x, 1, d->hidden)) return rc;
    auto ty = [&](int t) { return t ? t : d->ggml_type; };
    for (int l = 0; l < d->n_layers; l++) {
        const cima_decoder_layer& L = d->layers[l];
        if ((L.wk == nullptr) != (L.wv == nullptr))
            return fail(CIMA_E_INVALID, "%s: layer %d sets one of wk / wv", api, l);
        if (L.w_up && ty(L.type_gate) != ty(L.type_up))
            return fail(CIMA_E_INVALID, "%s: layer %d: gate and up formats differ (%d, %d)", api, l,
                        ty(L.type_gate), ty(L.type_up));
        // rmsnorm -> q|k|v GEMV with bias (forward_chunk_at :1030-1098):
        // one launch over the fused matrix, or one per projection into its
        // slice of qkv
        if (!L.wk) {
            if (int rc = cima_hip_rmsnorm_gguf_gemv(ctx, ty(L.type_q), d->x, L.attn_norm, d->rms_eps, L.wqkv, L.bqkv,
                                                    d->qkv, qd + 2 * kvd, d->hidden, 0, CIMA_DT_F16))
                return rc;
        } else {
            const void* w3[3] = {L.wqkv, L.wk, L.wv};
            const int t3[3] = {ty(L.type_q), ty(L.type_k), ty(L.type_v)};
            const int n3[3] = {qd, kvd, kvd}, o3[3] = {0, qd, qd + kvd};
            for (int j = 0; j < 3; j++) {
                const void* b = L.bqkv ? static_cast<const uint16_t*>(L.bqkv) + o3[j] : nullptr;
                if (int rc = cima_hip_rmsnorm_gguf_gemv(ctx, t3[j], d->x, L.attn_norm, d->rms_eps, w3[j], b,
                                                        static_cast<uint16_t*>(d->qkv) + o3[j], n3[j], d->hidden, 0,
                                                        CIMA_DT_F16))
                    return rc;
            }
        }
        // rope q, k; kv append; split attention (:1100-1160)
        if (int rc = attn_fused(ctx, d->qkv, L.k_cache, L.v_cache, d->part, d->q_heads, d->kv_heads, hd, d->max_seq,
                                csz, nch, d->rope_theta, scale, L.window, d->pos, api))
            return rc;
        // merge of the partials -> o projection + residual (:1161-1238)
        if (int rc = cima_hip_attn_gguf_gemv(ctx, ty(L.type_o), d->part, d->q_heads, hd, csz, nch, d->max_seq,
                                             L.window, d->pos, L.wo, nullptr, d->x, d->hidden, 1))
            return rc;
        // rmsnorm -> gate|up SwiGLU -> down + residual (:1240-1260)
        if (!L.w_up) {
            if (int rc = cima_hip_rmsnorm_gguf_gemv(ctx, ty(L.type_gate), d->x, L.ffn_norm, d->rms_eps, L.w_gate_up,
                                                    nullptr, d->act, d->ffn, d->hidden, 2, CIMA_DT_F16))
                return rc;
        } else if (int rc = gemv_common(ctx, ty(L.type_gate), d->x, L.w_gate_up, L.w_up, nullptr, nullptr, d->act,
                                        d->ffn, d->hidden, 2, CIMA_DT_F16, true, api, L.ffn_norm, d->rms_eps)) {
            return rc;
        }
        if (int rc = cima_hip_gguf_gemv(ctx, ty(L.type_down), d->act, L.w_down, nullptr, d->x, d->hidden, d->ffn, 1,
                                        CIMA_DT_F16))
            return rc;
    }
    // final norm -> head with argmax -> ids[0], pos += 1
    if (int rc = cima_hip_gguf_gemv_argmax(ctx, head_type, d->x, d->final_norm, d->rms_eps, head, d->logits, d->vocab,
                                           d->hidden, d->slot))
        return rc;
    return cima_hip_argmax_to_ids(ctx, d->slot, d->ids, d->pos);
}

// ---------------------------------------------------------------- graphs

struct cima_hip_graph {
    hipGraphExec_t exec = nullptr;
};

int cima_hip_capture_begin(cima_hip_ctx* ctx) {
    if (int rc = ready(ctx, "cima_hip_capture_begin")) return rc;
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeGlobal);
    return e == hipSuccess ? 0 : hip_fail(e, "hipStreamBeginCapture");
}

int cima_hip_capture_end(cima_hip_ctx* ctx, cima_hip_graph** out) {
    if (int rc = ready(ctx, "cima_hip_capture_end")) return rc;
    if (!out) return fail(CIMA_E_INVALID, "cima_hip_capture_end: null out pointer");
    *out = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiateWithFlags(&exec, graph, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiateWithFlags");
    auto* g = new cima_hip_graph();
    g->exec = exec;
    *out = g;
    return 0;
}

int cima_hip_graph_launch(cima_hip_ctx* ctx, cima_hip_graph* g) {
    if (int rc = ready(ctx, "cima_hip_graph_launch")) return rc;
    if (!g || !g->exec) return fail(CIMA_E_INVALID, "cima_hip_graph_launch: null graph");
    hipError_t e = hipGraphLaunch(g->exec, ctx->stream);
    return e == hipSuccess ? 0 : hip_fail(e, "hipGraphLaunch");
}

int cima_hip_graph_destroy(cima_hip_graph* g) {
    if (!g) return 0;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    delete g;
    return 0;
}

int cima_hip_stream_read_cfg(cima_hip_ctx* ctx, const void* src, long long nbytes, unsigned int* sink, int dest,
                             int depth, int width, int wgs_per_cu) {
    const char* api = "cima_hip_stream_read_cfg";
    if (int rc = ready(ctx, api)) return rc;
    if (nbytes < 0 || !src || !sink || !aligned(src, 16))
        return fail(CIMA_E_INVALID, "%s: null or misaligned (16 B) pointer, or nbytes < 0", api);
    if (wgs_per_cu < 1 || wgs_per_cu > 8) return fail(CIMA_E_INVALID, "%s: %d workgroups per CU", api, wgs_per_cu);
    char name[64];
    long long per_wg;  // bytes one workgroup takes per round
    if (dest == 0) {
        const bool ok = (width == 16 && (depth == 1 || depth == 2 || depth == 4 || depth == 8 || depth == 16)) ||
                        (width == 8 && (depth == 4 || depth == 8 || depth == 16));
        if (!ok) return fail(CIMA_E_INVALID, "%s: register reads of %d x %d B are not built", api, depth, width);
        snprintf(name, sizeof name, "cima_stream_read_r%d_w%d", depth, width);
        per_wg = 256LL * depth * width;
    } else if (dest == 1) {
        if (width != 16 || !(depth == 2 || depth == 4 || depth == 8 || depth == 16))
            return fail(CIMA_E_INVALID, "%s: LDS rings of %d KB per wave are not built", api, depth);
        snprintf(name, sizeof name, "cima_stream_read_l%d", depth);
        per_wg = 4LL * 1024 * depth;
    } else {
        return fail(CIMA_E_INVALID, "%s: destination %d is not 0 (registers) or 1 (LDS)", api, dest);
    }
    if (nbytes < 1024) return 0;
    long long grid = (nbytes + per_wg - 1) / per_wg;
    if (grid > (long long)wgs_per_cu * ctx->num_cu) grid = (long long)wgs_per_cu * ctx->num_cu;
    void* args[] = {&src, &nbytes, &sink};
    return launch_named(ctx, name, (unsigned)grid, 256, args, api);
}

int cima_hip_stream_read(cima_hip_ctx* ctx, const void* src, long long nbytes, unsigned int* sink) {
    const char* api = "cima_hip_stream_read";
    if (int rc = ready(ctx, api)) return rc;
    if (nbytes < 0 || !src || !sink || !aligned(src, 16))
        return fail(CIMA_E_INVALID, "%s: null or misaligned (16 B) pointer, or nbytes < 0", api);
    nbytes &= ~15LL;
    if (nbytes == 0) return 0;
    long long grid = (nbytes / 16 + 4 * 256 - 1) / (4 * 256);
    if (grid > 2L * ctx->num_cu) grid = 2L * ctx->num_cu;
    void* args[] = {&src, &nbytes, &sink};
    return launch_named(ctx, "cima_stream_read", (unsigned)grid, 256, args, api);
}

}  // extern "C"

// ------------------------------------------------------------ bitsandbytes 4-bit

int cima_hip_set_nf4_tuning(cima_hip_ctx* ctx, int rows, int kernel) {
    if (!ctx) return fail(CIMA_E_NOT_INIT, "cima_hip_set_nf4_tuning: null context");
    if (rows != 0 && rows != 1 && rows != 2 && rows != 4)
        return fail(CIMA_E_INVALID, "cima_hip_set_nf4_tuning: rows %d is not 0, 1, 2 or 4", rows);
    if (kernel < 0 || kernel > 2) return fail(CIMA_E_INVALID, "cima_hip_set_nf4_tuning: kernel %d is not 0, 1 or 2", kernel);
    ctx->tune_nf4_rows = rows;
    ctx->tune_nf4_kernel = kernel;
    return 0;
}

int cima_hip_nf4_dequant(cima_hip_ctx* ctx, const void* packed, const float* absmax, const float* qmap, void* out,
                         long long n, int blocksize) {
    const char* api = "cima_hip_nf4_dequant";
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "%s: context is not initialised", api);
    if (n < 0 || blocksize <= 0) return fail(CIMA_E_INVALID, "%s: n=%lld blocksize=%d", api, n, blocksize);
    if (n == 0) return 0;
    if (!packed || !absmax || !qmap || !out) return fail(CIMA_E_INVALID, "%s: null pointer", api);
    if (!aligned(absmax, 4) || !aligned(qmap, 4) || !aligned(out, 2))
        return fail(CIMA_E_INVALID, "%s: misaligned absmax / qmap (4 B) or out (2 B)", api);
    const void* pk = packed;
    const float* am = absmax;
    const float* qm = qmap;
    void* o = out;
    if (n % 32 == 0 && blocksize % 32 == 0 && aligned(packed, 16) && aligned(out, 16)) {
        long long nseg = n / 32;
        int spb = blocksize / 32;
        long long grid = (nseg + 255) / 256;
        if (grid > 0x7fffffffLL) return fail(CIMA_E_INVALID, "%s: n=%lld is too large", api, n);
        void* args[] = {&pk, &am, &qm, &o, &nseg, &spb};
        return launch_named(ctx, "cima_nf4_dequant_v", (unsigned)grid, 256, args, api);
    }
    long long nn = n;
    int bs = blocksize;
    long long grid = (n + 255) / 256;
    if (grid > 0x7fffffffLL) return fail(CIMA_E_INVALID, "%s: n=%lld is too large", api, n);
    void* args[] = {&pk, &am, &qm, &o, &nn, &bs};
    return launch_named(ctx, "cima_nf4_dequant_e", (unsigned)grid, 256, args, api);
}

int cima_hip_nf4_gemv(cima_hip_ctx* ctx, const void* x, const void* packed, const float* absmax, const float* qmap,
                      void* y, int n, int k, int blocksize, int act_dtype) {
    const char* api = "cima_hip_nf4_gemv";
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "%s: context is not initialised", api);
    if (act_dtype != CIMA_DT_F32 && act_dtype != CIMA_DT_F16)
        return fail(CIMA_E_INVALID, "%s: act_dtype %d is not CIMA_DT_F32 or CIMA_DT_F16", api, act_dtype);
    if (n < 0 || k <= 0 || blocksize <= 0) return fail(CIMA_E_INVALID, "%s: n=%d k=%d blocksize=%d", api, n, k, blocksize);
    if (n == 0) return 0;
    if (!x || !packed || !absmax || !qmap || !y) return fail(CIMA_E_INVALID, "%s: null pointer", api);
    const int esz = act_dtype == CIMA_DT_F32 ? 4 : 2;
    if (!aligned(x, esz) || !aligned(y, esz) || !aligned(absmax, 4) || !aligned(qmap, 4))
        return fail(CIMA_E_INVALID, "%s: misaligned x / y (%d B) or absmax / qmap (4 B)", api, esz);
    const char* an = act_dtype == CIMA_DT_F32 ? "f32" : "f16";
    const void* xp = x;
    const void* pk = packed;
    const float* am = absmax;
    const float* qm = qmap;
    void* yp = y;
    int nn = n, kk = k;
    const bool pow2 = (blocksize & (blocksize - 1)) == 0;
    const long long segs_total = (long long)n * (k / 32);
    const long long tab_lds = 65536LL + 2LL * k;  // pair table + x
    if (k % 32 == 0 && blocksize >= 32 && pow2 && aligned(packed, 16) && aligned(x, 16) && segs_total < (1LL << 32) &&
        2LL * k <= ctx->max_lds) {
        int bshift = 0;
        while ((32 << bshift) < blocksize) bshift++;
        // the pair table when it fits next to x (1024-thread workgroups, one
        // per CU), else the codebook in registers (256-thread workgroups)
        bool tab = tab_lds <= ctx->max_lds;
        if (ctx->tune_nf4_kernel == 1 && !tab)
            return fail(CIMA_E_INVALID, "%s: k=%d does not leave room for the pair table in LDS", api, k);
        if (ctx->tune_nf4_kernel == 2) tab = false;
        const int wpg = tab ? 16 : 4;  // waves per workgroup
        // two workgroups per CU where the LDS holds them; rows per wave: the
        // fewest row-steps for the busiest wave, ties to 2 rows, then 1
        // (measured on MI355X, weights cold: 14336x4096 9.9 us at 2 rows
        // against 10.7 at 1; 4096x14336, one workgroup per CU, 10.7 at 1
        // row against 13.8 at 2)
        const long long wgs = ctx->tune_wgs ? ctx->tune_wgs : (!tab || 2 * tab_lds <= ctx->max_lds ? 2 : 1);
        const long long waves = wgs * ctx->num_cu * wpg;
        int r = ctx->tune_nf4_rows;
        if (!r) {
            long long best = -1;
            for (int cand : {2, 1, 4}) {
                const long long groups_c = (n + cand - 1) / cand;
                const long long cost = (groups_c + waves - 1) / waves * cand;
                if (best < 0 || cost < best) {
                    best = cost;
                    r = cand;
                }
            }
        }
        const long long groups = (n + r - 1) / r;
        long long grid = (groups + wpg - 1) / wpg;
        if (grid > wgs * ctx->num_cu) grid = wgs * ctx->num_cu;
        // a wave keeps the sums of its rows in one register until the end: at most 64 rows per wave
        const long long min_waves = (groups * r + 63) / 64;
        if (grid < (min_waves + wpg - 1) / wpg) grid = (min_waves + wpg - 1) / wpg;
        char name[64];
        snprintf(name, sizeof name, "cima_nf4_gemv_%s_r%d_%s_%s", tab ? "t" : "c", r, an, an);
        hipFunction_t f;
        if (int rc = get_fn(ctx, name, &f)) return rc;
        void* args[] = {&xp, &pk, &am, &qm, &yp, &nn, &kk, &bshift};
        return launch(ctx, f, (unsigned)grid, 64 * wpg, args, api, (unsigned)(tab ? tab_lds : 2LL * k));
    }
    int bs = blocksize;
    char name[64];
    snprintf(name, sizeof name, "cima_nf4_gemv_e_%s_%s", an, an);
    void* args[] = {&xp, &pk, &am, &qm, &yp, &nn, &kk, &bs};
    return launch_named(ctx, name, (unsigned)((n + 3) / 4), 256, args, api);
}

int cima_hip_nf4_gemm_slab(cima_hip_ctx* ctx, const void* x, const void* packed, const float* absmax,
                           const float* qmap, void* y, int m, int n, int k, int blocksize, int x_dtype, int y_dtype,
                           void* slab, unsigned long long slab_bytes) {
    const char* api = "cima_hip_nf4_gemm_slab";
    if (!ctx || !ctx->loaded) return fail(CIMA_E_NOT_INIT, "%s: context is not initialised", api);
    if (m < 0 || n < 0 || k <= 0 || k % 8 || blocksize <= 0)
        return fail(CIMA_E_INVALID, "%s: m=%d n=%d k=%d blocksize=%d (k must be a positive multiple of 8)", api, m, n,
                    k, blocksize);
    if (x_dtype < CIMA_DT_F32 || x_dtype > CIMA_DT_BF16 || (y_dtype != CIMA_DT_F32 && y_dtype != CIMA_DT_F16))
        return fail(CIMA_E_INVALID, "%s: x_dtype %d / y_dtype %d not supported", api, x_dtype, y_dtype);
    if (m == 0 || n == 0) return 0;
    if (!x || !packed || !absmax || !qmap || !y || !slab) return fail(CIMA_E_INVALID, "%s: null pointer", api);
    if (!aligned(x, 16) || !aligned(y, 4) || !aligned(slab, 256))
        return fail(CIMA_E_INVALID, "%s: misaligned x (16 B), y (4 B) or slab (256 B)", api);
    if ((long long)m * k * (x_dtype == CIMA_DT_F32 ? 4 : 2) > 0xffffffffLL)
        return fail(CIMA_E_INVALID, "%s: X of %d x %d is 4 GiB or more", api, m, k);
    // The slab must hold one row slice of the f16 weight, as the
    // reference's lin_gemm needs of its scratch (both routes check it, so
    // a caller sized for the reference behaves the same here).  A slice
    // starts on an absmax block boundary: g rows is the smallest count whose
    // elements are whole blocks.
    long long g = blocksize;
    {
        long long a = blocksize, b = k;
        while (b) {
            const long long t2 = a % b;
            a = b;
            b = t2;
        }
        g = blocksize / a;  // blocksize / gcd(blocksize, k)
    }
    long long rows = (long long)(slab_bytes / (2ULL * (unsigned long long)k)) / g * g;
    if (rows > n) rows = n;
    if (rows < 1)
        return fail(CIMA_E_INVALID, "%s: slab of %llu bytes holds no %lld-row slice of the f16 weight (k=%d)", api,
                    slab_bytes, g, k);
    // Fused route: the MFMA tiles decode the packed weight themselves
    // (cima_gemm_nf4_*), the slab is not touched.  It takes every
    // bitsandbytes checkpoint shape: k % 64 == 0, 32-element runs sharing
    // one absmax (blocksize % 32 == 0), 16-byte aligned packed rows.
    if (k % 64 == 0 && blocksize % 32 == 0 && aligned(packed, 16) && aligned(absmax, 4)) {
        const int sh = (blocksize & (blocksize - 1)) == 0 ? log2i(blocksize) : -1;
        return gemm_launch(ctx, "nf4", x, packed, y, m, n, k, n, x_dtype, y_dtype,
                           GemmExt{absmax, qmap, (long long)blocksize, sh, nullptr, nullptr, 1}, api);
    }
    // Slab route for the other shapes: W is decoded into the slab a row
    // slice at a time (the reference's lin_gemm works through its 32 MiB
    // DQ_SCRATCH the same way, src/models/transformer.rs:630-653) and each
    // slice is multiplied by this library's f16-weight GEMM into its
    // columns of Y (leading dimension n): the MFMA tiles when k % 64 == 0,
    // else a plain one-thread-per-output kernel.
    static const char* const xn[] = {"f32", "f16", "bf16"};
    hipFunction_t small = nullptr;
    if (k % 64) {
        char name[64];
        snprintf(name, sizeof name, "cima_gemm_f16w_small_%s_%s", xn[x_dtype], y_dtype == CIMA_DT_F32 ? "f32" : "f16");
        if (int rc = get_fn(ctx, name, &small)) return rc;
    }
    const int yes = y_dtype == CIMA_DT_F32 ? 4 : 2;
    for (long long r0 = 0; r0 < n; r0 += rows) {
        const int nr = (int)std::min(rows, (long long)n - r0);
        const long long e0 = r0 * k;
        if (int rc = cima_hip_nf4_dequant(ctx, static_cast<const uint8_t*>(packed) + e0 / 2, absmax + e0 / blocksize,
                                          qmap, slab, (long long)nr * k, blocksize))
            return rc;
        void* ys = static_cast<uint8_t*>(y) + (size_t)r0 * yes;
        if (!small) {
            if (int rc = gemm_launch(ctx, "f16w", x, slab, ys, m, nr, k, n, x_dtype, y_dtype, GemmExt{}, api))
                return rc;
        } else {
            const void* xa = x;
            const void* wa = slab;
            void* ya = ys;
            int mm = m, nn = nr, kk = k, ld = n;
            void* args[] = {&xa, &wa, &ya, &mm, &nn, &kk, &ld};
            const long long outs = (long long)m * nr;
            if (int rc = launch(ctx, small, (unsigned)((outs + 255) / 256), 256, args, api)) return rc;
        }
    }
    return 0;
}
