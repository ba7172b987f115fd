/*
 * cima_hip.h -- C ABI of the MI355X (gfx950) GGUF dequant-GEMV library.
 *
 * This is the drop-in boundary for the reference engine's GGUF hot path:
 * each entry point replaces one method of the reference's CudaCtx (Rust,
 * src/cuda.rs), with the same argument order and meaning.  Pointers are
 * device pointers (hipMalloc'd or any HIP-visible device memory), sizes are
 * element or row counts, and every call is asynchronous on the context's
 * stream.  No call allocates device memory or calls a library kernel, so
 * all are safe inside HIP graph capture once the context exists.
 *
 * Return value: 0 on success; a positive hipError_t when the HIP runtime
 * failed; a negative CIMA_E_* code when the arguments were rejected before
 * anything was launched.  cima_hip_last_error() gives the message of the
 * last failure on the calling thread.
 *
 * Formats are ggml tensor type ids (src/formats.rs:90-117): 8 = Q8_0,
 * 2 = Q4_0, 3 = Q4_1, 6 = Q5_0, 7 = Q5_1, 12 = Q4_K, 13 = Q5_K, 14 = Q6_K,
 * 23 = IQ4_XS -- every GGUF block format the reference executes.
 */
#ifndef CIMA_HIP_H
#define CIMA_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids */
#define CIMA_GGML_Q4_0 2
#define CIMA_GGML_Q4_1 3
#define CIMA_GGML_Q5_0 6
#define CIMA_GGML_Q5_1 7
#define CIMA_GGML_Q8_0 8
#define CIMA_GGML_Q4_K 12
#define CIMA_GGML_Q5_K 13
#define CIMA_GGML_Q6_K 14
#define CIMA_GGML_IQ4_XS 23

/* activation / output element types */
#define CIMA_DT_F32 0
#define CIMA_DT_F16 1
#define CIMA_DT_BF16 2

/* argument errors (negative; hipError_t values are positive) */
#define CIMA_E_INVALID -1     /* bad pointer, shape, mode or alignment */
#define CIMA_E_FORMAT -2      /* not a supported GGUF block format */
#define CIMA_E_NO_KERNEL -3   /* code object lacks the kernel */
#define CIMA_E_NOT_INIT -4    /* null or destroyed context */
#define CIMA_E_LIBRARY -5     /* kept for the reference's error set; no entry point returns it now */

typedef struct cima_hip_ctx cima_hip_ctx;

/* Context creation: replaces CudaCtx::init (src/cuda.rs:691-908) -- device
 * selection, one non-blocking stream, then loading the prebuilt gfx950 code
 * objects (cima_gemv_a/b/c.hsaco, cima_gemm.hsaco, cima_dequant.hsaco,
 * cima_decode.hsaco) with
 * hipModuleLoad and resolving every kernel (the reference JIT-compiles with
 * NVRTC and resolves its KernelSet, src/cuda.rs:808-877).
 * code_dir: directory holding the code objects, or NULL for the directory
 * of this library. */
int cima_hip_init(int device, const char* code_dir, cima_hip_ctx** out);

/* Releases the module and the context's own stream. */
int cima_hip_destroy(cima_hip_ctx* ctx);

/* Per-thread binding: replaces CudaCtx::bind (src/cuda.rs:681-685,
 * cuCtxSetCurrent) with hipSetDevice. */
int cima_hip_bind(cima_hip_ctx* ctx);

/* Launch stream: every later call launches on hip_stream exactly as given
 * -- NULL is the device's null (legacy default) stream, which orders with
 * every blocking stream.  The caller keeps ownership of a stream it sets. */
int cima_hip_set_stream(cima_hip_ctx* ctx, void* hip_stream);
/* Launches go back to the context's own non-blocking stream, the one the
 * reference's CudaCtx creates at init (src/cuda.rs:740-744). */
int cima_hip_use_own_stream(cima_hip_ctx* ctx);
void* cima_hip_get_stream(cima_hip_ctx* ctx);

/* hipStreamSynchronize on the launch stream: CudaCtx::sync. */
int cima_hip_sync(cima_hip_ctx* ctx);

/* Message of the last failure on this thread ("" if none). */
const char* cima_hip_last_error(void);

/* 1 if `code` is a sticky device fault after which the context must be
 * rebuilt: the classification of cu_fatal (src/cuda.rs:122-127). */
int cima_hip_is_fatal(int code);

/* Number of compute units of the context's device. */
int cima_hip_num_cu(cima_hip_ctx* ctx);

/* GEMV launch tuning (no counterpart in the reference): rows per lane group
 * (1 or 2) and lanes per group (16..256, a power of two) for every
 * later gguf_gemv call on this context; 0 restores the built-in heuristic.
 * The environment variables CIMA_GEMV_ROWS / CIMA_GEMV_LPR set the initial
 * values at cima_hip_init (CIMA_GEMV_RING=1 / 2 forces / forbids the
 * item-ring main loop for one-unit rows). */
int cima_hip_set_gemv_tuning(cima_hip_ctx* ctx, int rows, int lanes_per_row);

/* GEMV main-loop choice (no counterpart in the reference): 0 = built-in
 * heuristic, 1 = the direct-to-LDS streaming kernels with one item in flight
 * per wave wherever they are built and fit, 3 = the same with two where
 * built (the gate+up pair, rows of one unit at 16 or 32 lanes; else one),
 * 2 = never them (the register-ring kernels).  Environment variable
 * CIMA_GEMV_DMA at init.  A set_gemv_tuning override of rows selects the
 * register kernels; one of lanes does too under the heuristic (mode 0) and
 * picks the streaming kernels' lanes per row (16, 32 or 64) under 1 or 3. */
int cima_hip_set_gemv_dma(cima_hip_ctx* ctx, int mode);

/* GEMV rows split over the workgroup's four waves (no counterpart in the
 * reference): for rows of more than 128 units (k > 8192 at Q4_K, k > 4096
 * at Q8_0) each wave takes a quarter of every row with its x fragment in
 * registers, and the four partial sums add in a fixed order.  0 = built-in
 * heuristic (Q6_K), 1 = wherever it applies (plain and epilogue GEMVs,
 * rows of at most 512 units), 2 = never.  Environment variable
 * CIMA_GEMV_WSPLIT at init. */
int cima_hip_set_gemv_wsplit(cima_hip_ctx* ctx, int mode);

/* GEMV grid tuning (no counterpart in the reference): the persistent grid
 * holds at most this many 256-thread workgroups per CU (0 = the default of 1, or fewer
 * if fewer fit; environment variable CIMA_GEMV_WGS at init). */
int cima_hip_set_gemv_grid(cima_hip_ctx* ctx, int wgs_per_cu);

/* X range flags of the prefill GEMMs (no counterpart in the reference).
 * The MFMA tiles round X to f16: exact for bf16 X of 2^-17 <= |x| < 65536
 * and zero, while larger values become +-inf and smaller nonzero ones may
 * lose bits; f32 X of |x| >= 65520 becomes inf.  Every gguf_gemm /
 * gguf_gemm_slab / nf4_gemm_slab call ORs into a per-context word: bit 0 =
 * X held values beyond f16's range, inf or NaN; bit 1 = X (bf16) held
 * nonzero values below 2^-17.  This call waits for the context's stream,
 * returns the word in *flags and clears it when `clear` is nonzero.  Not
 * for use during graph capture (it synchronises).  The check reads each X
 * element once more (its share in every workgroup, from L2); the
 * environment variable CIMA_GEMM_XCHECK=0 at cima_hip_init switches it off. */
#define CIMA_XRANGE_OVERFLOW 1u
#define CIMA_XRANGE_TINY 2u
int cima_hip_gemm_status(cima_hip_ctx* ctx, unsigned int* flags, int clear);

/* Prefill GEMM tuning (no counterpart in the reference): token-tile width
 * (16, 32, 64, 128 or 256) for later gguf_gemm calls; 0 = the built-in
 * choice (16 up to 32 tokens; 32 up to 128 while that grid has at most one
 * workgroup per CU, else 64; beyond, 256 where 128-token tiles would need
 * more than 1.5 workgroups per CU and 256-token tiles fit one per CU, else
 * 128). */
int cima_hip_set_gemm_tile(cima_hip_ctx* ctx, int tokens);

/* Fused dequant-GEMV: replaces CudaCtx::gguf_gemv (src/cuda.rs:2161-2220).
 *   y[r] = sum_j W[r, j] * x[j] for r in [0, n), W packed GGUF rows of k
 *   elements (row r at r * storage_bytes(fmt, k)).
 *   mode 0: y = dot (+ bias[r])
 *   mode 1: y = y + dot (+ bias[r])                  residual epilogue
 *   mode 2: W is the [2n, k] gate|up pair (rows [0,n) gate, [n,2n) up),
 *           bias (if any) has 2n entries:
 *           y = silu(g + bias[r]) * (u + bias[n + r])  (k_gemv_f16 mode 2,
 *           src/kernels.cu:493-538)
 *   act_dtype: CIMA_DT_F32 (x, bias, y fp32) or CIMA_DT_F16 (x, bias, y f16,
 *   the engine's activation type).  bias may be NULL.
 * Requires k % 32 == 0 (Q8_0, Q4_0) or k % 256 == 0 (Q4_K, Q6_K); x, bias
 * and y aligned to their element size (2 bytes f16, 4 bytes f32) as the
 * reference's pointers are, so a caller may pass a sub-slice at any element
 * offset; W 16-byte aligned for Q4_K and 2-byte aligned otherwise.
 * Unlike the reference, x is not quantised to 8-bit q8_1: each workgroup
 * stages it as 16-bit fixed point per 32-element block (x ~= s (256 hi +
 * lo), hi and lo int8, error <= amax/65278 per element); the weight quants
 * are dotted exactly in int32 (v_dot4_i32_i8 against the hi and lo planes)
 * and the block sums scaled in fp32. */
int cima_hip_gguf_gemv(cima_hip_ctx* ctx, int ggml_type, const void* x, const void* w,
                       const void* bias, void* y, int n, int k, int mode, int act_dtype);

/* RMSNorm fused into the GEMV: the same as cima_hip_gguf_gemv (modes 0, 1,
 * 2) applied to h = rmsnorm(x) = f16(sat(x) * rsqrt(mean(sat(x)^2) + eps) *
 * norm_w) (f32 activations: h stays fp32), where sat clamps to +-65000.
 * Replaces CudaCtx::rmsnorm (src/cuda.rs:1180-1198, k_rmsnorm
 * src/kernels.cu:37-50) followed by gguf_gemv on its output, as
 * forward_chunk_at runs them (src/models/transformer.rs:1030-1060, 1240-1252)
 * -- h is never written to memory.  norm_w has k entries of act_dtype,
 * 16-byte aligned. */
int cima_hip_rmsnorm_gguf_gemv(cima_hip_ctx* ctx, int ggml_type, const void* x, const void* norm_w, float eps,
                               const void* w, const void* bias, void* y, int n, int k, int mode, int act_dtype);
/* Fused gate+up SwiGLU GEMV over two separately stored weights (the
 * reference runs gate GEMV, up GEMV and k_swiglu, src/models/
 * transformer.rs:1249-1252): y = silu(Wg.x + bg) * (Wu.x + bu).
 * bias_gate / bias_up may be NULL. */
int cima_hip_gguf_gemv_swiglu(cima_hip_ctx* ctx, int ggml_type, const void* x,
                              const void* w_gate, const void* w_up, const void* bias_gate,
                              const void* bias_up, void* y, int n, int k, int act_dtype);

/* Prefill dequant-GEMM on MFMA: Y[m, n] (row stride ldy >= n) =
 * X[m, k] . dequant(W)[n, k]^T for m tokens.  Replaces the reference's
 * lin_gemm (src/models/transformer.rs:618-655): gguf_dequant of W into an
 * f16 slab (src/cuda.rs:2285) followed by gemm_f16 / gemm_strided_out
 * (src/cuda.rs:2468-2570), with no slab -- each workgroup dequantises its
 * W tile, bit-exact f16, into LDS (128-token tiles) or straight into the
 * MFMA operand registers (up to 64 tokens), and multiplies with f16 MFMA,
 * fp32 accumulate.  x_dtype: CIMA_DT_F32, CIMA_DT_F16 or CIMA_DT_BF16,
 * converted to f16 -- exact for bf16 of 2^-17 <= |x| < 65536; beyond,
 * values overflow to +-inf and below may lose bits as f16 subnormals, which
 * the call reports through cima_hip_gemm_status (the engine's activations
 * are f16 already, saturated to +-65000 by its RMSNorm, so nothing is lost
 * there); y_dtype: CIMA_DT_F32 or CIMA_DT_F16.
 * Requires k % 64 == 0 (and k % 256 for K-quants), x 16-byte aligned. */
int cima_hip_gguf_gemm(cima_hip_ctx* ctx, int ggml_type, const void* x, const void* w, void* y,
                       int m, int n, int k, int ldy, int x_dtype, int y_dtype);

/* Prefill GEMM with the engine's scratch slab: the signature of the
 * reference's lin_gemm / WTensor::gemm route (src/models/transformer.rs:
 * 618-655, src/quant.rs:120-129), whose gguf_dequant into the DQ_SCRATCH
 * slab + gemm_dispatch (src/cuda.rs:2285-2320, 2468-2541) runs here as the
 * fused MFMA kernels of cima_hip_gguf_gemm: W is dequantised tile by tile
 * and never expanded, and any slab size, 0 included, works.  No library
 * GEMM is involved.  At up to 32 tokens a weight too narrow to fill the
 * CUs is split along k over more workgroups, with the S partial tiles
 * (S x m x n fp32, S = 2 or 4) in the slab (256-byte aligned) and summed
 * into Y in a fixed order by a second launch; without room in the slab
 * the call runs unsplit.  The slab's contents are then scratch: calls that
 * share a slab must not overlap. */
int cima_hip_gguf_gemm_slab(cima_hip_ctx* ctx, int ggml_type, const void* x, const void* w, void* y,
                            int m, int n, int k, int ldy, int x_dtype, int y_dtype, void* slab,
                            unsigned long long slab_bytes);

/* Dequantise nblocks consecutive blocks to f16, bit-exact with the host
 * decoders: replaces CudaCtx::gguf_dequant (src/cuda.rs:2285-2320). */
int cima_hip_gguf_dequant(cima_hip_ctx* ctx, int ggml_type, const void* src, void* out_f16,
                          long long nblocks);

/* Embedding gather from a packed table: out[i, :] = dequant(table[ids[i]])
 * as f16; replaces CudaCtx::gguf_gather (src/cuda.rs:2226-2283).
 * ids are u32 row indices; they are not range-checked on the device. */
int cima_hip_gguf_gather(cima_hip_ctx* ctx, int ggml_type, const void* table,
                         const unsigned int* ids, void* out_f16, int n, int hidden);

/* ---------------------------------------------------------------------
 * Decode-step support (f16 activations).  These are the non-GEMV launches
 * of one batch-1 decode step of the reference's transformer family, each
 * with the argument meaning of the CudaCtx method it replaces.  pos_dev,
 * where accepted, is a device int holding the current position (graph
 * replay); NULL uses the host value.  Attention needs head_dim 64 or 128,
 * chunk sizes up to 256 and n_chunks * csz >= max_seq.
 * --------------------------------------------------------------------- */

/* y[r] = f16(sat(x[r]) * rsqrt(mean(sat(x[r])^2) + eps) * w) for rows
 * r < rows of n elements; w NULL = unit weight.  CudaCtx::rmsnorm
 * (src/cuda.rs:1180-1198). */
int cima_hip_rmsnorm(cima_hip_ctx* ctx, const void* x, const void* w, void* y, int rows, int n, float eps);
/* In-place NeoX RoPE over x [rows, heads, dim]; row r at position pos0 + r
 * (or *pos_dev + r); pairs >= nfreqs unrotated.  CudaCtx::rope
 * (src/cuda.rs:1302-1340) without frequency factors. */
int cima_hip_rope(cima_hip_ctx* ctx, void* x, int rows, int heads, int dim, int pos0, float theta, int nfreqs,
                  const int* pos_dev);
/* k, v [rows, kv_heads*dim] -> caches [kv_heads, max_seq, dim] at position
 * pos + r (or *pos_dev + r); positions >= max_seq are dropped.
 * CudaCtx::kv_append (src/cuda.rs:1344-1375). */
int cima_hip_kv_append(cima_hip_ctx* ctx, const void* k, const void* v, void* k_cache, void* v_cache, int rows,
                       int kv_heads, int dim, int pos, int max_seq, const int* pos_dev);
/* Per-(head, chunk) partial attention {m, l, acc[dim]} fp32 into part
 * [q_heads, n_chunks, dim + 2] for the query q [q_heads, dim] against the
 * first seq (or *pos_dev + 1) cache positions.  CudaCtx::attn_decode_split
 * (src/cuda.rs:1418-1474). */
int cima_hip_attn_decode_split(cima_hip_ctx* ctx, const void* q, const void* k_cache, const void* v_cache,
                               float* part, int q_heads, int kv_heads, int dim, int seq, int max_seq, int csz,
                               int n_chunks, float scale, int window, const int* pos_dev);
/* Log-sum-exp merge of the partials into out [q_heads, dim] f16.
 * CudaCtx::attn_reduce (src/cuda.rs:1476-1505). */
int cima_hip_attn_reduce(cima_hip_ctx* ctx, const float* part, void* out, int q_heads, int dim, int csz,
                         int n_chunks, int seq, int max_seq, int window, const int* pos_dev);
/* Split decode attention and its merge in one call that allocates
 * nothing: cima_hip_attn_decode_split + cima_hip_attn_reduce (same
 * arguments and results), their partials kept in a fixed 4 MiB device
 * array of the decode code object instead of a caller's workspace.  No
 * counterpart in the reference: for callers that cannot allocate (HIP
 * graph capture, tight serving loops, harnesses that forbid it).  Limit:
 * q_heads * n_chunks * (dim + 2) * 4 bytes <= 4 MiB, else CIMA_E_INVALID.
 * The array belongs to the context: each context loads its own copy of
 * the decode code object, so each holds its own 4 MiB of device memory
 * until it is destroyed.  Calls on one context share that array and keep
 * the last call's contents: calls on one context that overlap (on other
 * streams) race; calls on different contexts do not. */
int cima_hip_attn_decode_noalloc(cima_hip_ctx* ctx, const void* q, const void* k_cache, const void* v_cache,
                                 void* out, int q_heads, int kv_heads, int dim, int seq, int max_seq, int csz,
                                 int n_chunks, float scale, int window, const int* pos_dev);
/* One launch for a layer's decode attention partials at position
 * *pos_dev: RoPE of q and k from qkv = [q | k | v] (the fused q/k/v GEMV
 * output), append of the new k and v to the caches, and the split
 * attention of every (query head, chunk) into part (as for
 * cima_hip_attn_decode_split, window > 0 keeping the last `window`
 * positions).  Replaces rope x2 + kv_append + attn_decode_split
 * (src/models/transformer.rs:1100-1160; window as the split kernel's,
 * src/kernels.cu:557-559); the merge is cima_hip_attn_reduce or, fused,
 * cima_hip_attn_gguf_gemv with the same window.  Chunks past the position
 * or wholly before the window write nothing. */
int cima_hip_attn_decode(cima_hip_ctx* ctx, const void* qkv, void* k_cache, void* v_cache, float* part, int q_heads,
                         int kv_heads, int dim, int max_seq, int csz, int n_chunks, float theta, float scale,
                         int window, const int* pos_dev);
/* The o projection of merged attention: cima_hip_gguf_gemv (f16, mode 0 or
 * 1, k = q_heads * dim) whose x is merged, inside the GEMV, from the split
 * partials of the first *pos_dev + 1 positions (window > 0: of the chunks
 * from the window's first position on, as k_attn_reduce,
 * src/kernels.cu:619-621): x[h*dim + d] = f16(sum_c e^(m_c - M) acc_c[d] /
 * sum_c e^(m_c - M) l_c).  Replaces attn_reduce + gguf_gemv
 * (src/models/transformer.rs:1161-1238). */
int cima_hip_attn_gguf_gemv(cima_hip_ctx* ctx, int ggml_type, const float* part, int q_heads, int dim, int csz,
                            int n_chunks, int max_seq, int window, const int* pos_dev, const void* w,
                            const void* bias, void* y, int n, int mode);
/* The head GEMV with the greedy argmax folded in: y = W . rmsnorm(x)
 * (norm_w NULL: W . x), f16, and *slot = max(*slot, argmax key of every
 * y[r]) with the key of cima_hip_argmax (no softcap).  *slot must be 0 on
 * entry.  Replaces head_project + argmax_softcap_enqueue
 * (src/models/transformer.rs:1361-1390, src/cuda.rs:2036-2056). */
int cima_hip_gguf_gemv_argmax(cima_hip_ctx* ctx, int ggml_type, const void* x, const void* norm_w, float eps,
                              const void* w, void* y, int n, int k, unsigned long long* slot);
/* Greedy argmax of f16 logits x[n] (softcap cap > 0: cap * tanh(x / cap))
 * into *slot as (orderable f32 bits << 32 | index), ties to the higher
 * index.  *slot must be 0 on entry (cima_hip_argmax_to_ids leaves it 0).
 * CudaCtx::argmax_softcap_enqueue (src/cuda.rs:2036-2056) without its
 * memset, which would not be safe to capture. */
int cima_hip_argmax(cima_hip_ctx* ctx, const void* x, unsigned long long* slot, int n, float cap);
/* ids[0] = index in *slot (ids may be NULL), *slot = 0, and *pos_dev += 1
 * when pos_dev is not NULL: CudaCtx::argmax_to_ids + pos_bump
 * (src/cuda.rs:2058-2073). */
int cima_hip_argmax_to_ids(cima_hip_ctx* ctx, unsigned long long* slot, unsigned int* ids, int* pos_dev);
/* *pos_dev += 1: CudaCtx::pos_bump (src/cuda.rs:2068-2073). */
int cima_hip_pos_bump(cima_hip_ctx* ctx, int* pos_dev);

/* One layer of a Qwen2/Llama-family decoder, weights in GGUF blocks. */
typedef struct cima_decoder_layer {
    const void* attn_norm;  /* f16 [hidden] */
    const void* wqkv;       /* [(q_heads + 2 kv_heads) * head_dim, hidden]: q rows, k rows, v rows */
    const void* bqkv;       /* f16 [(q_heads + 2 kv_heads) * head_dim], or NULL */
    const void* wo;         /* [hidden, q_heads * head_dim] */
    const void* ffn_norm;   /* f16 [hidden] */
    const void* w_gate_up;  /* [2 ffn, hidden]: gate rows then up rows */
    const void* w_down;     /* [hidden, ffn] */
    void* k_cache;          /* f16 [kv_heads, max_seq, head_dim] */
    void* v_cache;          /* f16 [kv_heads, max_seq, head_dim] */
    /* Per-tensor formats, as GGUF files mix them (a Q4_K_M file keeps some
     * v and down projections in Q6_K, 896-wide rows in Q5_0 / Q8_0):
     * 0 = the decoder's ggml_type.  With wk and wv set, wqkv is the q
     * projection alone and k, v are separate matrices (type_q / type_k /
     * type_v); with w_up set, w_gate_up is the gate projection alone
     * (type_gate must equal type_up). */
    const void* wk;         /* [kv_heads * head_dim, hidden], or NULL */
    const void* wv;         /* [kv_heads * head_dim, hidden], or NULL */
    const void* w_up;       /* [ffn, hidden], or NULL */
    int type_q, type_k, type_v, type_o, type_gate, type_up, type_down;
    /* sliding-window attention: > 0 keeps the last `window` positions
     * (the reference's per-layer window, src/models/gemma4/mod.rs:1396-1421);
     * 0 = full causal attention */
    int window;
} cima_decoder_layer;

/* A decoder and its device workspace for cima_hip_decode_step. */
typedef struct cima_decoder {
    int ggml_type;    /* block format of every layer weight */
    int embed_type;   /* block format of the embedding table */
    int head_type;    /* block format of head (ignored when tied) */
    int n_layers, hidden, q_heads, kv_heads, head_dim, ffn, vocab, max_seq;
    int attn_chunk;   /* positions per attention chunk, <= 256 (0 = 256) */
    float rope_theta, rms_eps;
    const void* embed;       /* [vocab, hidden] */
    const void* head;        /* [vocab, hidden], NULL = tied to embed */
    const void* final_norm;  /* f16 [hidden] */
    const cima_decoder_layer* layers;  /* host array of n_layers */
    /* workspace, all device memory */
    void* x;          /* f16 [hidden] residual stream */
    void* qkv;        /* f16 [(q_heads + 2 kv_heads) * head_dim] */
    void* act;        /* f16 [ffn] */
    void* logits;     /* f16 [vocab] */
    float* part;      /* q_heads * ceil(max_seq / attn_chunk) * (head_dim + 2) floats */
    unsigned long long* slot;  /* zero */
    unsigned int* ids;         /* [1]: input token; receives the greedy next token */
    int* pos;                  /* [1]: position of the input token; advanced by one */
} cima_decoder;

/* One greedy batch-1 decode step, all on the context's stream and safe to
 * capture in a HIP graph (positions come from *pos, nothing is allocated):
 * gather ids[0] -> per layer [rmsnorm + q|k|v GEMV + bias, RoPE + KV append
 * + split attention, merge + o GEMV + residual, rmsnorm + gate|up SwiGLU
 * GEMV, down GEMV + residual] -> rmsnorm + head GEMV + argmax -> ids[0],
 * pos += 1.  Replaces
 * enqueue_decode_device (src/models/transformer.rs:1440-1461) and
 * forward_chunk_at's rows == 1 path (:1012-1300): 5 launches per layer
 * where the reference issues about 12 (7 with separate q, k, v matrices). */
int cima_hip_decode_step(cima_hip_ctx* ctx, const cima_decoder* d);

/* ---------------------------------------------------------------------
 * Graph capture of the context's stream (CudaCtx::capture_begin /
 * capture_end / graph_launch, src/cuda.rs:1069-1095): every call between
 * begin and end is recorded instead of run; the instantiated graph replays
 * the whole sequence with one launch.  The stream must be a non-default
 * stream (the context's own, or one set with cima_hip_set_stream).
 * --------------------------------------------------------------------- */
typedef struct cima_hip_graph cima_hip_graph;
int cima_hip_capture_begin(cima_hip_ctx* ctx);
int cima_hip_capture_end(cima_hip_ctx* ctx, cima_hip_graph** out);
int cima_hip_graph_launch(cima_hip_ctx* ctx, cima_hip_graph* graph);
int cima_hip_graph_destroy(cima_hip_graph* graph);

/* ---------------------------------------------------------------------
 * bitsandbytes 4-bit weights (NF4 / FP4), src/quant.rs:18-437: a
 * row-major [n, k] weight resident as n*k/2 packed bytes (element 2j in the
 * HIGH nibble of byte j), absmax[n*k / blocksize] f32 (the double
 * quantisation folded on the host, src/quant.rs:258-330) and the 16-entry
 * f32 codebook qmap.  Element i = qmap[nibble(i)] * absmax[i / blocksize].
 * --------------------------------------------------------------------- */
/* out[i] = f16(qmap[nibble(i)] * absmax[i / blocksize]) for i < n, bit-exact
 * (one fp32 product rounded to nearest even).  Replaces CudaCtx::nf4_dequant
 * (src/cuda.rs:2321-2345, k_nf4_dequant src/kernels.cu:320-329).  absmax /
 * qmap 4-byte, out 2-byte aligned; n % 32 == 0, blocksize % 32 == 0 with
 * 16-byte aligned packed and out take the vector kernel. */
int cima_hip_nf4_dequant(cima_hip_ctx* ctx, const void* packed, const float* absmax, const float* qmap, void* out_f16,
                         long long n, int blocksize);
/* Fused decode GEMV y[n] = W[n, k] . x[k] over the packed weight.  Replaces
 * CudaCtx::nf4_gemv (src/cuda.rs:2347-2381, k_nf4_gemv / k_nf4_gemv_ref
 * src/kernels.cu:331-387).  act_dtype CIMA_DT_F16 (x, y f16, as the
 * reference) or CIMA_DT_F32 (x, y fp32; x rounded to f16 inside).  Codes
 * are used as f16 (relative error <= 2^-11 each), fp32 accumulation.
 * k % 32 == 0, blocksize a power of two >= 32 and 16-byte aligned packed
 * and x take the fast kernels; any other shape a general one. */
int cima_hip_nf4_gemv(cima_hip_ctx* ctx, const void* x, const void* packed, const float* absmax, const float* qmap,
                      void* y, int n, int k, int blocksize, int act_dtype);
/* Tuning of the fast NF4 GEMV (no counterpart in the reference): rows each
 * wave walks together (0 = heuristic, 1, 2 or 4) and the kernel (0 =
 * heuristic, 1 = LDS pair table, 2 = codebook in registers).  The grid
 * width follows cima_hip_set_gemv_grid. */
int cima_hip_set_nf4_tuning(cima_hip_ctx* ctx, int rows, int kernel);
/* Prefill GEMM over the packed weight, Y[m, n] (row stride n) = X[m, k] .
 * W[n, k]^T: WTensor::gemm's Nf4 arm (src/quant.rs:131-162), which runs
 * nf4_dequant into the engine's slab, then gemm_f16.  Here, for every
 * bitsandbytes checkpoint shape (k % 64 == 0, blocksize % 32 == 0, packed
 * 16-byte aligned) the f16-MFMA prefill tiles of cima_hip_gguf_gemm decode
 * W themselves -- each weight bit-exactly f16(code * absmax), X rounded to
 * f16, fp32 accumulation -- and the slab is not touched.  Any other shape
 * (k % 8 == 0) decodes W into the caller's 256-byte aligned slab one row
 * slice at a time (slices starting on absmax block boundaries, as the
 * reference works through its 32 MiB DQ_SCRATCH,
 * src/models/transformer.rs:630-653) and multiplies each slice with this
 * library's f16-weight GEMM into its columns of Y.  x 16-byte aligned;
 * CIMA_E_INVALID if the slab holds no slice. */
int cima_hip_nf4_gemm_slab(cima_hip_ctx* ctx, const void* x, const void* packed, const float* absmax,
                           const float* qmap, void* y, int m, int n, int k, int blocksize, int x_dtype,
                           int y_dtype, void* slab, unsigned long long slab_bytes);

/* Bandwidth reference (no counterpart in the reference): reads nbytes
 * (16-byte aligned src, whole 16-byte words) once with plain streaming
 * loads; *sink is written only in an improbable case.  The HBM read rate a
 * kernel can reach, measured the way the GEMVs are. */
int cima_hip_stream_read(cima_hip_ctx* ctx, const void* src, long long nbytes, unsigned int* sink);
/* The same read in a chosen form, for sweeping the read ceiling (no
 * counterpart in the reference): dest 0 = into registers, `depth` loads of
 * `width` bytes (16: depth 1, 2, 4, 8 or 16; 8: depth 4, 8 or 16) in flight
 * per thread, grid-stride; dest 1 = into LDS through
 * global_load_lds_dwordx4, a ring of `depth` (2, 4, 8, 16) 1 KB copies in
 * flight per wave (width 16; whole 1 KB runs).  256-thread workgroups, at
 * most wgs_per_cu (1..8) per CU. */
int cima_hip_stream_read_cfg(cima_hip_ctx* ctx, const void* src, long long nbytes, unsigned int* sink, int dest,
                             int depth, int width, int wgs_per_cu);

#ifdef __cplusplus
}
#endif

#endif /* CIMA_HIP_H */
