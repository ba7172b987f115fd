/*
 * cima_hip.h -- C ABI of the MI355X (gfx950) GGUF dequant-GEMV library.
 *
 * This is the drop-in boundary for the reference engine's GGUF hot path:
 * each entry point replaces one method of the reference's CudaCtx (Rust,
 * src/cuda.rs), with the same argument order and meaning.  Pointers are
 * device pointers (hipMalloc'd or any HIP-visible device memory), sizes are
 * element or row counts, and every call is asynchronous on the context's
 * stream.  No call allocates device memory, so all are safe inside HIP
 * graph capture once the context exists.
 *
 * Return value: 0 on success; a positive hipError_t when the HIP runtime
 * failed; a negative CIMA_E_* code when the arguments were rejected before
 * anything was launched.  cima_hip_last_error() gives the message of the
 * last failure on the calling thread.
 *
 * Formats are ggml tensor type ids (src/formats.rs:90-117): 8 = Q8_0,
 * 2 = Q4_0, 12 = Q4_K, 14 = Q6_K.
 */
#ifndef CIMA_HIP_H
#define CIMA_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids */
#define CIMA_GGML_Q4_0 2
#define CIMA_GGML_Q8_0 8
#define CIMA_GGML_Q4_K 12
#define CIMA_GGML_Q6_K 14

/* activation / output element types */
#define CIMA_DT_F32 0
#define CIMA_DT_F16 1
#define CIMA_DT_BF16 2

/* argument errors (negative; hipError_t values are positive) */
#define CIMA_E_INVALID -1     /* bad pointer, shape, mode or alignment */
#define CIMA_E_FORMAT -2      /* not a supported GGUF block format */
#define CIMA_E_NO_KERNEL -3   /* code object lacks the kernel */
#define CIMA_E_NOT_INIT -4    /* null or destroyed context */

typedef struct cima_hip_ctx cima_hip_ctx;

/* Context creation: replaces CudaCtx::init (src/cuda.rs:691-908) -- device
 * selection, one non-blocking stream, then loading the prebuilt gfx950 code
 * objects (cima_gemv.hsaco, cima_gemm.hsaco, cima_dequant.hsaco) with
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

/* Launch stream.  NULL restores the context's own non-blocking stream
 * (src/cuda.rs:740-744).  The caller keeps ownership of a stream it sets. */
int cima_hip_set_stream(cima_hip_ctx* ctx, void* hip_stream);
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
 * values at cima_hip_init. */
int cima_hip_set_gemv_tuning(cima_hip_ctx* ctx, int rows, int lanes_per_row);

/* GEMV grid tuning (no counterpart in the reference): the persistent grid
 * holds at most this many workgroups per CU (0 = the default of 2, or fewer
 * if fewer fit; environment variable CIMA_GEMV_WGS at init). */
int cima_hip_set_gemv_grid(cima_hip_ctx* ctx, int wgs_per_cu);

/* Prefill GEMM tuning (no counterpart in the reference): token-tile width
 * (16, 64 or 128) for later gguf_gemm calls; 0 = the smallest built width
 * covering m (128 beyond). */
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
 * Requires k % 32 == 0 (Q8_0, Q4_0) or k % 256 == 0 (Q4_K, Q6_K), x and y
 * 16-byte aligned, W 16-byte aligned for Q4_K and 2-byte aligned otherwise.
 * Unlike the reference, x is not quantised to q8_1: the dot runs in fp32. */
int cima_hip_gguf_gemv(cima_hip_ctx* ctx, int ggml_type, const void* x, const void* w,
                       const void* bias, void* y, int n, int k, int mode, int act_dtype);

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
 * (src/cuda.rs:2468-2570), with no slab -- W is dequantised tile by tile
 * into LDS, bit-exact f16, and multiplied with f16 MFMA, fp32 accumulate.
 * x_dtype: CIMA_DT_F32, CIMA_DT_F16 or CIMA_DT_BF16 (converted to f16;
 * exact for |x| >= 2^-14); y_dtype: CIMA_DT_F32 or CIMA_DT_F16.
 * Requires k % 64 == 0 (and k % 256 for K-quants), x 8-byte aligned. */
int cima_hip_gguf_gemm(cima_hip_ctx* ctx, int ggml_type, const void* x, const void* w, void* y,
                       int m, int n, int k, int ldy, int x_dtype, int y_dtype);

/* Dequantise nblocks consecutive blocks to f16, bit-exact with the host
 * decoders: replaces CudaCtx::gguf_dequant (src/cuda.rs:2285-2320). */
int cima_hip_gguf_dequant(cima_hip_ctx* ctx, int ggml_type, const void* src, void* out_f16,
                          long long nblocks);

/* Embedding gather from a packed table: out[i, :] = dequant(table[ids[i]])
 * as f16; replaces CudaCtx::gguf_gather (src/cuda.rs:2226-2283).
 * ids are u32 row indices; they are not range-checked on the device. */
int cima_hip_gguf_gather(cima_hip_ctx* ctx, int ggml_type, const void* table,
                         const unsigned int* ids, void* out_f16, int n, int hidden);

#ifdef __cplusplus
}
#endif

#endif /* CIMA_HIP_H */
