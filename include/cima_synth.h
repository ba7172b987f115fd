/*
 * cima_synth.h -- seeded synthetic inputs for the GGUF GEMV benchmarks and
 * tests (host only, no GPU).
 *
 * No counterpart in the reference: the reference only decodes GGUF blocks
 * (src/quant.rs:571-896) and has no quantiser.  These quantisers produce
 * valid blocks in the reference's layouts from seeded fp32 weights; parity
 * does not depend on how they choose scales, because the GPU kernels and
 * the CPU oracle decode the same packed bytes.
 */
#ifndef CIMA_SYNTH_H
#define CIMA_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[i] ~ N(0, stddev^2) for i in [0, count): counter-based splitmix64 +
 * Box-Muller, so the values depend only on (seed, i), not on `threads`. */
void cima_synth_normal(uint64_t seed, float stddev, float* out, size_t count, int threads);

/* Quantise `rows` rows of k fp32 values into packed GGUF blocks
 * (rows * storage_bytes(type, k) bytes).  Returns 0, or -1 for an
 * unsupported type or a k that is not a block multiple.
 *   Q8_0: d = f16(amax/127), q = round(x/d) clamped to +-127
 *   Q4_0: d = f16(x_absmax_signed / -8), q = clamp(round(x/d) + 8, 0, 15)
 *   Q4_K: per 32-element sub-block min/max fit, 6-bit scales and mins
 *   Q6_K: per 16-element sub-block absmax fit, int8 scales, q in [-32, 31] */
int cima_synth_quantize(int ggml_type, const float* src, size_t rows, size_t k, uint8_t* dst, int threads);

/* Seeded N(0, stddev^2) weights of rows x k, quantised straight into dst
 * without materialising the fp32 matrix (row r uses counter range
 * [r*k, (r+1)*k) of the seed's stream, so the result equals
 * cima_synth_normal followed by cima_synth_quantize). */
int cima_synth_weights(int ggml_type, uint64_t seed, float stddev, size_t rows, size_t k, uint8_t* dst,
                       int threads);

#ifdef __cplusplus
}
#endif

#endif /* CIMA_SYNTH_H */
