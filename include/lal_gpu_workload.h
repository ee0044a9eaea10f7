/*
 * lal_gpu_workload.h -- synthetic workloads for benchmarks and parity tests.
 *
 * Not part of the sampling path: these kernels fill device buffers with the
 * shapes the sampler is measured on (Gaussian rows with outliers or per-row
 * offsets, Zipf-shaped rows over a per-row permutation, Bernoulli allow masks,
 * uniform int8 weights) so that a 623 MB batch need not be generated on the
 * host.  Values are deterministic for a given seed and launch; parity tests copy
 * them back and run the CPU oracle on the same bytes.
 */
#ifndef LAL_GPU_WORKLOAD_H
#define LAL_GPU_WORKLOAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* x[b][v] = sigma * N(0,1) + offset_b, offset_b ~ U(-offset_range, offset_range);
 * then n_outliers seeded positions per row are set to outlier_value. */
int lal_gpu_synth_gauss(float *d_out, int batch, int vocab, int ld,
                        unsigned long long seed, float sigma, float offset_range,
                        int n_outliers, float outlier_value, void *stream);

/* x[b][v] = -slope * ln(rank_b(v)) + noise * N(0,1), rank_b a per-row
 * permutation of 1..vocab (affine in v modulo vocab, seeded per row). */
int lal_gpu_synth_zipf(float *d_out, int batch, int vocab, int ld,
                       unsigned long long seed, float slope, float noise,
                       void *stream);

/* bits[b][w]: bit j set with probability p_one for token 32w+j < vocab. */
int lal_gpu_synth_bits(uint32_t *d_out, int batch, int vocab, int words_ld,
                       unsigned long long seed, float p_one, void *stream);

/* uniform integers in [lo, hi] as int8 */
int lal_gpu_synth_int8(int8_t *d_out, size_t n, unsigned long long seed,
                       int lo, int hi, void *stream);

/* uniform floats in [lo, hi) */
int lal_gpu_synth_uniform(float *d_out, size_t n, unsigned long long seed,
                          float lo, float hi, void *stream);

/* sigma * N(0,1) */
int lal_gpu_synth_normal(float *d_out, size_t n, unsigned long long seed,
                         float sigma, void *stream);

/* uniform token ids in [0, vocab) */
int lal_gpu_synth_ids(int *d_out, size_t n, unsigned long long seed, int vocab,
                      void *stream);

/* dst <- src, bytes a multiple of 16 and both 16-byte aligned: a plain
 * streaming copy, the yardstick that hardware byte counters are scaled by. */
int lal_gpu_copy(void *d_dst, const void *d_src, size_t bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif
