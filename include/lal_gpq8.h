/*
 * lal_gpq8.h -- GPQ8 weight files and the LM head's load-time preparation on
 * the MI355X (part of liblal_gpu.so).
 *
 * What each entry point replaces in samaidev/lal:
 *   lal_gpq8_open / _find   tools/server/qwen7b_server.c:497-571 (load_gpq8,
 *                           gp_find, get_q8): mmap the file, walk its tensor
 *                           directory, look tensors up by key
 *   lal_gpu_quantize_w_q8   runtime/lal_q8_kernel.h:357-372
 *                           (lal_quantize_q8_per_row), run at start-up by
 *                           qwen7b_server.c:1106-1112 on lm_head.weight
 *   lal_gpu_load_lm_head    qwen7b_server.c:1106-1112 as a whole: F32
 *                           lm_head.weight from the file, quantized on the GPU
 *                           into the packed layout of lal_gpu_lm_head_q8_packed
 *
 * File layout (little-endian; scripts/convert_qwen7b_q8_0.py:14-19):
 *   "GPQ8", int32 n_tensors, then per tensor: int32 key_len, key bytes,
 *   int32 ndim, int32 shape[ndim], uint8 qtype (0 F32, 1 Q8 with per-row
 *   scales, 2 Q4_0, 3 Q8_0), uint64 data_len, data, int32 n_scale,
 *   float scale[n_scale].
 * Unlike the reference loader, every length is checked against the file size;
 * a malformed file is an LAL_GPU_E_INVAL return, not an exit.
 */
#ifndef LAL_GPQ8_H
#define LAL_GPQ8_H

#include <stddef.h>
#include <stdint.h>

#include "lal_gpu_sample.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LAL_GPQ8_F32   0
#define LAL_GPQ8_Q8    1   /* int8 [out][in] + float scale[out] */
#define LAL_GPQ8_Q4_0  2
#define LAL_GPQ8_Q8_0  3   /* 32-element blocks: fp16 scale + 32 int8 */
#define LAL_GPQ8_MAX_DIMS 4

typedef struct lal_gpq8_file lal_gpq8_file;

typedef struct lal_gpq8_tensor {
    const char  *key;        /* NUL-terminated, owned by the file handle */
    int          ndim;
    int          shape[LAL_GPQ8_MAX_DIMS];
    int          qtype;      /* LAL_GPQ8_* */
    uint64_t     data_len;   /* bytes */
    const void  *data;       /* inside the mapping */
    int          n_scale;
    const float *scale;      /* inside the mapping (may be unaligned), or NULL */
} lal_gpq8_tensor;

/* Map `path` read-only and parse its directory. */
int  lal_gpq8_open(const char *path, lal_gpq8_file **out);
void lal_gpq8_close(lal_gpq8_file *f);
int  lal_gpq8_count(const lal_gpq8_file *f);
int  lal_gpq8_tensor_at(const lal_gpq8_file *f, int i, lal_gpq8_tensor *out);
/* LAL_GPU_E_RANGE when no tensor has this key. */
int  lal_gpq8_find(const lal_gpq8_file *f, const char *key, lal_gpq8_tensor *out);

/* Per-row int8 quantization of an F32 weight [vocab][n] in device memory:
 * scale[v] = max|w[v]| / 127 (at least 1e-8), q = lroundf(w * (1/scale))
 * clamped to [-127, 127].  Writes the row-major int8 matrix to d_wq and/or
 * the packed layout (lal_gpu_pack_q8) to d_wpk (either may be NULL, not
 * both) and the scales to d_sw. */
int  lal_gpu_quantize_w_q8(lal_gpu_ctx *ctx, const float *d_w, int vocab, int n, int8_t *d_wq,
                           int8_t *d_wpk, float *d_sw, void *stream);

/* Tensor `key` ([vocab][n], F32 or Q8) of an open file -> the packed int8
 * layout (d_wpk, lal_gpu_q8_packed_bytes(vocab, n) bytes) and per-row scales
 * (d_sw, vocab floats) on the device.  F32 rows are uploaded in chunks and
 * quantized on the GPU; Q8 rows are uploaded as stored.  *vocab / *n receive
 * the shape; with d_wpk == NULL only the shape is returned (ctx may then be
 * NULL).  Synchronous. */
int  lal_gpu_load_lm_head(lal_gpu_ctx *ctx, const lal_gpq8_file *f, const char *key, int8_t *d_wpk,
                          float *d_sw, int *vocab, int *n, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* LAL_GPQ8_H */
