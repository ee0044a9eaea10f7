/*
 * Harness that exposes the reference int8 LM-head routines
 * (runtime/lal_q8_kernel.h, static inline) as exported symbols.  XQ_MAX is the
 * value tools/server/qwen7b_server.c defines before including the header.
 * Compiled twice: with AVX2 (the server build) and without (the scalar path).
 */
#include <stdint.h>
#define XQ_MAX 18944
#include "runtime/lal_q8_kernel.h"

#ifndef REF_SUFFIX
#define REF_SUFFIX avx2
#endif
#define CAT2(a, b) a##_##b
#define CAT(a, b) CAT2(a, b)

float CAT(lal_ref_quantize_x_int8, REF_SUFFIX)(const float *x, int8_t *xq, int n)
{
    return lal_quantize_x_int8(x, xq, n);
}

void CAT(lal_ref_lm_head_int8_range, REF_SUFFIX)(float *logits, const int8_t *xq,
        float sx, const int8_t *w, const float *sw, int v0, int v1, int n)
{
    lal_lm_head_int8_range(logits, xq, sx, w, sw, v0, v1, n);
}

void CAT(lal_ref_lm_head_int8_range_abs_8row, REF_SUFFIX)(float *logits,
        const int8_t *xq, float sx, const int8_t *w, const float *sw,
        int v0, int v1, int n)
{
    static uint8_t ax[XQ_MAX];
    lal_compute_abs_xq(xq, ax, n);
    lal_lm_head_int8_range_abs_8row(logits, xq, ax, sx, w, sw, v0, v1, n);
}

void CAT(lal_ref_quantize_q8_per_row, REF_SUFFIX)(const float *w, int8_t *q,
        float *scale, int in_dim, int out_dim)
{
    lal_quantize_q8_per_row(w, q, scale, in_dim, out_dim);
}
