/*
 * lal_oracle.h -- CPU restatement of LAL's token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * sampler in lal_amd/csrc/lal_gpu_sample.hip.  Only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it; the
 * product path never calls it.
 *
 * Every function follows a reference routine (paths relative to the
 * samaidev/lal tree):
 *   lal_oracle_sample_row   runtime/lal_sampling.h:46-125 (variant BASIC),
 *                           tools/server/qwen7b_server.c:219-295 (FILTERED),
 *                           tools/server/qwen_server.c:418-527 (BASIC + F_DRAW_GPT2),
 *                           tools/mini_server.c:267-363 (FILTERED + F_FALLBACK_ZERO
 *                           + F_GREEDY_FILTER, the filter's last token given),
 *                           tools/server/gpt2_server.c:2908-2955 (top-p),
 *                           compiler/lal.py:2220-2242 (ban_last/ban_repeat/
 *                           ban_token on the top-k keep mask)
 *   lal_oracle_uniforms     runtime/lal_sampling.h:116 (one rand() per row)
 *   lal_oracle_quantize_x   runtime/lal_q8_kernel.h:375-442
 *   lal_oracle_lm_head      runtime/lal_q8_kernel.h:463-499
 *   lal_oracle_quantize_w   runtime/lal_q8_kernel.h:357-372
 *   lal_oracle_recent_push  runtime/lal_sampling.h:133-136
 *
 * How each part is pinned (tests/):
 *   top-k / softmax / draw / penalty / filtered variant / plugin bans:
 *       golden vectors written by the reference's own C code
 *       (test_oracle_golden.py) and oracle/_ref called directly;
 *   qwen_server / mini_server flags: against those servers' samplers
 *       compiled in oracle/_ref (test_oracle_pins.py);
 *   logit-space ops (bias, allow bitmask, mask_recent): against the
 *       reference sampler run on the op-applied row (test_oracle_pins.py);
 *   top-p nucleus: the reference has no callable entry point; pinned by its
 *       definition (prefix of the stable descending order that first reaches
 *       top_p, p -> 0, p >= 1, renormalisation, draw end points) in
 *       test_oracle_pins.py;
 *   uniforms, Q8 quantizers, LM head, recent_push: golden vectors.
 *
 * Unlike the reference, every routine is reentrant (per-call scratch, the
 * uniform is passed in), so the batch driver can run rows under OpenMP.
 */
#ifndef LAL_ORACLE_H
#define LAL_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LAL_ORACLE_VARIANT_BASIC    0 /* lal_sampling.h: greedy test before penalty */
#define LAL_ORACLE_VARIANT_FILTERED 1 /* qwen7b_server.c: penalty first, k in [1,V], sum<=0 -> argmax */

#define LAL_ORACLE_F_DRAW_GPT2 0x2u   /* gpt2_server.c:2997-3002, qwen_server.c:518-524: the
                                        draw runs over every id, r == 0 returns token 0 */
#define LAL_ORACLE_F_FALLBACK_ZERO 0x4u  /* mini_server.c:339-347: 0 when no sum reaches r */
#define LAL_ORACLE_F_GREEDY_FILTER 0x8u  /* mini_server.c:284-288: the argmax goes through
                                            the filter as a one-element keep mask */

typedef int (*lal_oracle_decode_fn)(int token_id, char *out_buf, int max_len);
typedef int (*lal_oracle_filter_fn)(int *keep_mask, int n_vocab, int last_token,
                                    const int *recent_tokens, int n_recent,
                                    lal_oracle_decode_fn decode_fn);

typedef struct {
    float temperature;
    int top_k;
    float top_p;
    float rep_penalty;
    int variant;
    unsigned flags;
    int ban_last;       /* lal.py ban_last */
    int ban_repeat;     /* lal.py ban_repeat(n), 0 = off */
    int n_ban_ids;      /* lal.py ban_token(id) list */
    const int *ban_ids;
    int mask_recent;    /* last n history ids -> -inf before top-k */
    /* the filter's last token (mini_server.c:267, `last_tok`) in place of
     * hist[n_hist-1]: has_last = 1 and last_token, or, for the batch driver,
     * last_tokens[B] */
    int has_last;
    int last_token;
    const int *last_tokens;
} lal_oracle_params;

typedef struct {
    float threshold;  /* k-th largest processed logit (with multiplicity) */
    int n_cand;       /* #processed logits >= threshold */
    int n_kept;       /* #tokens in the final sampling set */
    float sum;        /* softmax denominator over the final set */
    int used_uniform; /* 1 when the draw consumed the row's uniform */
    int greedy;       /* 1 when the greedy path returned */
} lal_oracle_info;

/* expf as called by the reference (glibc). */
float lal_oracle_expf(float x);

/*
 * Sample one row.  `row` is modified in place exactly as the reference does
 * (repetition penalty only).  `hist`/`n_hist` are the row's recent ids.
 * `allow` (bit v&31 of word v>>5) and `bias` ([V]) are the logit-space ops
 * applied before selection, in the order penalty -> bias -> allow -> mask_recent.
 * `u` is the row's uniform in [0,1].  The optional candidate arrays receive the
 * ids >= threshold in ascending order (cand_kept[i] = 1 when in the final set,
 * cand_probs[i] = e_i/sum for kept ids, 0 otherwise).
 */
int lal_oracle_sample_row(float *row, int V, const lal_oracle_params *p,
                          const int *hist, int n_hist,
                          const uint32_t *allow, const float *bias, float u,
                          lal_oracle_filter_fn filter, lal_oracle_decode_fn decode,
                          lal_oracle_info *info,
                          int cand_cap, int *cand_ids, float *cand_probs,
                          unsigned char *cand_kept);

/* Batch driver: rows independent, OpenMP over rows (nthreads <= 0: default). */
void lal_oracle_sample_batch(float *logits, int B, int V, int ld,
                             const lal_oracle_params *p,
                             const int *hist, int hist_ld, const int *hist_len,
                             const uint32_t *allow, int allow_ld,
                             const float *bias, const float *uniforms,
                             int *out_token, float *out_threshold,
                             int *out_n_cand, int *out_n_kept, float *out_sum,
                             int cand_ld, int *cand_ids, float *cand_probs,
                             unsigned char *cand_kept, int nthreads);

/* srand(seed), then n x ((float)rand()/(float)RAND_MAX); gpt2 != 0 uses
 * (float)(rand()%1000000)/1000000.0f (gpt2_server.c:2997). */
void lal_oracle_uniforms(unsigned seed, int n, float *out, int gpt2);

/* lal_quantize_x_int8: mode 0 = AVX2 build (RNE on the multiple-of-8 prefix,
 * truncation on the tail), mode 1 = scalar build (truncation). */
float lal_oracle_quantize_x(const float *x, int8_t *xq, int n, int mode);

/* logits[v] = (sx*sw[v]) * (float)dot(xq, W[v]) for v in [v0, v1). */
void lal_oracle_lm_head(float *logits, const int8_t *xq, float sx,
                        const int8_t *W, const float *sw, int v0, int v1,
                        int n, int nthreads);

/* lal_quantize_q8_per_row. */
void lal_oracle_quantize_w(const float *W, int8_t *q, float *scale,
                           int in_dim, int out_dim);

/* gpt2_server.c:2155-2215: the reference min-heap of R over logits[0..V)
 * (pass-1 int8 logits), then each kept id re-scored in fp32 from x[n] and
 * the int8 row wq[v] * ws[v] (eight fused multiply-add lanes over i mod 8,
 * summed in lane order; the tail with fused multiply-adds).  Updates logits
 * in place; ids (R entries, or NULL) receive the kept ids in heap order.
 * Returns the number kept (min(R, V)). */
int lal_oracle_gpt2_rerank(float *logits, const float *x, const int8_t *wq,
                           const float *ws, int V, int n, int R, int *ids);

typedef struct { int tokens[256]; int n; } lal_oracle_recent;
void lal_oracle_recent_push(lal_oracle_recent *rt, int tok);

/* lal_filter_topk plugins as compiler/lal.py emits them for ban_last plus
 * ban_repeat(4) (demos/mini_antirepeat.lal) and ban_repeat(6). */
int lal_oracle_filter_antirepeat4(int *keep_mask, int n_vocab, int last_token,
                                  const int *recent, int n_recent,
                                  lal_oracle_decode_fn decode_fn);
int lal_oracle_filter_norepeat6(int *keep_mask, int n_vocab, int last_token,
                                const int *recent, int n_recent,
                                lal_oracle_decode_fn decode_fn);

/* Hash of glibc expf over all inputs with high half-word in
 * [first_hi, first_hi+nhi): see lal_gpu_expf_check. */
void lal_oracle_expf_checksums(unsigned first_hi, int nhi, uint64_t *out);

/* Exact k-th largest (with multiplicity) by brute-force sort: a pin for the
 * heap selection that does not share its code. */
float lal_oracle_kth_largest_sorted(const float *x, int n, int k);

#ifdef __cplusplus
}
#endif
#endif
