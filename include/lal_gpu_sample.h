/*
 * lal_gpu_sample.h -- C ABI of the MI355X (gfx950) token sampler.
 *
 * One shared library (liblal_gpu.so, built from lal_amd/csrc/lal_gpu_sample.hip)
 * exports these plain-C entry points.  Pointers named d_* / marked "device"
 * are HIP device pointers; streams are hipStream_t passed as void*.  Calls are
 * asynchronous on the given stream unless stated otherwise and never exit():
 * errors are returned as negative LAL_GPU_E_* codes.
 *
 * What each entry point replaces in samaidev/lal (the reference is CPU-only,
 * header-only C; its interface is source-level):
 *   lal_gpu_sample         runtime/lal_sampling.h:46-125   lal_sample_token
 *                          tools/server/qwen7b_server.c:219-295
 *                                                  lal_sample_token_filtered
 *                          tools/server/gpt2_server.c:2862-3012 (top-p)
 *                          compiler/lal.py:2218-2242 lal_filter_topk bans
 *                          (ban_last / ban_repeat(n) / ban_token(id)) on the
 *                          top-k pool, batched over rows
 *   lal_gpu_sample_finish  tools/server/qwen7b_server.c:268-294, the softmax and
 *                          draw after a lal_filter_topk plugin (keep-mask
 *                          adapter for loaded .lal filters)
 *   lal_gpu_quantize_x     runtime/lal_q8_kernel.h:375-442 lal_quantize_x_int8
 *   lal_gpu_lm_head_q8     runtime/lal_q8_kernel.h:463-543
 *                          lal_lm_head_int8_range[_abs], caller
 *                          tools/server/qwen7b_server.c:829-845
 *   lal_gpu_lm_head_rerank tools/server/gpt2_server.c:2155-2215, the fp32
 *                          re-score of the int8 LM head's top 512
 *   lal_gpu_pack_q8 +      the same LM head over a weight layout made once
 *   lal_gpu_lm_head_q8_packed  at load time (qwen7b_server.c:1106-1112 keeps
 *                          the row-major int8 copy instead)
 *   lal_gpu_uniforms_rand  runtime/lal_sampling.h:116 ((float)rand()/RAND_MAX)
 * The source-compatible drop-in for runtime/lal_sampling.h is
 * include/lal_sampling.h, built on these entry points.
 */
#ifndef LAL_GPU_SAMPLE_H
#define LAL_GPU_SAMPLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LAL_GPU_ABI_VERSION 3

/* Limits.  top_k is capped at 512, the largest heap the reference samplers
 * hold (tools/server/qwen7b_server.c:239); beyond it the reference is
 * undefined behaviour. */
#define LAL_GPU_MAX_K        512
#define LAL_GPU_MAX_HISTORY  512   /* history ids per row (the reference ring holds 256) */
#define LAL_GPU_MAX_BAN_IDS  64    /* ban_token ids per call */

/* Return codes */
#define LAL_GPU_OK        0
#define LAL_GPU_E_INVAL  (-1)  /* null or inconsistent argument */
#define LAL_GPU_E_RANGE  (-2)  /* size above a context or library limit */
#define LAL_GPU_E_HIP    (-3)  /* HIP runtime error (see lal_gpu_last_hip_error) */
#define LAL_GPU_E_NOMEM  (-4)
#define LAL_GPU_E_NODEV  (-5)

/* Sampler variants */
#define LAL_GPU_VARIANT_BASIC    0 /* lal_sample_token: greedy test before the
                                      penalty (lal_sampling.h:51-67) */
#define LAL_GPU_VARIANT_FILTERED 1 /* lal_sample_token_filtered: penalty first,
                                      sum<=0 -> argmax of the kept set without
                                      a draw (qwen7b_server.c:223-286) */

/* Flags */
#define LAL_GPU_F_WRITEBACK  0x1u /* write the penalised value back into
                                     logits[row][t] for every history id t, the
                                     reference's in-place side effect */
#define LAL_GPU_F_DRAW_GPT2  0x2u /* the draw scans every id with cum += e_v
                                     (0 for ids not kept), so r == 0 returns
                                     token 0: gpt2_server.c:2997-3002 and
                                     qwen_server.c:518-524 */
#define LAL_GPU_F_DRAW_ALL_IDS LAL_GPU_F_DRAW_GPT2
#define LAL_GPU_F_FALLBACK_ZERO 0x4u /* when no running sum reaches r (a nan
                                     sum), return 0 instead of vocab-1
                                     (tools/mini_server.c:339-347) */
#define LAL_GPU_F_GREEDY_FILTER 0x8u /* greedy rows go through the lal_filter_topk
                                     bans too, as mini_server.c:284-288 passes
                                     the argmax as a one-element keep mask
                                     (&km): a ban of id 0 makes the token 0
                                     (bans of other ids fall outside that
                                     one-element array and do nothing) */

/* The other reference samplers as parameter sets:
 *   tools/server/qwen_server.c:418-527 sample_next_token
 *       VARIANT_BASIC | F_DRAW_ALL_IDS (no sum <= 0 branch; r == 0 -> id 0)
 *   tools/mini_server.c:267-363 sample_next_token
 *       VARIANT_FILTERED | F_FALLBACK_ZERO | F_GREEDY_FILTER, without
 *       F_WRITEBACK (it penalises a copy of the row), io.last_tokens = the
 *       caller's last token (it is not recent[n-1] once its 256-entry recent
 *       array is full) */

typedef struct lal_gpu_ctx lal_gpu_ctx;

typedef struct lal_gpu_sample_params {
    float temperature;  /* <= 0: greedy (first index of the maximum) */
    int   top_k;        /* <= 0: greedy; clamped to vocab, then <= LAL_GPU_MAX_K */
    float top_p;        /* nucleus over the top-k pool when 0 < top_p < 1 */
    float rep_penalty;  /* applied when > 1: x>0 ? x/p : x*p per occurrence */
    int   variant;      /* LAL_GPU_VARIANT_* */
    unsigned flags;     /* LAL_GPU_F_* */
    /* lal_filter_topk ops on the top-k pool (post-selection, no refill; the
     * pool is restored when they drop every token) */
    int   ban_last;     /* 1: drop history[len-1] */
    int   ban_repeat;   /* n > 0: drop history[max(0,len-n) .. len-1] */
    int   n_ban_ids;    /* ban_token(id) list, device int[n_ban_ids] */
    const int *ban_ids;
    /* logit-space op before selection: the last n history ids become -inf */
    int   mask_recent;
} lal_gpu_sample_params;

typedef struct lal_gpu_sample_io {
    /* inputs (device) */
    float          *logits;      /* [batch][ld] fp32; read-only unless WRITEBACK */
    int             ld;          /* row stride in floats, >= vocab */
    const int      *history;     /* [batch][history_ld] token ids, or NULL */
    int             history_ld;
    const int      *history_len; /* [batch] ids used per row, or NULL: history_ld */
    const uint32_t *allow_bits;  /* [batch][allow_ld] words, token v allowed when
                                    bit (v&31) of word (v>>5) is set; or NULL */
    int             allow_ld;    /* >= ceil(vocab/32) */
    const float    *bias;        /* [vocab] additive logit bias, or NULL */
    const float    *uniforms;    /* [batch] one uniform in [0,1] per row */
    /* outputs (device) */
    int            *out_token;   /* [batch] sampled ids */
    /* optional outputs (device, NULL to skip) */
    float          *out_threshold; /* [batch] k-th largest processed logit */
    int            *out_n_cand;    /* [batch] #processed logits >= threshold */
    int            *out_n_kept;    /* [batch] #tokens in the final set */
    float          *out_sum;       /* [batch] softmax denominator of the final set */
    int             cand_ld;       /* per-row capacity of the candidate arrays */
    int            *cand_ids;      /* [batch][cand_ld] pool ids, ascending */
    float          *cand_probs;    /* [batch][cand_ld] e/sum if kept, else 0 */
    uint8_t        *cand_kept;     /* [batch][cand_ld] 1 if in the final set */
    float          *out_history_vals; /* [batch][history_ld] logits[t] after the
                                         penalty for each history position */
    float          *cand_vals;     /* [batch][cand_ld] processed logit of each pool id */
    /* optional input (device): [batch] the token ban_last drops, in place of
     * history[len-1] (mini_server.c passes its last token separately); NULL:
     * history[len-1] */
    const int      *last_tokens;
} lal_gpu_sample_io;

/* Finish over a pool filtered on the host: the keep-mask half of
 * tools/server/qwen7b_server.c:257-294.  lal_gpu_sample (greedy off, no ban
 * operations, cand_ld >= the pool size) yields the pool: out_n_cand,
 * cand_ids (ascending) and cand_vals.  A lal_filter_topk plugin
 * (compiler/lal.py:2205-2208) then clears entries of a keep mask; keep[i] = 1
 * for pool entry i it left set, 0 for one it cleared.  Ids the plugin set
 * outside the pool may follow the pool entries (any order, *n_cand counting
 * them, cand_vals their processed logits) with keep = 2: like the reference
 * they count as "something kept" and for the argmax, not for the softmax.
 * This call restores the whole pool when nothing is kept, takes the softmax
 * over the kept pool entries in id order and draws with the row's uniform
 * (variant FILTERED: first id of the largest kept value, without a draw, when
 * the sum is <= 0).  A row whose entries exceed cand_ld gets token -1. */
typedef struct lal_gpu_finish_io {
    const int      *n_cand;      /* [batch] */
    int             cand_ld;
    const int      *cand_ids;    /* [batch][cand_ld] */
    const float    *cand_vals;   /* [batch][cand_ld] */
    const uint8_t  *keep;        /* [batch][cand_ld] 0, 1 or 2 (see above) */
    const float    *uniforms;    /* [batch] */
    int            *out_token;   /* [batch] */
    int            *out_n_kept;  /* [batch] or NULL */
    float          *out_sum;     /* [batch] or NULL */
} lal_gpu_finish_io;

/* Context: owns per-device scratch for up to max_batch rows (candidate lists
 * exchanged between the workgroups of one row, 64 KiB per row, and one counter
 * per row).  One context per host thread / stream: calls that overlap on one
 * context race.  Rows may be split into slices, one workgroup each, when the
 * batch is too small to fill the GPU; the environment variable
 * LAL_GPU_SLICES (1..64), read when the context is created, overrides that
 * choice (tuning only; results do not depend on it). */
int  lal_gpu_create(lal_gpu_ctx **out, int device, int max_batch, int max_vocab);
void lal_gpu_destroy(lal_gpu_ctx *ctx);

/* Batched sampler: one token per row.  Rows may hold any float values:
 * -inf, +inf and nan are handled as the reference's comparisons treat them
 * (a nan never enters the pool; a row with nans takes an exact, slower path
 * that replays the reference's heap).  out_token[b] = -1 would report an
 * internal capacity error; the library's bounds exclude it (a returned
 * LAL_GPU_OK never comes with -1), and callers may treat -1 as fatal. */
int  lal_gpu_sample(lal_gpu_ctx *ctx, int batch, int vocab,
                    const lal_gpu_sample_params *params,
                    const lal_gpu_sample_io *io, void *stream);

/* lal_gpu_sample without a context and without allocating: no counterpart in
 * the reference.  For callers that cannot allocate device memory on the
 * sampling path (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, checks and results as
 * lal_gpu_sample, on the current device; it calls no hipMalloc or hipFree.
 * The candidate lists that the workgroups of a sliced row exchange live in a
 * static per-device scratch array of LAL_GPU_NOALLOC_MAX_ROWS rows (about
 * 3.3 MB, held by each GPU the library runs on until the process ends), set up
 * on the first call on each device.  Batches of up to that many rows are
 * sliced as lal_gpu_sample slices them; larger batches run one workgroup per
 * row and use no scratch (results never depend on slicing).  A forced slice
 * count (LAL_GPU_SLICES) with a larger batch is LAL_GPU_E_RANGE.  A call with
 * a bias keeps the bias's nonzero map in the same array, for vocabularies of
 * up to LAL_GPU_NOALLOC_MAX_BIAS_VOCAB ids (larger: LAL_GPU_E_RANGE).  Every call
 * on one GPU shares that GPU's scratch: calls that overlap on one GPU (two
 * streams, two threads) race; calls in one stream order are safe. */
#define LAL_GPU_NOALLOC_MAX_ROWS 64
#define LAL_GPU_NOALLOC_MAX_BIAS_VOCAB (1 << 20)
int  lal_gpu_sample_noalloc(int batch, int vocab, const lal_gpu_sample_params *params,
                            const lal_gpu_sample_io *io, void *stream);

int  lal_gpu_sample_finish(lal_gpu_ctx *ctx, int batch, int vocab,
                           const lal_gpu_sample_params *params,
                           const lal_gpu_finish_io *io, void *stream);

/* Int8 LM head front end (runtime/lal_q8_kernel.h).
 * lal_gpu_quantize_x: x[batch][n] fp32 -> xq[batch][n] int8, sx[batch];
 *   mode 0 = AVX2 build semantics (round-to-nearest-even on the multiple-of-8
 *   prefix, truncation on the tail), mode 1 = scalar build (truncation).
 * lal_gpu_lm_head_q8: logits[b][v] = (sx[b]*sw[v]) * (float)dot(xq[b], W[v])
 *   with exact int32 accumulation; W row-major [vocab][n] int8.  */
int  lal_gpu_quantize_x(lal_gpu_ctx *ctx, const float *d_x, int batch, int n,
                        int mode, int8_t *d_xq, float *d_sx, void *stream);
int  lal_gpu_lm_head_q8(lal_gpu_ctx *ctx, const int8_t *d_xq, const float *d_sx,
                        int batch, int n, const int8_t *d_w, const float *d_sw,
                        int vocab, float *d_logits, int ld, void *stream);

/* Packed weight layout for the matrix-core LM head, made once at load time
 * (the weights are static):  block (T, c), T < ceil(vocab/16), c < ceil(n/64),
 * is 1024 bytes at offset (T * ceil(n/64) + c) * 1024; its byte 16*l + j
 * (l < 64, j < 16) holds W[16T + l%16][64c + 16*(l/16) + j], zero past the
 * matrix.  Each 1 KB block is the B operand of one 16x16x64 int8 MFMA, so a
 * wave streams its 16 vocab rows as one contiguous run.
 * lal_gpu_lm_head_q8_packed computes the same logits as lal_gpu_lm_head_q8
 * (bit for bit) from that layout; it needs n % 16 == 0 and 16-byte aligned
 * d_xq / d_wpk. */
size_t lal_gpu_q8_packed_bytes(int vocab, int n);
int  lal_gpu_pack_q8(lal_gpu_ctx *ctx, const int8_t *d_w, int vocab, int n, int8_t *d_wpk,
                     void *stream);
int  lal_gpu_lm_head_q8_packed(lal_gpu_ctx *ctx, const int8_t *d_xq, const float *d_sx,
                               int batch, int n, const int8_t *d_wpk, const float *d_sw,
                               int vocab, float *d_logits, int ld, void *stream);

/* One decode step's LM head and token choice (tools/server/qwen7b_server.c:
 * 829-848: lal_quantize_x, lal_lm_head_q8 over every vocabulary row, then the
 * sampler): d_x [batch][n] fp32 -> d_xq / d_sx (quantize_x mode 0, also
 * outputs) -> logits over the packed head into d_logits [batch][ld] -> the
 * sampler with params / io (io->logits and io->ld are ignored: the step's
 * logits are used).  Results are bit for bit those of lal_gpu_quantize_x +
 * lal_gpu_lm_head_q8_packed + lal_gpu_sample.  For up to LAL_GPU_LIST_ROWS
 * rows (default 16, at most 16) without a bias or allow mask the head keeps,
 * per row, the logits at or above a bound taken from a fixed sample of its
 * tiles (with LAL_GPU_HEAD_QX=1 it also quantizes up to 4 rows itself), and the
 * sampler reads that list instead of the row; a row whose list cannot be
 * shown to hold its top-k pool (fewer than k values at or above the bound, a
 * nan logit, a full list) is read whole, as lal_gpu_sample reads it.
 * LAL_GPU_LIST_ROWS, LAL_GPU_HEAD_QX and LAL_GPU_LIST_KS (the bound's rank,
 * for tests) are read when the context is created.
 * Needs n % 16 == 0, 16-byte aligned d_xq / d_wpk, batch <= max_batch and
 * vocab <= max_vocab of the context. */
int  lal_gpu_lm_head_sample(lal_gpu_ctx *ctx, const float *d_x, int batch, int n,
                            int8_t *d_xq, float *d_sx, const int8_t *d_wpk,
                            const float *d_sw, int vocab, float *d_logits, int ld,
                            const lal_gpu_sample_params *params,
                            const lal_gpu_sample_io *io, void *stream);

/* GPT-2 int8 LM head, pass 2 (tools/server/gpt2_server.c:2155-2215): d_logits
 * holds pass 1 (lal_gpu_lm_head_q8 over wte rows quantized by
 * lal_gpu_quantize_x mode 1, as gpt2_server.c:3752-3761 does at load).  The
 * rerank_n (<= 512; the reference uses 512) largest logits of each row -- the
 * set the reference's min-heap keeps, ties at the boundary included -- are
 * re-scored in fp32 from the hidden state d_x [batch][n] (n <= 8192):
 * w = (float)wq[v][i] * ws[v], eight fused multiply-add lanes over i mod 8
 * summed in lane order, then the tail (the AVX2 build's order), written in
 * place; every other logit keeps its int8 value. */
int  lal_gpu_lm_head_rerank(lal_gpu_ctx *ctx, const float *d_x, int batch, int n,
                            const int8_t *d_wq, const float *d_ws, int vocab, int rerank_n,
                            float *d_logits, int ld, void *stream);

/* Host helper: srand(seed) then n draws of (float)rand()/(float)RAND_MAX
 * (gpt2 != 0: (float)(rand()%1000000)/1000000.0f), the reference's RNG
 * stream, written to host memory. */
void lal_gpu_uniforms_rand(unsigned seed, int n, float *out, int gpt2);

/* Device/stream plumbing so C and ctypes callers need no other HIP binding. */
int  lal_gpu_device_count(int *count);
int  lal_gpu_set_device(int device);
int  lal_gpu_malloc(void **d_ptr, size_t bytes);
int  lal_gpu_free(void *d_ptr);
int  lal_gpu_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes, void *stream);
int  lal_gpu_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes, void *stream);
int  lal_gpu_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes, void *stream);
int  lal_gpu_memset(void *d_dst, int value, size_t bytes, void *stream);
int  lal_gpu_stream_create(void **stream);
int  lal_gpu_stream_destroy(void *stream);
int  lal_gpu_stream_sync(void *stream);
int  lal_gpu_device_sync(void);
int  lal_gpu_event_create(void **event);
int  lal_gpu_event_destroy(void *event);
int  lal_gpu_event_record(void *event, void *stream);
int  lal_gpu_event_elapsed_ms(float *ms, void *start, void *stop);
int  lal_gpu_last_hip_error(void);
const char *lal_gpu_strerror(int code);
int  lal_gpu_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* LAL_GPU_SAMPLE_H */
