#ifndef LAL_SAMPLING_H
#define LAL_SAMPLING_H
/*
 * lal_sampling.h -- source-compatible replacement for runtime/lal_sampling.h
 * that samples on an MI355X through liblal_gpu.so (include/lal_gpu_sample.h).
 *
 * Same names, signatures and side effects as the reference header
 * (runtime/lal_sampling.h:26-136), so a LAL server builds against it unchanged:
 *
 *   lal_sampling_init()                       runtime/lal_sampling.h:30-32
 *   lal_sample_token(logits, V, T, k, p,      runtime/lal_sampling.h:46-125
 *                    recent, n_recent)
 *   LalRecentTokens / lal_recent_push         runtime/lal_sampling.h:128-136
 *   lal_g_temperature / lal_g_top_k /         runtime/lal_sampling.h:26-28
 *   lal_g_rep_penalty
 *   lal_sample_token_top_p(logits, n, T, k,   docs/MINIMAL.md:116 (proposed);
 *                          top_p)             nucleus of tools/server/gpt2_server.c:2908-2955
 *   lal_sample_token_filtered(...)            tools/server/qwen7b_server.c:219-295,
 *                                             only with LAL_SAMPLING_FILTERED defined
 *   lal_sampling_set_filter_plugin(fn, dec)   qwen7b_server.c:160-215, 257-270: a
 *                                             loaded lal_filter_topk plugin
 *
 * Behaviour kept from the reference:
 *   - logits is modified in place by the repetition penalty, once per
 *     occurrence of an id in recent[] (the penalised values are computed on
 *     the GPU and written back into the caller's array);
 *   - exactly one rand() is consumed per non-greedy call, as
 *     (float)rand()/(float)RAND_MAX; greedy calls consume none;
 *     lal_sample_token_filtered consumes none when its softmax sum is <= 0;
 *   - no error codes: the token id is always returned.
 * Differences: a GPU error or a size beyond the library's limits
 * (top_k > LAL_GPU_MAX_K, n_recent > LAL_GPU_MAX_HISTORY) prints a message
 * and aborts instead of sampling on the CPU.  lal_sample_token accepts
 * 64 < top_k <= 512, where the reference's 64-slot heap overflows.
 *
 * Link with -llal_gpu.  Like the reference, the functions keep static state
 * (one device context, one stream, staging buffers) and are not reentrant.
 * The GPU is chosen by the environment variable LAL_GPU_DEVICE (default 0).
 */

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "lal_gpu_sample.h"

/* The reference declares the temperature global as int (lal_sampling.h:26);
 * kept as is, so code that reads it sees the same value (0). */
static int   lal_g_temperature = 0.8f;
static int   lal_g_top_k = 40;
static float lal_g_rep_penalty = 1.1f;

static void lal_sampling_init(void) { srand((unsigned)time(NULL)); }

typedef struct {
    int tokens[256];
    int n;
} LalRecentTokens;

/* Append; once 256 ids are held, drop the oldest. */
static void lal_recent_push(LalRecentTokens *rt, int tok)
{
    if (rt->n < 256) {
        rt->tokens[rt->n++] = tok;
        return;
    }
    memmove(rt->tokens, rt->tokens + 1, 255 * sizeof(int));
    rt->tokens[255] = tok;
}

/* ---- device state shared by the entry points below -------------------- */
/* The plugin ABI of compiler/lal.py:2205-2208 (loaded .lal filters). */
typedef int (*lal_token_decode_fn)(int token_id, char *out_buf, int max_len);
typedef int (*lal_filter_topk_fn)(int *keep_mask, int n_vocab, int last_token,
                                  const int *recent_tokens, int n_recent,
                                  lal_token_decode_fn decode_fn);

typedef struct {
    lal_gpu_ctx *ctx;
    void *stream;
    int vocab_cap;
    float *d_row;
    int *d_hist, *d_tok, *d_ban;
    float *d_u, *d_sum, *d_hvals;
    int ban_last, ban_repeat, n_ban;
    int h_ban[LAL_GPU_MAX_BAN_IDS];  /* host copy, uploaded again when the
                                        device buffers are re-created */
    /* keep-mask adapter for a loaded lal_filter_topk plugin */
    lal_filter_topk_fn plugin;
    lal_token_decode_fn decode;
    int *d_cids, *d_ncand;
    float *d_cvals;
    unsigned char *d_keep;
    int *h_mask, *h_cids;
    float *h_xvals;
    unsigned char *h_keep;
} lal_sampling_gpu_state;

static lal_sampling_gpu_state lal__gs;

static void lal__die(const char *what, int rc)
{
    fprintf(stderr, "lal_sampling (GPU): %s failed: %s (HIP error %d)\n", what,
            lal_gpu_strerror(rc), lal_gpu_last_hip_error());
    abort();
}

#define LAL__CHECK(call, what)          \
    do {                                \
        int lal__rc = (call);           \
        if (lal__rc != LAL_GPU_OK)      \
            lal__die(what, lal__rc);    \
    } while (0)

static void lal__release(void)
{
    lal_sampling_gpu_state *g = &lal__gs;
    if (!g->ctx) return;
    lal_gpu_free(g->d_row);
    lal_gpu_free(g->d_hist);
    lal_gpu_free(g->d_tok);
    lal_gpu_free(g->d_ban);
    lal_gpu_free(g->d_u);
    lal_gpu_free(g->d_sum);
    lal_gpu_free(g->d_hvals);
    lal_gpu_free(g->d_cids);
    lal_gpu_free(g->d_ncand);
    lal_gpu_free(g->d_cvals);
    lal_gpu_free(g->d_keep);
    free(g->h_mask);
    free(g->h_cids);
    free(g->h_keep);
    free(g->h_xvals);
    g->h_mask = g->h_cids = NULL;
    g->h_keep = NULL;
    g->h_xvals = NULL;
    lal_gpu_destroy(g->ctx);
    g->ctx = NULL;
}

/* Create the context and staging buffers on first use, or grow them when a
 * larger vocabulary arrives. */
static void lal__ensure(int vocab)
{
    lal_sampling_gpu_state *g = &lal__gs;
    if (g->ctx && vocab <= g->vocab_cap) return;
    if (!g->stream) {
        const char *dev = getenv("LAL_GPU_DEVICE");
        LAL__CHECK(lal_gpu_set_device(dev ? atoi(dev) : 0), "lal_gpu_set_device");
        LAL__CHECK(lal_gpu_stream_create(&g->stream), "lal_gpu_stream_create");
    }
    lal__release();
    const char *dev = getenv("LAL_GPU_DEVICE");
    LAL__CHECK(lal_gpu_create(&g->ctx, dev ? atoi(dev) : 0, 1, vocab), "lal_gpu_create");
    g->vocab_cap = vocab;
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_row, (size_t)vocab * sizeof(float)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_hist, LAL_GPU_MAX_HISTORY * sizeof(int)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_tok, sizeof(int)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_ban, LAL_GPU_MAX_BAN_IDS * sizeof(int)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_u, sizeof(float)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_sum, sizeof(float)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_hvals, LAL_GPU_MAX_HISTORY * sizeof(float)),
               "lal_gpu_malloc");
    /* the pool can be the whole row (ties), so the adapter's buffers hold V */
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_cids, (size_t)vocab * sizeof(int)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_ncand, sizeof(int)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_cvals, (size_t)vocab * sizeof(float)), "lal_gpu_malloc");
    LAL__CHECK(lal_gpu_malloc((void **)&g->d_keep, (size_t)vocab), "lal_gpu_malloc");
    if (g->n_ban > 0) {
        LAL__CHECK(lal_gpu_memcpy_h2d(g->d_ban, g->h_ban, (size_t)g->n_ban * sizeof(int), g->stream),
                   "upload ban ids");
        LAL__CHECK(lal_gpu_stream_sync(g->stream), "stream sync");
    }
    g->h_mask = (int *)malloc((size_t)vocab * sizeof(int));
    g->h_cids = (int *)malloc((size_t)vocab * sizeof(int));
    g->h_keep = (unsigned char *)malloc((size_t)vocab);
    g->h_xvals = (float *)malloc((size_t)vocab * sizeof(float));
    if (!g->h_mask || !g->h_cids || !g->h_keep || !g->h_xvals)
        lal__die("host allocation", LAL_GPU_E_NOMEM);
}

/* One row through lal_gpu_sample.  Uploads the row and history, runs the
 * kernel with uniform u, and returns the token and softmax sum; the
 * penalised history values land in hvals[0..n_hist). */
static int lal__run_io(const float *logits, int vocab, const lal_gpu_sample_params *p,
                       const int *recent, int n_recent, float u, float *sum, float *hvals,
                       int with_pool)
{
    lal_sampling_gpu_state *g = &lal__gs;
    lal_gpu_sample_io io;
    memset(&io, 0, sizeof io);
    if (with_pool) {
        /* the pool (ids ascending, processed logits, final kept flags) for a
         * later lal_gpu_sample_finish; it can hold the whole row (ties) */
        io.out_n_cand = g->d_ncand;
        io.cand_ld = vocab;
        io.cand_ids = g->d_cids;
        io.cand_vals = g->d_cvals;
        io.cand_kept = g->d_keep;
    }
    LAL__CHECK(lal_gpu_memcpy_h2d(g->d_row, logits, (size_t)vocab * sizeof(float), g->stream),
               "upload logits");
    if (n_recent > 0) {
        LAL__CHECK(lal_gpu_memcpy_h2d(g->d_hist, recent, (size_t)n_recent * sizeof(int), g->stream),
                   "upload history");
        io.history = g->d_hist;
        io.history_ld = n_recent;
        io.out_history_vals = g->d_hvals;
    }
    LAL__CHECK(lal_gpu_memcpy_h2d(g->d_u, &u, sizeof u, g->stream), "upload uniform");
    io.logits = g->d_row;
    io.ld = vocab;
    io.uniforms = g->d_u;
    io.out_token = g->d_tok;
    io.out_sum = g->d_sum;
    LAL__CHECK(lal_gpu_sample(g->ctx, 1, vocab, p, &io, g->stream), "lal_gpu_sample");
    int tok = 0;
    LAL__CHECK(lal_gpu_memcpy_d2h(&tok, g->d_tok, sizeof tok, g->stream), "download token");
    LAL__CHECK(lal_gpu_memcpy_d2h(sum, g->d_sum, sizeof *sum, g->stream), "download sum");
    if (n_recent > 0 && hvals)
        LAL__CHECK(lal_gpu_memcpy_d2h(hvals, g->d_hvals, (size_t)n_recent * sizeof(float), g->stream),
                   "download history values");
    LAL__CHECK(lal_gpu_stream_sync(g->stream), "stream sync");
    if (tok < 0) lal__die("lal_gpu_sample (internal capacity error, token -1)", LAL_GPU_E_RANGE);
    return tok;
}

static int lal__run(const float *logits, int vocab, const lal_gpu_sample_params *p,
                    const int *recent, int n_recent, float u, float *sum, float *hvals)
{
    return lal__run_io(logits, vocab, p, recent, n_recent, u, sum, hvals, 0);
}

/* The draw over the pool the last lal__run_io(with_pool) left on the device,
 * with uniform u (the softmax and draw of qwen7b_server.c:275-294 over the
 * kept flags the sampler computed): a pool-sized launch instead of a second
 * upload and pass over the row. */
static int lal__draw_pool(int vocab, const lal_gpu_sample_params *p, float u)
{
    lal_sampling_gpu_state *g = &lal__gs;
    lal_gpu_finish_io fio;
    memset(&fio, 0, sizeof fio);
    LAL__CHECK(lal_gpu_memcpy_h2d(g->d_u, &u, sizeof u, g->stream), "upload uniform");
    fio.n_cand = g->d_ncand;
    fio.cand_ld = vocab;
    fio.cand_ids = g->d_cids;
    fio.cand_vals = g->d_cvals;
    fio.keep = g->d_keep;
    fio.uniforms = g->d_u;
    fio.out_token = g->d_tok;
    LAL__CHECK(lal_gpu_sample_finish(g->ctx, 1, vocab, p, &fio, g->stream), "lal_gpu_sample_finish");
    int tok = 0;
    LAL__CHECK(lal_gpu_memcpy_d2h(&tok, g->d_tok, sizeof tok, g->stream), "download token");
    if (tok < 0) lal__die("lal_gpu_sample_finish (pool above its buffer)", LAL_GPU_E_RANGE);
    return tok;
}

/* Reproduce the in-place penalty on the caller's row. */
static void lal__write_back(float *logits, int vocab, const int *recent, int n_recent,
                            const float *hvals)
{
    for (int i = 0; i < n_recent; i++) {
        const int t = recent[i];
        if (t >= 0 && t < vocab) logits[t] = hvals[i];
    }
}

static int lal__prepare(int vocab, int top_k, const int *recent, int *n_recent)
{
    if (!recent || *n_recent < 0) *n_recent = 0;
    if (*n_recent > LAL_GPU_MAX_HISTORY) lal__die("history longer than LAL_GPU_MAX_HISTORY", LAL_GPU_E_RANGE);
    if ((top_k < vocab ? top_k : vocab) > LAL_GPU_MAX_K)
        lal__die("top_k above LAL_GPU_MAX_K", LAL_GPU_E_RANGE);
    if (vocab <= 0) return 0;
    lal__ensure(vocab);
    return 1;
}

static float lal__uniform(void) { return (float)rand() / (float)RAND_MAX; }

/* Filtered sampler with a loaded lal_filter_topk plugin
 * (tools/server/qwen7b_server.c:257-294): the GPU selects the pool, the host
 * builds the keep mask over the whole vocabulary as the server does and calls
 * the plugin, the GPU finishes (softmax over the kept pool entries, draw).
 * Plugins from compiler/lal.py only clear entries; ids a plugin sets outside
 * the pool go to the finish call as keep = 2 entries with their penalised
 * logits, since the reference lets them block the restore of an emptied pool
 * and win its sum <= 0 argmax. */
static int lal__run_plugin(const float *logits, int vocab, lal_gpu_sample_params *p,
                           const int *recent, int n_recent, float *hvals)
{
    lal_sampling_gpu_state *g = &lal__gs;
    lal_gpu_sample_io io;
    memset(&io, 0, sizeof io);
    p->ban_last = p->ban_repeat = p->n_ban_ids = 0;
    p->ban_ids = NULL;
    LAL__CHECK(lal_gpu_memcpy_h2d(g->d_row, logits, (size_t)vocab * sizeof(float), g->stream),
               "upload logits");
    if (n_recent > 0) {
        LAL__CHECK(lal_gpu_memcpy_h2d(g->d_hist, recent, (size_t)n_recent * sizeof(int), g->stream),
                   "upload history");
        io.history = g->d_hist;
        io.history_ld = n_recent;
        io.out_history_vals = g->d_hvals;
    }
    const float zero = 0.0f;
    LAL__CHECK(lal_gpu_memcpy_h2d(g->d_u, &zero, sizeof zero, g->stream), "upload uniform");
    io.logits = g->d_row;
    io.ld = vocab;
    io.uniforms = g->d_u;
    io.out_token = g->d_tok;
    io.out_n_cand = g->d_ncand;
    io.cand_ld = vocab;
    io.cand_ids = g->d_cids;
    io.cand_vals = g->d_cvals;
    LAL__CHECK(lal_gpu_sample(g->ctx, 1, vocab, p, &io, g->stream), "lal_gpu_sample");
    int nc = 0;
    LAL__CHECK(lal_gpu_memcpy_d2h(&nc, g->d_ncand, sizeof nc, g->stream), "download pool size");
    if (n_recent > 0)
        LAL__CHECK(lal_gpu_memcpy_d2h(hvals, g->d_hvals, (size_t)n_recent * sizeof(float), g->stream),
                   "download history values");
    LAL__CHECK(lal_gpu_stream_sync(g->stream), "stream sync");
    if (nc < 1 || nc > vocab) lal__die("pool size", LAL_GPU_E_RANGE);
    LAL__CHECK(lal_gpu_memcpy_d2h(g->h_cids, g->d_cids, (size_t)nc * sizeof(int), g->stream),
               "download pool ids");
    LAL__CHECK(lal_gpu_stream_sync(g->stream), "stream sync");
    /* keep_mask[v] = (v in the pool), then the plugin */
    memset(g->h_mask, 0, (size_t)vocab * sizeof(int));
    for (int i = 0; i < nc; i++) g->h_mask[g->h_cids[i]] = 1;
    const int last = (n_recent > 0) ? recent[n_recent - 1] : -1;
    (void)g->plugin(g->h_mask, vocab, last, recent, n_recent, g->decode);
    for (int i = 0; i < nc; i++) {
        int *m = &g->h_mask[g->h_cids[i]];
        g->h_keep[i] = *m ? 1 : 0;
        *m = 0;
    }
    int nt = nc;  /* what is still set lies outside the pool */
    for (int v = 0; v < vocab; v++) {
        if (!g->h_mask[v]) continue;
        float x = logits[v];
        for (int j = 0; j < n_recent; j++)
            if (recent[j] == v) x = hvals[j];
        g->h_cids[nt] = v;
        g->h_xvals[nt - nc] = x;
        g->h_keep[nt] = 2;
        nt++;
    }
    LAL__CHECK(lal_gpu_memcpy_h2d(g->d_keep, g->h_keep, (size_t)nt, g->stream), "upload keep flags");
    if (nt > nc) {
        const size_t ne = (size_t)(nt - nc);
        LAL__CHECK(lal_gpu_memcpy_h2d(g->d_cids + nc, g->h_cids + nc, ne * sizeof(int), g->stream),
                   "upload extra ids");
        LAL__CHECK(lal_gpu_memcpy_h2d(g->d_cvals + nc, g->h_xvals, ne * sizeof(float), g->stream),
                   "upload extra values");
        LAL__CHECK(lal_gpu_memcpy_h2d(g->d_ncand, &nt, sizeof nt, g->stream), "upload entry count");
    }
    lal_gpu_finish_io fio;
    memset(&fio, 0, sizeof fio);
    fio.n_cand = g->d_ncand;
    fio.cand_ld = vocab;
    fio.cand_ids = g->d_cids;
    fio.cand_vals = g->d_cvals;
    fio.keep = g->d_keep;
    fio.uniforms = g->d_u;
    fio.out_token = g->d_tok;
    fio.out_sum = g->d_sum;
    /* as in lal__sample_common: u = 0 first, one rand() only if the sum is > 0 */
    int tok = 0;
    float sum = 0.0f;
    LAL__CHECK(lal_gpu_sample_finish(g->ctx, 1, vocab, p, &fio, g->stream), "lal_gpu_sample_finish");
    LAL__CHECK(lal_gpu_memcpy_d2h(&tok, g->d_tok, sizeof tok, g->stream), "download token");
    LAL__CHECK(lal_gpu_memcpy_d2h(&sum, g->d_sum, sizeof sum, g->stream), "download sum");
    LAL__CHECK(lal_gpu_stream_sync(g->stream), "stream sync");
    if (sum > 0.0f) {
        const float u = lal__uniform();
        if (u != 0.0f) {
            LAL__CHECK(lal_gpu_memcpy_h2d(g->d_u, &u, sizeof u, g->stream), "upload uniform");
            LAL__CHECK(lal_gpu_sample_finish(g->ctx, 1, vocab, p, &fio, g->stream), "lal_gpu_sample_finish");
            LAL__CHECK(lal_gpu_memcpy_d2h(&tok, g->d_tok, sizeof tok, g->stream), "download token");
            LAL__CHECK(lal_gpu_stream_sync(g->stream), "stream sync");
        }
    }
    return tok;
}

static int lal__sample_common(float *logits, int vocab_size, float temperature, int top_k,
                              float top_p, float rep_penalty, const int *recent, int n_recent,
                              int variant)
{
    if (!lal__prepare(vocab_size, top_k, recent, &n_recent)) return 0;
    lal_gpu_sample_params p;
    memset(&p, 0, sizeof p);
    p.temperature = temperature;
    p.top_k = top_k;
    p.top_p = top_p;
    p.rep_penalty = rep_penalty;
    p.variant = variant;
    const int greedy = (temperature <= 0.0f || top_k <= 0);
    if (variant == LAL_GPU_VARIANT_FILTERED) {
        lal_sampling_gpu_state *g = &lal__gs;
        p.ban_last = g->ban_last;
        p.ban_repeat = g->ban_repeat;
        p.n_ban_ids = g->n_ban;
        p.ban_ids = g->n_ban ? g->d_ban : NULL;
    }
    float hv[LAL_GPU_MAX_HISTORY];
    float sum = 0.0f;
    int tok;
    if (greedy) {
        tok = lal__run(logits, vocab_size, &p, recent, n_recent, 0.0f, &sum, hv);
    } else if (variant != LAL_GPU_VARIANT_FILTERED) {
        tok = lal__run(logits, vocab_size, &p, recent, n_recent, lal__uniform(), &sum, hv);
    } else if (lal__gs.plugin) {
        tok = lal__run_plugin(logits, vocab_size, &p, recent, n_recent, hv);
    } else {
        /* The filtered sampler draws only when its softmax sum is positive.
         * Run with u = 0 first, keeping the pool on the device: when sum <= 0
         * that token (the argmax of the kept set) is final and no rand() is
         * consumed; when the drawn u is 0 it is final as well; otherwise the
         * draw with u runs over the pool alone. */
        tok = lal__run_io(logits, vocab_size, &p, recent, n_recent, 0.0f, &sum, hv, 1);
        if (sum > 0.0f) {
            const float u = lal__uniform();
            if (u != 0.0f) tok = lal__draw_pool(vocab_size, &p, u);
        }
    }
    lal__write_back(logits, vocab_size, recent, n_recent, hv);
    return tok;
}

/* lal_sampling.h:46-125: greedy test first, then the penalty, top-k with
 * ties, softmax over the pool and one draw. */
static int lal_sample_token(float *logits, int vocab_size, float temperature, int top_k,
                            float rep_penalty, const int *recent, int n_recent)
{
    return lal__sample_common(logits, vocab_size, temperature, top_k, 0.0f, rep_penalty, recent,
                              n_recent, LAL_GPU_VARIANT_BASIC);
}

/* Top-k, then the nucleus of gpt2_server.c:2908-2955 (stable descending
 * order, inclusive cumulative cutoff at top_p), then one draw over the kept
 * tokens in ascending id order with u = (float)rand()/(float)RAND_MAX.
 * No history, so no penalty. */
static int lal_sample_token_top_p(float *logits, int n, float temperature, int top_k, float top_p)
{
    return lal__sample_common(logits, n, temperature, top_k, top_p, 1.0f, NULL, 0,
                              LAL_GPU_VARIANT_BASIC);
}

/* The lal_filter_topk operations that the GPU applies itself on the top-k
 * pool (compiler/lal.py:2218-2242): ban_last, ban_repeat(n) and ban_token(id).
 * Stands in for a loaded .lal filter plugin made only of these operations. */
static void lal_sampling_set_filter_ops(int ban_last, int ban_repeat, const int *ban_ids, int n_ban_ids)
{
    lal_sampling_gpu_state *g = &lal__gs;
    if (n_ban_ids < 0 || n_ban_ids > LAL_GPU_MAX_BAN_IDS || (n_ban_ids > 0 && !ban_ids))
        lal__die("ban_token list above LAL_GPU_MAX_BAN_IDS", LAL_GPU_E_RANGE);
    if (!g->ctx) lal__ensure(1);
    g->ban_last = ban_last;
    g->ban_repeat = ban_repeat;
    g->n_ban = n_ban_ids;
    if (n_ban_ids > 0) {
        memcpy(g->h_ban, ban_ids, (size_t)n_ban_ids * sizeof(int));
        LAL__CHECK(lal_gpu_memcpy_h2d(g->d_ban, g->h_ban, (size_t)n_ban_ids * sizeof(int), g->stream),
                   "upload ban ids");
        LAL__CHECK(lal_gpu_stream_sync(g->stream), "stream sync");
    }
}

/* Route lal_sample_token_filtered through a loaded lal_filter_topk plugin
 * (the keep-mask adapter); NULL goes back to the operations set by
 * lal_sampling_set_filter_ops.  decode_fn is passed to the plugin. */
static void lal_sampling_set_filter_plugin(lal_filter_topk_fn fn, lal_token_decode_fn decode_fn)
{
    lal__gs.plugin = fn;
    lal__gs.decode = decode_fn;
}

#ifdef LAL_SAMPLING_FILTERED
/* qwen7b_server.c:219-295: penalty first, top-k pool (k clamped to [1, V],
 * up to 512), the filter operations set by lal_sampling_set_filter_ops, pool
 * restored when they drop every token, softmax over the kept set, argmax
 * without a draw when its sum is <= 0. */
static int lal_sample_token_filtered(float *logits, int vocab_size, float temperature, int top_k,
                                     float rep_penalty, const int *recent, int n_recent)
{
    return lal__sample_common(logits, vocab_size, temperature, top_k, 0.0f, rep_penalty, recent,
                              n_recent, LAL_GPU_VARIANT_FILTERED);
}
#endif

#endif /* LAL_SAMPLING_H */
