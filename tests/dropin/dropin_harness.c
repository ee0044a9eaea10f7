/*
 * Test harness: a translation unit that includes include/lal_sampling.h the
 * way a LAL server includes runtime/lal_sampling.h, exporting thin wrappers
 * so the parity tests can drive the drop-in through ctypes.
 */
#define LAL_SAMPLING_FILTERED 1
#include "lal_sampling.h"

void dh_srand(unsigned seed) { srand(seed); }
int dh_rand(void) { return rand(); }

int dh_sample_token(float *logits, int vocab_size, float temperature, int top_k, float rep_penalty,
                    const int *recent, int n_recent)
{
    return lal_sample_token(logits, vocab_size, temperature, top_k, rep_penalty, recent, n_recent);
}

int dh_sample_token_filtered(float *logits, int vocab_size, float temperature, int top_k,
                             float rep_penalty, const int *recent, int n_recent)
{
    return lal_sample_token_filtered(logits, vocab_size, temperature, top_k, rep_penalty, recent,
                                     n_recent);
}

int dh_sample_token_top_p(float *logits, int n, float temperature, int top_k, float top_p)
{
    return lal_sample_token_top_p(logits, n, temperature, top_k, top_p);
}

void dh_set_filter_ops(int ban_last, int ban_repeat, const int *ban_ids, int n_ban_ids)
{
    lal_sampling_set_filter_ops(ban_last, ban_repeat, ban_ids, n_ban_ids);
}

void dh_recent_push(int *tokens256, int *n, int tok)
{
    LalRecentTokens rt;
    memcpy(rt.tokens, tokens256, sizeof rt.tokens);
    rt.n = *n;
    lal_recent_push(&rt, tok);
    memcpy(tokens256, rt.tokens, sizeof rt.tokens);
    *n = rt.n;
}

void dh_globals(int *temperature, int *top_k, float *rep_penalty)
{
    *temperature = lal_g_temperature;
    *top_k = lal_g_top_k;
    *rep_penalty = lal_g_rep_penalty;
}

void dh_release(void) { lal__release(); }

void dh_set_filter_plugin(void *fn)
{
    lal_sampling_set_filter_plugin((lal_filter_topk_fn)fn, NULL);
}

/* Test plugins with the lal_filter_topk ABI, beyond what compiler/lal.py
 * emits: they exercise the adapter's restore and outside-the-pool paths. */
int dh_plugin_clear_all(int *keep_mask, int n_vocab, int last_token, const int *recent,
                        int n_recent, lal_token_decode_fn decode_fn)
{
    (void)last_token; (void)recent; (void)n_recent; (void)decode_fn;
    int d = 0;
    for (int v = 0; v < n_vocab; v++)
        if (keep_mask[v]) { keep_mask[v] = 0; d++; }
    return d;
}

/* keep every third kept id (in id order), starting with the second */
int dh_plugin_thin3(int *keep_mask, int n_vocab, int last_token, const int *recent,
                    int n_recent, lal_token_decode_fn decode_fn)
{
    (void)last_token; (void)recent; (void)n_recent; (void)decode_fn;
    int i = 0, d = 0;
    for (int v = 0; v < n_vocab; v++) {
        if (!keep_mask[v]) continue;
        if (i++ % 3 != 1) { keep_mask[v] = 0; d++; }
    }
    return d;
}

/* clear the pool and set ids outside it: the recent ids and id 7 */
int dh_plugin_swap_out(int *keep_mask, int n_vocab, int last_token, const int *recent,
                       int n_recent, lal_token_decode_fn decode_fn)
{
    (void)last_token; (void)decode_fn;
    int pool[4096], np = 0;
    for (int v = 0; v < n_vocab; v++)
        if (keep_mask[v]) {
            if (np < 4096) pool[np++] = v;
            keep_mask[v] = 0;
        }
    for (int i = 0; i < n_recent; i++)
        if (recent[i] >= 0 && recent[i] < n_vocab) keep_mask[recent[i]] = 1;
    if (n_vocab > 7) keep_mask[7] = 1;
    for (int i = 0; i < np; i++) keep_mask[pool[i]] = 0;
    return np;
}

/* keep the pool and also set ids outside it (ignored by the softmax) */
int dh_plugin_add_out(int *keep_mask, int n_vocab, int last_token, const int *recent,
                      int n_recent, lal_token_decode_fn decode_fn)
{
    (void)last_token; (void)recent; (void)n_recent; (void)decode_fn;
    for (int v = 3; v < n_vocab; v += 997) keep_mask[v] = 1;
    return 0;
}
