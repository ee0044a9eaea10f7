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
