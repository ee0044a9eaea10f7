/*
 * Harness that exposes sample_next_token (a static function of
 * tools/server/qwen_server.c:418-527, the Qwen2 server's sampler) by
 * compiling that translation unit with its main() renamed.  The sampler reads
 * the server's globals (g_logits over VOCAB_SIZE = 151936 ids, temperature,
 * top-k, penalty, the recent-token ring and the loaded filter), which the
 * wrapper sets before the call.
 */
#define main lal_ref_qwen_server_main
#include "tools/server/qwen_server.c"
#undef main

int lal_ref_qwen_server_sample(float *logits, float temperature, int top_k, float rep_penalty,
                               const int *recent, int n_recent, void *filter)
{
    if (n_recent > 256) n_recent = 256;
    g_logits = logits;
    g_temperature = temperature;
    g_top_k = top_k;
    g_rep_penalty = rep_penalty;
    for (int i = 0; i < n_recent; i++) g_recent_tokens[i] = recent[i];
    g_n_recent = n_recent;
    g_lal_filter = (int (*)(int *, int, int, const int *, int, lal_token_decode_fn))filter;
    int tok = sample_next_token();
    g_lal_filter = NULL;
    return tok;
}

int lal_ref_qwen_server_vocab(void) { return VOCAB_SIZE; }
