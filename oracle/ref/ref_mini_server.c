/*
 * Harness that exposes sample_next_token (a static function of
 * tools/mini_server.c:267-363, the mini character model's sampler) by
 * compiling that translation unit with its main() renamed.  The sampler
 * copies the row it is given, reads the server's globals (vocabulary size,
 * temperature, top-k, penalty, the recent-token array and the loaded filter)
 * and takes the last token as an argument.
 */
#define main lal_ref_mini_server_main
#include "tools/mini_server.c"
#undef main

int lal_ref_mini_server_sample(const float *lm, int vocab, float temperature, int top_k,
                               float rep_penalty, const int *recent, int n_recent, int last_tok,
                               void *filter)
{
    if (n_recent > 256) n_recent = 256;
    G_V = vocab;
    g_temperature = temperature;
    g_top_k = top_k;
    g_rep_penalty = rep_penalty;
    for (int i = 0; i < n_recent; i++) g_recent[i] = recent[i];
    g_n_recent = n_recent;
    g_lal_filter = (int (*)(int *, int, int, const int *, int, lal_token_decode_fn))filter;
    int tok = sample_next_token(lm, last_tok);
    g_lal_filter = NULL;
    return tok;
}
