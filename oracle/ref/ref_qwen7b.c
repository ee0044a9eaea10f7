/*
 * Harness that exposes lal_sample_token_filtered (a static function of
 * tools/server/qwen7b_server.c:219-295) by compiling that translation unit
 * with its main() renamed.  The server's plugin pointer can be set so the
 * filter contract (qwen7b_server.c:260-269) is exercised exactly as the
 * server runs it.
 */
#define main lal_ref_qwen7b_main
#include "tools/server/qwen7b_server.c"
#undef main

int lal_ref_sample_token_filtered(float *logits, int vocab_size,
                                  float temperature, int top_k,
                                  float rep_penalty, const int *recent,
                                  int n_recent)
{
    return lal_sample_token_filtered(logits, vocab_size, temperature, top_k,
                                     rep_penalty, recent, n_recent);
}

void lal_ref_set_filter(void *fn)
{
    g_lal_filter = (int (*)(int *, int, int, const int *, int,
                            lal_token_decode_fn))fn;
}

int lal_ref_vocab_capacity(void) { return VOCAB_SIZE; }

/* Install a tokenizer vocabulary (id -> vocab string) in place of
 * load_tokenizer's, so that the server's decode_fn (qwen7b_decode_for_filter
 * -> decode_token, qwen7b_server.c:885-888) decodes for a loaded plugin. */
void lal_ref_qwen7b_set_vocab(char **strs, int n)
{
    g_vocab_str = strs;
    g_vocab_str_n = n;
}
