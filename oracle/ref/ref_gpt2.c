/*
 * Harness that exposes the GPT-2 server's int8 LM head with its fp32 re-rank
 * (lm_head_int8_parallel, a static function of
 * tools/server/gpt2_server.c:2125-2215) and its row quantizer
 * (lm_head_quantize_x, :1982-1998) by compiling that translation unit with
 * its main() renamed.  The shapes are the server's own (VOCAB_SIZE x N_EMBD).
 */
#define main lal_ref_gpt2_main
#include "tools/server/gpt2_server.c"
#undef main

/* logits[VOCAB_SIZE] <- pass 1 (int8) + pass 2 (fp32 re-rank of the top 512) */
void lal_ref_gpt2_lm_head(float *logits, const float *x, int8_t *wq, float *ws)
{
    g_wte_q = wq;
    g_wte_scale = ws;
    lm_head_int8_parallel(logits, x, 1);
    g_wte_q = NULL;
    g_wte_scale = NULL;
}

float lal_ref_gpt2_quantize_row(const float *x, int8_t *q, int n)
{
    return lm_head_quantize_x(x, q, n);
}

int lal_ref_gpt2_vocab(void) { return VOCAB_SIZE; }
int lal_ref_gpt2_embd(void) { return N_EMBD; }
