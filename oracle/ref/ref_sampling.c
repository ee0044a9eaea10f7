/*
 * Harness that exposes the reference sampler (runtime/lal_sampling.h, a
 * header of static functions) as exported symbols, so the oracle can be
 * checked against the reference's own code.  Built from the header where it
 * lies in the reference tree (see oracle/Makefile); nothing is copied.
 */
#include <stdint.h>
#include <time.h>
#include "runtime/lal_sampling.h"

void lal_ref_srand(unsigned seed) { srand(seed); }
int lal_ref_rand(void) { return rand(); }

int lal_ref_sample_token(float *logits, int vocab_size, float temperature,
                         int top_k, float rep_penalty, const int *recent,
                         int n_recent)
{
    return lal_sample_token(logits, vocab_size, temperature, top_k,
                            rep_penalty, recent, n_recent);
}

void lal_ref_recent_push(int *tokens256, int *n, int tok)
{
    LalRecentTokens rt;
    memcpy(rt.tokens, tokens256, sizeof rt.tokens);
    rt.n = *n;
    lal_recent_push(&rt, tok);
    memcpy(tokens256, rt.tokens, sizeof rt.tokens);
    *n = rt.n;
}
