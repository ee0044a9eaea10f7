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

/* ---- a lal_filter_topk plugin that uses decode_fn --------------------------
 * A stub tokenizer (id -> plain ASCII word, decoded unchanged by the
 * reference's byte-level BPE decoder) and a plugin with the anti-repeat bans
 * and two ban_relation rules of demos/qwen_filter.lal, written from the
 * semantics of compiler/lal.py:2243-2317: the recent ids are decoded into a
 * text (at most 1024 bytes); when it ends with the trigger and the character
 * before the trigger is a boundary, every kept id whose decoded text is not
 * an allow word (exactly, or followed by a boundary character) is dropped. */
#define DH_VOCAB 4096
static char *dh_vocab[DH_VOCAB];

char **dh_vocab_table(void)
{
    static const char *named[] = {" the", " capital", " of", " France", " Japan", " is", " Paris",
                                  " Tokyo", " Berlin", "Paris", " Paris.", " Parisian", " Rome",
                                  ",", " city", "Tokyo!", " Tokyo", " Osaka", "\n", " capital?",
                                  " xcapital"};
    const int nn = (int)(sizeof named / sizeof named[0]);
    if (!dh_vocab[0]) {
        for (int i = 0; i < DH_VOCAB; i++) {
            char buf[32];
            if (i < nn) snprintf(buf, sizeof buf, "%s", named[i]);
            else if (i % 5 == 0) snprintf(buf, sizeof buf, "%s", named[i % nn]);
            else snprintf(buf, sizeof buf, " w%d", i);
            dh_vocab[i] = strdup(buf);
        }
    }
    return dh_vocab;
}

int dh_decode_stub(int token_id, char *out_buf, int max_len)
{
    char **t = dh_vocab_table();
    if (token_id < 0 || token_id >= DH_VOCAB || max_len <= 0) {
        if (max_len > 0) out_buf[0] = 0;
        return 0;
    }
    int n = (int)strlen(t[token_id]);
    if (n > max_len - 1) n = max_len - 1;
    memcpy(out_buf, t[token_id], (size_t)n);
    out_buf[n] = 0;
    return n;
}

static int dh_boundary(char c)
{
    return c == ' ' || c == '\n' || c == '\t' || c == '.' || c == ',' || c == '!' || c == '?' ||
           c == ':' || c == ';' || c == '(' || c == '"';
}

static int dh_relation(int *keep_mask, int n_vocab, const int *recent, int n_recent,
                       lal_token_decode_fn decode_fn, const char *trigger, const char *allow)
{
    if (!decode_fn) return 0;
    char buf[128], text[1024];
    int tl = 0, dropped = 0;
    text[0] = 0;
    for (int i = 0; i < n_recent && tl < (int)sizeof text - 64; i++) {
        int n = decode_fn(recent[i], buf, (int)sizeof buf - 1);
        if (n > 0) {
            buf[n] = 0;
            int bl = (int)strlen(buf);
            if (tl + bl < (int)sizeof text) {
                memcpy(text + tl, buf, (size_t)bl);
                tl += bl;
            }
        }
    }
    text[tl] = 0;
    const int gl = (int)strlen(trigger);
    if (gl == 0 || tl < gl || memcmp(text + tl - gl, trigger, (size_t)gl) != 0) return 0;
    if (!dh_boundary(tl == gl ? ' ' : text[tl - gl - 1])) return 0;
    const int al = (int)strlen(allow);
    for (int v = 0; v < n_vocab; v++) {
        if (!keep_mask[v]) continue;
        int dn = decode_fn(v, buf, (int)sizeof buf - 1);
        if (dn <= 0) { keep_mask[v] = 0; dropped++; continue; }
        buf[dn] = 0;
        int ok = strcmp(buf, allow) == 0 ||
                 ((int)strlen(buf) >= al && memcmp(buf, allow, (size_t)al) == 0 &&
                  (buf[al] == 0 || dh_boundary(buf[al])));
        if (!ok) { keep_mask[v] = 0; dropped++; }
    }
    return dropped;
}

int dh_plugin_relation(int *keep_mask, int n_vocab, int last_token, const int *recent,
                       int n_recent, lal_token_decode_fn decode_fn)
{
    int d = 0;
    if (last_token >= 0 && last_token < n_vocab && keep_mask[last_token]) { keep_mask[last_token] = 0; d++; }
    const int s = n_recent > 6 ? n_recent - 6 : 0;
    for (int i = s; i < n_recent; i++) {
        int t = recent[i];
        if (t >= 0 && t < n_vocab && keep_mask[t]) { keep_mask[t] = 0; d++; }
    }
    d += dh_relation(keep_mask, n_vocab, recent, n_recent, decode_fn, "capital of France", " Paris");
    d += dh_relation(keep_mask, n_vocab, recent, n_recent, decode_fn, "capital of Japan", " Tokyo");
    return d;
}

void dh_set_filter_plugin_decode(void *fn, void *decode)
{
    lal_sampling_set_filter_plugin((lal_filter_topk_fn)fn, (lal_token_decode_fn)decode);
}
