/*
 * lal_oracle.c -- CPU restatement of LAL's token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker).  It is never linked into the
 * product library; only tests/, the smoke check and bench.py's cpu_baseline
 * leg load it.  Reference anchors are given per function; the full list is in
 * lal_oracle.h.
 */
#include "lal_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

float lal_oracle_expf(float x) { return expf(x); }

/* ---------------------------------------------------------------------------
 * k-th largest with multiplicity, by a size-k min-heap whose root is replaced
 * only by a strictly larger value (runtime/lal_sampling.h:69-104,
 * tools/server/qwen7b_server.c:237-256).
 * ------------------------------------------------------------------------- */
static float heap_kth_largest(const float *y, int n, int k, float *heap)
{
    int size = 0;
    heap[0] = -INFINITY;
    for (int v = 0; v < n; v++) {
        float val = y[v];
        if (size < k) {
            int c = size++;
            heap[c] = val;
            while (c > 0) {
                int up = (c - 1) >> 1;
                if (heap[up] <= heap[c]) break;
                float t = heap[up]; heap[up] = heap[c]; heap[c] = t;
                c = up;
            }
        } else if (val > heap[0]) {
            heap[0] = val;
            int at = 0;
            for (;;) {
                int a = 2 * at + 1, b = a + 1, lo = at;
                if (a < size && heap[a] < heap[lo]) lo = a;
                if (b < size && heap[b] < heap[lo]) lo = b;
                if (lo == at) break;
                float t = heap[at]; heap[at] = heap[lo]; heap[lo] = t;
                at = lo;
            }
        }
    }
    return heap[0];
}

static int cmp_desc(const void *a, const void *b)
{
    float x = *(const float *)a, y = *(const float *)b;
    return (x < y) - (x > y);
}

float lal_oracle_kth_largest_sorted(const float *x, int n, int k)
{
    float *tmp = (float *)malloc((size_t)n * sizeof(float));
    memcpy(tmp, x, (size_t)n * sizeof(float));
    qsort(tmp, (size_t)n, sizeof(float), cmp_desc);
    float r = tmp[k - 1];
    free(tmp);
    return r;
}

/* Stable descending sort of (prob, id) pairs: equal probabilities keep their
 * input (ascending-id) order, which is what the insertion sort of
 * gpt2_server.c:2934-2945 produces.  Bottom-up merge sort so that large tie
 * groups stay O(n log n). */
static void stable_sort_desc(float *p, int *id, int n, float *tp, int *tid)
{
    for (int w = 1; w < n; w *= 2) {
        for (int lo = 0; lo < n; lo += 2 * w) {
            int mid = lo + w < n ? lo + w : n;
            int hi = lo + 2 * w < n ? lo + 2 * w : n;
            int i = lo, j = mid, o = lo;
            while (i < mid && j < hi) {
                /* take from the right only when strictly larger */
                if (p[j] > p[i]) { tp[o] = p[j]; tid[o++] = id[j++]; }
                else             { tp[o] = p[i]; tid[o++] = id[i++]; }
            }
            while (i < mid) { tp[o] = p[i]; tid[o++] = id[i++]; }
            while (j < hi)  { tp[o] = p[j]; tid[o++] = id[j++]; }
        }
        memcpy(p, tp, (size_t)n * sizeof(float));
        memcpy(id, tid, (size_t)n * sizeof(int));
    }
}

static void apply_penalty(float *row, int V, float pen, const int *hist, int n_hist)
{
    /* lal_sampling.h:59-67: once per history occurrence, in order */
    if (!(pen > 1.0f) || !hist || n_hist <= 0) return;
    for (int i = 0; i < n_hist; i++) {
        int t = hist[i];
        if (t < 0 || t >= V) continue;
        if (row[t] > 0) row[t] = row[t] / pen;
        else            row[t] = row[t] * pen;
    }
}

static int argmax_first(const float *y, int V)
{
    int best = 0;
    for (int v = 1; v < V; v++)
        if (y[v] > y[best]) best = v;
    return best;
}

int lal_oracle_sample_row(float *row, int V, const lal_oracle_params *p,
                          const int *hist, int n_hist,
                          const uint32_t *allow, const float *bias, float u,
                          lal_oracle_filter_fn filter, lal_oracle_decode_fn decode,
                          lal_oracle_info *info,
                          int cand_cap, int *cand_ids, float *cand_probs,
                          unsigned char *cand_kept)
{
    lal_oracle_info inf;
    memset(&inf, 0, sizeof inf);
    const float T = p->temperature;
    const int greedy = (T <= 0.0f || p->top_k <= 0);
    int token = V - 1;

    if (p->variant == LAL_ORACLE_VARIANT_FILTERED)
        apply_penalty(row, V, p->rep_penalty, hist, n_hist);
    else if (!greedy)
        apply_penalty(row, V, p->rep_penalty, hist, n_hist);

    /* processed logits: bias -> allow bitmask -> hard anti-repeat */
    float *y = (float *)malloc((size_t)V * sizeof(float));
    for (int v = 0; v < V; v++) {
        float x = row[v];
        if (bias) x = x + bias[v];
        if (allow && !((allow[v >> 5] >> (v & 31)) & 1u)) x = -INFINITY;
        y[v] = x;
    }
    if (p->mask_recent > 0 && hist) {
        int s = n_hist > p->mask_recent ? n_hist - p->mask_recent : 0;
        for (int i = s; i < n_hist; i++) {
            int t = hist[i];
            if (t >= 0 && t < V) y[t] = -INFINITY;
        }
    }

    if (greedy) {
        token = argmax_first(y, V);
        /* the selection's threshold and pool: the argmax value */
        inf.threshold = y[token];
        if (p->flags & LAL_ORACLE_F_GREEDY_FILTER) {
            /* mini_server.c:284-288 hands &km (km = the argmax) to the filter
             * as its keep mask: element 0 is the token id.  Only id 0 lies
             * inside that one-element array, so a ban of id 0 clears it
             * (token 0); the filter is called with n_vocab = 1 so that the ids
             * it would read past the array stay out of range. */
            int km = token;
            const int last = p->has_last ? p->last_token : ((n_hist > 0 && hist) ? hist[n_hist - 1] : -1);
            if (p->ban_last && last == 0) km = 0;
            if (p->ban_repeat > 0 && hist) {
                int s = n_hist > p->ban_repeat ? n_hist - p->ban_repeat : 0;
                for (int i = s; i < n_hist; i++)
                    if (hist[i] == 0) km = 0;
            }
            for (int i = 0; i < p->n_ban_ids; i++)
                if (p->ban_ids[i] == 0) km = 0;
            if (filter) {
                int m1 = km;
                filter(&m1, 1, last, hist, n_hist, decode);
                km = m1;
            }
            token = km;
        }
        inf.greedy = 1;
        int n = 0;
        for (int v = 0; v < V; v++) n += (y[v] >= inf.threshold);
        inf.n_cand = n;
        inf.n_kept = 1;
        if (cand_ids || cand_probs || cand_kept) {
            int i = 0;
            for (int v = 0; v < V && i < cand_cap; v++) {
                if (!(y[v] >= inf.threshold)) continue;
                if (cand_ids) cand_ids[i] = v;
                if (cand_kept) cand_kept[i] = (unsigned char)(v == token);
                if (cand_probs) cand_probs[i] = (v == token) ? 1.0f : 0.0f;
                i++;
            }
        }
        if (info) *info = inf;
        free(y);
        return token;
    }

    int k = p->top_k;
    if (k > V) k = V;
    if (k < 1) k = 1;
    float *heap = (float *)malloc((size_t)k * sizeof(float));
    const float thr = heap_kth_largest(y, V, k, heap);
    free(heap);

    int *cand = (int *)malloc((size_t)V * sizeof(int));
    int *keep = (int *)malloc((size_t)V * sizeof(int));
    int n_cand = 0;
    for (int v = 0; v < V; v++) {
        int c = (y[v] >= thr);
        if (c) cand[n_cand++] = v;
        keep[v] = c;
    }

    /* top-p nucleus over the top-k pool (gpt2_server.c:2908-2955) */
    if (p->top_p > 0.0f && p->top_p < 1.0f && n_cand > 0) {
        float *pr = (float *)malloc((size_t)n_cand * sizeof(float));
        int *id = (int *)malloc((size_t)n_cand * sizeof(int));
        float *tp = (float *)malloc((size_t)n_cand * sizeof(float));
        int *tid = (int *)malloc((size_t)n_cand * sizeof(int));
        float amax = -1e30f;
        for (int i = 0; i < n_cand; i++)
            if (y[cand[i]] > amax) amax = y[cand[i]];
        float se = 0.0f;
        for (int i = 0; i < n_cand; i++) {
            pr[i] = expf((y[cand[i]] - amax) / T);
            se += pr[i];
            id[i] = cand[i];
        }
        float inv = 1.0f / (se + 1e-12f);
        for (int i = 0; i < n_cand; i++) pr[i] *= inv;
        stable_sort_desc(pr, id, n_cand, tp, tid);
        for (int i = 0; i < n_cand; i++) keep[cand[i]] = 0;
        float cum = 0.0f;
        for (int i = 0; i < n_cand; i++) {
            keep[id[i]] = 1;
            cum += pr[i];
            if (cum >= p->top_p) break;
        }
        free(pr); free(id); free(tp); free(tid);
    }

    /* lal.py filter ops on the keep mask (compiler/lal.py:2220-2242), then an
     * optional plugin with the lal_filter_topk ABI, then restore-if-empty
     * (qwen7b_server.c:260-269). */
    {
        int last = p->has_last ? p->last_token : ((n_hist > 0 && hist) ? hist[n_hist - 1] : -1);
        if (p->ban_last && last >= 0 && last < V) keep[last] = 0;
        if (p->ban_repeat > 0 && hist) {
            int s = n_hist > p->ban_repeat ? n_hist - p->ban_repeat : 0;
            for (int i = s; i < n_hist; i++) {
                int t = hist[i];
                if (t >= 0 && t < V) keep[t] = 0;
            }
        }
        for (int i = 0; i < p->n_ban_ids; i++) {
            int t = p->ban_ids[i];
            if (t >= 0 && t < V) keep[t] = 0;
        }
        if (filter) filter(keep, V, last, hist, n_hist, decode);
        int any = 0;
        for (int i = 0; i < n_cand; i++) if (keep[cand[i]]) { any = 1; break; }
        /* a plugin may only clear entries; anything it sets outside the pool
         * is still honoured as the reference does (keep_mask is read as-is) */
        if (!any) {
            for (int v = 0; v < V; v++) if (keep[v]) { any = 1; break; }
        }
        if (!any)
            for (int i = 0; i < n_cand; i++) keep[cand[i]] = 1;
    }

    /* softmax over the kept set, ascending id, sequential fp32 */
    float mx = -1e30f;
    for (int v = 0; v < V; v++)
        if (keep[v] && y[v] >= thr && y[v] > mx) mx = y[v];
    float sum = 0.0f;
    int n_kept = 0;
    for (int v = 0; v < V; v++)
        if (keep[v] && y[v] >= thr) { sum += expf((y[v] - mx) / T); n_kept++; }

    inf.threshold = thr;
    inf.n_cand = n_cand;
    inf.n_kept = n_kept;
    inf.sum = sum;

    if (p->variant == LAL_ORACLE_VARIANT_FILTERED && sum <= 0) {
        /* qwen7b_server.c:285-286: argmax over the kept set, no draw */
        int best = 0;
        float bv = -1e30f;
        for (int v = 0; v < V; v++)
            if (keep[v] && y[v] > bv) { bv = y[v]; best = v; }
        token = best;
    } else {
        inf.used_uniform = 1;
        float r = u * sum;
        token = (p->flags & LAL_ORACLE_F_FALLBACK_ZERO) ? 0 : V - 1;
        if ((p->flags & LAL_ORACLE_F_DRAW_GPT2) && r == 0.0f) {
            token = 0;
        } else {
            float acc = 0.0f;
            for (int v = 0; v < V; v++) {
                if (keep[v] && y[v] >= thr) {
                    acc += expf((y[v] - mx) / T);
                    if (r <= acc) { token = v; break; }
                }
            }
        }
    }

    if (cand_ids || cand_probs || cand_kept) {
        int m = n_cand < cand_cap ? n_cand : cand_cap;
        for (int i = 0; i < m; i++) {
            int v = cand[i];
            int kp = keep[v] != 0;
            if (cand_ids) cand_ids[i] = v;
            if (cand_kept) cand_kept[i] = (unsigned char)kp;
            if (cand_probs) cand_probs[i] = kp ? expf((y[v] - mx) / T) / sum : 0.0f;
        }
    }
    free(cand); free(keep); free(y);
    if (info) *info = inf;
    return token;
}

void lal_oracle_sample_batch(float *logits, int B, int V, int ld,
                             const lal_oracle_params *p,
                             const int *hist, int hist_ld, const int *hist_len,
                             const uint32_t *allow, int allow_ld,
                             const float *bias, const float *uniforms,
                             int *out_token, float *out_threshold,
                             int *out_n_cand, int *out_n_kept, float *out_sum,
                             int cand_ld, int *cand_ids, float *cand_probs,
                             unsigned char *cand_kept, int nthreads)
{
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int b = 0; b < B; b++) {
        lal_oracle_info inf;
        const int *h = hist ? hist + (size_t)b * hist_ld : NULL;
        int nh = hist ? (hist_len ? hist_len[b] : hist_ld) : 0;
        const uint32_t *al = allow ? allow + (size_t)b * allow_ld : NULL;
        size_t co = (size_t)b * (cand_ld > 0 ? cand_ld : 0);
        lal_oracle_params pb = *p;
        if (p->last_tokens) {
            pb.has_last = 1;
            pb.last_token = p->last_tokens[b];
        }
        out_token[b] = lal_oracle_sample_row(
            logits + (size_t)b * ld, V, &pb, h, nh, al, bias, uniforms[b],
            NULL, NULL, &inf, cand_ld,
            cand_ids ? cand_ids + co : NULL,
            cand_probs ? cand_probs + co : NULL,
            cand_kept ? cand_kept + co : NULL);
        if (out_threshold) out_threshold[b] = inf.threshold;
        if (out_n_cand) out_n_cand[b] = inf.n_cand;
        if (out_n_kept) out_n_kept[b] = inf.n_kept;
        if (out_sum) out_sum[b] = inf.sum;
    }
#ifndef _OPENMP
    (void)nthreads;
#endif
}

void lal_oracle_uniforms(unsigned seed, int n, float *out, int gpt2)
{
    srand(seed);
    for (int i = 0; i < n; i++) {
        if (gpt2) out[i] = (float)(rand() % 1000000) / 1000000.0f;
        else      out[i] = (float)rand() / (float)RAND_MAX;
    }
}

/* lal_q8_kernel.h:375-442.  The AVX2 build converts the multiple-of-8 prefix
 * with round-to-nearest-even (cvtps_epi32 under the default MXCSR) and the
 * remainder with C truncation; the scalar build truncates everything. */
/* x86 float -> int32 conversions as the reference's builds execute them
 * (cvtps2dq rounds to nearest even; cvttss2si, C's (int) cast, truncates):
 * a nan or a value outside the int32 range gives INT_MIN ("integer
 * indefinite"). */
static int x86_cvt(float v, int round_even)
{
    if (!(v >= -2147483648.0f && v < 2147483648.0f)) return INT_MIN;
    return round_even ? (int)nearbyintf(v) : (int)v;
}

/* _mm_max_ps / _mm256_max_ps: the first operand if it is greater, else the
 * second (so a nan in either operand gives the second). */
static float x86_maxps(float a, float b)
{
    return (a > b) ? a : b;
}

/* lal_q8_kernel.h:375-445 (lal_quantize_x_int8).  mode 0, the AVX2 build
 * (:376-428): |x| maxima in 8 lanes over the first n & ~7 values (lane j
 * sees x[8c + j] in order, from 0), reduced as hi/lo halves then two shuffled
 * steps (:387-392), the tail folded in with `a > max` (:393); values of the 8-
 * aligned prefix rounded by cvtps2dq (:402-404), the tail truncated (:415);
 * both clamped to [-127, 127].  mode 1, the scalar build (:429-443): `a > max`
 * over all values, every value truncated and clamped. */
float lal_oracle_quantize_x(const float *x, int8_t *xq, int n, int mode)
{
    float m = 0.0f;
    int n8 = 0;
    if (mode == 0) {
        n8 = n & ~7;
        float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int i = 0; i < n8; i++) lane[i & 7] = x86_maxps(lane[i & 7], fabsf(x[i]));
        float h[4];
        for (int j = 0; j < 4; j++) h[j] = x86_maxps(lane[j], lane[j + 4]);
        /* _MM_SHUFFLE(1,0,3,2): (h2, h3, h0, h1) */
        const float s1[4] = {h[2], h[3], h[0], h[1]};
        for (int j = 0; j < 4; j++) h[j] = x86_maxps(h[j], s1[j]);
        /* _MM_SHUFFLE(0,0,0,1): element 0 takes h1 */
        m = x86_maxps(h[0], h[1]);
    }
    for (int i = n8; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > m) m = a;
    }
    float scale = m / 127.0f;
    if (scale < 1e-8f) scale = 1e-8f;
    float inv = 1.0f / scale;
    for (int i = 0; i < n; i++) {
        int q = x86_cvt(x[i] * inv, i < n8);
        if (q > 127) q = 127;
        if (q < -127) q = -127;
        xq[i] = (int8_t)q;
    }
    return scale;
}

/* lal_q8_kernel.h:463-499: exact int32 dot, then (sx*sw[v])*(float)dot */
void lal_oracle_lm_head(float *logits, const int8_t *xq, float sx,
                        const int8_t *W, const float *sw, int v0, int v1,
                        int n, int nthreads)
{
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int v = v0; v < v1; v++) {
        const int8_t *w = W + (size_t)v * n;
        int32_t dot = 0;
        for (int i = 0; i < n; i++) dot += (int32_t)xq[i] * (int32_t)w[i];
        logits[v] = sx * sw[v] * (float)dot;
    }
#ifndef _OPENMP
    (void)nthreads;
#endif
}

/* lal_q8_kernel.h:357-372: per-row absmax, lroundf (half away from zero) */
void lal_oracle_quantize_w(const float *W, int8_t *q, float *scale,
                           int in_dim, int out_dim)
{
    for (int j = 0; j < out_dim; j++) {
        const float *r = W + (size_t)j * in_dim;
        float m = 0.0f;
        for (int i = 0; i < in_dim; i++) {
            float a = fabsf(r[i]);
            if (a > m) m = a;
        }
        float s = m / 127.0f;
        if (s < 1e-8f) s = 1e-8f;
        scale[j] = s;
        float inv = 1.0f / s;
        for (int i = 0; i < in_dim; i++) {
            long t = lroundf(r[i] * inv);
            if (t > 127) t = 127;
            if (t < -127) t = -127;
            q[(size_t)j * in_dim + i] = (int8_t)t;
        }
    }
}

/* gpt2_server.c:2155-2192: min-heap of (value, id), root = smallest kept;
 * a value enters while there is room, later only when it exceeds the root. */
int lal_oracle_gpt2_rerank(float *logits, const float *x, const int8_t *wq,
                           const float *ws, int V, int n, int R, int *ids)
{
    float *hv = (float *)malloc((size_t)R * sizeof(float));
    int *hi = (int *)malloc((size_t)R * sizeof(int));
    int size = 0;
    for (int v = 0; v < V; v++) {
        const float val = logits[v];
        if (size < R) {
            int c = size++;
            hv[c] = val;
            hi[c] = v;
            while (c > 0) {
                const int up = (c - 1) >> 1;
                if (hv[up] <= hv[c]) break;
                float t = hv[up]; hv[up] = hv[c]; hv[c] = t;
                int ti = hi[up]; hi[up] = hi[c]; hi[c] = ti;
                c = up;
            }
        } else if (val > hv[0]) {
            hv[0] = val;
            hi[0] = v;
            int at = 0;
            for (;;) {
                const int a = 2 * at + 1, b = a + 1;
                int lo = at;
                if (a < size && hv[a] < hv[lo]) lo = a;
                if (b < size && hv[b] < hv[lo]) lo = b;
                if (lo == at) break;
                float t = hv[at]; hv[at] = hv[lo]; hv[lo] = t;
                int ti = hi[at]; hi[at] = hi[lo]; hi[lo] = ti;
                at = lo;
            }
        }
    }
    /* gpt2_server.c:2200-2213 */
    float *w = (float *)malloc((size_t)n * sizeof(float));
    for (int j = 0; j < size; j++) {
        const int v = hi[j];
        const float sc = ws[v];
        for (int i = 0; i < n; i++) w[i] = (float)wq[(size_t)v * n + i] * sc;
        float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int i = 0;
        for (; i + 8 <= n; i += 8)
            for (int c = 0; c < 8; c++) lane[c] = fmaf(x[i + c], w[i + c], lane[c]);
        float s = lane[0];
        for (int c = 1; c < 8; c++) s = s + lane[c];
        for (; i < n; i++) s = fmaf(x[i], w[i], s);
        logits[v] = s;
        if (ids) ids[j] = v;
    }
    free(w);
    free(hv);
    free(hi);
    return size;
}

/* Filter plugins with the lal_filter_topk ABI (compiler/lal.py:2205-2242):
 * each ban clears a still-kept id and counts it.  antirepeat4 is what
 * demos/mini_antirepeat.lal declares (ban_last; ban_repeat(4)); norepeat6 is
 * the id rules of demos/qwen_filter.lal (ban_last; ban_repeat(6)). */
static int ban_recent(int *keep, int V, int last, const int *rec, int n, int rep)
{
    int dropped = 0;
    if (last >= 0 && last < V && keep[last]) { keep[last] = 0; dropped++; }
    int s = n > rep ? n - rep : 0;
    for (int i = s; i < n; i++) {
        int t = rec[i];
        if (t >= 0 && t < V && keep[t]) { keep[t] = 0; dropped++; }
    }
    return dropped;
}

int lal_oracle_filter_antirepeat4(int *keep_mask, int n_vocab, int last_token,
                                  const int *recent, int n_recent,
                                  lal_oracle_decode_fn decode_fn)
{
    (void)decode_fn;
    return ban_recent(keep_mask, n_vocab, last_token, recent, n_recent, 4);
}

int lal_oracle_filter_norepeat6(int *keep_mask, int n_vocab, int last_token,
                                const int *recent, int n_recent,
                                lal_oracle_decode_fn decode_fn)
{
    (void)decode_fn;
    return ban_recent(keep_mask, n_vocab, last_token, recent, n_recent, 6);
}

/* Per-chunk hash of glibc expf over every float input x = (hi<<16)|lo,
 * lo in [0, 65536): out[i] for hi = first_hi + i.  The GPU's expf
 * restatement is checked against these sums (same mixing function). */
static uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void lal_oracle_expf_checksums(unsigned first_hi, int nhi, uint64_t *out)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 16)
#endif
    for (int i = 0; i < nhi; i++) {
        uint64_t h = 0;
        uint32_t hi = first_hi + (uint32_t)i;
        for (uint32_t lo = 0; lo < 65536u; lo++) {
            uint32_t ux = (hi << 16) | lo, rb;
            float x, r;
            memcpy(&x, &ux, 4);
            r = expf(x);
            memcpy(&rb, &r, 4);
            if (r != r) rb = 0x7fc00000u;
            h += mix64(((uint64_t)ux << 32) | rb);
        }
        out[i] = h;
    }
}

/* lal_sampling.h:133-136: append, or drop the oldest once 256 are held */
void lal_oracle_recent_push(lal_oracle_recent *rt, int tok)
{
    if (rt->n < 256) {
        rt->tokens[rt->n++] = tok;
        return;
    }
    memmove(rt->tokens, rt->tokens + 1, 255 * sizeof(int));
    rt->tokens[255] = tok;
}
