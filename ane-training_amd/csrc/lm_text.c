/*
 * lm_text.c — the text side of the token loop (C11, host only): the llama2.c
 * tokenizer, a drand48-compatible random stream and the three samplers of
 * training/training_dynamic/generate.m.
 *
 *   tokenizer   load generate.m:37-56, decode :58-65, encode :68-126
 *   samplers    argmax :129-136, temperature :138-162, top-p :164-209
 *
 * Behaviour follows the reference exactly, quirks included (encode maps each
 * byte to its single-character token and skips bytes without one, then merges
 * the adjacent pair whose concatenation scores highest, earliest pair on ties;
 * no BOS and no leading space are added).  The reference finds merge
 * candidates by scanning the whole vocabulary for every pair; here the
 * vocabulary is sorted once and searched, which gives the same token: for a
 * string present several times the entry the scan would keep is the one with
 * the highest score, lowest index among equal scores.
 */
#include "stories_lm.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct LMTokenizer {
    char **vocab;
    float *scores;
    int n;
    int max_token_length;
    int single[256];   /* first token whose string is exactly that one byte, or -1 */
    int *order;        /* token ids sorted by (string, score desc, id asc) */
};

static const LMTokenizer *g_sort_tok;   /* qsort context (load is not re-entrant) */

static int cmp_entry(const void *a, const void *b)
{
    const int i = *(const int *)a, j = *(const int *)b;
    const int c = strcmp(g_sort_tok->vocab[i], g_sort_tok->vocab[j]);
    if (c) return c;
    const float si = g_sort_tok->scores[i], sj = g_sort_tok->scores[j];
    if (si != sj) return si > sj ? -1 : 1;
    return (i > j) - (i < j);
}

void lm_tokenizer_free(LMTokenizer *t)
{
    if (!t) return;
    if (t->vocab)
        for (int i = 0; i < t->n; i++) free(t->vocab[i]);
    free(t->vocab);
    free(t->scores);
    free(t->order);
    free(t);
}

LMTokenizer *lm_tokenizer_load(const char *path, int vocab_size, int *status)
{
    int st = LM_OK;
    LMTokenizer *t = NULL;
    FILE *f = NULL;
    if (!path || vocab_size < 1) {
        st = LM_ERR_INVALID;
        goto done;
    }
    f = fopen(path, "rb");
    if (!f) {
        st = LM_ERR_IO;
        goto done;
    }
    t = (LMTokenizer *)calloc(1, sizeof(LMTokenizer));
    if (!t) {
        st = LM_ERR_OOM;
        goto done;
    }
    t->vocab = (char **)calloc((size_t)vocab_size, sizeof(char *));
    t->scores = (float *)malloc((size_t)vocab_size * sizeof(float));
    t->order = (int *)malloc((size_t)vocab_size * sizeof(int));
    if (!t->vocab || !t->scores || !t->order) {
        st = LM_ERR_OOM;
        goto done;
    }
    if (fread(&t->max_token_length, sizeof(int), 1, f) != 1) {
        st = LM_ERR_FORMAT;
        goto done;
    }
    for (int i = 0; i < vocab_size; i++) {
        int len = 0;
        if (fread(&t->scores[i], sizeof(float), 1, f) != 1 || fread(&len, sizeof(int), 1, f) != 1 ||
            len < 0 || len > (1 << 20)) {
            st = LM_ERR_FORMAT;
            goto done;
        }
        t->vocab[i] = (char *)malloc((size_t)len + 1);
        if (!t->vocab[i]) {
            st = LM_ERR_OOM;
            goto done;
        }
        t->n = i + 1;
        if (fread(t->vocab[i], 1, (size_t)len, f) != (size_t)len) {
            st = LM_ERR_FORMAT;
            goto done;
        }
        t->vocab[i][len] = '\0';
    }
    for (int c = 0; c < 256; c++) t->single[c] = -1;
    for (int i = vocab_size - 1; i >= 0; i--) {
        const unsigned char *s = (const unsigned char *)t->vocab[i];
        if (s[0] && !s[1]) t->single[s[0]] = i;   /* descending: the first id wins */
    }
    for (int i = 0; i < vocab_size; i++) t->order[i] = i;
    g_sort_tok = t;
    qsort(t->order, (size_t)vocab_size, sizeof(int), cmp_entry);
    g_sort_tok = NULL;
done:
    if (f) fclose(f);
    if (st != LM_OK) {
        lm_tokenizer_free(t);
        t = NULL;
    }
    if (status) *status = st;
    return t;
}

int lm_tokenizer_vocab_size(const LMTokenizer *t) { return t ? t->n : LM_ERR_INVALID; }

const char *lm_tokenizer_decode(const LMTokenizer *t, int token)
{
    if (!t || token < 0 || token >= t->n) return "";
    return t->vocab[token];
}

/* The entry of string s the reference's scan would pick (highest score, then
 * lowest id), or -1. */
static int find_best(const LMTokenizer *t, const char *s)
{
    int lo = 0, hi = t->n;   /* first position whose string is >= s */
    while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (strcmp(t->vocab[t->order[mid]], s) < 0) lo = mid + 1;
        else hi = mid;
    }
    if (lo < t->n && strcmp(t->vocab[t->order[lo]], s) == 0) return t->order[lo];
    return -1;
}

int lm_tokenizer_encode(const LMTokenizer *t, const char *text, int *tokens, int max_tokens)
{
    if (!t || !tokens || max_tokens < 0) return LM_ERR_INVALID;
    if (!text || !*text || max_tokens == 0) return 0;
    const size_t len = strlen(text);
    int *ct = (int *)malloc(len * sizeof(int));
    if (!ct) return LM_ERR_OOM;
    int n = 0;
    for (const unsigned char *p = (const unsigned char *)text; *p && n < max_tokens; p++) {
        const int v = t->single[*p];
        if (v >= 0) ct[n++] = v;   /* bytes with no single-byte token are dropped */
    }
    char merged[256];
    while (n > 1) {
        float best_score = -1e10f;
        int best_idx = -1, best_tok = -1;
        for (int i = 0; i < n - 1; i++) {
            /* the reference builds the pair in a 256-byte buffer (truncating) */
            snprintf(merged, sizeof(merged), "%s%s", t->vocab[ct[i]], t->vocab[ct[i + 1]]);
            const int v = find_best(t, merged);
            if (v >= 0 && t->scores[v] > best_score) {
                best_score = t->scores[v];
                best_idx = i;
                best_tok = v;
            }
        }
        if (best_idx < 0) break;
        ct[best_idx] = best_tok;
        memmove(ct + best_idx + 1, ct + best_idx + 2, (size_t)(n - best_idx - 2) * sizeof(int));
        n--;
    }
    const int out = n < max_tokens ? n : max_tokens;
    memcpy(tokens, ct, (size_t)out * sizeof(int));
    free(ct);
    return out;
}

/* ---- random stream: the drand48 recurrence ---------------------------------
 * X' = (0x5DEECE66D * X + 0xB) mod 2^48, value X' / 2^48; seeding sets the high
 * 32 bits of X to the low 32 bits of the seed and the low 16 bits to 0x330E
 * (POSIX drand48 / srand48).  The state is explicit, so sessions do not share
 * a hidden global stream. */

void lm_rng_seed(LMRng *r, uint64_t seed)
{
    if (r) r->x = ((seed & 0xFFFFFFFFull) << 16) | 0x330Eull;
}

double lm_rng_next(LMRng *r)
{
    r->x = (0x5DEECE66Dull * r->x + 0xBull) & 0xFFFFFFFFFFFFull;
    return (double)r->x / 281474976710656.0;   /* 2^48 */
}

/* ---- loss -------------------------------------------------------------------- */

/* Mean next-token cross-entropy of S logit rows (training/forward.h:174-183):
 * for t < S-1, -(logits[t, tokens[t+1]] - max_t - log(sum_i exp(logits[t, i] -
 * max_t))), averaged over S-1; sums in the reference's order, in fp32. */
int lm_mean_ce(const float *logits, const int *tokens, int S, int V, float *loss)
{
    if (!logits || !tokens || !loss || S < 2 || V < 1) return LM_ERR_INVALID;
    for (int t = 1; t < S; t++)
        if (tokens[t] < 0 || tokens[t] >= V) return LM_ERR_RANGE;
    float total = 0.f;
    for (int t = 0; t < S - 1; t++) {
        const float *row = logits + (size_t)t * V;
        float mx = -1e9f;
        for (int i = 0; i < V; i++)
            if (row[i] > mx) mx = row[i];
        float sm = 0.f;
        for (int i = 0; i < V; i++) sm += expf(row[i] - mx);
        const float log_prob = row[tokens[t + 1]] - mx - logf(sm);
        total -= log_prob;
    }
    *loss = total / (S - 1);
    return LM_OK;
}

/* ---- samplers --------------------------------------------------------------- */

int lm_sample_argmax(const float *logits, int n)
{
    if (!logits || n < 1) return LM_ERR_INVALID;
    int best = 0;
    float best_val = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > best_val) {   /* strict: lowest index on ties */
            best_val = logits[i];
            best = i;
        }
    return best;
}

/* probs[i] = exp((l_i - max) / temp) / sum, in the reference's order */
static float *softmax_t(const float *logits, int n, float temp)
{
    float *p = (float *)malloc((size_t)n * sizeof(float));
    if (!p) return NULL;
    float maxv = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > maxv) maxv = logits[i];
    float sum = 0.f;
    for (int i = 0; i < n; i++) {
        p[i] = expf((logits[i] - maxv) / temp);
        sum += p[i];
    }
    for (int i = 0; i < n; i++) p[i] /= sum;
    return p;
}

int lm_sample_temperature(const float *logits, int n, float temp, LMRng *r)
{
    if (!logits || n < 1 || !r || !(temp > 0.f)) return LM_ERR_INVALID;
    float *p = softmax_t(logits, n, temp);
    if (!p) return LM_ERR_OOM;
    const float u = (float)lm_rng_next(r);
    float cum = 0.f;
    int out = n - 1;
    for (int i = 0; i < n; i++) {
        cum += p[i];
        if (cum >= u) {
            out = i;
            break;
        }
    }
    free(p);
    return out;
}

int lm_sample_topp(const float *logits, int n, float temp, float topp, LMRng *r)
{
    if (!logits || n < 1 || !r || !(temp > 0.f)) return LM_ERR_INVALID;
    float *p = softmax_t(logits, n, temp);
    int *idx = (int *)malloc((size_t)n * sizeof(int));
    if (!p || !idx) {
        free(p);
        free(idx);
        return LM_ERR_OOM;
    }
    for (int i = 0; i < n; i++) idx[i] = i;
    /* selection sort by probability, descending, stopped once the sorted head
     * holds topp of the mass (the reference's partial sort, swap for swap, so
     * ties come out in its order) */
    float cum = 0.f;
    for (int i = 0; i < n - 1; i++) {
        int best = i;
        for (int j = i + 1; j < n; j++)
            if (p[idx[j]] > p[idx[best]]) best = j;
        if (best != i) {
            const int tmp = idx[i];
            idx[i] = idx[best];
            idx[best] = tmp;
        }
        cum += p[idx[i]];
        if (cum >= topp) break;
    }
    /* nucleus: the shortest head of idx reaching topp */
    float c = 0.f, cutoff_sum = 0.f;
    int cutoff = 0;
    for (int i = 0; i < n; i++) {
        c += p[idx[i]];
        cutoff = i + 1;
        cutoff_sum = c;
        if (c >= topp) break;
    }
    const float u = (float)lm_rng_next(r) * cutoff_sum;
    float cs = 0.f;
    int out = idx[0];
    for (int i = 0; i < cutoff; i++) {
        cs += p[idx[i]];
        if (cs >= u) {
            out = idx[i];
            break;
        }
    }
    free(p);
    free(idx);
    return out;
}
