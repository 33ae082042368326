/*
 * lm_gen.c — the generation session of ane_gen.h over the C ABI of
 * stories_lm.h (C11, host).
 *
 * ane_gen_run follows the reference's loop (training/training_dynamic/
 * ane_train.m:1469-1612) token for token: context = BOS + the encoded prompt
 * (at most seq_len - 2 tokens), the text starts with the prompt's pieces,
 * every step samples the logits of the last context position, EOS (2) stops
 * without being appended, a full window drops the token after BOS, the
 * callback may stop the run.  The reference recomputes the whole window each
 * step; here the K/V cache carries it, so a step is one lm_forward, except
 * after a window shift (every position moves), where the window is prefilled
 * again.  Both give the logits of the same causal forward.
 *
 * Arithmetic: the first window (BOS + prompt) goes through lm_forward one
 * position at a time, the fp32 decode chain whose logits follow the
 * reference's fp32 forward to summation order, so the ids match the
 * reference's until the first window shift.  A shift re-prefills the
 * seq_len - 1 positions of the window through the fp16 MFMA prefill (logits within atol 2e-2
 * + rtol 1e-2 of the reference): from there on an id can differ from the
 * reference's only where two logits are that close.
 */
#define _POSIX_C_SOURCE 200809L
#include "ane_gen.h"
#include "stories_lm.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define BOS 1
#define EOS 2

struct ANEGenSession {
    LMModel *m;
    LMTokenizer *tok;
    Config cfg;
    int seq;          /* context window (the model's seq_len) */
    int *context;     /* [seq] */
    float *logits;    /* [V] */
};

const char *ane_train_error_str(ANETrainError err)
{
    switch (err) {
    case ANE_TRAIN_OK: return "ok";
    case ANE_TRAIN_ERR_ANE: return "GPU device error (no gfx950 device, or a HIP failure)";
    case ANE_TRAIN_ERR_COMPILE: return "model shape not supported by the kernels";
    case ANE_TRAIN_ERR_MEMORY: return "out of memory";
    case ANE_TRAIN_ERR_CONFIG: return "invalid configuration";
    case ANE_TRAIN_ERR_CHECKPOINT: return "checkpoint load failure";
    case ANE_TRAIN_ERR_DATA: return "tokenizer load failure";
    default: return "unknown error";
    }
}

ANEGenConfig ane_gen_default_config(void)
{
    ANEGenConfig c;
    c.temperature = 0.8f;
    c.top_p = 0.9f;
    c.max_tokens = 256;
    c.seed = 0;
    return c;
}

static ANETrainError map_status(int st)
{
    switch (st) {
    case LM_ERR_NO_DEVICE:
    case LM_ERR_NOT_GFX950:
    case LM_ERR_HIP:
    case LM_ERR_NOT_INIT: return ANE_TRAIN_ERR_ANE;
    case LM_ERR_OOM: return ANE_TRAIN_ERR_MEMORY;
    case LM_ERR_UNSUPPORTED: return ANE_TRAIN_ERR_COMPILE;
    case LM_ERR_INVALID:
    case LM_ERR_RANGE: return ANE_TRAIN_ERR_CONFIG;
    default: return ANE_TRAIN_ERR_CHECKPOINT;
    }
}

/* The checkpoint's format and context window: BLZT files start with the
 * magic 'BLZT' (int32) and hold seq_len as their tenth int32; llama2.c files
 * start with a Config (seq_len its seventh int32).  0 when unreadable. */
static int peek_window(const char *path, int *blzt)
{
    FILE *f = fopen(path, "rb");
    if (!f) return 0;
    int32_t h[10];
    const size_t n = fread(h, sizeof(int32_t), 10, f);
    fclose(f);
    *blzt = n >= 1 && h[0] == 0x424C5A54;
    if (*blzt) return n == 10 ? h[9] : 0;
    return n >= 7 ? h[6] : 0;
}

void ane_gen_destroy(ANEGenSession *g)
{
    if (!g) return;
    lm_free(g->m);
    lm_tokenizer_free(g->tok);
    free(g->context);
    free(g->logits);
    free(g);
}

ANEGenSession *ane_gen_create(const char *checkpoint_path, const char *tokenizer_path,
                              ANETrainError *err)
{
    ANETrainError e = ANE_TRAIN_OK;
    ANEGenSession *g = NULL;
    int st = 0;
    if (!checkpoint_path || !tokenizer_path) {
        e = ANE_TRAIN_ERR_CONFIG;
        goto fail;
    }
    if ((st = lm_init()) != LM_OK) {
        e = ANE_TRAIN_ERR_ANE;
        goto fail;
    }
    g = (ANEGenSession *)calloc(1, sizeof(ANEGenSession));
    if (!g) {
        e = ANE_TRAIN_ERR_MEMORY;
        goto fail;
    }
    /* one batch slot with the checkpoint's window as cache length */
    int blzt = 0;
    const int window = peek_window(checkpoint_path, &blzt);
    if (window < 2) {
        e = ANE_TRAIN_ERR_CHECKPOINT;
        goto fail;
    }
    g->m = blzt ? lm_load_blzt(checkpoint_path, 1, window, &st)
                : lm_load_llama2c(checkpoint_path, 1, window, &st);
    if (!g->m) {
        e = map_status(st);
        goto fail;
    }
    lm_get_config(g->m, &g->cfg);
    g->seq = window;
    /* the reference forward keeps K and V in fp32 (forward.h:118-128) */
    if ((st = lm_set_option(g->m, LM_OPT_KV_F32, 1)) != LM_OK) {
        e = map_status(st);
        goto fail;
    }
    const int V = g->cfg.vocab_size < 0 ? -g->cfg.vocab_size : g->cfg.vocab_size;
    g->tok = lm_tokenizer_load(tokenizer_path, V, &st);
    if (!g->tok) {
        e = st == LM_ERR_OOM ? ANE_TRAIN_ERR_MEMORY : ANE_TRAIN_ERR_DATA;
        goto fail;
    }
    g->context = (int *)calloc((size_t)g->seq, sizeof(int));
    g->logits = (float *)malloc((size_t)V * sizeof(float));
    if (!g->context || !g->logits) {
        e = ANE_TRAIN_ERR_MEMORY;
        goto fail;
    }
    if (err) *err = ANE_TRAIN_OK;
    return g;
fail:
    ane_gen_destroy(g);
    if (err) *err = e;
    return NULL;
}

static double now_ms(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

typedef struct {
    char *p;
    size_t len, cap;
} Text;

static int text_add(Text *t, const char *piece)
{
    const size_t n = strlen(piece);
    if (t->len + n + 1 > t->cap) {
        size_t cap = t->cap ? t->cap : 4096;
        while (t->len + n + 1 > cap) cap *= 2;
        char *q = (char *)realloc(t->p, cap);
        if (!q) return -1;
        t->p = q;
        t->cap = cap;
    }
    memcpy(t->p + t->len, piece, n);
    t->len += n;
    t->p[t->len] = '\0';
    return 0;
}

/* Logits of the last of the ctx_len context tokens with the window cached in
 * slot 0 (positions 0 .. ctx_len-1): step by step through the fp32 decode
 * chain (exact), or as one MFMA prefill of the window. */
static int window_logits(ANEGenSession *g, int ctx_len, int exact)
{
    const int V = g->cfg.vocab_size < 0 ? -g->cfg.vocab_size : g->cfg.vocab_size;
    if (exact) {
        const float *lg = NULL;
        for (int p = 0; p < ctx_len; p++)
            if (!(lg = lm_forward(g->m, g->context[p], p))) return LM_ERR_HIP;
        memcpy(g->logits, lg, (size_t)V * sizeof(float));
        return LM_OK;
    }
    const int slot = 0;
    return lm_prefill_batch(g->m, 1, &slot, g->context, ctx_len, LM_LOGITS_LAST, g->logits);
}

ANEGenResult ane_gen_run(ANEGenSession *g, const char *prompt, const ANEGenConfig *cfg,
                         ANEGenTokenFn on_token, void *ctx)
{
    ANEGenResult result;
    memset(&result, 0, sizeof(result));
    if (!g) {
        result.stop_reason = ANE_GEN_STOP_ERROR;
        return result;
    }
    const float temperature = cfg ? cfg->temperature : 0.8f;
    const float topp = cfg ? cfg->top_p : 0.9f;
    const int max_tokens = cfg ? cfg->max_tokens : 256;
    const uint64_t seed = cfg ? cfg->seed : 0;
    const int V = g->cfg.vocab_size < 0 ? -g->cfg.vocab_size : g->cfg.vocab_size;
    const int SEQ = g->seq;
    LMRng rng;
    lm_rng_seed(&rng, seed ? seed : (uint64_t)time(NULL));

    int ctx_len = 0;
    g->context[ctx_len++] = BOS;
    if (prompt) {
        int *pt = (int *)malloc((size_t)SEQ * sizeof(int));
        if (!pt) {
            result.stop_reason = ANE_GEN_STOP_ERROR;
            return result;
        }
        const int n = lm_tokenizer_encode(g->tok, prompt, pt, SEQ - 2);
        for (int i = 0; i < n && ctx_len < SEQ; i++) g->context[ctx_len++] = pt[i];
        free(pt);
    }
    Text text = {NULL, 0, 0};
    if (text_add(&text, "")) {
        result.stop_reason = ANE_GEN_STOP_ERROR;
        return result;
    }
    for (int i = 1; i < ctx_len; i++)
        if (text_add(&text, lm_tokenizer_decode(g->tok, g->context[i]))) goto oom;

    const double t0 = now_ms();
    int generated = 0;
    int stale = 1;   /* the cache does not hold the current window */
    int shifted = 0; /* a window shift has happened */
    for (int gen = 0; gen < max_tokens; gen++) {
        if (stale) {
            if (window_logits(g, ctx_len, !shifted) != LM_OK) {
                result.stop_reason = ANE_GEN_STOP_ERROR;
                break;
            }
            stale = 0;
        }
        int next;
        if (temperature < 1e-6f) next = lm_sample_argmax(g->logits, V);
        else if (topp > 0.0f && topp < 1.0f) next = lm_sample_topp(g->logits, V, temperature, topp, &rng);
        else next = lm_sample_temperature(g->logits, V, temperature, &rng);
        if (next < 0) {
            result.stop_reason = ANE_GEN_STOP_ERROR;
            break;
        }
        if (next == EOS) {
            result.stop_reason = ANE_GEN_STOP_EOS;
            break;
        }
        if (ctx_len >= SEQ) {   /* drop the oldest token after BOS */
            memmove(g->context + 1, g->context + 2, (size_t)(SEQ - 2) * sizeof(int));
            ctx_len = SEQ - 1;
            stale = 1;
            shifted = 1;
        }
        g->context[ctx_len++] = next;
        generated++;
        const char *piece = lm_tokenizer_decode(g->tok, next);
        if (text_add(&text, piece)) goto oom;
        if (on_token && !on_token(piece, next, ctx)) {
            result.stop_reason = ANE_GEN_STOP_CALLBACK;
            generated++;   /* counted twice, as the reference does (ane_train.m:1590) */
            break;
        }
        if (gen == max_tokens - 1) {
            result.stop_reason = ANE_GEN_STOP_MAX;
            break;
        }
        if (!stale) {   /* the cache holds positions 0 .. ctx_len-2: one step */
            const float *lg = lm_forward(g->m, next, ctx_len - 1);
            if (!lg) {
                result.stop_reason = ANE_GEN_STOP_ERROR;
                break;
            }
            memcpy(g->logits, lg, (size_t)V * sizeof(float));
        }
    }
    const double ms = now_ms() - t0;
    result.text = text.p;
    result.tokens_generated = generated;
    result.total_ms = ms;
    result.ms_per_token = generated > 0 ? ms / generated : 0.0;
    return result;
oom:
    free(text.p);
    memset(&result, 0, sizeof(result));
    result.stop_reason = ANE_GEN_STOP_ERROR;
    return result;
}

void ane_gen_result_free(ANEGenResult *r)
{
    if (r && r->text) {
        free(r->text);
        r->text = NULL;
    }
}
