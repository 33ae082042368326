/*
 * generate.c — command-line greedy generator over the C ABI (stories_lm.h).
 *
 * The token loop of training/training_dynamic/generate.m:427-516 on the MI355X
 * library: start from BOS (token 1, generate.m:397), take the argmax of every
 * step's logits (sample_argmax, generate.m:129-136), stop at EOS (token 2,
 * generate.m:501), report ms/token and tok/s (generate.m:518-523).  The KV
 * cache replaces the reference's full-window recompute, so a run of n tokens
 * needs max_seq >= n instead of the 256-token sliding window.
 *
 *   stories_generate [--ckpt model.bin | --synth SEED] [--steps N]
 *                    [--first TOKEN] [--stepwise] [--print]
 *   stories_generate --ckpt model --tokenizer tokenizer.bin [--prompt TEXT]
 *                    [--temp T] [--topp P] [--seed S] [--steps N]
 *
 * --ckpt      llama2.c model file (training/model.h:78-164 layout), or with
 *             --tokenizer also a BLZT v4 checkpoint
 * --synth     seeded N(0, 0.02) fp16 Stories-110M weights (untied classifier)
 * --stepwise  one lm_forward call per token with the argmax taken on the host
 *             (the loop shape of generate.m); default: lm_generate_greedy, which
 *             keeps the argmax feedback on the device
 * --tokenizer text mode through the generation session (ane_gen.h): prompt,
 *             sampling (temperature / top-p, generate.m:488-497) and streamed
 *             text, as generate.m prints it
 */
#include "ane_gen.h"
#include "stories_lm.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static double now_ms(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

static int argmax_first(const float *v, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;   /* strict '>': lowest index on ties */
    return best;
}

static bool print_piece(const char *piece, int id, void *ctx)
{
    (void)id;
    (void)ctx;
    fputs(piece, stdout);
    fflush(stdout);
    return true;
}

static int run_text(const char *ckpt, const char *tokenizer, const char *prompt, float temp,
                    float topp, unsigned long long seed, int steps)
{
    ANETrainError err;
    ANEGenSession *g = ane_gen_create(ckpt, tokenizer, &err);
    if (!g) {
        fprintf(stderr, "ane_gen_create: %s\n", ane_train_error_str(err));
        return 1;
    }
    ANEGenConfig cfg = ane_gen_default_config();
    cfg.temperature = temp;
    cfg.top_p = topp;
    cfg.max_tokens = steps;
    cfg.seed = seed;
    if (prompt) fputs(prompt, stdout);
    ANEGenResult r = ane_gen_run(g, prompt, &cfg, print_piece, NULL);
    static const char *why[] = {"EOS", "max tokens", "callback", "error"};
    printf("\n%d tokens, %.3f ms/token, %.1f tok/s (stop: %s)\n", r.tokens_generated, r.ms_per_token,
           r.ms_per_token > 0 ? 1e3 / r.ms_per_token : 0.0, why[r.stop_reason & 3]);
    const int rc = r.stop_reason == ANE_GEN_STOP_ERROR;
    ane_gen_result_free(&r);
    ane_gen_destroy(g);
    return rc;
}

int main(int argc, char **argv)
{
    const char *ckpt = NULL, *tokenizer = NULL, *prompt = NULL;
    unsigned long long seed = 1;
    int steps = 256, first = 1, stepwise = 0, print = 0;
    float temp = 0.8f, topp = 0.9f;
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--ckpt") && i + 1 < argc) ckpt = argv[++i];
        else if (!strcmp(argv[i], "--synth") && i + 1 < argc) seed = strtoull(argv[++i], NULL, 10);
        else if (!strcmp(argv[i], "--seed") && i + 1 < argc) seed = strtoull(argv[++i], NULL, 10);
        else if (!strcmp(argv[i], "--steps") && i + 1 < argc) steps = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--first") && i + 1 < argc) first = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--tokenizer") && i + 1 < argc) tokenizer = argv[++i];
        else if (!strcmp(argv[i], "--prompt") && i + 1 < argc) prompt = argv[++i];
        else if (!strcmp(argv[i], "--temp") && i + 1 < argc) temp = (float)atof(argv[++i]);
        else if (!strcmp(argv[i], "--topp") && i + 1 < argc) topp = (float)atof(argv[++i]);
        else if (!strcmp(argv[i], "--stepwise")) stepwise = 1;
        else if (!strcmp(argv[i], "--print")) print = 1;
        else {
            fprintf(stderr, "usage: %s [--ckpt model.bin | --synth SEED] [--steps N] "
                            "[--first TOKEN] [--stepwise] [--print]\n"
                            "       %s --ckpt model --tokenizer tokenizer.bin [--prompt TEXT] "
                            "[--temp T] [--topp P] [--seed S] [--steps N]\n", argv[0], argv[0]);
            return 2;
        }
    }
    if (steps < 1) return 2;
    if (tokenizer) {
        if (!ckpt) {
            fprintf(stderr, "--tokenizer needs --ckpt\n");
            return 2;
        }
        return run_text(ckpt, tokenizer, prompt, temp, topp, seed, steps);
    }
    int rc = lm_init();
    if (rc) {
        fprintf(stderr, "lm_init: %s\n", lm_strerror(rc));
        return 1;
    }
    int st = 0;
    LMModel *m = NULL;
    if (ckpt) {
        m = lm_load_llama2c(ckpt, 1, steps, &st);
    } else {
        Config cfg = {768, 2048, 12, 12, 12, 32000, 256};
        size_t n = lm_weights_numel(&cfg, 1);
        uint16_t *w16 = (uint16_t *)malloc(n * sizeof(uint16_t));
        if (!w16) return 1;
        lm_synth_weights_f16(&cfg, seed, 0.02f, 1, w16);
        LMWeights w;
        lm_weights_view(&cfg, LM_DTYPE_F16, w16, 1, &w);
        m = lm_create(&cfg, &w, 1, steps, &st);
        free(w16);
    }
    if (!m) {
        fprintf(stderr, "model: %s\n", lm_strerror(st));
        return 1;
    }
    Config cfg;
    lm_get_config(m, &cfg);
    int *ids = (int *)malloc((size_t)steps * sizeof(int));
    if (!ids) return 1;
    double t0 = now_ms();
    if (stepwise) {
        int tok = first;
        for (int p = 0; p < steps; p++) {
            const float *lg = lm_forward(m, tok, p);
            if (!lg) {
                fprintf(stderr, "lm_forward failed at position %d\n", p);
                return 1;
            }
            tok = argmax_first(lg, cfg.vocab_size);
            ids[p] = tok;
        }
    } else {
        int pos0 = 0;
        rc = lm_generate_greedy(m, 1, &first, &pos0, steps, ids);
        if (rc) {
            fprintf(stderr, "lm_generate_greedy: %s\n", lm_strerror(rc));
            return 1;
        }
    }
    double ms = now_ms() - t0;
    int n_out = steps;
    for (int p = 0; p < steps; p++)
        if (ids[p] == 2) {   /* EOS ends the text (generate.m:501) */
            n_out = p + 1;
            break;
        }
    if (print) {
        for (int p = 0; p < n_out; p++) printf("%d%c", ids[p], p + 1 < n_out ? ' ' : '\n');
    }
    printf("%d tokens (%d before EOS) in %.2f ms: %.3f ms/token, %.1f tok/s (%s)\n", steps, n_out, ms,
           ms / steps, steps / (ms * 1e-3), stepwise ? "stepwise" : "device loop");
    free(ids);
    lm_free(m);
    return 0;
}
