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
 *
 * --ckpt     llama2.c model file (training/model.h:78-164 layout)
 * --synth    seeded N(0, 0.02) fp16 Stories-110M weights (untied classifier)
 * --stepwise one lm_forward call per token with the argmax taken on the host
 *            (the loop shape of generate.m); default: lm_generate_greedy, which
 *            keeps the argmax feedback on the device
 */
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

int main(int argc, char **argv)
{
    const char *ckpt = NULL;
    unsigned long long seed = 1;
    int steps = 256, first = 1, stepwise = 0, print = 0;
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--ckpt") && i + 1 < argc) ckpt = argv[++i];
        else if (!strcmp(argv[i], "--synth") && i + 1 < argc) seed = strtoull(argv[++i], NULL, 10);
        else if (!strcmp(argv[i], "--steps") && i + 1 < argc) steps = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--first") && i + 1 < argc) first = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--stepwise")) stepwise = 1;
        else if (!strcmp(argv[i], "--print")) print = 1;
        else {
            fprintf(stderr, "usage: %s [--ckpt model.bin | --synth SEED] [--steps N] "
                            "[--first TOKEN] [--stepwise] [--print]\n", argv[0]);
            return 2;
        }
    }
    if (steps < 1) return 2;
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
