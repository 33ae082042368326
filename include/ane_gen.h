/*
 * ane_gen.h — text generation session over the MI355X token loop.
 *
 * The names, types and meanings are those of the reference's generation API
 * (training/training_dynamic/ane_train.h:198-261, with the error codes of
 * ane_train.h:30-38), so a caller of that API links against
 * libstories_lm.so unchanged.  A session owns one model (batch 1, a K/V cache
 * of seq_len positions) and one tokenizer; generation runs on the GPU with the
 * reference's sampling and stopping rules (ane_train.m:1469-1612): BOS then the
 * encoded prompt, argmax below temperature 1e-6, nucleus sampling for
 * 0 < top_p < 1, plain temperature sampling otherwise, EOS (token 2) stops, and
 * a full context window drops its oldest token after BOS.
 *
 * Checkpoints: BLZT v4 (the reference's training checkpoints; the optimizer
 * state is skipped and the classifier is the embedding) or llama2.c files.
 */
#ifndef ANE_GEN_H
#define ANE_GEN_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    ANE_TRAIN_OK = 0,
    ANE_TRAIN_ERR_ANE = 1,          /* device: no gfx950 GPU, or a HIP failure */
    ANE_TRAIN_ERR_COMPILE = 2,      /* model shape the kernels do not support   */
    ANE_TRAIN_ERR_MEMORY = 3,
    ANE_TRAIN_ERR_CONFIG = 4,
    ANE_TRAIN_ERR_CHECKPOINT = 5,
    ANE_TRAIN_ERR_DATA = 6,         /* tokenizer file                           */
} ANETrainError;

/* Static text for an error code. */
const char *ane_train_error_str(ANETrainError err);

typedef struct {
    float temperature;   /* default 0.8; below 1e-6 greedy (argmax) */
    float top_p;         /* default 0.9; nucleus sampling when in (0, 1) */
    int max_tokens;      /* default 256 */
    uint64_t seed;       /* 0: seeded from the clock */
} ANEGenConfig;

ANEGenConfig ane_gen_default_config(void);

/* Called with each generated token's text and id; returning false stops. */
typedef bool (*ANEGenTokenFn)(const char *token, int token_id, void *ctx);

typedef enum {
    ANE_GEN_STOP_EOS = 0,
    ANE_GEN_STOP_MAX = 1,
    ANE_GEN_STOP_CALLBACK = 2,
    ANE_GEN_STOP_ERROR = 3,
} ANEGenStopReason;

typedef struct {
    char *text;                    /* prompt pieces + generated pieces; free with ane_gen_result_free */
    int tokens_generated;
    double total_ms;
    double ms_per_token;
    ANEGenStopReason stop_reason;
} ANEGenResult;

typedef struct ANEGenSession ANEGenSession;

/* NULL on failure with *err set (when err != NULL). */
ANEGenSession *ane_gen_create(const char *checkpoint_path, const char *tokenizer_path,
                              ANETrainError *err);

ANEGenResult ane_gen_run(ANEGenSession *g, const char *prompt, const ANEGenConfig *cfg,
                         ANEGenTokenFn on_token, void *ctx);

void ane_gen_result_free(ANEGenResult *r);

void ane_gen_destroy(ANEGenSession *g);

#ifdef __cplusplus
}
#endif

#endif /* ANE_GEN_H */
