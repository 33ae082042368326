/*
 * host_sanitize.c — the product's host-only C code (weight files, fp16
 * conversion, RoPE table, tokenizer, samplers, mean loss) and the CPU oracle,
 * driven under AddressSanitizer and UndefinedBehaviorSanitizer by
 * tests/test_host_sanitize.py (which builds this file with the sources and
 * writes the input files).  No device code is involved.
 *
 * Usage: host_sanitize <dir>
 *   every <dir>/<name>.llama2c is read with lmh_read_llama2c, every
 *   <dir>/<name>.blzt with lmh_read_blzt, every <dir>/<name>.<V>.tok loaded as
 *   a tokenizer of V entries (then every id decoded and a set of strings
 *   encoded); one line "<file> <status>" per file, then the built-in checks
 *   (exit status 1 on a failed check; a sanitizer report aborts the run).
 */
#define _DEFAULT_SOURCE
#include <dirent.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lm_internal.h"
#include "oracle.h"

static int failures;

#define CHECK(cond, ...)                         \
    do {                                         \
        if (!(cond)) {                           \
            fprintf(stderr, "FAIL: " __VA_ARGS__); \
            fputc('\n', stderr);                 \
            failures++;                          \
        }                                        \
    } while (0)

static int ends_with(const char *s, const char *suffix)
{
    size_t n = strlen(s), m = strlen(suffix);
    return n >= m && strcmp(s + n - m, suffix) == 0;
}

static size_t config_numel(const Config *c, int untied)
{
    size_t sz[LMH_NTENSORS], n = 0;
    lmh_tensor_sizes(c, untied, sz);
    for (int t = 0; t < LMH_NTENSORS; t++) n += sz[t];
    return n;
}

static void read_files(const char *dir)
{
    DIR *d = opendir(dir);
    if (!d) {
        fprintf(stderr, "cannot open %s\n", dir);
        exit(2);
    }
    struct dirent *e;
    char path[4096];
    while ((e = readdir(d))) {
        snprintf(path, sizeof path, "%s/%s", dir, e->d_name);
        if (ends_with(e->d_name, ".llama2c")) {
            Config c;
            int untied = 0;
            float *w = NULL;
            const int rc = lmh_read_llama2c(path, &c, &untied, &w);
            if (rc == LM_OK) {
                const size_t n = config_numel(&c, untied);
                double s = 0;
                for (size_t i = 0; i < n; i++) s += w[i];   /* every element readable */
                CHECK(isfinite(s), "%s: non-finite weights", e->d_name);
            } else {
                CHECK(w == NULL, "%s: failed read left a buffer", e->d_name);
            }
            free(w);
            printf("%s %d\n", e->d_name, rc);
        } else if (ends_with(e->d_name, ".blzt")) {
            Config c;
            float *w = NULL;
            const int rc = lmh_read_blzt(path, &c, &w);
            if (rc == LM_OK) {
                const size_t n = config_numel(&c, 0);
                double s = 0;
                for (size_t i = 0; i < n; i++) s += w[i];
                CHECK(isfinite(s), "%s: non-finite weights", e->d_name);
            }
            free(w);
            printf("%s %d\n", e->d_name, rc);
        } else if (ends_with(e->d_name, ".tok")) {
            /* <name>.<V>.tok */
            char name[256];
            snprintf(name, sizeof name, "%s", e->d_name);
            name[strlen(name) - 4] = 0;
            const char *dot = strrchr(name, '.');
            const int V = dot ? atoi(dot + 1) : 0;
            int st = 0;
            LMTokenizer *t = lm_tokenizer_load(path, V, &st);
            if (t) {
                CHECK(lm_tokenizer_vocab_size(t) == V, "%s: vocab size", e->d_name);
                size_t total = 0;
                for (int i = -1; i <= V; i++) {   /* out-of-range ids included */
                    const char *p = lm_tokenizer_decode(t, i);
                    if (p) total += strlen(p);
                }
                static const char *texts[] = {"", "a", "abcabc ab", " ca bc", "\xff\xfe\x01",
                                              "a longer text with spaces and repeated words words"};
                int toks[256];
                for (size_t k = 0; k < sizeof texts / sizeof *texts; k++) {
                    for (int cap = 0; cap <= 64; cap += 8) {
                        const int n = lm_tokenizer_encode(t, texts[k], toks, cap);
                        CHECK(n <= cap, "%s: encode wrote %d ids into %d", e->d_name, n, cap);
                        for (int i = 0; i < n; i++)
                            CHECK(toks[i] >= 0 && toks[i] < V, "%s: id %d", e->d_name, toks[i]);
                    }
                }
                (void)total;
                lm_tokenizer_free(t);
            }
            printf("%s %d\n", e->d_name, t ? LM_OK : st);
        }
    }
    closedir(d);
}

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static double urand(void)
{
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (double)(rng_state >> 11) / 9007199254740992.0;
}

static void check_fp16(void)
{
    for (uint32_t h = 0; h < 65536; h++) {
        const float f = lmh_f16_to_f32((uint16_t)h);
        const uint16_t back = lmh_f32_to_f16(f);
        if (isnan(f)) CHECK(isnan(lmh_f16_to_f32(back)), "fp16 NaN %04x", h);
        else CHECK(back == h, "fp16 round trip %04x -> %04x", h, back);
    }
    float src[1024];
    uint16_t hv[1024];
    float out[1024];
    for (int i = 0; i < 1024; i++) src[i] = (float)((urand() - 0.5) * pow(2.0, 40.0 * urand() - 20.0));
    src[0] = INFINITY; src[1] = -INFINITY; src[2] = NAN; src[3] = 65520.f; src[4] = 1e-8f;
    lm_f32_to_f16(src, hv, 1024);
    lm_f16_to_f32(hv, out, 1024);
    for (int i = 5; i < 1024; i++)
        CHECK(fabsf(out[i] - src[i]) <= fmaxf(fabsf(src[i]) * 1e-3f, 6e-8f) || fabsf(src[i]) > 65504.f,
              "fp16 conversion of %g gave %g", src[i], out[i]);
}

static void check_weights_round_trip(const char *dir)
{
    static const int shapes[][7] = {{256, 512, 2, 4, 4, -512, 64}, {512, 1024, 1, 4, 2, 700, 32}};
    for (int s = 0; s < 2; s++) {
        Config c = {shapes[s][0], shapes[s][1], shapes[s][2], shapes[s][3], shapes[s][4], shapes[s][5],
                    shapes[s][6]};
        const int untied = c.vocab_size < 0;
        c.vocab_size = abs(c.vocab_size);
        const size_t n = lm_weights_numel(&c, untied);
        uint16_t *w16 = malloc(n * 2);
        CHECK(lm_synth_weights_f16(&c, 7 + s, 0.02f, untied, w16) == LM_OK, "synth");
        LMWeights w;
        CHECK(lm_weights_view(&c, LM_DTYPE_F16, w16, untied, &w) == LM_OK, "view");
        char path[4096];
        snprintf(path, sizeof path, "%s/roundtrip%d.bin", dir, s);
        Config cw = c;
        if (untied) cw.vocab_size = -c.vocab_size;
        CHECK(lm_write_llama2c(path, &cw, &w) == LM_OK, "write");
        Config cr;
        int ur = -1;
        float *r = NULL;
        CHECK(lmh_read_llama2c(path, &cr, &ur, &r) == LM_OK, "read back");
        CHECK(ur == untied && cr.dim == c.dim && cr.n_layers == c.n_layers, "header back");
        if (r) {
            float *f = malloc(n * 4);
            lm_f16_to_f32(w16, f, n);
            CHECK(memcmp(f, r, n * 4) == 0, "weights back (shape %d)", s);
            free(f);
        }
        free(r);
        free(w16);
        remove(path);
    }
    const Config bad[] = {{0, 512, 2, 4, 4, 512, 64}, {256, 512, 2, 3, 3, 512, 64},
                          {256, 512, 2, 4, 3, 512, 64}, {256, -1, 2, 4, 4, 512, 64},
                          {256, 512, 2, 4, 4, 0, 64}};
    for (size_t i = 0; i < sizeof bad / sizeof *bad; i++)
        CHECK(lmh_check_config(&bad[i]) != LM_OK, "bad config %zu accepted", i);
}

static void check_samplers(void)
{
    LMRng r;
    lm_rng_seed(&r, 42);
    static float lg[32000];
    const int sizes[] = {1, 2, 7, 512, 32000};
    const float temps[] = {1e-3f, 0.5f, 1.0f, 3.0f};
    const float topps[] = {0.f, 0.1f, 0.9f, 1.0f};
    for (size_t a = 0; a < sizeof sizes / sizeof *sizes; a++) {
        const int n = sizes[a];
        for (int i = 0; i < n; i++) lg[i] = (float)(urand() * 8.0 - 4.0);
        if (n > 4) lg[3] = lg[1];   /* a tie */
        const int am = lm_sample_argmax(lg, n);
        CHECK(am >= 0 && am < n, "argmax");
        for (size_t b = 0; b < sizeof temps / sizeof *temps; b++) {
            const int t = lm_sample_temperature(lg, n, temps[b], &r);
            CHECK(t >= 0 && t < n, "temperature sample %d of %d", t, n);
            for (size_t c = 0; c < sizeof topps / sizeof *topps; c++) {
                const int p = lm_sample_topp(lg, n, temps[b], topps[c], &r);
                CHECK(p >= 0 && p < n, "top-p sample %d of %d", p, n);
            }
        }
    }
    int toks[64];
    for (int i = 0; i < 64; i++) toks[i] = (int)(urand() * 512);
    float *logits = malloc(64 * 512 * 4), loss = 0.f;
    for (int i = 0; i < 64 * 512; i++) logits[i] = (float)(urand() * 6.0 - 3.0);
    CHECK(lm_mean_ce(logits, toks, 64, 512, &loss) == LM_OK && isfinite(loss) && loss > 0.f, "mean CE");
    CHECK(lm_mean_ce(logits, toks, 1, 512, &loss) != LM_OK || isfinite(loss), "mean CE of one row");
    free(logits);
}

static void check_rope(void)
{
    const int S = 640, hd = 128;
    float *c = malloc((size_t)S * hd / 2 * 4), *s = malloc((size_t)S * hd / 2 * 4);
    CHECK(lm_rope_table(S, hd, c, s) == LM_OK, "rope table");
    for (int i = 0; i < S * hd / 2; i++)
        CHECK(fabsf(c[i] * c[i] + s[i] * s[i] - 1.f) < 1e-5f, "rope entry %d not a rotation", i);
    CHECK(lm_rope_table(S, 3, c, s) != LM_OK, "odd head dim accepted");
    free(c);
    free(s);
}

static void check_oracle(void)
{
    const int cfg[7] = {256, 512, 2, 4, 2, 300, 48};
    Config c = {256, 512, 2, 4, 2, 300, 48};
    const size_t n = lm_weights_numel(&c, 1);
    uint16_t *w16 = malloc(n * 2);
    float *w = malloc(n * 4);
    lm_synth_weights_f16(&c, 3, 0.02f, 1, w16);
    lm_f16_to_f32(w16, w, n);
    OracleModel *o = oracle_create(cfg, w, 1, 48, 1);
    CHECK(o != NULL, "oracle_create");
    int toks[20];
    for (int i = 0; i < 20; i++) toks[i] = (int)(urand() * 300);
    float *full = malloc(20 * 300 * 4), *row = malloc(300 * 4);
    CHECK(oracle_forward_full(o, toks, 20, full) == 0, "oracle full forward");
    OracleModel *o2 = oracle_create(cfg, w, 1, 48, 1);
    for (int p = 0; p < 20; p++) {
        CHECK(oracle_decode_step(o2, toks[p], p, row) == 0, "oracle decode step");
        CHECK(memcmp(row, full + (size_t)p * 300, 300 * 4) == 0, "decode step %d != full row", p);
    }
    CHECK(isfinite(oracle_loss(full, toks, 20, 300)), "oracle loss");
    oracle_free(o);
    oracle_free(o2);
    free(full);
    free(row);
    free(w);
    free(w16);
}

int main(int argc, char **argv)
{
    if (argc != 2) {
        fprintf(stderr, "usage: %s <dir>\n", argv[0]);
        return 2;
    }
    read_files(argv[1]);
    check_fp16();
    check_weights_round_trip(argv[1]);
    check_samplers();
    check_rope();
    check_oracle();
    printf("checks failed: %d\n", failures);
    return failures ? 1 : 0;
}
