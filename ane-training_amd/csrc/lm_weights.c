/*
 * lm_weights.c — host-side weight utilities of the Stories C ABI (plain C99).
 *
 *  - IEEE binary16 <-> binary32 conversion with round-to-nearest-even, the
 *    rounding of the reference's fp16 path (cvt_f32_f16,
 *    training/training_dynamic/io.h:33-50; ane_weight_fp16, libane/ane.m:592-607).
 *  - The llama2.c weight layout: tensor order of model_load_weights
 *    (training/model.h:78-164), negative vocab_size = untied classifier
 *    (model.h:85-86,155-160).  K/V sizes use n_kv_heads*head_dim rows, which is
 *    model.h's dim*dim when n_kv_heads == n_heads.
 *  - Seeded synthetic weights (SplitMix64 counters -> Box-Muller -> fp16).
 *  - The fp32 RoPE table with the expressions of training/forward.h:58-61.
 */
#include "lm_internal.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* binary16 <-> binary32                                                      */
/* ------------------------------------------------------------------------- */

uint16_t lmh_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf / nan */
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                        /* below 2^-14: half subnormal */
        uint32_t e = ax >> 23;
        if (e < 102u) return (uint16_t)sign;       /* < 2^-25 rounds to zero */
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                 /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - 0x38000000u;                 /* rebias 127 -> 15 */
    r += 0xFFFu + ((r >> 13) & 1u);                /* round to nearest, ties even */
    return (uint16_t)(sign | (r >> 13));
}

float lmh_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            e = 113;
            while (!(m & 0x400u)) { m <<= 1; e--; }
            bits = sign | (e << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void lm_f32_to_f16(const float *src, uint16_t *dst, size_t n)
{
    if (!src || !dst) return;
    #pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; i++) dst[i] = lmh_f32_to_f16(src[i]);
}

void lm_f16_to_f32(const uint16_t *src, float *dst, size_t n)
{
    if (!src || !dst) return;
    #pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; i++) dst[i] = lmh_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------- */
/* llama2.c layout                                                            */
/* ------------------------------------------------------------------------- */

int lmh_check_config(const Config *c)
{
    if (!c) return LM_ERR_INVALID;
    int V = c->vocab_size < 0 ? -c->vocab_size : c->vocab_size;
    if (c->dim <= 0 || c->hidden_dim <= 0 || c->n_layers <= 0 || c->n_heads <= 0 ||
        c->n_kv_heads <= 0 || V <= 0)
        return LM_ERR_FORMAT;
    if (c->dim % c->n_heads) return LM_ERR_FORMAT;
    if (c->n_kv_heads > c->n_heads || c->n_heads % c->n_kv_heads) return LM_ERR_FORMAT;
    if (c->dim > (1 << 16) || c->hidden_dim > (1 << 18) || c->n_layers > 4096 ||
        V > (1 << 24))
        return LM_ERR_FORMAT;
    return LM_OK;
}

void lmh_tensor_sizes(const Config *c, int untied, size_t sz[LMH_NTENSORS])
{
    size_t D = (size_t)c->dim, F = (size_t)c->hidden_dim, L = (size_t)c->n_layers;
    size_t V = (size_t)(c->vocab_size < 0 ? -c->vocab_size : c->vocab_size);
    size_t hd = D / (size_t)c->n_heads;
    size_t NQ = (size_t)c->n_heads * hd, NKV = (size_t)c->n_kv_heads * hd;
    sz[LMH_T_EMBED] = V * D;
    sz[LMH_T_RMS_ATT] = L * D;
    sz[LMH_T_WQ] = L * NQ * D;
    sz[LMH_T_WK] = L * NKV * D;
    sz[LMH_T_WV] = L * NKV * D;
    sz[LMH_T_WO] = L * D * NQ;
    sz[LMH_T_RMS_FFN] = L * D;
    sz[LMH_T_W1] = L * F * D;
    sz[LMH_T_W2] = L * D * F;
    sz[LMH_T_W3] = L * F * D;
    sz[LMH_T_RMS_FINAL] = D;
    sz[LMH_T_WCLS] = untied ? V * D : 0;
}

size_t lm_weights_numel(const Config *cfg, int untied)
{
    if (lmh_check_config(cfg) != LM_OK) return 0;
    size_t sz[LMH_NTENSORS], n = 0;
    lmh_tensor_sizes(cfg, untied, sz);
    for (int t = 0; t < LMH_NTENSORS; t++) n += sz[t];
    return n;
}

int lm_weights_view(const Config *cfg, LMDType dtype, const void *base, int untied,
                    LMWeights *out)
{
    if (!cfg || !base || !out) return LM_ERR_INVALID;
    if (dtype != LM_DTYPE_F32 && dtype != LM_DTYPE_F16) return LM_ERR_INVALID;
    int rc = lmh_check_config(cfg);
    if (rc) return rc;
    size_t sz[LMH_NTENSORS];
    lmh_tensor_sizes(cfg, untied, sz);
    size_t es = dtype == LM_DTYPE_F32 ? 4 : 2;
    const char *p = (const char *)base;
    const void *ptr[LMH_NTENSORS];
    for (int t = 0; t < LMH_NTENSORS; t++) {
        ptr[t] = p;
        p += sz[t] * es;
    }
    out->dtype = dtype;
    out->token_embedding = ptr[LMH_T_EMBED];
    out->rms_att_w = ptr[LMH_T_RMS_ATT];
    out->wq = ptr[LMH_T_WQ];
    out->wk = ptr[LMH_T_WK];
    out->wv = ptr[LMH_T_WV];
    out->wo = ptr[LMH_T_WO];
    out->rms_ffn_w = ptr[LMH_T_RMS_FFN];
    out->w1 = ptr[LMH_T_W1];
    out->w2 = ptr[LMH_T_W2];
    out->w3 = ptr[LMH_T_W3];
    out->rms_final_w = ptr[LMH_T_RMS_FINAL];
    out->wcls = untied ? ptr[LMH_T_WCLS] : NULL;
    return LM_OK;
}

const void *lmh_weights_ptr(const LMWeights *w, int t)
{
    switch (t) {
    case LMH_T_EMBED: return w->token_embedding;
    case LMH_T_RMS_ATT: return w->rms_att_w;
    case LMH_T_WQ: return w->wq;
    case LMH_T_WK: return w->wk;
    case LMH_T_WV: return w->wv;
    case LMH_T_WO: return w->wo;
    case LMH_T_RMS_FFN: return w->rms_ffn_w;
    case LMH_T_W1: return w->w1;
    case LMH_T_W2: return w->w2;
    case LMH_T_W3: return w->w3;
    case LMH_T_RMS_FINAL: return w->rms_final_w;
    case LMH_T_WCLS: return w->wcls;
    default: return NULL;
    }
}

int lmh_weights_untied(const LMWeights *w)
{
    return w->wcls != NULL && w->wcls != w->token_embedding;
}

/* ------------------------------------------------------------------------- */
/* Seeded synthetic weights                                                   */
/* ------------------------------------------------------------------------- */

static inline uint64_t splitmix64_mix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

#define SM_GAMMA 0x9E3779B97F4A7C15ull

/* Standard normal number `i` of stream `base` (Box-Muller, cosine branch). */
static inline double synth_normal(uint64_t base, uint64_t i)
{
    uint64_t a = splitmix64_mix(base + (2 * i + 1) * SM_GAMMA);
    uint64_t b = splitmix64_mix(base + (2 * i + 2) * SM_GAMMA);
    double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;   /* (0, 1] */
    double u2 = (double)(b >> 11) * 0x1.0p-53;         /* [0, 1) */
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

int lm_synth_weights_f16(const Config *cfg, uint64_t seed, float std, int untied,
                         uint16_t *out)
{
    if (!cfg || !out) return LM_ERR_INVALID;
    int rc = lmh_check_config(cfg);
    if (rc) return rc;
    size_t sz[LMH_NTENSORS];
    lmh_tensor_sizes(cfg, untied, sz);
    uint16_t *p = out;
    const uint16_t one = lmh_f32_to_f16(1.0f);
    for (int t = 0; t < LMH_NTENSORS; t++) {
        size_t n = sz[t];
        int is_norm = (t == LMH_T_RMS_ATT || t == LMH_T_RMS_FFN || t == LMH_T_RMS_FINAL);
        if (is_norm) {
            for (size_t i = 0; i < n; i++) p[i] = one;
        } else {
            uint64_t base = splitmix64_mix(seed ^ (0xD1B54A32D192ED03ull * (uint64_t)(t + 1)));
            #pragma omp parallel for schedule(static)
            for (size_t i = 0; i < n; i++) {
                float v = (float)((double)std * synth_normal(base, (uint64_t)i));
                p[i] = lmh_f32_to_f16(v);
            }
        }
        p += n;
    }
    return LM_OK;
}

/* ------------------------------------------------------------------------- */
/* llama2.c file I/O                                                          */
/* ------------------------------------------------------------------------- */

int lm_write_llama2c(const char *path, const Config *cfg, const LMWeights *w)
{
    if (!path || !cfg || !w) return LM_ERR_INVALID;
    int rc = lmh_check_config(cfg);
    if (rc) return rc;
    int untied = lmh_weights_untied(w);
    Config hdr = *cfg;
    int V = cfg->vocab_size < 0 ? -cfg->vocab_size : cfg->vocab_size;
    hdr.vocab_size = untied ? -V : V;
    FILE *f = fopen(path, "wb");
    if (!f) {
        fprintf(stderr, "lm_write_llama2c: cannot open %s\n", path);
        return LM_ERR_IO;
    }
    size_t sz[LMH_NTENSORS];
    lmh_tensor_sizes(cfg, untied, sz);
    int ok = fwrite(&hdr, sizeof(Config), 1, f) == 1;
    const size_t CH = 1u << 20;
    float *tmp = ok ? (float *)malloc(CH * sizeof(float)) : NULL;
    if (!tmp) ok = 0;
    for (int t = 0; t < LMH_NTENSORS && ok; t++) {
        const void *src = lmh_weights_ptr(w, t);
        if (sz[t] == 0) continue;
        if (!src) { ok = 0; break; }
        for (size_t off = 0; off < sz[t] && ok; off += CH) {
            size_t n = sz[t] - off < CH ? sz[t] - off : CH;
            if (w->dtype == LM_DTYPE_F32)
                memcpy(tmp, (const float *)src + off, n * 4);
            else
                lm_f16_to_f32((const uint16_t *)src + off, tmp, n);
            ok = fwrite(tmp, 4, n, f) == n;
        }
    }
    free(tmp);
    if (fclose(f) != 0) ok = 0;
    if (!ok) {
        fprintf(stderr, "lm_write_llama2c: write failed for %s\n", path);
        return LM_ERR_IO;
    }
    return LM_OK;
}

/* Bytes from the current position of f to its end (0 when unknown). */
static unsigned long long bytes_left(FILE *f)
{
    const long here = ftell(f);
    if (here < 0 || fseek(f, 0, SEEK_END) != 0) return 0;
    const long end = ftell(f);
    if (fseek(f, here, SEEK_SET) != 0 || end < here) return 0;
    return (unsigned long long)(end - here);
}

int lmh_read_llama2c(const char *path, Config *cfg, int *untied, float **data)
{
    *data = NULL;
    FILE *f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "lm_load_llama2c: cannot open %s\n", path);
        return LM_ERR_IO;
    }
    Config hdr;
    if (fread(&hdr, sizeof(Config), 1, f) != 1) {
        fprintf(stderr, "lm_load_llama2c: failed to read config from %s\n", path);
        fclose(f);
        return LM_ERR_FORMAT;
    }
    int rc = lmh_check_config(&hdr);
    if (rc) {
        fprintf(stderr, "lm_load_llama2c: inconsistent header in %s "
                "(dim=%d hidden=%d layers=%d heads=%d kv_heads=%d vocab=%d seq=%d)\n",
                path, hdr.dim, hdr.hidden_dim, hdr.n_layers, hdr.n_heads, hdr.n_kv_heads,
                hdr.vocab_size, hdr.seq_len);
        fclose(f);
        return LM_ERR_FORMAT;
    }
    int u = hdr.vocab_size < 0;                    /* model.h:85-86 */
    if (u) hdr.vocab_size = -hdr.vocab_size;
    size_t n = lm_weights_numel(&hdr, u);
    /* a file shorter than its header says is refused before the allocation */
    const unsigned long long left = bytes_left(f);
    if (left < (unsigned long long)n * sizeof(float)) {
        fprintf(stderr, "lm_load_llama2c: %s holds %llu bytes of weights, its header needs %llu "
                "(file truncated?)\n", path, left, (unsigned long long)n * sizeof(float));
        fclose(f);
        return LM_ERR_FORMAT;
    }
    float *buf = (float *)malloc(n * sizeof(float));
    if (!buf) {
        fclose(f);
        return LM_ERR_OOM;
    }
    size_t got = fread(buf, sizeof(float), n, f);
    fclose(f);
    if (got != n) {
        fprintf(stderr, "lm_load_llama2c: short read on %s: got %zu of %zu floats "
                "(file truncated?)\n", path, got, n);
        free(buf);
        return LM_ERR_FORMAT;
    }
    *cfg = hdr;
    *untied = u;
    *data = buf;
    return LM_OK;
}

/* ------------------------------------------------------------------------- */
/* BLZT v4 checkpoints (the reference's training checkpoints)                 */
/* ------------------------------------------------------------------------- */

/* Header of a BLZT checkpoint, 96 bytes (training/training_dynamic/config.h:78-86,
 * read by generate.m:212-248): magic 'BLZT', version 4, training counters,
 * model shape (with the GQA fields kv_heads, head_dim, q_dim in version 4). */
typedef struct {
    int32_t magic, version, step, total_steps;
    int32_t n_layers, vocab_size, dim, hidden_dim, n_heads, seq_len;
    float lr, loss;
    double cum_compile, cum_train, cum_wall;
    int32_t cum_steps, cum_batches, adam_t;
    int32_t kv_heads, head_dim, q_dim;
} BlztHeader;

#define BLZT_MAGIC 0x424C5A54

static int read_f32(FILE *f, float *dst, size_t n)
{
    return fread(dst, sizeof(float), n, f) == n ? LM_OK : LM_ERR_FORMAT;
}

static int skip_f32(FILE *f, size_t n)
{
    /* long is 64-bit on the LP64 hosts this builds for */
    return fseek(f, (long)(n * sizeof(float)), SEEK_CUR) == 0 ? LM_OK : LM_ERR_FORMAT;
}

/* Weights of a BLZT v4 file into a llama2.c-ordered fp32 buffer (tied
 * classifier: the embedding).  Per layer the file holds Wq, Wk, Wv, Wo, W1,
 * W2, W3, rms_att, rms_ffn followed by the Adam m and v of each; then
 * rms_final (+ Adam) and the embedding (generate.m:228-246). */
int lmh_read_blzt(const char *path, Config *cfg, float **data)
{
    *data = NULL;
    FILE *f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "lm_load_blzt: cannot open %s\n", path);
        return LM_ERR_IO;
    }
    BlztHeader h;
    if (fread(&h, sizeof(h), 1, f) != 1 || h.magic != BLZT_MAGIC || h.version != 4) {
        fprintf(stderr, "lm_load_blzt: %s is not a BLZT version 4 checkpoint\n", path);
        fclose(f);
        return LM_ERR_FORMAT;
    }
    Config c;
    c.dim = h.dim;
    c.hidden_dim = h.hidden_dim;
    c.n_layers = h.n_layers;
    c.n_heads = h.n_heads;
    c.n_kv_heads = h.kv_heads > 0 ? h.kv_heads : h.n_heads;
    c.vocab_size = h.vocab_size;
    c.seq_len = h.seq_len;
    const int hd = h.head_dim > 0 ? h.head_dim : (h.n_heads > 0 ? h.dim / h.n_heads : 0);
    const int qd = h.q_dim > 0 ? h.q_dim : h.n_heads * hd;
    if (lmh_check_config(&c) || c.vocab_size < 1 || qd != c.dim || hd * c.n_heads != c.dim) {
        fprintf(stderr, "lm_load_blzt: unsupported shape in %s (dim=%d heads=%d head_dim=%d "
                "q_dim=%d kv_heads=%d vocab=%d): this loop needs q_dim == dim\n",
                path, h.dim, h.n_heads, hd, qd, c.n_kv_heads, h.vocab_size);
        fclose(f);
        return LM_ERR_FORMAT;
    }
    size_t sz[LMH_NTENSORS];
    lmh_tensor_sizes(&c, 0, sz);
    const size_t L = (size_t)c.n_layers, D = (size_t)c.dim;
    const size_t wq = sz[LMH_T_WQ] / L, wk = sz[LMH_T_WK] / L, wv = sz[LMH_T_WV] / L;
    const size_t wo = sz[LMH_T_WO] / L, w1 = sz[LMH_T_W1] / L, w2 = sz[LMH_T_W2] / L;
    const size_t w3 = sz[LMH_T_W3] / L;
    /* the weights and their Adam m and v: three values per parameter, up to
     * the embedding, whose Adam state the loop does not read */
    const size_t per_layer = wq + wk + wv + wo + w1 + w2 + w3 + 2 * D;
    const unsigned long long need =
        4ull * (3 * (L * per_layer + D) + (unsigned long long)c.vocab_size * D);
    if (bytes_left(f) < need) {
        fprintf(stderr, "lm_load_blzt: %s is truncated\n", path);
        fclose(f);
        return LM_ERR_FORMAT;
    }
    float *buf = (float *)malloc(lm_weights_numel(&c, 0) * sizeof(float));
    if (!buf) {
        fclose(f);
        return LM_ERR_OOM;
    }
    LMWeights w;
    lm_weights_view(&c, LM_DTYPE_F32, buf, 0, &w);
    float *emb = (float *)w.token_embedding, *ra = (float *)w.rms_att_w, *rf = (float *)w.rms_ffn_w;
    float *q = (float *)w.wq, *k = (float *)w.wk, *v = (float *)w.wv, *o = (float *)w.wo;
    float *p1 = (float *)w.w1, *p2 = (float *)w.w2, *p3 = (float *)w.w3, *fin = (float *)w.rms_final_w;
    int rc = LM_OK;
    for (size_t l = 0; l < L && rc == LM_OK; l++) {
        rc = read_f32(f, q + l * wq, wq);
        if (!rc) rc = read_f32(f, k + l * wk, wk);
        if (!rc) rc = read_f32(f, v + l * wv, wv);
        if (!rc) rc = read_f32(f, o + l * wo, wo);
        if (!rc) rc = read_f32(f, p1 + l * w1, w1);
        if (!rc) rc = read_f32(f, p2 + l * w2, w2);
        if (!rc) rc = read_f32(f, p3 + l * w3, w3);
        if (!rc) rc = read_f32(f, ra + l * D, D);
        if (!rc) rc = read_f32(f, rf + l * D, D);
        if (!rc) rc = skip_f32(f, 2 * (wq + wk + wv + wo + w1 + w2 + w3 + 2 * D));
    }
    if (!rc) rc = read_f32(f, fin, D);
    if (!rc) rc = skip_f32(f, 2 * D);
    if (!rc) rc = read_f32(f, emb, (size_t)c.vocab_size * D);
    fclose(f);
    if (rc) {
        fprintf(stderr, "lm_load_blzt: %s is truncated\n", path);
        free(buf);
        return rc;
    }
    *cfg = c;
    *data = buf;
    return LM_OK;
}

int lm_blzt_to_llama2c(const char *blzt_path, const char *out_path)
{
    if (!blzt_path || !out_path) return LM_ERR_INVALID;
    Config c;
    float *data = NULL;
    int rc = lmh_read_blzt(blzt_path, &c, &data);
    if (rc) return rc;
    LMWeights w;
    lm_weights_view(&c, LM_DTYPE_F32, data, 0, &w);
    rc = lm_write_llama2c(out_path, &c, &w);
    free(data);
    return rc;
}

/* ------------------------------------------------------------------------- */
/* RoPE table                                                                 */
/* ------------------------------------------------------------------------- */

int lm_rope_table(int max_seq, int head_dim, float *cos_out, float *sin_out)
{
    if (max_seq <= 0 || head_dim <= 0 || (head_dim & 1) || !cos_out || !sin_out)
        return LM_ERR_INVALID;
    int half = head_dim / 2;
    for (int t = 0; t < max_seq; t++)
        for (int i = 0; i < head_dim; i += 2) {          /* forward.h:58-61 */
            float freq = 1.0f / powf(10000.0f, (float)i / head_dim);
            float val = t * freq;
            cos_out[(size_t)t * half + i / 2] = cosf(val);
            sin_out[(size_t)t * half + i / 2] = sinf(val);
        }
    return LM_OK;
}
