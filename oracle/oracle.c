/*
 * oracle.c — CPU oracle of the Stories / Llama-2 forward.  TEST
 * INFRASTRUCTURE ONLY (see oracle.h): the checker the HIP path is compared
 * against, never part of the product.
 *
 * Every function cites the reference lines it restates.  Matrix-vector
 * products run over a transposed copy of each weight matrix so that the inner
 * loop vectorises across output rows; each output still accumulates its
 * inputs one at a time, in ascending order, with one fused multiply-add per
 * term, exactly the order of training/forward.h:36-44.  OpenMP splits work
 * across outputs and tokens only, which cannot change any result.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

struct OracleModel {
    int D, F, L, H, Hkv, hd, NQ, NKV, V, max_seq, kv_f16;
    float *embed;                 /* [V][D] row-major                 */
    float *rms_att, *rms_ffn;     /* [L][D]                           */
    float *rms_final;             /* [D]                              */
    float *wqT, *wkT, *wvT, *woT; /* per layer, transposed [in][out]  */
    float *w1T, *w2T, *w3T;
    float *wclsT;                 /* [D][V]                           */
    float *kc, *vc;               /* [L][max_seq][NKV]                */
};

/* ---------------------------------------------------------------- helpers */

float oracle_round_f16(float x)
{
    /* IEEE binary16 round-to-nearest-even and back (io.h:33-50 semantics). */
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = u & 0x80000000u, ax = u & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return x;
    if (ax >= 0x477FF000u) { u = sign | 0x7F800000u; memcpy(&x, &u, 4); return x; }
    if (ax < 0x38800000u) {
        /* half subnormal grid: multiples of 2^-24 */
        float a = fabsf(x) * 16777216.0f;      /* exact scaling by 2^24 */
        float r = nearbyintf(a);               /* default rounding: ties to even */
        float y = r / 16777216.0f;
        return sign ? -y : y;
    }
    uint32_t lsb = (ax >> 13) & 1u;
    ax = (ax + 0xFFFu + lsb) & ~0x1FFFu;
    u = sign | ax;
    memcpy(&x, &u, 4);
    return x;
}

static void transpose(const float *W, float *WT, int out, int in)
{
    #pragma omp parallel for schedule(static)
    for (int j = 0; j < in; j++)
        for (int i = 0; i < out; i++) WT[(size_t)j * out + i] = W[(size_t)i * in + j];
}

/* y[t, i] = sum_j W[i, j] x[t, j] from WT = W^T ([in][out]).  Blocks of 8
 * tokens x 64 outputs; each output's sum runs j = 0..in-1 with fmaf. */
#define OB 64
#define TB 8
static void matmul_T(const float *WT, const float *x, float *y, int S, int in, int out)
{
    const int nob = (out + OB - 1) / OB, ntb = (S + TB - 1) / TB;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int tb = 0; tb < ntb; tb++)
        for (int ob = 0; ob < nob; ob++) {
            const int t0 = tb * TB, nt = S - t0 < TB ? S - t0 : TB;
            const int i0 = ob * OB, n = out - i0 < OB ? out - i0 : OB;
            float acc[TB][OB];
            for (int tt = 0; tt < TB; tt++)
                for (int i = 0; i < OB; i++) acc[tt][i] = 0.0f;
            for (int j = 0; j < in; j++) {
                const float *w = WT + (size_t)j * out + i0;
                for (int tt = 0; tt < nt; tt++) {
                    const float xj = x[(size_t)(t0 + tt) * in + j];
                    for (int i = 0; i < n; i++) acc[tt][i] = fmaf(w[i], xj, acc[tt][i]);
                }
            }
            for (int tt = 0; tt < nt; tt++)
                memcpy(y + (size_t)(t0 + tt) * out + i0, acc[tt], (size_t)n * 4);
        }
}

/* ------------------------------------------------- public building blocks */

/* training/forward.h:36-44 (cpu_matmul), W[out][in] row-major. */
void oracle_matmul(const float *W, const float *x, float *y, int S, int in_dim, int out_dim)
{
    for (int t = 0; t < S; t++)
        for (int i = 0; i < out_dim; i++) {
            float sum = 0;
            for (int j = 0; j < in_dim; j++)
                sum = fmaf(W[(size_t)i * in_dim + j], x[(size_t)t * in_dim + j], sum);
            y[(size_t)t * out_dim + i] = sum;
        }
}

/* training/forward.h:46-53 (cpu_rmsnorm); same arithmetic as the channel-first
 * rmsnorm of training/stories_cpu_ops.h:6-21. */
void oracle_rmsnorm(float *out, const float *x, const float *w, int S, int D)
{
    for (int t = 0; t < S; t++) {
        float ss = 0;
        for (int i = 0; i < D; i++) ss = fmaf(x[(size_t)t * D + i], x[(size_t)t * D + i], ss);
        ss = 1.0f / sqrtf(ss / D + 1e-5f);
        for (int i = 0; i < D; i++) out[(size_t)t * D + i] = x[(size_t)t * D + i] * ss * w[i];
    }
}

/* training/forward.h:55-70 (cpu_rope), interleaved pairs (2i, 2i+1), token t at
 * position pos0 + t; k has n_kv_heads heads (dashboard.py:228-234). */
void oracle_rope(float *q, float *k, int S, int n_heads, int n_kv_heads, int head_dim, int pos0)
{
    const int NQ = n_heads * head_dim, NKV = n_kv_heads * head_dim;
    for (int t = 0; t < S; t++) {
        const int p = pos0 + t;
        for (int h = 0; h < n_heads; h++)
            for (int i = 0; i < head_dim; i += 2) {
                float freq = 1.0f / powf(10000.0f, (float)i / head_dim);
                float val = p * freq;
                float cos_v = cosf(val), sin_v = sinf(val);
                size_t off = (size_t)t * NQ + h * head_dim + i;
                float q0 = q[off], q1 = q[off + 1];
                q[off] = fmaf(q0, cos_v, -(q1 * sin_v));
                q[off + 1] = fmaf(q0, sin_v, q1 * cos_v);
                if (h < n_kv_heads) {
                    size_t ko = (size_t)t * NKV + h * head_dim + i;
                    float k0 = k[ko], k1 = k[ko + 1];
                    k[ko] = fmaf(k0, cos_v, -(k1 * sin_v));
                    k[ko + 1] = fmaf(k0, sin_v, k1 * cos_v);
                }
            }
    }
}

/* Causal attention of one query row against keys/values 0..n-1 of one head
 * (the inner body of training/forward.h:78-95). */
static void attend_row(float *out, const float *qh, const float *kbase, const float *vbase,
                       size_t kv_stride, int n, int head_dim, float *scores)
{
    const float scale = 1.0f / sqrtf((float)head_dim);
    float mx = -1e9f;
    for (int s = 0; s < n; s++) {
        float dot = 0;
        for (int i = 0; i < head_dim; i++) dot = fmaf(qh[i], kbase[(size_t)s * kv_stride + i], dot);
        scores[s] = dot * scale;
        if (scores[s] > mx) mx = scores[s];
    }
    float sm = 0;
    for (int s = 0; s < n; s++) { scores[s] = expf(scores[s] - mx); sm += scores[s]; }
    for (int s = 0; s < n; s++) scores[s] /= sm;
    for (int i = 0; i < head_dim; i++) {
        float val = 0;
        for (int s = 0; s < n; s++) val = fmaf(scores[s], vbase[(size_t)s * kv_stride + i], val);
        out[i] = val;
    }
}

/* training/forward.h:72-99 (cpu_attention); query head h reads kv head
 * h / (n_heads / n_kv_heads) (dashboard.py:244-245). */
void oracle_attention(float *out, const float *q, const float *k, const float *v, int S,
                      int n_heads, int n_kv_heads, int head_dim)
{
    const int NQ = n_heads * head_dim, NKV = n_kv_heads * head_dim, grp = n_heads / n_kv_heads;
    #pragma omp parallel
    {
        float *scores = (float *)malloc((size_t)S * sizeof(float));
        #pragma omp for collapse(2) schedule(dynamic, 4)
        for (int h = 0; h < n_heads; h++)
            for (int t = 0; t < S; t++) {
                const int kvh = h / grp;
                attend_row(out + (size_t)t * NQ + h * head_dim, q + (size_t)t * NQ + h * head_dim,
                           k + kvh * head_dim, v + kvh * head_dim, NKV, t + 1, head_dim, scores);
            }
        free(scores);
    }
}

static inline float silu_f(float x) { return x / (1.0f + expf(-x)); }   /* forward.h:101 */

/* ------------------------------------------------------------------- model */

OracleModel *oracle_create(const int *c, const float *w, int untied, int max_seq, int kv_f16)
{
    if (!c || !w || max_seq < 1) return NULL;
    int D = c[0], F = c[1], L = c[2], H = c[3], Hkv = c[4], V = c[5] < 0 ? -c[5] : c[5];
    if (D <= 0 || F <= 0 || L <= 0 || H <= 0 || Hkv <= 0 || V <= 0 || D % H || H % Hkv)
        return NULL;
    OracleModel *o = (OracleModel *)calloc(1, sizeof(OracleModel));
    if (!o) return NULL;
    o->D = D; o->F = F; o->L = L; o->H = H; o->Hkv = Hkv; o->V = V;
    o->hd = D / H; o->NQ = H * o->hd; o->NKV = Hkv * o->hd;
    o->max_seq = max_seq; o->kv_f16 = kv_f16;
    const size_t d = D, f = F, nq = o->NQ, nkv = o->NKV, v = V, l = L;
    o->embed = (float *)malloc(v * d * 4);
    o->rms_att = (float *)malloc(l * d * 4);
    o->rms_ffn = (float *)malloc(l * d * 4);
    o->rms_final = (float *)malloc(d * 4);
    o->wqT = (float *)malloc(l * nq * d * 4);
    o->wkT = (float *)malloc(l * nkv * d * 4);
    o->wvT = (float *)malloc(l * nkv * d * 4);
    o->woT = (float *)malloc(l * d * nq * 4);
    o->w1T = (float *)malloc(l * f * d * 4);
    o->w2T = (float *)malloc(l * d * f * 4);
    o->w3T = (float *)malloc(l * f * d * 4);
    o->wclsT = (float *)malloc(v * d * 4);
    o->kc = (float *)calloc(l * (size_t)max_seq * nkv, 4);
    o->vc = (float *)calloc(l * (size_t)max_seq * nkv, 4);
    if (!o->embed || !o->rms_att || !o->rms_ffn || !o->rms_final || !o->wqT || !o->wkT ||
        !o->wvT || !o->woT || !o->w1T || !o->w2T || !o->w3T || !o->wclsT || !o->kc || !o->vc) {
        oracle_free(o);
        return NULL;
    }
    /* llama2.c order: embed, rms_att, wq, wk, wv, wo, rms_ffn, w1, w2, w3,
     * rms_final, [wcls] (training/model.h:94-160). */
    const float *p = w;
    memcpy(o->embed, p, v * d * 4); p += v * d;
    memcpy(o->rms_att, p, l * d * 4); p += l * d;
    for (size_t i = 0; i < l; i++) transpose(p + i * nq * d, o->wqT + i * nq * d, nq, d);
    p += l * nq * d;
    for (size_t i = 0; i < l; i++) transpose(p + i * nkv * d, o->wkT + i * nkv * d, nkv, d);
    p += l * nkv * d;
    for (size_t i = 0; i < l; i++) transpose(p + i * nkv * d, o->wvT + i * nkv * d, nkv, d);
    p += l * nkv * d;
    for (size_t i = 0; i < l; i++) transpose(p + i * d * nq, o->woT + i * d * nq, d, nq);
    p += l * d * nq;
    memcpy(o->rms_ffn, p, l * d * 4); p += l * d;
    for (size_t i = 0; i < l; i++) transpose(p + i * f * d, o->w1T + i * f * d, f, d);
    p += l * f * d;
    for (size_t i = 0; i < l; i++) transpose(p + i * d * f, o->w2T + i * d * f, d, f);
    p += l * d * f;
    for (size_t i = 0; i < l; i++) transpose(p + i * f * d, o->w3T + i * f * d, f, d);
    p += l * f * d;
    memcpy(o->rms_final, p, d * 4); p += d;
    transpose(untied ? p : o->embed, o->wclsT, V, D);   /* tied: wcls = embed (model.h:155-157) */
    return o;
}

void oracle_free(OracleModel *o)
{
    if (!o) return;
    free(o->embed); free(o->rms_att); free(o->rms_ffn); free(o->rms_final);
    free(o->wqT); free(o->wkT); free(o->wvT); free(o->woT);
    free(o->w1T); free(o->w2T); free(o->w3T); free(o->wclsT);
    free(o->kc); free(o->vc);
    free(o);
}

static void round_kv(float *a, size_t n)
{
    for (size_t i = 0; i < n; i++) a[i] = oracle_round_f16(a[i]);
}

/* The layer stack and classifier over S rows at positions pos0..pos0+S-1.
 * mode_full: attention over the S rows themselves (forward.h:127-128);
 * otherwise the rows' K/V are appended to the cache at pos0.. and row t
 * attends to cached positions 0..pos0+t (dashboard.py:236-251, one row at a
 * time there; the same values and summation order for several rows).
 * last_only: the classifier of the last row only (generate.m:474-487). */
static int forward_rows(OracleModel *o, const int *tokens, int S, int pos0, int mode_full,
                        int last_only, float *logits)
{
    const int D = o->D, F = o->F, NQ = o->NQ, NKV = o->NKV, hd = o->hd;
    const size_t s = (size_t)S;
    float *x = (float *)malloc(s * D * 4), *xn = (float *)malloc(s * D * 4);
    float *q = (float *)malloc(s * NQ * 4), *k = (float *)malloc(s * NKV * 4);
    float *v = (float *)malloc(s * NKV * 4), *att = (float *)malloc(s * NQ * 4);
    float *o_out = (float *)malloc(s * D * 4);
    float *h1 = (float *)malloc(s * F * 4), *h3 = (float *)malloc(s * F * 4);
    int rc = 0;
    if (!x || !xn || !q || !k || !v || !att || !o_out || !h1 || !h3) { rc = -4; goto done; }

    for (int t = 0; t < S; t++)                                   /* forward.h:108-110 */
        memcpy(x + (size_t)t * D, o->embed + (size_t)tokens[t] * D, (size_t)D * 4);

    for (int l = 0; l < o->L; l++) {
        const size_t L = l;
        oracle_rmsnorm(xn, x, o->rms_att + L * D, S, D);           /* :115 */
        matmul_T(o->wqT + L * NQ * D, xn, q, S, D, NQ);           /* :122-124 */
        matmul_T(o->wkT + L * NKV * D, xn, k, S, D, NKV);
        matmul_T(o->wvT + L * NKV * D, xn, v, S, D, NKV);
        oracle_rope(q, k, S, o->H, o->Hkv, hd, pos0);             /* :127 */
        if (o->kv_f16) { round_kv(k, s * NKV); round_kv(v, s * NKV); }
        if (mode_full) {
            oracle_attention(att, q, k, v, S, o->H, o->Hkv, hd);   /* :128 */
        } else {
            float *kc = o->kc + L * o->max_seq * NKV, *vc = o->vc + L * o->max_seq * NKV;
            memcpy(kc + (size_t)pos0 * NKV, k, s * NKV * 4);       /* dashboard.py:236-240 */
            memcpy(vc + (size_t)pos0 * NKV, v, s * NKV * 4);
            const int grp = o->H / o->Hkv, H = o->H;
            #pragma omp parallel
            {
                float *scores = (float *)malloc((size_t)(pos0 + S) * sizeof(float));
                #pragma omp for collapse(2) schedule(dynamic, 4)
                for (int h = 0; h < H; h++)                        /* dashboard.py:243-251 */
                    for (int t = 0; t < S; t++)
                        attend_row(att + (size_t)t * NQ + h * hd, q + (size_t)t * NQ + h * hd,
                                   kc + (h / grp) * hd, vc + (h / grp) * hd, NKV, pos0 + t + 1,
                                   hd, scores);
                free(scores);
            }
        }
        matmul_T(o->woT + L * D * NQ, att, o_out, S, NQ, D);      /* :134 */
        for (size_t i = 0; i < s * D; i++) x[i] += o_out[i];       /* :136 */
        oracle_rmsnorm(xn, x, o->rms_ffn + L * D, S, D);           /* :139 */
        matmul_T(o->w1T + L * F * D, xn, h1, S, D, F);            /* :145-146 */
        matmul_T(o->w3T + L * F * D, xn, h3, S, D, F);
        for (size_t i = 0; i < s * F; i++) h1[i] = silu_f(h1[i]) * h3[i];   /* :149-151 */
        matmul_T(o->w2T + L * D * F, h1, o_out, S, F, D);          /* :157 */
        for (size_t i = 0; i < s * D; i++) x[i] += o_out[i];       /* :159 */
    }
    oracle_rmsnorm(xn, x, o->rms_final, S, D);                     /* :164 */
    if (last_only)
        matmul_T(o->wclsT, xn + (s - 1) * D, logits, 1, D, o->V);  /* generate.m:486 */
    else
        matmul_T(o->wclsT, xn, logits, S, D, o->V);                /* :169 */
done:
    free(x); free(xn); free(q); free(k); free(v); free(att); free(o_out); free(h1); free(h3);
    return rc;
}

int oracle_forward_full(OracleModel *o, const int *tokens, int S, float *logits)
{
    if (!o || !tokens || !logits || S < 1) return -3;
    for (int t = 0; t < S; t++)
        if (tokens[t] < 0 || tokens[t] >= o->V) return -8;
    return forward_rows(o, tokens, S, 0, 1, 0, logits);
}

int oracle_forward_last(OracleModel *o, const int *tokens, int S, float *logits)
{
    if (!o || !tokens || !logits || S < 1) return -3;
    for (int t = 0; t < S; t++)
        if (tokens[t] < 0 || tokens[t] >= o->V) return -8;
    return forward_rows(o, tokens, S, 0, 1, 1, logits);
}

int oracle_decode_step(OracleModel *o, int token, int pos, float *logits)
{
    if (!o || !logits) return -3;
    if (token < 0 || token >= o->V || pos < 0 || pos >= o->max_seq) return -8;
    return forward_rows(o, &token, 1, pos, 0, 0, logits);
}

int oracle_forward_cached(OracleModel *o, const int *tokens, int S, int pos0, int last_only,
                          float *logits)
{
    if (!o || !tokens || !logits || S < 1) return -3;
    if (pos0 < 0 || pos0 + S > o->max_seq) return -8;
    for (int t = 0; t < S; t++)
        if (tokens[t] < 0 || tokens[t] >= o->V) return -8;
    return forward_rows(o, tokens, S, pos0, 0, last_only, logits);
}

/* training/forward.h:174-183 */
float oracle_loss(const float *logits, const int *tokens, int S, int vs)
{
    float loss = 0;
    for (int t = 0; t < S - 1; t++) {
        const float *lg = logits + (size_t)t * vs;
        float mx = -1e9f;
        for (int i = 0; i < vs; i++) if (lg[i] > mx) mx = lg[i];
        float sm = 0;
        for (int i = 0; i < vs; i++) sm += expf(lg[i] - mx);
        float log_prob = lg[tokens[t + 1]] - mx - logf(sm);
        loss -= log_prob;
    }
    return loss / (S - 1);
}

/* training/training_dynamic/generate.m:129-136 */
int oracle_argmax(const float *logits, int n)
{
    int best = 0;
    float best_val = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > best_val) { best_val = logits[i]; best = i; }
    return best;
}

int oracle_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
