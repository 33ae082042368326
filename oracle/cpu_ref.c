/*
 * cpu_ref.c — the reference's portable CPU forward with OpenBLAS in place of
 * Apple Accelerate, timed as the CPU baseline of bench.py.  BENCHMARK AND TEST
 * INFRASTRUCTURE ONLY: the product library never loads it.
 *
 * What it restates (paths under the reference repository):
 *   RMSNorm       stories_cpu_ops.h:6-21 (sum of squares over d, then
 *                 ss/d + 1e-5, reciprocal square root, x * ss * w), row-major
 *                 as training/forward.h:46-53 lays rows out
 *   embedding     stories_cpu_ops.h:113-121 / forward.h:108-110
 *   projections   y = W x per row; the reference's CPU paths call Accelerate's
 *                 cblas_sgemv / cblas_sgemm for these (generate.m:486,
 *                 train_large.m:456-459): here OpenBLAS's sgemv (one row) and
 *                 sgemm (several rows)
 *   RoPE          forward.h:55-70 (interleaved pairs)
 *   attention     forward.h:72-99, causal, over the K/V cache
 *   SwiGLU        forward.h:101,149-151; residuals forward.h:136,159
 *   classifier    forward.h:163-170 (untied) or the embedding (tied,
 *                 generate.m:486-487); on the last row only for the
 *                 per-token window recompute of generate.m:427-516
 * All arithmetic is fp32 on fp32 weights (the same fp16-exact values the GPU
 * holds).  BLAS: OpenBLAS is opened at run time from the path the caller
 * gives (numpy bundles one: libscipy_openblas64_, exporting
 * scipy_cblas_sgemm64_ / scipy_cblas_sgemv64_ with 64-bit integers); without
 * it, plain loops stand in, and cpuref_blas_name says which ran.  Every
 * parallel part runs inside OpenBLAS: the projections, and attention per head
 * as two products (scores = Q K^T, out = P V).  The elementwise work between
 * them is serial, so no second thread pool competes with OpenBLAS's.
 */
#include <dlfcn.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* CBLAS enum values (cblas.h) */
#define ROW_MAJOR 101
#define NO_TRANS 111
#define TRANS 112

typedef void (*sgemm64_t)(int, int, int, int64_t, int64_t, int64_t, float, const float *, int64_t,
                          const float *, int64_t, float, float *, int64_t);
typedef void (*sgemv64_t)(int, int, int64_t, int64_t, float, const float *, int64_t, const float *,
                          int64_t, float, float *, int64_t);
typedef void (*set_threads_t)(int);

static sgemm64_t g_sgemm;
static sgemv64_t g_sgemv;
static set_threads_t g_set_threads;
static char g_blas_name[256] = "in-repo serial loops (no OpenBLAS opened)";

int cpuref_blas_open(const char *path)
{
    if (!path) return -1;
    void *h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!h) return -1;
    sgemm64_t gm = (sgemm64_t)dlsym(h, "scipy_cblas_sgemm64_");
    sgemv64_t gv = (sgemv64_t)dlsym(h, "scipy_cblas_sgemv64_");
    if (!gm) gm = (sgemm64_t)dlsym(h, "cblas_sgemm64_");
    if (!gv) gv = (sgemv64_t)dlsym(h, "cblas_sgemv64_");
    if (!gm || !gv) return -2;
    g_sgemm = gm;
    g_sgemv = gv;
    g_set_threads = (set_threads_t)dlsym(h, "scipy_openblas_set_num_threads64_");
    if (!g_set_threads) g_set_threads = (set_threads_t)dlsym(h, "openblas_set_num_threads64_");
    typedef char *(*cfg_t)(void);
    cfg_t cf = (cfg_t)dlsym(h, "scipy_openblas_get_config64_");
    const char *base = strrchr(path, '/');
    snprintf(g_blas_name, sizeof(g_blas_name), "OpenBLAS %s (%s)", cf ? cf() : "",
             base ? base + 1 : path);
    return 0;
}

const char *cpuref_blas_name(void) { return g_blas_name; }

int cpuref_set_threads(int n)
{
    if (n < 1) return -1;
    if (g_set_threads) g_set_threads(n);
    return 0;
}

/* C[M, N] = alpha A[M, K] B^T (B [N, K], row strides lda, ldb, ldc) */
static void gemm_nt(int M, int N, int K, float alpha, const float *A, int lda, const float *B,
                    int ldb, float *C, int ldc)
{
    if (g_sgemm) {
        g_sgemm(ROW_MAJOR, NO_TRANS, TRANS, M, N, K, alpha, A, lda, B, ldb, 0.0f, C, ldc);
        return;
    }
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float s = 0.f;
            for (int k = 0; k < K; k++) s += A[(size_t)m * lda + k] * B[(size_t)n * ldb + k];
            C[(size_t)m * ldc + n] = alpha * s;
        }
}

/* C[M, N] = A[M, K] B[K, N] (row strides lda, ldb, ldc) */
static void gemm_nn(int M, int N, int K, const float *A, int lda, const float *B, int ldb, float *C,
                    int ldc)
{
    if (g_sgemm) {
        g_sgemm(ROW_MAJOR, NO_TRANS, NO_TRANS, M, N, K, 1.0f, A, lda, B, ldb, 0.0f, C, ldc);
        return;
    }
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float s = 0.f;
            for (int k = 0; k < K; k++) s += A[(size_t)m * lda + k] * B[(size_t)k * ldb + n];
            C[(size_t)m * ldc + n] = s;
        }
}

/* Y[S, out] = X[S, in] W[out, in]^T: sgemv for one row, sgemm for several */
static void proj(const float *W, const float *X, float *Y, int S, int in, int out)
{
    if (S == 1 && g_sgemv) {
        g_sgemv(ROW_MAJOR, NO_TRANS, out, in, 1.0f, W, in, X, 1, 0.0f, Y, 1);
        return;
    }
    gemm_nt(S, out, in, 1.0f, X, in, W, in, Y, out);
}

typedef struct {
    int D, F, L, H, Hkv, hd, NQ, NKV, V, max_seq;
    const float *embed, *rms_att, *rms_ffn, *rms_final, *wcls;
    const float **wq, **wk, **wv, **wo, **w1, **w2, **w3;
    float *kc, *vc;           /* [L][max_seq][NKV] */
    float *w;                 /* owned copy of the weights */
} CpuRef;

void cpuref_free(CpuRef *r)
{
    if (!r) return;
    free(r->wq); free(r->wk); free(r->wv); free(r->wo); free(r->w1); free(r->w2); free(r->w3);
    free(r->kc); free(r->vc); free(r->w);
    free(r);
}

/* cfg7 {dim, hidden, layers, heads, kv_heads, vocab, seq_len}; w: the fp32
 * weights in llama2.c order (training/model.h:94-160), classifier last when
 * untied. */
CpuRef *cpuref_create(const int *c, const float *w, int untied, int max_seq)
{
    CpuRef *r = (CpuRef *)calloc(1, sizeof(CpuRef));
    if (!r) return NULL;
    r->D = c[0]; r->F = c[1]; r->L = c[2]; r->H = c[3]; r->Hkv = c[4];
    r->V = c[5] < 0 ? -c[5] : c[5];
    r->hd = r->D / r->H; r->NQ = r->H * r->hd; r->NKV = r->Hkv * r->hd; r->max_seq = max_seq;
    const size_t D = r->D, F = r->F, L = r->L, NQ = r->NQ, NKV = r->NKV, V = r->V;
    const size_t n = V * D + L * D * 2 + L * (NQ * D + 2 * NKV * D + D * NQ + 3 * F * D) + D +
                     (untied ? V * D : 0);
    r->w = (float *)malloc(n * 4);
    const float **pp[7];
    for (int i = 0; i < 7; i++) pp[i] = (const float **)malloc(L * sizeof(float *));
    r->wq = pp[0]; r->wk = pp[1]; r->wv = pp[2]; r->wo = pp[3]; r->w1 = pp[4]; r->w2 = pp[5];
    r->w3 = pp[6];
    r->kc = (float *)calloc(L * (size_t)max_seq * NKV, 4);
    r->vc = (float *)calloc(L * (size_t)max_seq * NKV, 4);
    if (!r->w || !r->kc || !r->vc || !pp[0] || !pp[1] || !pp[2] || !pp[3] || !pp[4] || !pp[5] ||
        !pp[6]) {
        cpuref_free(r);
        return NULL;
    }
    memcpy(r->w, w, n * 4);
    const float *p = r->w;
    r->embed = p; p += V * D;
    r->rms_att = p; p += L * D;
    for (size_t l = 0; l < L; l++) r->wq[l] = p + l * NQ * D;
    p += L * NQ * D;
    for (size_t l = 0; l < L; l++) r->wk[l] = p + l * NKV * D;
    p += L * NKV * D;
    for (size_t l = 0; l < L; l++) r->wv[l] = p + l * NKV * D;
    p += L * NKV * D;
    for (size_t l = 0; l < L; l++) r->wo[l] = p + l * D * NQ;
    p += L * D * NQ;
    r->rms_ffn = p; p += L * D;
    for (size_t l = 0; l < L; l++) r->w1[l] = p + l * F * D;
    p += L * F * D;
    for (size_t l = 0; l < L; l++) r->w2[l] = p + l * D * F;
    p += L * D * F;
    for (size_t l = 0; l < L; l++) r->w3[l] = p + l * F * D;
    p += L * F * D;
    r->rms_final = p; p += D;
    r->wcls = untied ? p : r->embed;
    return r;
}

/* stories_cpu_ops.h:6-21 on row-major rows */
static void rmsnorm_rows(float *out, const float *x, const float *w, int S, int D)
{
    for (int t = 0; t < S; t++) {
        const float *xr = x + (size_t)t * D;
        float ss = 0.f;
        for (int i = 0; i < D; i++) ss += xr[i] * xr[i];
        ss = 1.0f / sqrtf(ss / D + 1e-5f);
        for (int i = 0; i < D; i++) out[(size_t)t * D + i] = xr[i] * ss * w[i];
    }
}

/* forward.h:55-70 at positions pos0 + t */
static void rope_rows(float *q, float *k, int S, int H, int Hkv, int hd, int pos0)
{
    const int NQ = H * hd, NKV = Hkv * hd;
    for (int t = 0; t < S; t++)
        for (int i = 0; i < hd; i += 2) {
            const float freq = 1.0f / powf(10000.0f, (float)i / hd);
            const float a = (pos0 + t) * freq, c = cosf(a), s = sinf(a);
            for (int h = 0; h < H; h++) {
                float *v = q + (size_t)t * NQ + h * hd + i;
                const float v0 = v[0], v1 = v[1];
                v[0] = v0 * c - v1 * s;
                v[1] = v0 * s + v1 * c;
            }
            for (int h = 0; h < Hkv; h++) {
                float *v = k + (size_t)t * NKV + h * hd + i;
                const float v0 = v[0], v1 = v[1];
                v[0] = v0 * c - v1 * s;
                v[1] = v0 * s + v1 * c;
            }
        }
}

/* S rows at positions pos0.. : append K/V to the cache, attend causally
 * (forward.h:72-99 over the cache), classifier of every row or the last. */
static int forward_rows(CpuRef *r, const int *tok, int S, int pos0, int last_only, float *logits)
{
    const int D = r->D, F = r->F, NQ = r->NQ, NKV = r->NKV, hd = r->hd, H = r->H;
    const size_t s = S;
    float *x = (float *)malloc(s * D * 4), *xn = (float *)malloc(s * D * 4);
    float *q = (float *)malloc(s * NQ * 4), *att = (float *)malloc(s * NQ * 4);
    float *o = (float *)malloc(s * D * 4), *h1 = (float *)malloc(s * F * 4),
          *h3 = (float *)malloc(s * F * 4);
    float *sc = (float *)malloc(s * (size_t)(pos0 + S) * 4);
    int rc = 0;
    if (!x || !xn || !q || !att || !o || !h1 || !h3 || !sc) { rc = -4; goto done; }
    for (int t = 0; t < S; t++) memcpy(x + (size_t)t * D, r->embed + (size_t)tok[t] * D, D * 4);
    for (int l = 0; l < r->L; l++) {
        float *kc = r->kc + (size_t)l * r->max_seq * NKV, *vc = r->vc + (size_t)l * r->max_seq * NKV;
        rmsnorm_rows(xn, x, r->rms_att + (size_t)l * D, S, D);
        proj(r->wq[l], xn, q, S, D, NQ);
        proj(r->wk[l], xn, kc + (size_t)pos0 * NKV, S, D, NKV);
        proj(r->wv[l], xn, vc + (size_t)pos0 * NKV, S, D, NKV);
        rope_rows(q, kc + (size_t)pos0 * NKV, S, H, r->Hkv, hd, pos0);
        /* causal attention per head as two products over the cache
         * (forward.h:78-95): scores = Q K^T / sqrt(hd), masked past each row's
         * position, softmax with the max subtracted, out = P V */
        const int grp = H / r->Hkv, n = pos0 + S;
        const float scale = 1.0f / sqrtf((float)hd);
        for (int h = 0; h < H; h++) {
            const float *kb = kc + (h / grp) * hd, *vb = vc + (h / grp) * hd;
            gemm_nt(S, n, hd, scale, q + h * hd, NQ, kb, NKV, sc, n);
            for (int t = 0; t < S; t++) {
                float *row = sc + (size_t)t * n;
                const int vis = pos0 + t + 1;
                float mx = -1e9f, sum = 0.f;
                for (int j = 0; j < vis; j++) mx = row[j] > mx ? row[j] : mx;
                for (int j = 0; j < vis; j++) { row[j] = expf(row[j] - mx); sum += row[j]; }
                for (int j = 0; j < vis; j++) row[j] /= sum;
                for (int j = vis; j < n; j++) row[j] = 0.f;
            }
            gemm_nn(S, hd, n, sc, n, vb, NKV, att + h * hd, NQ);
        }
        proj(r->wo[l], att, o, S, NQ, D);
        for (size_t i = 0; i < s * D; i++) x[i] += o[i];
        rmsnorm_rows(xn, x, r->rms_ffn + (size_t)l * D, S, D);
        proj(r->w1[l], xn, h1, S, D, F);
        proj(r->w3[l], xn, h3, S, D, F);
        for (size_t i = 0; i < s * F; i++) h1[i] = h1[i] / (1.0f + expf(-h1[i])) * h3[i];
        proj(r->w2[l], h1, o, S, F, D);
        for (size_t i = 0; i < s * D; i++) x[i] += o[i];
    }
    if (last_only) {
        rmsnorm_rows(xn, x + (s - 1) * D, r->rms_final, 1, D);
        proj(r->wcls, xn, logits, 1, D, r->V);
    } else {
        rmsnorm_rows(xn, x, r->rms_final, S, D);
        proj(r->wcls, xn, logits, S, D, r->V);
    }
done:
    free(x); free(xn); free(q); free(att); free(o); free(h1); free(h3); free(sc);
    return rc;
}

/* One KV-cache decode step (the token loop with a cache, dashboard.py:205-267). */
int cpuref_decode_step(CpuRef *r, int token, int pos, float *logits)
{
    if (!r || !logits || token < 0 || token >= r->V || pos < 0 || pos >= r->max_seq) return -3;
    return forward_rows(r, &token, 1, pos, 0, logits);
}

/* The full causal forward of S tokens from position 0 (forward.h:104-170),
 * logits of every row, or of the last row only (generate.m's per-token
 * window recompute). */
int cpuref_forward(CpuRef *r, const int *tokens, int S, int last_only, float *logits)
{
    if (!r || !tokens || !logits || S < 1 || S > r->max_seq) return -3;
    for (int t = 0; t < S; t++)
        if (tokens[t] < 0 || tokens[t] >= r->V) return -3;
    return forward_rows(r, tokens, S, 0, last_only, logits);
}
