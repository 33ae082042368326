/*
 * oracle.h — CPU oracle of the Stories / Llama-2 forward.  TEST INFRASTRUCTURE
 * ONLY: the parity checker for the HIP path.  Only tests/, the smoke check and
 * the benchmark's CPU-baseline leg may load it; the product library never does.
 *
 * It restates, in portable C11 with fp32 arithmetic, the reference's CPU forward
 * (training/forward.h:36-184, RMSNorm/embedding of training/stories_cpu_ops.h:6-21,
 * 113-121) and the KV-cache decode structure of training/dashboard.py:186-276.
 *
 * Floating-point contract.  The reference is built with Apple clang -O2
 * (training/Makefile:1-2), whose default -ffp-contract=on fuses a multiply
 * into the add of the same statement.  The oracle writes those fusions out
 * with fmaf() and is compiled with -ffp-contract=off so nothing else fuses:
 *   matmul   sum = fmaf(W[i,j], x[j], sum), j ascending        (forward.h:40-41)
 *   rmsnorm  ss = fmaf(x, x, ss); out = x * ss * w             (forward.h:49-51)
 *   rope     a' = fmaf(a, cos, -(b*sin)); b' = fmaf(a, sin, b*cos) (forward.h:64-68)
 *   attn     dot = fmaf(q, k, dot); val = fmaf(p, v, val)     (forward.h:83,93)
 * Every output element keeps the reference's sequential summation order, so
 * mode (i) and mode (ii) below agree bit for bit.
 */
#ifndef STORIES_ORACLE_H
#define STORIES_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct OracleModel OracleModel;

/* cfg7 = {dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len}
 * (training/model.h:19-21; vocab_size sign ignored).  `w` holds the fp32
 * weights contiguously in llama2.c order (training/model.h:94-160), the
 * classifier last when untied.  kv_f16 != 0 rounds cached K/V to binary16
 * (RNE) like the device cache; 0 keeps them fp32 like forward.h.  NULL on
 * bad arguments. */
OracleModel *oracle_create(const int *cfg7, const float *w, int untied, int max_seq,
                           int kv_f16);
void oracle_free(OracleModel *o);

/* Mode (i): full causal forward of S tokens at positions 0..S-1,
 * logits [S, vocab] row-major (training/forward.h:104-170). */
int oracle_forward_full(OracleModel *o, const int *tokens, int S, float *logits);

/* The same forward with the classifier applied to the last row only, logits
 * [vocab]: the reference's per-token window recompute (generate.m:437-487,
 * cblas_sgemv on the last position). */
int oracle_forward_last(OracleModel *o, const int *tokens, int S, float *logits);

/* Mode (ii): one KV-cache decode step of `token` at `pos`; positions < pos
 * must have been stepped before (training/dashboard.py:205-267 with
 * forward.h's arithmetic).  logits [vocab]. */
int oracle_decode_step(OracleModel *o, int token, int pos, float *logits);

/* Mode (ii) over S rows: tokens at positions pos0..pos0+S-1 append their K/V
 * to the cache and attend to cached positions 0..pos0+t; positions < pos0 must
 * have been filled before.  With pos0 = 0 the logits equal mode (i)'s bit for
 * bit, and S = 1 is oracle_decode_step.  logits [S, vocab], or [vocab] with
 * last_only. */
int oracle_forward_cached(OracleModel *o, const int *tokens, int S, int pos0, int last_only,
                          float *logits);

/* Mean next-token cross-entropy over S-1 positions (training/forward.h:174-183). */
float oracle_loss(const float *logits, const int *tokens, int S, int vocab);

/* First index of the maximum, strict '>' scan (generate.m:129-136). */
int oracle_argmax(const float *logits, int n);

/* Building blocks, exposed for closed-form tests. */
void oracle_matmul(const float *W, const float *x, float *y, int S, int in_dim, int out_dim);
void oracle_rmsnorm(float *out, const float *x, const float *w, int S, int D);
void oracle_rope(float *q, float *k, int S, int n_heads, int n_kv_heads, int head_dim, int pos0);
void oracle_attention(float *out, const float *q, const float *k, const float *v, int S,
                      int n_heads, int n_kv_heads, int head_dim);

/* OpenMP threads the oracle's parallel loops use. */
int oracle_num_threads(void);

/* binary16 round trip used by the kv_f16 mode. */
float oracle_round_f16(float x);

#ifdef __cplusplus
}
#endif

#endif
