/*
 * lm_internal.h — private declarations shared by the C host runtime
 * (lm_runtime.c, lm_weights.c, C99) and the HIP kernel translation units
 * (k_*.hip).  Kernel launchers are plain C functions: raw device pointers,
 * sizes and a hipStream_t, returning a hipError_t value (0 = success).
 */
#ifndef LM_INTERNAL_H
#define LM_INTERNAL_H

#include "../../include/stories_lm.h"

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tensor order of a llama2.c weight file (training/model.h:94-160). */
enum {
    LMH_T_EMBED = 0, LMH_T_RMS_ATT, LMH_T_WQ, LMH_T_WK, LMH_T_WV, LMH_T_WO,
    LMH_T_RMS_FFN, LMH_T_W1, LMH_T_W2, LMH_T_W3, LMH_T_RMS_FINAL, LMH_T_WCLS,
    LMH_NTENSORS
};

uint16_t lmh_f32_to_f16(float f);
float lmh_f16_to_f32(uint16_t h);
int lmh_check_config(const Config *c);
void lmh_tensor_sizes(const Config *c, int untied, size_t sz[LMH_NTENSORS]);
const void *lmh_weights_ptr(const LMWeights *w, int t);
int lmh_weights_untied(const LMWeights *w);
int lmh_read_llama2c(const char *path, Config *cfg, int *untied, float **data);
int lmh_read_blzt(const char *path, Config *cfg, float **data);

/* Rows of W1 and W3 are stored interleaved in blocks of LMK_GATE_BLOCK rows:
 * block j = [W1 rows j*G .. j*G+G-1, W3 rows j*G .. j*G+G-1], so any 2G-wide
 * output tile of the fused W1|W3 product holds matching h1/h3 columns. */
#define LMK_GATE_BLOCK 16

/* Argmax partial: best value and its index (lowest index on ties). */
typedef struct { float val; int idx; } LMArgPart;

/* ---- decode kernels (k_decode.hip) ---------------------------------------
 * Activations are fp32 [B, ...]; weights fp16 row-major W[out, in].
 * KV cache of one layer: [max_batch][Hkv][max_seq][hd] fp16 (or fp32), slot b
 * = row b. */

/* xn = rmsnorm(x[b]) * w; rows of [Wq;Wk;Wv] . xn; RoPE on q,k rows at pos[b];
 * q -> q[b, :NQ] fp32, k,v -> cache[b][h][pos[b]][:] (fp16, or fp32 when
 * kv_f32).  With emb != NULL the input rows are the fp16 embedding rows
 * emb[tok[b]] instead of x, and x[b] is set to them (first layer). */
int lmk_qkv_rope(hipStream_t s, float *x, const uint16_t *emb, const int *tok,
                 const float *rms_w, const uint16_t *wqkv, int D, int NQ, int NKV, int hd,
                 const float *rope_cos, const float *rope_sin, const int *pos,
                 int B, float *q, void *kc, void *vc, int kv_f32, int max_seq);

/* Tagged hand-off words of the batch 1-4 chain (LM_TAG_WORDS of them): q, k
 * and v of up to LM_TAG_B rows, then LM_TA_COPIES copies of the head
 * outputs, LM_TX_COPIES of x after Wo and LM_TG_COPIES of the FFN gate, each
 * reading work-group taking one copy, so that the readers of one value spread
 * over more memory channels. */
#define LM_TAG_B 4
/* Microseconds (real-time counter) before a hand-off wait gives up: the
 * second int of the flag buffer the launchers take as `err`.  Waits inside a
 * launch last microseconds; the limit only ends a launch that cannot make
 * progress. */
#define LM_HANDOFF_US 100000
/* Copies of the head outputs (LM_TA_COPIES), x after Wo (LM_TX_COPIES) and
 * the gate (LM_TG_COPIES).  C0 with one layer per launch, same-box A/Bs, two
 * alternating runs each, us/token with the fp32 cache: 4/4/4 153.1-153.9
 * against 1/8/1 150.2-150.5; then 1/8/1 152.9-153.1 against 2/8/1
 * 151.7-151.8, 1/8/2 153.2-153.3, 1/8/4 153.6-153.9; then 2/8/1 150.6-150.8
 * against 4/8/1 151.4-151.6 and 8/8/1 150.5-150.7 (binary16 K/V 1.2 us
 * slower); x in 12 or 16 copies 154-157.  Each copy costs its writers one
 * more partial-line store per value: the 512 W1/W3 readers of x gain from
 * more, the 96 readers of the gate, written by 512 work-groups, do not.
 * Reader a takes copy a % copies: with work-group ids going to XCDs mod 8,
 * each XCD's readers of x share one copy (spreading a copy's readers over
 * the XCDs cost 4 us/token). */
#ifndef LM_TA_COPIES
#define LM_TA_COPIES 2
#endif
#ifndef LM_TX_COPIES
#define LM_TX_COPIES 8
#endif
#ifndef LM_TG_COPIES
#define LM_TG_COPIES 1
#endif
#define LM_TAG_WORDS(NQ, NKV, D, F) \
    ((size_t)LM_TAG_B * ((NQ) + 2 * (NKV) + LM_TA_COPIES * (NQ) + LM_TG_COPIES * (F) + LM_TX_COPIES * (D)))

/* lmk_qkv_rope and the attention of every (head, row) in one launch: the
 * QKV work-groups hand q, k, v of the current position to the attention
 * work-groups through tagged words (`tagged`: LM_TAG_WORDS(NQ, NKV, D, F)
 * 64-bit words, zero at allocation), tagged with *epoch * n_layers + layer +
 * 1; the head outputs go to out[b, h*hd ..] (fp32), or, with wo (the layer's
 * Wo [D, NQ]), on through tagged words to Wo work-groups in the same launch
 * that add Wo . attn to x (lmk_wo_residual's work; out unused).  With w13 too
 * (rms_ffn, w13 and w2 of the layer, hidden width F), the Wo work-groups hand
 * x on through tagged words to W1/W3 work-groups (lmk_ffn13's work), and
 * those the gate to W2 work-groups that write x (lmk_w2_residual's work): the
 * whole layer in one launch.  err: two ints, the flag a hand-off wait that
 * gives up sets (the kernel still ends) and the microseconds before one does
 * (LM_HANDOFF_US unless set by LM_OPT_HANDOFF_US).  B <= 4, hd 64 or
 * 128.  wgs_per_cu (1-4; 0 = as registers and LDS allow): at most that many
 * work-groups of the whole-layer launch share a CU, enforced with dynamic
 * LDS, so the later roles' work-groups (W1/W3, W2) are dispatched as the
 * early ones finish instead of all at once. */
int lmk_qkv_attn(hipStream_t s, float *x, const uint16_t *emb, const int *tok,
                 const float *rms_w, const uint16_t *wqkv, int D, int NQ, int NKV, int hd,
                 const float *rope_cos, const float *rope_sin, const int *pos, int B,
                 void *kc, void *vc, int kv_f32, int max_seq, int H,
                 unsigned long long *tagged, const unsigned *epoch, int layer,
                 int n_layers, int *err, float *out, const uint16_t *wo,
                 const float *rms_ffn, const uint16_t *w13, const uint16_t *w2, int F,
                 int wgs_per_cu);

/* Whether the whole-layer form of lmk_qkv_attn (w13 given) is built for this
 * model width, hidden width and batch. */
int lmk_layer_fusable(int D, int F, int B);

/* Causal attention, one work-group per (head, row): out[b, h*hd ..] =
 * softmax(q_bh . K[0..pos[b]] / sqrt(hd)) . V over cache slot slot[b] (slot
 * NULL: slot b).  Serves decode rows and prefill rows alike. */
int lmk_attn_decode(hipStream_t s, const float *q, const void *kc,
                    const void *vc, int kv_f32, const int *pos, const int *slot, int B, int H,
                    int Hkv, int hd, int max_seq, float *out, uint16_t *out16);

/* x[b, r] += Wo[r, :] . attn[b] */
int lmk_wo_residual(hipStream_t s, const float *attn, const uint16_t *wo, int D,
                    int B, float *x);

/* xn = rmsnorm(x[b]) * w; g[b, i] = silu(W1[i] . xn) * (W3[i] . xn). */
int lmk_ffn13(hipStream_t s, float *x, const float *rms_w,
              const uint16_t *w13, int D, int F, int B, float *g);

/* x[b, r] += W2[r, :] . g[b, :] */
int lmk_w2_residual(hipStream_t s, const float *g, const uint16_t *w2, int D,
                    int F, int B, float *x);

/* xn = rmsnorm(x[b]) * w; logits[b, v] = Wcls[v] . xn (logits may be NULL);
 * argmax partials (lowest index on ties) to part[b * nblk + blk], nblk =
 * lmk_cls_nblk(V).  With fold_tw (2 * LM_TAG_B * nblk 64-bit words, zero at
 * allocation) the partials go out as tagged words instead, and one more
 * work-group of the launch reduces them as lmk_argmax_final does (tok, and
 * with hist the history and positions), then advances *epoch; a hand-off wait
 * that gives up sets *err. */
int lmk_cls_nblk(int V);
int lmk_cls(hipStream_t s, const float *x, const float *rms_w,
            const uint16_t *wcls, int D, int V, int B, float *logits,
            LMArgPart *part, unsigned long long *fold_tw, unsigned *epoch, int *tok,
            int *pos, int *hist, int hist_stride, int *err);

/* Reduce the argmax partials of each row b: tok[b] = argmax; when hist != NULL,
 * hist[b*hist_stride + pos[b] + 1] = tok[b] and pos[b] += 1 (device-resident
 * greedy loop state); with epoch, *epoch += 1 (the decode-step count that tags
 * lmk_qkv_attn's hand-off words). */
int lmk_argmax_final(hipStream_t s, const LMArgPart *part, int nblk, int B,
                     int *tok, int *pos, int *hist, int hist_stride, unsigned *epoch);

/* ---- prefill attention (k_attn.hip) ----------------------------------------
 * Rows come in nseq whole sequences of S consecutive rows (consecutive
 * positions from pos[first row], cache slot slot[first row]); every row's K/V
 * is already in the cache.  out[r, h*hd ..] = causal attention of row r (fp16). */
int lmk_attn_prefill(hipStream_t s, const float *q, const void *kc, const void *vc,
                     int kv_f32, const int *pos, const int *slot, int S, int nseq,
                     int H, int Hkv, int hd, int max_seq, uint16_t *out);

/* ---- MFMA GEMMs (k_gemm.hip) ----------------------------------------------
 * C[m, n] = sum_k A[m, k] W[n, k], A fp16 [M, lda], W fp16 [N, K], fp32
 * accumulation, on the LDS-tiled MFMA kernel (K % 64 == 0; the tile shape
 * follows M). */

#define LMK_EPI_STORE   0   /* out fp32 [M, ldc]                                   */
#define LMK_EPI_RESID   1   /* out[m, n] += C (fp32 residual stream)               */
#define LMK_EPI_GATE    2   /* g[m, i] = fp16(silu(h1) * h3), W1/W3 interleaved    */
#define LMK_EPI_QKV     3   /* RoPE; q -> fp32 [M, NQ]; k, v -> cache(slot, pos)   */
#define LMK_EPI_ARGMAX  4   /* out (may be NULL) + [M, ceil(N/32)] argmax partials */
#define LMK_EPI_RESNORM 5   /* out += C; u = fp16(out * gain); ss = row sums of out^2
                               per 32 columns (a row norm left to the next GEMM)   */

typedef struct {
    float *out;              /* STORE / RESID                                      */
    int ldc;
    int stream_out;          /* STORE / ARGMAX: out is not read again on the device
                                soon (logits): non-temporal stores                  */
    LMArgPart *part;         /* ARGMAX: [M, ceil(N/32)] argmax partials            */
    uint16_t *g;             /* GATE: [M, F] fp16                                  */
    int F;
    float *q;                /* QKV                                                 */
    void *kc, *vc;           /* layer's cache base: [max_batch][Hkv][max_seq][hd]   */
    int kv_f32, NQ, NKV, hd, Hkv, max_seq;
    const int *slot, *pos;   /* per row                                             */
    const float *rope_cos, *rope_sin;
    /* RESNORM: out[m, n] += C (the residual add), then u[m, n] = fp16(out[m, n] *
     * gain[n]) ([M, N], the next GEMM's operand before its row scale) and
     * ss[m, n/32] = sum of out[m, n]^2 over the 32 columns of block n/32 */
    const float *gain;
    uint16_t *u;
    float *ss;
    int *ovf;                /* RESNORM: set to 1 when a u value is not finite (fp16
                              * overflow of out * gain), or NULL; a device-visible
                              * address (pinned host memory) */
    /* GATE / QKV after a RESNORM GEMM: with rs_ss, product row m is
     * first scaled by 1/sqrt(sum_b rs_ss[m, b] / (32 nss) + 1e-5), the RMSNorm
     * of that row (forward.h:46-53) whose gain is already in the operand */
    const float *rs_ss;
    int nss;                 /* blocks of 32 columns per row of rs_ss / ss; with
                              * rs_ss a multiple of 4, <= 64, rs_ss 16-byte aligned */
} LMEpilogue;

int lmk_gemm(hipStream_t s, const uint16_t *A, int lda, const uint16_t *W, int M, int N,
             int K, int epi, const LMEpilogue *ep);


/* Decode rows after a K-split QKV GEMM: attention of head h, row b with q, k,
 * v summed from the ns partials part[s][b][..] (sstride floats apart) and
 * RoPE'd at pos[b]; k, v appended to the cache at (slot[b], pos[b]); the head
 * output to out16[b, h*hd ..] (fp16). */
int lmk_attn_decode_part(hipStream_t s, const float *part, size_t sstride, int ns, int NQ, int NKV,
                         const int *pos, const int *slot, int B, int H, int Hkv, int hd,
                         int max_seq, const float *rope_cos, const float *rope_sin, void *kc,
                         void *vc, int kv_f32, uint16_t *out16);
/* Arm the calling thread's next decode-chain kernel launch (qkv_rope,
 * qkv_attn, attn, wo_residual, ffn13, w2_residual, cls, argmax_final) to
 * record `start` at its dispatch's start and `stop` at its end (either may be
 * NULL). */
void lmk_time_next(hipEvent_t start, hipEvent_t stop);
/* GEMM with K cut into ns splits: part[s][M][N] (fp32) is split s's partial of
 * A W^T; lmk_pick_split chooses ns for a shape (1: do not split). */
#define LMK_MAX_SPLIT 16
#define LMK_MAX_DEC_SPLIT 8    /* most splits lmk_pick_split gives for M <= 64 */
#define LMK_MAX_ROW_SPLIT 4    /* most splits lmk_pick_split gives for M > 64 */
int lmk_pick_split(int M, int N, int K);
int lmk_gemm_split(hipStream_t s, const uint16_t *A, int lda, const uint16_t *W, int M, int N,
                   int K, int ns, float *part);

/* One work-group per row: with emb != NULL x[m] is first set to the embedding row
 * emb[tok[m]]; with ns > 0 the ns partials sp[s][m] (sstride floats apart) of a
 * K-split projection are added to x[m] first (the residual add); then
 * xn[m] = fp16(x[m] / sqrt(mean(x[m]^2) + 1e-5) * gain). */
int lmk_rownorm(hipStream_t s, float *x, int D, int M, const uint16_t *emb, const int *tok,
                const float *sp, int ns, size_t sstride, const float *gain, uint16_t *xn);

/* ---- loss terms (k_loss.hip) ---------------------------------------------- */

/* M logit rows [M, V] of M/S sequences of S rows, tokens tok[M]: lp[r] =
 * log softmax(logits[r])[tok[r+1]] for rows that are not the last of their
 * sequence (model_forward's loss terms, training/forward.h:174-183), 0 for
 * the last.  V % 4 == 0, S >= 2, M % S == 0. */
int lmk_row_logprob(hipStream_t s, const float *logits, int V, const int *tok, int S, int M,
                    float *lp);

/* ---- allocation-free entry point (k_noalloc.hip) -------------------------- */

/* Look up, once for the current device, the device address of the static
 * argmax-partials scratch of lm_gemm_argmax_noalloc (called by lm_init). */
int lmk_noalloc_setup(void);

/* ---- diagnostics kernels (k_decode.hip) ---------------------------------- */

/* Wave-reduction self-check: out[0..3] = sums computed with the production
 * DPP reduction and with a shuffle reduction over in[0..63]. */
int lmk_selftest_reduce(hipStream_t s, const float *in, float *out);

#ifdef __cplusplus
}
#endif

#endif /* LM_INTERNAL_H */
