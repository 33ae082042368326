/*
 * lm_runtime.c — the C-ABI runtime of the Stories token loop (C99 over the HIP
 * C runtime API).  It owns device memory, the stream, the per-batch decode
 * graphs and the host-facing entry points of stories_lm.h; every kernel is
 * reached through the lmk_* launchers of the HIP translation units.
 *
 * Device layout (all row-major, W[out, in]):
 *   layer block l (one allocation for all layers, layer after layer):
 *     Wqkv [NQ + 2*NKV, D]   Wq rows, then Wk rows, then Wv rows
 *     Wo   [D, NQ]
 *     W13  [2F, D]           W1/W3 rows interleaved in blocks of 16
 *     W2   [D, F]
 *   embed [V, D], wcls [V, D] (the embedding itself when tied)   fp16
 *   rms_att [L, D], rms_ffn [L, D], rms_final [D]                  fp32
 *   RoPE cos/sin [max_seq, hd/2]                                   fp32
 *   K/V cache, per layer [max_batch][Hkv][max_seq][hd]             fp16
 *   residual x [rows, D], q [rows, NQ], gate g [rows, F],
 *   logits [rows, V]                                               fp32
 */
#include "lm_internal.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define HIPCHK(call)                                                                 \
    do {                                                                             \
        hipError_t e_ = (call);                                                      \
        if (e_ != hipSuccess) {                                                      \
            fprintf(stderr, "stories_lm: %s failed at %s:%d: %s\n", #call, __FILE__, \
                    __LINE__, hipGetErrorString(e_));                                \
            return LM_ERR_HIP;                                                       \
        }                                                                            \
    } while (0)

#define MAX_GEMV_B 4
#define PREFILL_GRAPHS 4   /* prefill chunk shapes kept captured */

struct LMModel {
    Config cfg;                 /* vocab_size positive */
    int untied;
    int D, F, L, H, Hkv, hd, NQ, NKV, V;
    int max_batch, max_seq, max_rows;
    int cls_nblk;
    size_t layer_elems, off_wo, off_w13, off_w2;
    hipStream_t stream;
    hipEvent_t ev0, ev1;
    hipEvent_t ev_hand;         /* end of this handle's last hand-off launches */
    /* weights */
    uint16_t *d_layers, *d_embed, *d_wcls;
    float *d_rms_att, *d_rms_ffn, *d_rms_final;
    float *d_rope_cos, *d_rope_sin;
    /* cache + activations */
    void *d_kc, *d_vc;
    size_t kv_layer_elems;
    int kv_f32;                 /* cache element: 0 = binary16, 1 = fp32 */
    /* per-row activations, max_rows rows (decode rows, or a prefill chunk) */
    float *d_x, *d_q, *d_attn, *d_g, *d_logits;
    float *d_ss;                /* per-row sums of squares of x, D/32 per row  */
    float *d_part;              /* partials of K-split GEMMs, Wo/W2 products    */
    uint16_t *d_g16;            /* gate rows in fp16 (input of the W2 GEMM)    */
    uint16_t *d_xn16, *d_a16;   /* normalised rows / attention rows in fp16    */
    LMArgPart *d_amax;
    int *d_rin;                 /* prefill rows of a chunk of R: tokens, positions, slots
                                 * (R ints each, back to back), copied in one piece;
                                 * then R floats of loss terms (lm_prefill_loss)     */
    int *h_rin;                 /* their pinned host staging (same layout)          */
    /* per-slot greedy state */
    int *d_tok, *d_pos, *d_hist, *d_slot_id;
    /* batch 1-4 chain: QKV, attention (fuse_qa >= 1), Wo (>= 2) and the FFN
     * (3 at one row, 4 at every batch; chain_level) in one launch, handing q,
     * k, v, the head outputs, x and the gate over through tagged words; the
     * decode-step count that tags them; the flag a hand-off wait that gives up
     * sets, and the polls before one does */
    int fuse_qa;
    int prefill_fold;           /* LM_OPT_PREFILL_FOLD */
    int fold_off;               /* the folded norm is off for the rows being redone */
    int *d_ovf;                 /* device address of ovf_slot: RESNORM's overflow flag */
    int layer_wgs;              /* whole-layer work-groups per CU at most (0: no cap) */
    unsigned long long *d_tagged;
    unsigned long long *d_cls_tw;     /* the classifier's argmax partials as tagged words (level 3) */
    unsigned *d_epoch;
    int *d_err;
    /* pinned host staging */
    float *h_logits;
    int *h_io;
    /* captured decode graphs: [B][0] one step, [B][1] GRAPH_STEPS steps
     * (greedy feedback stays on the device) */
    hipGraphExec_t (*step_graph)[2];   /* [max_batch + 1][2]   */
    /* captured prefill chunks (the layers and, with all logits, the
     * classifier), by rows, rows per sequence and logits mode; replaced round
     * robin */
    struct {
        int R, S, all;
        hipGraphExec_t ge;
    } pgraph[PREFILL_GRAPHS];
    int pgraph_next;
    int use_graph;
};

static int g_init_status = 1; /* 1 = not attempted */

const char *lm_strerror(int status)
{
    switch (status) {
    case LM_OK: return "ok";
    case LM_ERR_NO_DEVICE: return "no HIP device";
    case LM_ERR_NOT_GFX950: return "device is not gfx950";
    case LM_ERR_INVALID: return "invalid argument";
    case LM_ERR_OOM: return "out of memory";
    case LM_ERR_HIP: return "HIP runtime error";
    case LM_ERR_IO: return "I/O error";
    case LM_ERR_FORMAT: return "bad or truncated weight file";
    case LM_ERR_RANGE: return "token, position, slot or length out of range";
    case LM_ERR_UNSUPPORTED: return "shape not supported by the kernels";
    case LM_ERR_NOT_INIT: return "lm_init not called or failed";
    default: return "unknown status";
    }
}

/* The device checks run once per process (pthread_once), so concurrent first
 * calls from several threads neither race on the status nor repeat the
 * setup; every call returns the one recorded status. */
static pthread_once_t g_init_once = PTHREAD_ONCE_INIT;

static void init_once(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        fprintf(stderr, "stories_lm: no HIP device visible\n");
        g_init_status = LM_ERR_NO_DEVICE;
        return;
    }
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) {
        g_init_status = LM_ERR_NO_DEVICE;
        return;
    }
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        fprintf(stderr, "stories_lm: device 0 is %s, kernels are built for gfx950\n",
                p.gcnArchName);
        g_init_status = LM_ERR_NOT_GFX950;
        return;
    }
    if (hipSetDevice(0) != hipSuccess) {
        g_init_status = LM_ERR_NO_DEVICE;
        return;
    }
    if (lmk_noalloc_setup() != hipSuccess) {
        fprintf(stderr, "stories_lm: lookup of the static scratch's device address failed\n");
        g_init_status = LM_ERR_HIP;
        return;
    }
    g_init_status = LM_OK;
}

int lm_init(void)
{
    if (pthread_once(&g_init_once, init_once) != 0) return LM_ERR_NOT_INIT;
    return g_init_status;
}

int lm_device_info(LMDeviceInfo *out)
{
    if (!out) return LM_ERR_INVALID;
    int rc = lm_init();
    if (rc) return rc;
    hipDeviceProp_t p;
    HIPCHK(hipGetDeviceProperties(&p, 0));
    memset(out, 0, sizeof(*out));
    snprintf(out->name, sizeof(out->name), "%.63s", p.name);
    snprintf(out->arch, sizeof(out->arch), "%.31s", p.gcnArchName);
    out->compute_units = p.multiProcessorCount;
    out->clock_khz = p.clockRate;
    out->l2_bytes = p.l2CacheSize;
    out->total_mem = p.totalGlobalMem;
    return LM_OK;
}

/* ------------------------------------------------------------------------- */
/* creation                                                                   */
/* ------------------------------------------------------------------------- */

static int dev_alloc(void **p, size_t bytes)
{
    *p = NULL;
    if (bytes == 0) return LM_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        fprintf(stderr, "stories_lm: hipMalloc(%zu) failed: %s\n", bytes, hipGetErrorString(e));
        *p = NULL;
        return LM_ERR_OOM;
    }
    return LM_OK;
}

/* Copy n elements of tensor src (fp32 or fp16) as fp16 into dst (host). */
static void to_f16(const void *src, LMDType dt, size_t off, size_t n, uint16_t *dst)
{
    if (dt == LM_DTYPE_F16)
        memcpy(dst, (const uint16_t *)src + off, n * 2);
    else
        lm_f32_to_f16((const float *)src + off, dst, n);
}

static void to_f32(const void *src, LMDType dt, size_t off, size_t n, float *dst)
{
    if (dt == LM_DTYPE_F32)
        memcpy(dst, (const float *)src + off, n * 4);
    else
        lm_f16_to_f32((const uint16_t *)src + off, dst, n);
}

/* Where the host weights come from: one contiguous block per tensor
 * (LMWeights) or per-layer pointer arrays (LMLayerWeights). */
typedef struct {
    LMDType dtype;
    const void *embed, *rms_final, *wcls;   /* wcls NULL: tied */
    const LMWeights *flat;
    const LMLayerWeights *per;
} WSrc;

static const void *const *per_layer_array(const LMLayerWeights *w, int t)
{
    switch (t) {
    case LMH_T_RMS_ATT: return w->rms_att_w;
    case LMH_T_WQ: return w->wq;
    case LMH_T_WK: return w->wk;
    case LMH_T_WV: return w->wv;
    case LMH_T_WO: return w->wo;
    case LMH_T_RMS_FFN: return w->rms_ffn_w;
    case LMH_T_W1: return w->w1;
    case LMH_T_W2: return w->w2;
    case LMH_T_W3: return w->w3;
    default: return NULL;
    }
}

/* Layer l's tensor t (n elements per layer) in the source's element type. */
static const void *src_layer(const WSrc *ws, int t, size_t l, size_t n)
{
    if (ws->per) return per_layer_array(ws->per, t)[l];
    const char *base = (const char *)lmh_weights_ptr(ws->flat, t);
    return base + l * n * (ws->dtype == LM_DTYPE_F16 ? 2 : 4);
}

static int upload_weights(LMModel *m, const WSrc *w)
{
    const size_t D = m->D, F = m->F, NQ = m->NQ, NKV = m->NKV, V = m->V, L = m->L;
    const size_t GB = LMK_GATE_BLOCK;
    const LMDType dt = w->dtype;
    uint16_t *stage = (uint16_t *)malloc(m->layer_elems * 2);
    float *nf = (float *)malloc(L * D * 4);
    if (!stage || !nf) { free(stage); free(nf); return LM_ERR_OOM; }
    int rc = LM_OK;
    for (size_t l = 0; l < L && rc == LM_OK; l++) {
        uint16_t *p = stage;
        to_f16(src_layer(w, LMH_T_WQ, l, NQ * D), dt, 0, NQ * D, p);    p += NQ * D;
        to_f16(src_layer(w, LMH_T_WK, l, NKV * D), dt, 0, NKV * D, p);  p += NKV * D;
        to_f16(src_layer(w, LMH_T_WV, l, NKV * D), dt, 0, NKV * D, p);  p += NKV * D;
        to_f16(src_layer(w, LMH_T_WO, l, D * NQ), dt, 0, D * NQ, p);    p += D * NQ;
        const void *w1 = src_layer(w, LMH_T_W1, l, F * D), *w3 = src_layer(w, LMH_T_W3, l, F * D);
        for (size_t j = 0; j < F / GB; j++) {
            to_f16(w1, dt, j * GB * D, GB * D, p); p += GB * D;
            to_f16(w3, dt, j * GB * D, GB * D, p); p += GB * D;
        }
        to_f16(src_layer(w, LMH_T_W2, l, D * F), dt, 0, D * F, p);
        if (hipMemcpy(m->d_layers + l * m->layer_elems, stage, m->layer_elems * 2,
                      hipMemcpyHostToDevice) != hipSuccess)
            rc = LM_ERR_HIP;
    }
    free(stage);
    if (rc == LM_OK) {
        uint16_t *e16 = (uint16_t *)malloc(V * D * 2);
        if (!e16) rc = LM_ERR_OOM;
        if (rc == LM_OK) {
            to_f16(w->embed, dt, 0, V * D, e16);
            if (hipMemcpy(m->d_embed, e16, V * D * 2, hipMemcpyHostToDevice) != hipSuccess)
                rc = LM_ERR_HIP;
            if (rc == LM_OK && m->untied) {
                to_f16(w->wcls, dt, 0, V * D, e16);
                if (hipMemcpy(m->d_wcls, e16, V * D * 2, hipMemcpyHostToDevice) != hipSuccess)
                    rc = LM_ERR_HIP;
            }
        }
        free(e16);
    }
    if (rc == LM_OK) {
        for (size_t l = 0; l < L; l++) to_f32(src_layer(w, LMH_T_RMS_ATT, l, D), dt, 0, D, nf + l * D);
        if (hipMemcpy(m->d_rms_att, nf, L * D * 4, hipMemcpyHostToDevice) != hipSuccess) rc = LM_ERR_HIP;
        for (size_t l = 0; l < L; l++) to_f32(src_layer(w, LMH_T_RMS_FFN, l, D), dt, 0, D, nf + l * D);
        if (rc == LM_OK && hipMemcpy(m->d_rms_ffn, nf, L * D * 4, hipMemcpyHostToDevice) != hipSuccess)
            rc = LM_ERR_HIP;
        to_f32(w->rms_final, dt, 0, D, nf);
        if (rc == LM_OK && hipMemcpy(m->d_rms_final, nf, D * 4, hipMemcpyHostToDevice) != hipSuccess)
            rc = LM_ERR_HIP;
    }
    free(nf);
    return rc;
}

static size_t kv_bytes(const LMModel *m)
{
    return (size_t)m->L * m->kv_layer_elems * (m->kv_f32 ? 4 : 2);
}

/* (Re)allocate the K/V cache in the current element type, zero-filled. */
static int alloc_kv(LMModel *m)
{
    if (m->d_kc) { hipFree(m->d_kc); m->d_kc = NULL; }
    if (m->d_vc) { hipFree(m->d_vc); m->d_vc = NULL; }
    int st = dev_alloc(&m->d_kc, kv_bytes(m));
    if (!st) st = dev_alloc(&m->d_vc, kv_bytes(m));
    if (st) return st;
    if (hipMemset(m->d_kc, 0, kv_bytes(m)) != hipSuccess ||
        hipMemset(m->d_vc, 0, kv_bytes(m)) != hipSuccess)
        return LM_ERR_HIP;
    return LM_OK;
}

static void drop_graphs(LMModel *m)
{
    for (int i = 0; i < PREFILL_GRAPHS; i++)
        if (m->pgraph[i].ge) {
            hipGraphExecDestroy(m->pgraph[i].ge);
            m->pgraph[i].ge = NULL;
        }
    if (!m->step_graph) return;
    for (int b = 0; b <= m->max_batch; b++)
        for (int k = 0; k < 2; k++)
            if (m->step_graph[b][k]) {
                hipGraphExecDestroy(m->step_graph[b][k]);
                m->step_graph[b][k] = NULL;
            }
}

static void free_rows(LMModel *m)
{
    void *dev[] = {m->d_x, m->d_q, m->d_attn, m->d_g, m->d_logits, m->d_ss, m->d_part, m->d_g16,
                   m->d_xn16, m->d_a16, m->d_amax, m->d_rin};
    for (size_t i = 0; i < sizeof(dev) / sizeof(dev[0]); i++)
        if (dev[i]) hipFree(dev[i]);
    if (m->h_rin) hipHostFree(m->h_rin);
    m->d_x = m->d_q = m->d_attn = m->d_g = m->d_logits = m->d_ss = m->d_part = NULL;
    m->d_g16 = m->d_xn16 = m->d_a16 = NULL;
    m->d_amax = NULL;
    m->d_rin = m->h_rin = NULL;
    m->max_rows = 0;
}

/* (Re)allocate the per-row activation buffers for R rows.  Captured graphs
 * hold the old addresses, so they are dropped. */
static int alloc_rows(LMModel *m, int R)
{
    if (m->stream && hipStreamSynchronize(m->stream) != hipSuccess) return LM_ERR_HIP;
    drop_graphs(m);
    free_rows(m);
    const size_t r = (size_t)R, D = m->D, F = m->F, NQ = m->NQ, V = m->V;
    int st;
    if ((st = dev_alloc((void **)&m->d_x, r * D * 4))) return st;
    if ((st = dev_alloc((void **)&m->d_q, r * NQ * 4))) return st;
    if ((st = dev_alloc((void **)&m->d_attn, r * NQ * 4))) return st;
    if ((st = dev_alloc((void **)&m->d_g, r * F * 4))) return st;
    if ((st = dev_alloc((void **)&m->d_g16, r * F * 2))) return st;
    if ((st = dev_alloc((void **)&m->d_xn16, r * D * 2))) return st;
    if ((st = dev_alloc((void **)&m->d_a16, r * NQ * 2))) return st;
    if ((st = dev_alloc((void **)&m->d_logits, r * V * 4))) return st;
    if ((st = dev_alloc((void **)&m->d_ss, r * (D / 32) * 4))) return st;
    {
        /* K-split partials (widest: QKV of decode rows), or one [R, D] product
         * of prefill rows */
        const size_t w = NQ + 2 * (size_t)m->NKV > D ? NQ + 2 * (size_t)m->NKV : D;
        const size_t rd = r < 64 ? r : 64;
        size_t n = LMK_MAX_SPLIT * rd * w;
        if (r > 64 && LMK_MAX_ROW_SPLIT * r * w > n) n = LMK_MAX_ROW_SPLIT * r * w;
        if (r * D > n) n = r * D;
        if ((st = dev_alloc((void **)&m->d_part, n * 4))) return st;
    }
    if ((st = dev_alloc((void **)&m->d_amax, r * m->cls_nblk * sizeof(LMArgPart)))) return st;
    /* tokens, positions and slots of a chunk's rows, then its rows' loss terms */
    if ((st = dev_alloc((void **)&m->d_rin, 4 * r * 4))) return st;
    if (hipHostMalloc((void **)&m->h_rin, 4 * r * 4, 0) != hipSuccess) {
        m->h_rin = NULL;
        return LM_ERR_OOM;
    }
    m->max_rows = R;
    return LM_OK;
}

static int supported_k(int k)
{
    return k == 256 || k == 512 || k == 768 || k == 1024 || k == 2048 || k == 5632;
}

static LMModel *create_model(const Config *cfg, const WSrc *w, int max_batch, int max_seq,
                             int *status);

LMModel *lm_create(const Config *cfg, const LMWeights *w, int max_batch, int max_seq, int *status)
{
    int st = LM_OK;
    if (!cfg || !w || max_batch < 1 || max_seq < 1 ||
        (w->dtype != LM_DTYPE_F32 && w->dtype != LM_DTYPE_F16))
        st = LM_ERR_INVALID;
    for (int t = 0; t < LMH_NTENSORS - 1 && st == LM_OK; t++)
        if (!lmh_weights_ptr(w, t)) {
            fprintf(stderr, "stories_lm: weight tensor %d is NULL\n", t);
            st = LM_ERR_INVALID;
        }
    if (st != LM_OK) {
        if (status) *status = st;
        fprintf(stderr, "stories_lm: lm_create failed: %s\n", lm_strerror(st));
        return NULL;
    }
    const WSrc ws = {w->dtype, w->token_embedding, w->rms_final_w,
                     lmh_weights_untied(w) ? w->wcls : NULL, w, NULL};
    return create_model(cfg, &ws, max_batch, max_seq, status);
}

LMModel *lm_create_layers(const Config *cfg, const LMLayerWeights *w, int max_batch, int max_seq,
                          int *status)
{
    int st = LM_OK;
    if (!cfg || !w || max_batch < 1 || max_seq < 1 || cfg->n_layers < 1 ||
        (w->dtype != LM_DTYPE_F32 && w->dtype != LM_DTYPE_F16) || !w->token_embedding ||
        !w->rms_final_w)
        st = LM_ERR_INVALID;
    for (int t = LMH_T_RMS_ATT; t <= LMH_T_W3 && st == LM_OK; t++) {
        const void *const *a = per_layer_array(w, t);
        if (!a) {
            fprintf(stderr, "stories_lm: per-layer weight array %d is NULL\n", t);
            st = LM_ERR_INVALID;
        }
        for (int l = 0; a && l < cfg->n_layers && st == LM_OK; l++)
            if (!a[l]) {
                fprintf(stderr, "stories_lm: weight tensor %d of layer %d is NULL\n", t, l);
                st = LM_ERR_INVALID;
            }
    }
    if (st != LM_OK) {
        if (status) *status = st;
        fprintf(stderr, "stories_lm: lm_create_layers failed: %s\n", lm_strerror(st));
        return NULL;
    }
    const WSrc ws = {w->dtype, w->token_embedding, w->rms_final_w,
                     w->wcls && w->wcls != w->token_embedding ? w->wcls : NULL, NULL, w};
    return create_model(cfg, &ws, max_batch, max_seq, status);
}

static LMModel *create_model(const Config *cfg, const WSrc *w, int max_batch, int max_seq,
                             int *status)
{
    int st = LM_OK;
    LMModel *m = NULL;
#define FAIL(code)      \
    do {                \
        st = (code);    \
        goto fail;      \
    } while (0)
    if ((st = lm_init()) != LM_OK) goto fail;
    if ((st = lmh_check_config(cfg)) != LM_OK) {
        fprintf(stderr, "stories_lm: inconsistent Config\n");
        goto fail;
    }
    m = (LMModel *)calloc(1, sizeof(LMModel));
    if (!m) FAIL(LM_ERR_OOM);
    m->cfg = *cfg;
    m->V = cfg->vocab_size < 0 ? -cfg->vocab_size : cfg->vocab_size;
    m->cfg.vocab_size = m->V;
    m->untied = w->wcls != NULL;
    m->D = cfg->dim; m->F = cfg->hidden_dim; m->L = cfg->n_layers;
    m->H = cfg->n_heads; m->Hkv = cfg->n_kv_heads;
    m->hd = m->D / m->H;
    m->NQ = m->H * m->hd;
    m->NKV = m->Hkv * m->hd;
    if ((m->hd != 64 && m->hd != 128) || !supported_k(m->D) || m->D == 5632 || !supported_k(m->F)) {
        fprintf(stderr, "stories_lm: unsupported shape dim=%d hidden=%d head_dim=%d "
                "(need head_dim 64/128, dim in {256,512,768,1024,2048}, hidden also 5632)\n",
                m->D, m->F, m->hd);
        FAIL(LM_ERR_UNSUPPORTED);
    }
    if (max_seq > (1 << 16) || max_batch > 4096) FAIL(LM_ERR_RANGE);
    m->max_batch = max_batch;
    m->max_seq = max_seq;
    m->cls_nblk = lmk_cls_nblk(m->V);
    m->use_graph = 1;

    const size_t D = m->D, F = m->F, NQ = m->NQ, NKV = m->NKV, V = m->V, L = m->L;
    m->off_wo = (NQ + 2 * NKV) * D;
    m->off_w13 = m->off_wo + D * NQ;
    m->off_w2 = m->off_w13 + 2 * F * D;
    m->layer_elems = m->off_w2 + D * F;
    m->kv_layer_elems = (size_t)max_batch * m->Hkv * max_seq * m->hd;
    const size_t NB = (size_t)max_batch;
    m->step_graph = (hipGraphExec_t(*)[2])calloc(NB + 1, sizeof(*m->step_graph));
    if (!m->step_graph) FAIL(LM_ERR_OOM);

    if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) FAIL(LM_ERR_HIP);
    if (hipEventCreate(&m->ev0) != hipSuccess || hipEventCreate(&m->ev1) != hipSuccess ||
        hipEventCreateWithFlags(&m->ev_hand, hipEventDisableTiming) != hipSuccess)
        FAIL(LM_ERR_HIP);
    if ((st = dev_alloc((void **)&m->d_layers, L * m->layer_elems * 2))) goto fail;
    if ((st = dev_alloc((void **)&m->d_embed, V * D * 2))) goto fail;
    if (m->untied) {
        if ((st = dev_alloc((void **)&m->d_wcls, V * D * 2))) goto fail;
    } else {
        m->d_wcls = m->d_embed;
    }
    if ((st = dev_alloc((void **)&m->d_rms_att, L * D * 4))) goto fail;
    if ((st = dev_alloc((void **)&m->d_rms_ffn, L * D * 4))) goto fail;
    if ((st = dev_alloc((void **)&m->d_rms_final, D * 4))) goto fail;
    if ((st = dev_alloc((void **)&m->d_rope_cos, (size_t)max_seq * m->hd / 2 * 4))) goto fail;
    if ((st = dev_alloc((void **)&m->d_rope_sin, (size_t)max_seq * m->hd / 2 * 4))) goto fail;
    if ((st = alloc_kv(m))) goto fail;
    if ((st = alloc_rows(m, max_batch))) goto fail;
    if ((st = dev_alloc((void **)&m->d_tok, NB * 4))) goto fail;
    if ((st = dev_alloc((void **)&m->d_pos, NB * 4))) goto fail;
    if ((st = dev_alloc((void **)&m->d_slot_id, NB * 4))) goto fail;
    if ((st = dev_alloc((void **)&m->d_hist, (size_t)max_batch * (max_seq + 1) * 4))) goto fail;
    const size_t ntag = LM_TAG_WORDS(NQ, NKV, D, F);
    if ((st = dev_alloc((void **)&m->d_tagged, ntag * 8))) goto fail;
    const size_t ncls = (size_t)2 * LM_TAG_B * m->cls_nblk;
    if ((st = dev_alloc((void **)&m->d_cls_tw, ncls * 8))) goto fail;
    if ((st = dev_alloc((void **)&m->d_epoch, 4))) goto fail;
    if ((st = dev_alloc((void **)&m->d_err, 8))) goto fail;   /* flag, wait limit (us) */
    if (hipMemset(m->d_tagged, 0, ntag * 8) != hipSuccess || hipMemset(m->d_cls_tw, 0, ncls * 8) != hipSuccess ||
        hipMemset(m->d_epoch, 0, 4) != hipSuccess || hipMemset(m->d_err, 0, 4) != hipSuccess)
        FAIL(LM_ERR_HIP);
    {
        const int lim_us = LM_HANDOFF_US;
        if (hipMemcpy(m->d_err + 1, &lim_us, 4, hipMemcpyHostToDevice) != hipSuccess) FAIL(LM_ERR_HIP);
    }
    m->fuse_qa = 3;
    m->layer_wgs = 2;
    m->prefill_fold = 1;
    if (hipHostMalloc((void **)&m->h_logits, (size_t)max_batch * V * 4, 0) != hipSuccess) FAIL(LM_ERR_OOM);
    if (hipHostMalloc((void **)&m->h_io, (size_t)4 * (max_batch + 1) * 4, 0) != hipSuccess) FAIL(LM_ERR_OOM);
    memset(m->h_io, 0, (size_t)4 * (max_batch + 1) * 4);
    /* RESNORM's overflow flag: the int after the hand-off flag's slot, written
     * by the device only when a prefill row overflows */
    if (hipHostGetDevicePointer((void **)&m->d_ovf, m->h_io + 4 * (size_t)max_batch + 1, 0) != hipSuccess)
        FAIL(LM_ERR_HIP);

    if ((st = upload_weights(m, w))) goto fail;
    {
        size_t n = (size_t)max_seq * m->hd / 2;
        float *c = (float *)malloc(n * 4), *s = (float *)malloc(n * 4);
        if (!c || !s) { free(c); free(s); FAIL(LM_ERR_OOM); }
        lm_rope_table(max_seq, m->hd, c, s);
        hipError_t e1 = hipMemcpy(m->d_rope_cos, c, n * 4, hipMemcpyHostToDevice);
        hipError_t e2 = hipMemcpy(m->d_rope_sin, s, n * 4, hipMemcpyHostToDevice);
        free(c); free(s);
        if (e1 != hipSuccess || e2 != hipSuccess) FAIL(LM_ERR_HIP);
    }
    if (hipMemset(m->d_hist, 0, (size_t)max_batch * (max_seq + 1) * 4) != hipSuccess ||
        hipMemset(m->d_pos, 0, NB * 4) != hipSuccess || hipMemset(m->d_tok, 0, NB * 4) != hipSuccess)
        FAIL(LM_ERR_HIP);
    {
        int *ids = (int *)malloc(NB * 4);
        if (!ids) FAIL(LM_ERR_OOM);
        for (int b = 0; b < max_batch; b++) ids[b] = b;
        hipError_t e = hipMemcpy(m->d_slot_id, ids, NB * 4, hipMemcpyHostToDevice);
        free(ids);
        if (e != hipSuccess) FAIL(LM_ERR_HIP);
    }
    if (hipDeviceSynchronize() != hipSuccess) FAIL(LM_ERR_HIP);
    if (status) *status = LM_OK;
    return m;
fail:
    if (status) *status = st;
    if (st != LM_OK) fprintf(stderr, "stories_lm: lm_create failed: %s\n", lm_strerror(st));
    lm_free(m);
    return NULL;
#undef FAIL
}

LMModel *lm_load_llama2c(const char *path, int max_batch, int max_seq, int *status)
{
    if (!path) {
        if (status) *status = LM_ERR_INVALID;
        return NULL;
    }
    Config cfg;
    int untied = 0;
    float *data = NULL;
    int rc = lmh_read_llama2c(path, &cfg, &untied, &data);
    if (rc) {
        if (status) *status = rc;
        return NULL;
    }
    LMWeights w;
    lm_weights_view(&cfg, LM_DTYPE_F32, data, untied, &w);
    LMModel *m = lm_create(&cfg, &w, max_batch, max_seq, status);
    free(data);
    return m;
}

LMModel *lm_load_blzt(const char *path, int max_batch, int max_seq, int *status)
{
    if (!path) {
        if (status) *status = LM_ERR_INVALID;
        return NULL;
    }
    Config cfg;
    float *data = NULL;
    int rc = lmh_read_blzt(path, &cfg, &data);
    if (rc) {
        if (status) *status = rc;
        return NULL;
    }
    LMWeights w;
    lm_weights_view(&cfg, LM_DTYPE_F32, data, 0, &w);
    LMModel *m = lm_create(&cfg, &w, max_batch, max_seq, status);
    free(data);
    return m;
}

/* Launches that hold hand-off waits (the batch 1-4 decode chain at fusion
 * levels 1-4) rely on in-order dispatch of their own work-groups on each XCD:
 * a launch's lowest unfinished work-group always finds its producers done or
 * running.  Two such launches of different handles in flight at once could
 * each hold the slots the other's lowest pending work-group needs.  So their
 * launches are ordered on the device: under g_hand_mu, a handle's stream first
 * waits for the last hand-off launches any other handle enqueued (g_hand_last),
 * then enqueues its own and records ev_hand, which becomes g_hand_last.  The
 * rest of the work of distinct handles (prefill, batched decode, copies) still
 * runs concurrently. */
static pthread_mutex_t g_hand_mu = PTHREAD_MUTEX_INITIALIZER;
static LMModel *g_hand_owner;   /* handle whose ev_hand g_hand_last is */

static int handoff_enter(LMModel *m)
{
    pthread_mutex_lock(&g_hand_mu);
    if (g_hand_owner && g_hand_owner != m &&
        hipStreamWaitEvent(m->stream, g_hand_owner->ev_hand, 0) != hipSuccess) {
        pthread_mutex_unlock(&g_hand_mu);
        fprintf(stderr, "stories_lm: hipStreamWaitEvent on another handle's decode failed\n");
        return LM_ERR_HIP;
    }
    return LM_OK;
}

/* rc: the status of what was enqueued since handoff_enter (passed through) */
static int handoff_leave(LMModel *m, int rc)
{
    if (hipEventRecord(m->ev_hand, m->stream) == hipSuccess) {
        g_hand_owner = m;
    } else {
        g_hand_owner = NULL;   /* nothing later waits on an unrecorded event */
        if (rc == LM_OK) rc = LM_ERR_HIP;
    }
    pthread_mutex_unlock(&g_hand_mu);
    return rc;
}

/* A handle being freed (its stream already synchronised) leaves the chain. */
static void handoff_forget(LMModel *m)
{
    pthread_mutex_lock(&g_hand_mu);
    if (g_hand_owner == m) g_hand_owner = NULL;
    pthread_mutex_unlock(&g_hand_mu);
}

void lm_free(LMModel *m)
{
    if (!m) return;
    if (m->stream) hipStreamSynchronize(m->stream);
    handoff_forget(m);
    drop_graphs(m);
    free(m->step_graph);
    free_rows(m);
    void *dev[] = {m->d_layers, m->d_embed, m->untied ? m->d_wcls : NULL, m->d_rms_att,
                   m->d_rms_ffn, m->d_rms_final, m->d_rope_cos, m->d_rope_sin, m->d_kc,
                   m->d_vc, m->d_tok, m->d_pos, m->d_hist, m->d_slot_id, m->d_tagged, m->d_cls_tw, m->d_epoch,
                   m->d_err};
    for (size_t i = 0; i < sizeof(dev) / sizeof(dev[0]); i++)
        if (dev[i]) hipFree(dev[i]);
    if (m->h_logits) hipHostFree(m->h_logits);
    if (m->h_io) hipHostFree(m->h_io);
    if (m->ev0) hipEventDestroy(m->ev0);
    if (m->ev1) hipEventDestroy(m->ev1);
    if (m->ev_hand) hipEventDestroy(m->ev_hand);
    if (m->stream) hipStreamDestroy(m->stream);
    free(m);
}

int lm_get_config(const LMModel *m, Config *out)
{
    if (!m || !out) return LM_ERR_INVALID;
    *out = m->cfg;
    return LM_OK;
}

int lm_set_option(LMModel *m, int option, int value)
{
    if (!m) return LM_ERR_INVALID;
    switch (option) {
    case LM_OPT_USE_GRAPH:
        m->use_graph = value ? 1 : 0;
        return LM_OK;
    case LM_OPT_FUSE_QKV_ATTN:
        if (value < 0 || value > 4) return LM_ERR_INVALID;
        if (value == m->fuse_qa) return LM_OK;
        HIPCHK(hipStreamSynchronize(m->stream));
        drop_graphs(m);
        m->fuse_qa = value;
        return LM_OK;
    case LM_OPT_LAYER_WGS:
        if (value < 0 || value > 4) return LM_ERR_INVALID;
        if (value == m->layer_wgs) return LM_OK;
        HIPCHK(hipStreamSynchronize(m->stream));
        drop_graphs(m);
        m->layer_wgs = value;
        return LM_OK;
    case LM_OPT_PREFILL_FOLD:
        if (value != 0 && value != 1) return LM_ERR_INVALID;
        if (value == m->prefill_fold) return LM_OK;
        HIPCHK(hipStreamSynchronize(m->stream));
        drop_graphs(m);
        m->prefill_fold = value;
        return LM_OK;
    case LM_OPT_HANDOFF_US:
        if (value < 1) return LM_ERR_INVALID;
        HIPCHK(hipStreamSynchronize(m->stream));
        HIPCHK(hipMemcpy(m->d_err + 1, &value, 4, hipMemcpyHostToDevice));
        return LM_OK;
    case LM_OPT_HANDOFF_ABORT:
        /* raise the give-up flag from the host: every hand-off wait of the
         * next call ends at once (the kernels still run to their end) and
         * the call reports LM_ERR_HIP, then clears the flag */
        if (value != 1) return LM_ERR_INVALID;
        HIPCHK(hipStreamSynchronize(m->stream));
        HIPCHK(hipMemcpy(m->d_err, &value, 4, hipMemcpyHostToDevice));
        return LM_OK;
    case LM_OPT_KV_F32:
        if ((value ? 1 : 0) == m->kv_f32) return LM_OK;
        HIPCHK(hipStreamSynchronize(m->stream));
        drop_graphs(m);
        m->kv_f32 = value ? 1 : 0;
        return alloc_kv(m);
    default:
        return LM_ERR_INVALID;
    }
}

/* ------------------------------------------------------------------------- */
/* decode step                                                                */
/* ------------------------------------------------------------------------- */

#define KCHK(call)                                                                    \
    do {                                                                              \
        int e_ = (call);                                                              \
        if (e_ != 0) {                                                                \
            fprintf(stderr, "stories_lm: launch %s failed: %s\n", #call,              \
                    hipGetErrorString((hipError_t)e_));                               \
            return LM_ERR_HIP;                                                        \
        }                                                                             \
    } while (0)

/* The decode chain's fusion level for B rows: fuse_qa, where 3 takes the
 * whole-layer launch for one row only (B = 2 and 4 ran faster at level 2:
 * 203 and 281 us/step against 207 and 385) and 4 takes it for every batch;
 * the whole-layer launch is built only for the (dim, hidden) pairs and
 * batches lmk_layer_fusable names, and level 2 runs elsewhere. */
static int chain_level(const LMModel *m, int B)
{
    int lvl = m->fuse_qa;
    if (lvl == 3 && B > 1) lvl = 2;
    if (lvl == 4) lvl = 3;
    return lvl == 3 && !lmk_layer_fusable(m->D, m->F, B) ? 2 : lvl;
}

/* Whether kernel family fam runs inside another family's launch at fusion
 * level lvl (the QKV launch; at level 3 the argmax inside the classifier's). */
static int fam_inside(int fam, int lvl)
{
    return (fam == LM_KERN_ATTN && lvl >= 1) || (fam == LM_KERN_WO && lvl >= 2) ||
           ((fam == LM_KERN_W13 || fam == LM_KERN_W2 || fam == LM_KERN_ARGMAX) && lvl >= 3);
}

/* Queue the kernel of family `fam` (LM_KERN_*) of layer l for rows 0..B-1
 * (nothing for a family that runs inside the QKV launch). */
static int enqueue_kernel(LMModel *m, int B, int fam, int l, float *logits)
{
    const int lvl = chain_level(m, B);
    if (fam_inside(fam, lvl)) return LM_OK;
    hipStream_t s = m->stream;
    const int D = m->D, F = m->F;
    const uint16_t *lw = m->d_layers + (size_t)l * m->layer_elems;
    const size_t kvo = (size_t)l * m->kv_layer_elems * (m->kv_f32 ? 4 : 2);
    void *kc = (char *)m->d_kc + kvo, *vc = (char *)m->d_vc + kvo;
    switch (fam) {
    case LM_KERN_QKV:
        if (lvl)   /* with the attention of every head (Wo from level 2, the FFN at 3) */
            KCHK(lmk_qkv_attn(s, m->d_x, l == 0 ? m->d_embed : NULL, m->d_tok,
                              m->d_rms_att + (size_t)l * D, lw, D, m->NQ, m->NKV, m->hd,
                              m->d_rope_cos, m->d_rope_sin, m->d_pos, B, kc, vc, m->kv_f32,
                              m->max_seq, m->H, m->d_tagged, m->d_epoch, l, m->L, m->d_err,
                              m->d_attn, lvl >= 2 ? lw + m->off_wo : NULL,
                              m->d_rms_ffn + (size_t)l * D, lvl == 3 ? lw + m->off_w13 : NULL,
                              lw + m->off_w2, F, m->layer_wgs));
        else
            KCHK(lmk_qkv_rope(s, m->d_x, l == 0 ? m->d_embed : NULL, m->d_tok,
                              m->d_rms_att + (size_t)l * D, lw, D, m->NQ, m->NKV, m->hd,
                              m->d_rope_cos, m->d_rope_sin, m->d_pos, B, m->d_q, kc, vc, m->kv_f32,
                              m->max_seq));
        break;
    case LM_KERN_ATTN:
        KCHK(lmk_attn_decode(s, m->d_q, kc, vc, m->kv_f32, m->d_pos, NULL, B, m->H, m->Hkv,
                             m->hd, m->max_seq, m->d_attn, NULL));
        break;
    case LM_KERN_WO:
        KCHK(lmk_wo_residual(s, m->d_attn, lw + m->off_wo, D, B, m->d_x));
        break;
    case LM_KERN_W13:
        KCHK(lmk_ffn13(s, m->d_x, m->d_rms_ffn + (size_t)l * D, lw + m->off_w13, D, F, B, m->d_g));
        break;
    case LM_KERN_W2:
        KCHK(lmk_w2_residual(s, m->d_g, lw + m->off_w2, D, F, B, m->d_x));
        break;
    case LM_KERN_CLS:
        KCHK(lmk_cls(s, m->d_x, m->d_rms_final, m->d_wcls, D, m->V, B, logits, m->d_amax,
                     lvl == 3 ? m->d_cls_tw : NULL, m->d_epoch, m->d_tok, m->d_pos, m->d_hist,
                     m->max_seq + 1, m->d_err));
        break;
    case LM_KERN_ARGMAX:
        KCHK(lmk_argmax_final(s, m->d_amax, m->cls_nblk, B, m->d_tok, m->d_pos, m->d_hist,
                              m->max_seq + 1, m->d_epoch));
        break;
    default:
        return LM_ERR_INVALID;
    }
    return LM_OK;
}

/* Queue one decode step for rows 0..B-1 (tokens in d_tok, positions in d_pos);
 * logits go to `logits` (device, B x V, may be NULL), the argmax to d_tok, and
 * the history/position advance to d_hist/d_pos. */
static int enqueue_decode_gemv(LMModel *m, int B, float *logits)
{
    static const int fams[5] = {LM_KERN_QKV, LM_KERN_ATTN, LM_KERN_WO, LM_KERN_W13, LM_KERN_W2};
    int rc;
    for (int l = 0; l < m->L; l++)
        for (int f = 0; f < 5; f++)
            if ((rc = enqueue_kernel(m, B, fams[f], l, NULL))) return rc;
    if ((rc = enqueue_kernel(m, B, LM_KERN_CLS, 0, logits))) return rc;
    return enqueue_kernel(m, B, LM_KERN_ARGMAX, 0, NULL);
}

/* ------------------------------------------------------------------------- */
/* MFMA path: prefill rows and decode batches above MAX_GEMV_B                 */
/* ------------------------------------------------------------------------- */

/* Largest decode batch of the MFMA decode step (one 64-row tile). */
#define MAX_GEMM_B 64
/* Rows per prefill chunk (whole sequences). */
#define PREFILL_ROWS 2048

/* Queue the layers for M rows (row r: token tok[r], position pos[r], cache slot
 * slot[r]; the K/V of every row is appended to the cache before attention, so
 * rows of one sequence attend causally to each other; seq_rows > 1: the rows
 * are whole sequences of seq_rows rows, attended by the MFMA prefill kernel,
 * else one row per slot, by the decode kernel), then with with_cls the
 * final rmsnorm + classifier of all M rows: logits to `logits` (prefill: only
 * when non-NULL; decode: may be NULL) and, for decode rows, the argmax partials
 * to d_amax. */
static int enqueue_rows(LMModel *m, int M, int seq_rows, const int *tok, const int *pos,
                        const int *slot, float *logits, int with_cls)
{
    hipStream_t s = m->stream;
    const int D = m->D, F = m->F, NQ = m->NQ, NKV = m->NKV, NQKV = NQ + 2 * NKV;
    const size_t sx = (size_t)M * D;   /* split stride of a [M, D] partial */
    /* Wo and W2 write their product, not x: into d_part as fp32 (decode rows
     * (M <= 64) run these narrow projections K-split, one partial per split),
     * and the row norm that next reads x adds it (the residual add).  Only
     * unsplit decode rows keep the residual add in the GEMM epilogue. */
    const int dec = M <= 64;
    const int ns_qkv = dec && seq_rows == 1 ? lmk_pick_split(M, NQKV, D) : 1;
    const int ns_wo = lmk_pick_split(M, D, NQ);
    const int ns_w2 = lmk_pick_split(M, D, F);
    const int sep_wo = !dec || ns_wo > 1, sep_w2 = !dec || ns_w2 > 1;
    /* Beyond 64 rows, an unsplit Wo or W2 folds the row norm that follows it
     * into the GEMMs: it adds its product to x and writes u = fp16(x * gain)
     * and the sums of squares of x per 32 columns (RESNORM), and the GEMM that
     * reads u scales its product rows by 1/sqrt(mean(x^2) + 1e-5), which
     * distributes over the row's dot products.  That saves the row-norm
     * launch and the product's round trip through memory.  K-split
     * projections keep the row norm, which adds their partials (an unsplit
     * 2048-row W2 took 20 us against 14 + 5.6 for the split and the norm);
     * so do layer 0 (embedding) and the classifier.  Only prefill rows fold
     * (LM_OPT_PREFILL_FOLD): u is rounded to fp16 before the row is
     * normalised, and a prefill chunk whose u overflows is redone with the
     * row norm apart (run_prefill); decode rows have no such retry. */
    const int can_fold = !dec && seq_rows > 1 && m->prefill_fold && !m->fold_off && D % 128 == 0 &&
                         D / 32 <= 64;
    const int fold_wo = can_fold && ns_wo == 1, fold_w2 = can_fold && ns_w2 == 1;
    int rs_next = 0;                   /* x's norm is pending in u for QKV */
    const float *pend = NULL;          /* W2 partials not yet added to x */
    int pend_ns = 0;
    LMEpilogue ep;
    for (int l = 0; l < m->L; l++) {
        const uint16_t *lw = m->d_layers + (size_t)l * m->layer_elems;
        const size_t kvo = (size_t)l * m->kv_layer_elems * (m->kv_f32 ? 4 : 2);
        void *kc = (char *)m->d_kc + kvo, *vc = (char *)m->d_vc + kvo;
        const float *rs = rs_next ? m->d_ss : NULL;   /* u's row scale */
        if (!rs)
            KCHK(lmk_rownorm(s, m->d_x, D, M, l == 0 ? m->d_embed : NULL, tok, pend, pend_ns, sx,
                             m->d_rms_att + (size_t)l * D, m->d_xn16));
        pend = NULL;
        pend_ns = 0;
        if (ns_qkv > 1) {
            /* decode rows, too few column tiles to fill the CUs: K-split QKV;
             * the attention kernel sums the partials, applies RoPE and appends
             * K/V itself */
            KCHK(lmk_gemm_split(s, m->d_xn16, D, lw, M, NQKV, D, ns_qkv, m->d_part));
            KCHK(lmk_attn_decode_part(s, m->d_part, (size_t)M * NQKV, ns_qkv, NQ, NKV, pos, slot, M,
                                      m->H, m->Hkv, m->hd, m->max_seq, m->d_rope_cos,
                                      m->d_rope_sin, kc, vc, m->kv_f32, m->d_a16));
        } else {
            /* QKV with RoPE and the K/V append in the GEMM epilogue (staged
             * through LDS and stored row-contiguously) */
            memset(&ep, 0, sizeof(ep));
            ep.q = m->d_q; ep.kc = kc; ep.vc = vc; ep.kv_f32 = m->kv_f32;
            ep.NQ = NQ; ep.NKV = NKV; ep.hd = m->hd; ep.Hkv = m->Hkv; ep.max_seq = m->max_seq;
            ep.slot = slot; ep.pos = pos; ep.rope_cos = m->d_rope_cos; ep.rope_sin = m->d_rope_sin;
            ep.rs_ss = rs; ep.nss = D / 32;
            KCHK(lmk_gemm(s, m->d_xn16, D, lw, M, NQKV, D, LMK_EPI_QKV, &ep));
        }
        if (ns_qkv > 1) {
        } else if (seq_rows > 1) {
            KCHK(lmk_attn_prefill(s, m->d_q, kc, vc, m->kv_f32, pos, slot, seq_rows,
                                  M / seq_rows, m->H, m->Hkv, m->hd, m->max_seq, m->d_a16));
        } else {
            KCHK(lmk_attn_decode(s, m->d_q, kc, vc, m->kv_f32, pos, slot, M, m->H, m->Hkv, m->hd,
                                 m->max_seq, NULL, m->d_a16));
        }
        if (fold_wo) {
            memset(&ep, 0, sizeof(ep));
            ep.out = m->d_x; ep.ldc = D;
            ep.gain = m->d_rms_ffn + (size_t)l * D; ep.u = m->d_xn16; ep.ss = m->d_ss; ep.nss = D / 32;
            ep.ovf = m->d_ovf;
            KCHK(lmk_gemm(s, m->d_a16, NQ, lw + m->off_wo, M, D, NQ, LMK_EPI_RESNORM, &ep));
        } else if (sep_wo) {
            if (ns_wo > 1) {
                KCHK(lmk_gemm_split(s, m->d_a16, NQ, lw + m->off_wo, M, D, NQ, ns_wo, m->d_part));
            } else {
                memset(&ep, 0, sizeof(ep));
                ep.out = m->d_part; ep.ldc = D;
                KCHK(lmk_gemm(s, m->d_a16, NQ, lw + m->off_wo, M, D, NQ, LMK_EPI_STORE, &ep));
            }
            KCHK(lmk_rownorm(s, m->d_x, D, M, NULL, NULL, m->d_part, ns_wo, sx,
                             m->d_rms_ffn + (size_t)l * D, m->d_xn16));
        } else {
            memset(&ep, 0, sizeof(ep));
            ep.out = m->d_x; ep.ldc = D;
            KCHK(lmk_gemm(s, m->d_a16, NQ, lw + m->off_wo, M, D, NQ, LMK_EPI_RESID, &ep));
            KCHK(lmk_rownorm(s, m->d_x, D, M, NULL, NULL, NULL, 0, 0,
                             m->d_rms_ffn + (size_t)l * D, m->d_xn16));
        }
        memset(&ep, 0, sizeof(ep));
        ep.g = m->d_g16; ep.F = F;
        if (fold_wo) { ep.rs_ss = m->d_ss; ep.nss = D / 32; }
        KCHK(lmk_gemm(s, m->d_xn16, D, lw + m->off_w13, M, 2 * F, D, LMK_EPI_GATE, &ep));
        rs_next = fold_w2 && l + 1 < m->L;
        if (fold_w2) {
            memset(&ep, 0, sizeof(ep));
            ep.out = m->d_x; ep.ldc = D;
            if (l + 1 < m->L) {   /* u of the next layer's attention norm */
                ep.gain = m->d_rms_att + (size_t)(l + 1) * D; ep.u = m->d_xn16; ep.ss = m->d_ss;
                ep.nss = D / 32; ep.ovf = m->d_ovf;
            }
            KCHK(lmk_gemm(s, m->d_g16, F, lw + m->off_w2, M, D, F,
                          l + 1 < m->L ? LMK_EPI_RESNORM : LMK_EPI_RESID, &ep));
        } else if (sep_w2) {
            if (ns_w2 > 1) {
                KCHK(lmk_gemm_split(s, m->d_g16, F, lw + m->off_w2, M, D, F, ns_w2, m->d_part));
            } else {
                memset(&ep, 0, sizeof(ep));
                ep.out = m->d_part; ep.ldc = D;
                KCHK(lmk_gemm(s, m->d_g16, F, lw + m->off_w2, M, D, F, LMK_EPI_STORE, &ep));
            }
            pend = m->d_part;
            pend_ns = ns_w2;
        } else {
            memset(&ep, 0, sizeof(ep));
            ep.out = m->d_x; ep.ldc = D;
            KCHK(lmk_gemm(s, m->d_g16, F, lw + m->off_w2, M, D, F, LMK_EPI_RESID, &ep));
        }
    }
    if (!with_cls) {
        /* x must hold the final residual for the caller: add pending partials */
        if (pend_ns)
            KCHK(lmk_rownorm(s, m->d_x, D, M, NULL, NULL, pend, pend_ns, sx, m->d_rms_final,
                             m->d_xn16));
        return LM_OK;
    }
    KCHK(lmk_rownorm(s, m->d_x, D, M, NULL, NULL, pend, pend_ns, sx, m->d_rms_final, m->d_xn16));
    memset(&ep, 0, sizeof(ep));
    ep.out = logits; ep.ldc = m->V; ep.stream_out = 1;
    if (seq_rows > 1) {   /* prefill: logits only */
        if (logits) KCHK(lmk_gemm(s, m->d_xn16, D, m->d_wcls, M, m->V, D, LMK_EPI_STORE, &ep));
    } else {              /* decode: argmax partials for the greedy step (+ logits) */
        ep.part = m->d_amax;
        KCHK(lmk_gemm(s, m->d_xn16, D, m->d_wcls, M, m->V, D, LMK_EPI_ARGMAX, &ep));
    }
    return LM_OK;
}

/* One greedy decode step of rows 0..B-1 on the MFMA path (slot b = row b). */
static int enqueue_decode_gemm(LMModel *m, int B, float *logits)
{
    int rc = enqueue_rows(m, B, 1, m->d_tok, m->d_pos, m->d_slot_id, logits, 1);
    if (rc) return rc;
    KCHK(lmk_argmax_final(m->stream, m->d_amax, m->cls_nblk, B, m->d_tok, m->d_pos, m->d_hist,
                          m->max_seq + 1, NULL));
    return LM_OK;
}

static int enqueue_decode(LMModel *m, int B, float *logits)
{
    return B <= MAX_GEMV_B ? enqueue_decode_gemv(m, B, logits) : enqueue_decode_gemm(m, B, logits);
}

/* Greedy steps captured per multi-step graph. */
#define GRAPH_STEPS 16

/* Run `nsteps` (1 or GRAPH_STEPS) decode steps of rows 0..B-1, replaying the
 * captured graph of that shape (captured on first use).  Single steps write
 * the logits to d_logits; multi-step runs only feed the argmax forward. */
static int enqueue_decode_steps(LMModel *m, int B, int nsteps)
{
    if (!m->use_graph) {
        for (int t = 0; t < nsteps; t++) {
            int rc = enqueue_decode(m, B, nsteps == 1 ? m->d_logits : NULL);
            if (rc) return rc;
        }
        return LM_OK;
    }
    hipGraphExec_t *ge = &m->step_graph[B][nsteps == 1 ? 0 : 1];
    if (!*ge) {
        hipGraph_t g;
        HIPCHK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
        int rc = LM_OK;
        for (int t = 0; t < nsteps && rc == LM_OK; t++)
            rc = enqueue_decode(m, B, nsteps == 1 ? m->d_logits : NULL);
        hipError_t e = hipStreamEndCapture(m->stream, &g);
        if (rc) return rc;
        HIPCHK(e);
        e = hipGraphInstantiateWithFlags(ge, g, 0);
        hipGraphDestroy(g);
        HIPCHK(e);
    }
    HIPCHK(hipGraphLaunch(*ge, m->stream));
    return LM_OK;
}

/* Whether the decode step of B rows holds hand-off waits (the batch 1-4
 * chain with QKV and attention in one launch, levels 1-4). */
static int step_waits(const LMModel *m, int B)
{
    return B <= MAX_GEMV_B && chain_level(m, B) >= 1;
}

static int run_decode_steps(LMModel *m, int B, int nsteps)
{
    if (B > MAX_GEMM_B) {
        fprintf(stderr, "stories_lm: decode batch %d > %d not supported\n", B, MAX_GEMM_B);
        return LM_ERR_UNSUPPORTED;
    }
    if (nsteps != 1 && nsteps != GRAPH_STEPS) return LM_ERR_INVALID;
    if (!step_waits(m, B)) return enqueue_decode_steps(m, B, nsteps);
    int rc = handoff_enter(m);
    if (rc) return rc;
    return handoff_leave(m, enqueue_decode_steps(m, B, nsteps));
}

static int run_decode_step(LMModel *m, int B) { return run_decode_steps(m, B, 1); }

/* The hand-off flag of the fused QKV + attention launches: queued to the host
 * with the results of a call, checked once the stream has synchronised. */
static int *err_slot(LMModel *m) { return m->h_io + 4 * (size_t)m->max_batch; }

static int queue_err_read(LMModel *m)
{
    return hipMemcpyAsync(err_slot(m), m->d_err, 4, hipMemcpyDeviceToHost, m->stream) == hipSuccess
               ? LM_OK
               : LM_ERR_HIP;
}

static int check_err(LMModel *m)
{
    if (!*err_slot(m)) return LM_OK;
    fprintf(stderr, "stories_lm: a hand-off wait inside a fused launch gave up (results invalid)\n");
    *err_slot(m) = 0;
    /* Once a wait has given up, every wait of the launch ends early, so the
     * argmax reducer can advance the step count while classifier work-groups
     * dispatched before it have yet to read it; their words then carry the
     * tags of the next step.  Clear every hand-off word (tag 0 matches no
     * step) with the flag, on the model's stream, before the next call. */
    HIPCHK(hipMemsetAsync(m->d_tagged, 0, LM_TAG_WORDS(m->NQ, m->NKV, m->D, m->F) * 8, m->stream));
    HIPCHK(hipMemsetAsync(m->d_cls_tw, 0, (size_t)2 * LM_TAG_B * m->cls_nblk * 8, m->stream));
    HIPCHK(hipMemsetAsync(m->d_err, 0, 4, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return LM_ERR_HIP;
}

static int check_tok_pos(const LMModel *m, const int *tokens, const int *pos, int B)
{
    for (int b = 0; b < B; b++) {
        if (tokens[b] < 0 || tokens[b] >= m->V) {
            fprintf(stderr, "stories_lm: token %d out of range [0,%d)\n", tokens[b], m->V);
            return LM_ERR_RANGE;
        }
        if (pos[b] < 0 || pos[b] >= m->max_seq) {
            fprintf(stderr, "stories_lm: position %d out of range [0,%d)\n", pos[b], m->max_seq);
            return LM_ERR_RANGE;
        }
    }
    return LM_OK;
}

int lm_forward_batch(LMModel *m, const int *tokens, const int *pos, int B, float *logits, int *argmax)
{
    if (!m || !tokens || !pos || B < 1) return LM_ERR_INVALID;
    if (B > m->max_batch) return LM_ERR_RANGE;
    int rc = check_tok_pos(m, tokens, pos, B);
    if (rc) return rc;
    int *hio = m->h_io;
    memcpy(hio, tokens, B * 4);
    memcpy(hio + B, pos, B * 4);
    HIPCHK(hipMemcpyAsync(m->d_tok, hio, B * 4, hipMemcpyHostToDevice, m->stream));
    HIPCHK(hipMemcpyAsync(m->d_pos, hio + B, B * 4, hipMemcpyHostToDevice, m->stream));
    if ((rc = run_decode_step(m, B))) return rc;
    if (argmax)
        HIPCHK(hipMemcpyAsync(hio + 2 * B, m->d_tok, B * 4, hipMemcpyDeviceToHost, m->stream));
    if (logits)
        HIPCHK(hipMemcpyAsync(m->h_logits, m->d_logits, (size_t)B * m->V * 4,
                              hipMemcpyDeviceToHost, m->stream));
    if ((rc = queue_err_read(m))) return rc;
    HIPCHK(hipStreamSynchronize(m->stream));
    if ((rc = check_err(m))) return rc;
    if (argmax) memcpy(argmax, hio + 2 * B, B * 4);
    if (logits) memcpy(logits, m->h_logits, (size_t)B * m->V * 4);
    return LM_OK;
}

const float *lm_forward(LMModel *m, int token, int pos)
{
    if (!m) {
        fprintf(stderr, "stories_lm: lm_forward on NULL handle\n");
        return NULL;
    }
    if (check_tok_pos(m, &token, &pos, 1)) return NULL;
    int *hio = m->h_io;
    hio[0] = token;
    hio[1] = pos;
    if (hipMemcpyAsync(m->d_tok, hio, 4, hipMemcpyHostToDevice, m->stream) != hipSuccess ||
        hipMemcpyAsync(m->d_pos, hio + 1, 4, hipMemcpyHostToDevice, m->stream) != hipSuccess)
        return NULL;
    if (run_decode_step(m, 1)) return NULL;
    if (hipMemcpyAsync(m->h_logits, m->d_logits, (size_t)m->V * 4, hipMemcpyDeviceToHost,
                       m->stream) != hipSuccess ||
        queue_err_read(m) != LM_OK || hipStreamSynchronize(m->stream) != hipSuccess) {
        fprintf(stderr, "stories_lm: lm_forward: HIP error\n");
        return NULL;
    }
    if (check_err(m)) return NULL;
    return m->h_logits;
}

int lm_generate_greedy(LMModel *m, int B, const int *first_tokens, const int *pos0, int n_steps,
                       int *out_tokens)
{
    if (!m || !first_tokens || !pos0 || !out_tokens || B < 1 || n_steps < 0) return LM_ERR_INVALID;
    if (B > m->max_batch) return LM_ERR_RANGE;
    int rc = check_tok_pos(m, first_tokens, pos0, B);
    if (rc) return rc;
    for (int b = 0; b < B; b++)
        if (pos0[b] + n_steps > m->max_seq) {
            fprintf(stderr, "stories_lm: pos0 %d + %d steps exceeds max_seq %d\n", pos0[b], n_steps,
                    m->max_seq);
            return LM_ERR_RANGE;
        }
    if (n_steps == 0) return LM_OK;
    int *hio = m->h_io;
    memcpy(hio, first_tokens, B * 4);
    memcpy(hio + B, pos0, B * 4);
    HIPCHK(hipMemcpyAsync(m->d_tok, hio, B * 4, hipMemcpyHostToDevice, m->stream));
    HIPCHK(hipMemcpyAsync(m->d_pos, hio + B, B * 4, hipMemcpyHostToDevice, m->stream));
    int t = 0;
    for (; t + GRAPH_STEPS <= n_steps; t += GRAPH_STEPS)
        if ((rc = run_decode_steps(m, B, GRAPH_STEPS))) return rc;
    for (; t < n_steps; t++)
        if ((rc = run_decode_step(m, B))) return rc;
    const size_t stride = (size_t)m->max_seq + 1;
    int *h = (int *)malloc((size_t)B * stride * 4);
    if (!h) return LM_ERR_OOM;
    hipError_t e = hipMemcpyAsync(h, m->d_hist, (size_t)B * stride * 4, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(err_slot(m), m->d_err, 4, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) {
        free(h);
        fprintf(stderr, "stories_lm: lm_generate_greedy: %s\n", hipGetErrorString(e));
        return LM_ERR_HIP;
    }
    if ((rc = check_err(m))) {
        free(h);
        return rc;
    }
    for (int t = 0; t < n_steps; t++)
        for (int b = 0; b < B; b++) out_tokens[(size_t)t * B + b] = h[b * stride + pos0[b] + 1 + t];
    free(h);
    return LM_OK;
}

/* Final rmsnorm + classifier of M rows held in x_rows (fp32 [M, D]): logits to
 * d_logits. */
static int enqueue_cls_rows(LMModel *m, float *x_rows, int M)
{
    hipStream_t s = m->stream;
    LMEpilogue ep;
    KCHK(lmk_rownorm(s, x_rows, m->D, M, NULL, NULL, NULL, 0, 0, m->d_rms_final, m->d_xn16));
    memset(&ep, 0, sizeof(ep));
    ep.out = m->d_logits; ep.ldc = m->V; ep.stream_out = 1;
    KCHK(lmk_gemm(s, m->d_xn16, m->D, m->d_wcls, M, m->V, m->D, LMK_EPI_STORE, &ep));
    return LM_OK;
}

/* Causal forward of nseq sequences of S tokens (sequence i: slot slots[i],
 * positions pos0[i] .. pos0[i]+S-1, positions below pos0[i] already cached)
 * on the MFMA path, in chunks of whole sequences.  logits_mode LM_LOGITS_ALL:
 * every row's logits; LM_LOGITS_LAST: the last row of each sequence.  Host
 * `logits` (may be NULL) receives them in sequence order; the last chunk's
 * logits stay in d_logits. */
/* The layers of a prefill chunk of R rows (sequences of S rows; tokens,
 * positions and slots in d_rin, R ints each) and, with `all`, the
 * classifier into d_logits: replayed from a captured graph of that shape
 * (captured on first use) unless graphs are off. */
static int run_rows(LMModel *m, int R, int S, int all)
{
    const int *tok = m->d_rin, *pos = m->d_rin + R, *slot = m->d_rin + 2 * (size_t)R;
    if (!m->use_graph || m->fold_off)   /* (the graphs hold the folded form) */
        return enqueue_rows(m, R, S, tok, pos, slot, all ? m->d_logits : NULL, all);
    int k = 0;
    while (k < PREFILL_GRAPHS &&
           !(m->pgraph[k].ge && m->pgraph[k].R == R && m->pgraph[k].S == S && m->pgraph[k].all == all))
        k++;
    if (k == PREFILL_GRAPHS) {
        k = m->pgraph_next;
        m->pgraph_next = (k + 1) % PREFILL_GRAPHS;
        if (m->pgraph[k].ge) {
            hipGraphExecDestroy(m->pgraph[k].ge);
            m->pgraph[k].ge = NULL;
        }
        hipGraph_t g;
        HIPCHK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue_rows(m, R, S, tok, pos, slot, all ? m->d_logits : NULL, all);
        hipError_t e = hipStreamEndCapture(m->stream, &g);
        if (rc) return rc;
        HIPCHK(e);
        e = hipGraphInstantiateWithFlags(&m->pgraph[k].ge, g, 0);
        hipGraphDestroy(g);
        HIPCHK(e);
        m->pgraph[k].R = R;
        m->pgraph[k].S = S;
        m->pgraph[k].all = all;
    }
    HIPCHK(hipGraphLaunch(m->pgraph[k].ge, m->stream));
    return LM_OK;
}

static int run_prefill(LMModel *m, int nseq, const int *slots, const int *pos0, const int *tokens,
                       int S, int logits_mode, float *logits, float *loss)
{
    const int V = m->V;
    unsigned char *seen = (unsigned char *)calloc((size_t)m->max_batch, 1);
    if (!seen) return LM_ERR_OOM;
    for (int i = 0; i < nseq; i++) {
        if (slots[i] < 0 || slots[i] >= m->max_batch || pos0[i] < 0 || pos0[i] + S > m->max_seq) {
            fprintf(stderr, "stories_lm: prefill sequence %d: slot %d / positions %d..%d out of "
                    "range (max_batch %d, max_seq %d)\n", i, slots[i], pos0[i], pos0[i] + S - 1,
                    m->max_batch, m->max_seq);
            free(seen);
            return LM_ERR_RANGE;
        }
        /* two sequences in one slot would write the same cache rows */
        if (seen[slots[i]]++) {
            fprintf(stderr, "stories_lm: prefill: slot %d given to more than one sequence\n",
                    slots[i]);
            free(seen);
            return LM_ERR_INVALID;
        }
        for (int t = 0; t < S; t++)
            if (tokens[(size_t)i * S + t] < 0 || tokens[(size_t)i * S + t] >= V) {
                fprintf(stderr, "stories_lm: prefill token %d out of range [0,%d)\n",
                        tokens[(size_t)i * S + t], V);
                free(seen);
                return LM_ERR_RANGE;
            }
    }
    free(seen);
    const int cs = S >= PREFILL_ROWS ? 1 : PREFILL_ROWS / S;   /* sequences per chunk */
    const int chunk_rows = (nseq < cs ? nseq : cs) * S;
    int rc;
    if (chunk_rows > m->max_rows && (rc = alloc_rows(m, chunk_rows))) return rc;
    int *h = m->h_rin;   /* pinned; each chunk ends with a stream synchronise */
    rc = LM_OK;
    for (int i0 = 0; i0 < nseq && rc == LM_OK; i0 += cs) {
        const int n = nseq - i0 < cs ? nseq - i0 : cs;
        const int R = n * S;
        for (int i = 0; i < n; i++)
            for (int t = 0; t < S; t++) {
                const int r = i * S + t;
                h[r] = tokens[(size_t)(i0 + i) * S + t];
                h[R + r] = pos0[i0 + i] + t;
                h[2 * R + r] = slots[i0 + i];
            }
        if (hipMemcpyAsync(m->d_rin, h, (size_t)3 * R * 4, hipMemcpyHostToDevice, m->stream) != hipSuccess) {
            rc = LM_ERR_HIP;
            break;
        }
        /* pass 1 only when pass 0's folded norm overflowed fp16 (its u is
         * x * gain before the row is normalised): the same rows again with
         * the row norm apart, rewriting the same cache entries */
        for (int pass = 0; pass < 2 && rc == LM_OK; pass++) {
            if (logits_mode == LM_LOGITS_ALL) {
                rc = run_rows(m, R, S, 1);
                if (rc == LM_OK && logits &&
                    hipMemcpyAsync(logits + (size_t)i0 * S * V, m->d_logits, (size_t)R * V * 4,
                                   hipMemcpyDeviceToHost, m->stream) != hipSuccess)
                    rc = LM_ERR_HIP;
                /* the chunk's loss terms, before the next chunk reuses d_logits */
                if (rc == LM_OK && loss) {
                    float *d_lp = (float *)(m->d_rin + 3 * (size_t)R);
                    if (lmk_row_logprob(m->stream, m->d_logits, V, m->d_rin, S, R, d_lp) != hipSuccess ||
                        hipMemcpyAsync(h + 3 * (size_t)R, d_lp, (size_t)R * 4, hipMemcpyDeviceToHost,
                                       m->stream) != hipSuccess)
                        rc = LM_ERR_HIP;
                }
            } else {
                rc = run_rows(m, R, S, 0);
                /* gather the last row of each sequence into d_attn (same row width) */
                if (rc == LM_OK &&
                    hipMemcpy2DAsync(m->d_attn, (size_t)m->D * 4, m->d_x + (size_t)(S - 1) * m->D,
                                     (size_t)S * m->D * 4, (size_t)m->D * 4, n,
                                     hipMemcpyDeviceToDevice, m->stream) != hipSuccess)
                    rc = LM_ERR_HIP;
                if (rc == LM_OK) rc = enqueue_cls_rows(m, m->d_attn, n);
                if (rc == LM_OK && logits &&
                    hipMemcpyAsync(logits + (size_t)i0 * V, m->d_logits, (size_t)n * V * 4,
                                   hipMemcpyDeviceToHost, m->stream) != hipSuccess)
                    rc = LM_ERR_HIP;
            }
            if (rc == LM_OK && hipStreamSynchronize(m->stream) != hipSuccess) rc = LM_ERR_HIP;
            volatile int *ovf = m->h_io + 4 * (size_t)m->max_batch + 1;
            if (rc != LM_OK || !*ovf) break;
            *ovf = 0;
            m->fold_off = 1;
        }
        m->fold_off = 0;
        if (rc == LM_OK && loss) {
            /* mean over each sequence, summed in the reference's order
             * (forward.h:174-183: loss -= log_prob; loss / (S-1)) */
            const float *lp = (const float *)(h + 3 * (size_t)R);
            for (int i = 0; i < n; i++) {
                float acc = 0.f;
                for (int t = 0; t < S - 1; t++) acc -= lp[(size_t)i * S + t];
                loss[i0 + i] = acc / (S - 1);
            }
        }
    }
    /* after a failure, let the copy out of the staging buffer finish before
     * a later call refills it */
    if (rc != LM_OK) (void)hipStreamSynchronize(m->stream);
    return rc;
}

int lm_prefill(LMModel *m, int slot, int pos0, const int *tokens, int S, float *logits)
{
    if (!m || !tokens || S < 1) return LM_ERR_INVALID;
    if (slot < 0 || slot >= m->max_batch || pos0 < 0 || pos0 + S > m->max_seq) return LM_ERR_RANGE;
    return run_prefill(m, 1, &slot, &pos0, tokens, S, LM_LOGITS_ALL, logits, NULL);
}

static int prefill_from_zero(LMModel *m, int nseq, const int *slots, const int *tokens, int S,
                             int logits_mode, float *logits, float *loss)
{
    int *sl = (int *)malloc((size_t)nseq * 2 * sizeof(int));
    if (!sl) return LM_ERR_OOM;
    for (int i = 0; i < nseq; i++) {
        sl[i] = slots ? slots[i] : i;
        sl[nseq + i] = 0;
    }
    int rc = run_prefill(m, nseq, sl, sl + nseq, tokens, S, logits_mode, logits, loss);
    free(sl);
    return rc;
}

int lm_prefill_batch(LMModel *m, int nseq, const int *slots, const int *tokens, int S,
                     int logits_mode, float *logits)
{
    if (!m || !tokens || nseq < 1 || S < 1 ||
        (logits_mode != LM_LOGITS_ALL && logits_mode != LM_LOGITS_LAST))
        return LM_ERR_INVALID;
    return prefill_from_zero(m, nseq, slots, tokens, S, logits_mode, logits, NULL);
}

int lm_prefill_loss(LMModel *m, int nseq, const int *slots, const int *tokens, int S, float *logits,
                    float *loss)
{
    if (!m || !tokens || !loss || nseq < 1 || S < 2) return LM_ERR_INVALID;
    if (m->V % 4) {   /* the loss kernel reads each logit row as 16-byte groups */
        fprintf(stderr, "stories_lm: lm_prefill_loss: vocab_size %d is not a multiple of 4\n", m->V);
        return LM_ERR_UNSUPPORTED;
    }
    return prefill_from_zero(m, nseq, slots, tokens, S, LM_LOGITS_ALL, logits, loss);
}

int lm_read_logits(LMModel *m, int row0, int nrows, float *dst)
{
    if (!m || !dst || row0 < 0 || nrows < 0) return LM_ERR_INVALID;
    if (row0 + nrows > m->max_rows) return LM_ERR_RANGE;
    HIPCHK(hipMemcpy(dst, m->d_logits + (size_t)row0 * m->V, (size_t)nrows * m->V * 4,
                     hipMemcpyDeviceToHost));
    return LM_OK;
}

/* ------------------------------------------------------------------------- */
/* timing                                                                     */
/* ------------------------------------------------------------------------- */

int lm_sync(LMModel *m)
{
    if (!m) return LM_ERR_INVALID;
    HIPCHK(hipStreamSynchronize(m->stream));
    return LM_OK;
}

int lm_timer_begin(LMModel *m)
{
    if (!m) return LM_ERR_INVALID;
    HIPCHK(hipEventRecord(m->ev0, m->stream));
    return LM_OK;
}

int lm_timer_end(LMModel *m, float *ms)
{
    if (!m || !ms) return LM_ERR_INVALID;
    HIPCHK(hipEventRecord(m->ev1, m->stream));
    HIPCHK(hipEventSynchronize(m->ev1));
    HIPCHK(hipEventElapsedTime(ms, m->ev0, m->ev1));
    return LM_OK;
}

/* Diagnostics: run the DPP reduction self-test (no model needed). */
int lm_selftest_reduce(const float *in64, float *out4)
{
    if (!in64 || !out4) return LM_ERR_INVALID;
    int rc = lm_init();
    if (rc) return rc;
    float *d = NULL;
    HIPCHK(hipMalloc((void **)&d, 68 * 4));
    hipError_t e = hipMemcpy(d, in64, 64 * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = (hipError_t)lmk_selftest_reduce(0, d, d + 64);
    if (e == hipSuccess) e = hipMemcpy(out4, d + 64, 16, hipMemcpyDeviceToHost);
    hipFree(d);
    HIPCHK(e);
    return LM_OK;
}

int lm_profile_chain(LMModel *m, int B, const int *tokens, const int *pos, int steps,
                     float *us_per_launch, int *launches_per_step)
{
    static const int fams[5] = {LM_KERN_QKV, LM_KERN_ATTN, LM_KERN_WO, LM_KERN_W13, LM_KERN_W2};
    if (!m || !tokens || !pos || !us_per_launch || B < 1 || steps < 1) return LM_ERR_INVALID;
    if (B > m->max_batch) return LM_ERR_RANGE;
    if (B > MAX_GEMV_B) return LM_ERR_UNSUPPORTED;
    int rc = check_tok_pos(m, tokens, pos, B);
    if (rc) return rc;
    for (int b = 0; b < B; b++)
        if (pos[b] + steps + 1 > m->max_seq) return LM_ERR_RANGE;
    const int lvl = chain_level(m, B), waits = step_waits(m, B);
    /* the launches of one step, in order: (family, layer) */
    const int nmax = 5 * m->L + 2;
    int *kf = (int *)calloc((size_t)nmax, sizeof(int)), *kl = (int *)calloc((size_t)nmax, sizeof(int));
    int nk = 0;
    if (!kf || !kl) rc = LM_ERR_OOM;
    for (int l = 0; l < m->L && rc == LM_OK; l++)
        for (int f = 0; f < 5; f++)
            if (!fam_inside(fams[f], lvl)) { kf[nk] = fams[f]; kl[nk++] = l; }   /* else inside QKV's */
    for (int f = LM_KERN_CLS; f <= LM_KERN_ARGMAX && rc == LM_OK; f++)
        if (!fam_inside(f, lvl)) { kf[nk] = f; kl[nk++] = 0; }   /* else inside the classifier's */
    /* Each run of consecutive launches of one family (at level 3 the L
     * whole-layer launches, then the classifier) is timed by one event pair,
     * the first launch's start to the last one's end, with no event between
     * them, so the launches meet each other as in the greedy loop's graphs;
     * the run's time is shared equally among its launches.  Steps are queued
     * back to back in runs of GRAPH_STEPS, as those graphs run them (the argmax
     * feeds each step's token to the next on the device); the stream is
     * synchronised and the events read once per run of steps. */
    int nrun = 0;
    for (int i = 0; i < nk; i++) nrun += i == 0 || kf[i] != kf[i - 1];
    const int chunk = GRAPH_STEPS;
    const size_t nev = 2 * (size_t)nrun * chunk;
    hipEvent_t *ev = (hipEvent_t *)calloc(nev, sizeof(hipEvent_t));
    double sum[LM_KERN_COUNT] = {0};
    int cnt[LM_KERN_COUNT] = {0};
    if (!ev) rc = LM_ERR_OOM;
    for (size_t i = 0; i < nev && rc == LM_OK; i++)
        if (hipEventCreate(&ev[i]) != hipSuccess) rc = LM_ERR_HIP;
    int *hio = m->h_io;
    if (rc == LM_OK) {
        memcpy(hio, tokens, B * 4);
        memcpy(hio + B, pos, B * 4);
        if (hipMemcpyAsync(m->d_tok, hio, B * 4, hipMemcpyHostToDevice, m->stream) != hipSuccess ||
            hipMemcpyAsync(m->d_pos, hio + B, B * 4, hipMemcpyHostToDevice, m->stream) != hipSuccess)
            rc = LM_ERR_HIP;
    }
    for (int st0 = 0; st0 <= steps && rc == LM_OK; st0 += chunk) {   /* step 0 untimed */
        const int nst = steps + 1 - st0 < chunk ? steps + 1 - st0 : chunk;
        if (waits && (rc = handoff_enter(m))) break;
        for (int t = 0, r = 0; t < nst && rc == LM_OK; t++)
            for (int i = 0; i < nk && rc == LM_OK; i++) {
                const int first = i == 0 || kf[i] != kf[i - 1], last = i == nk - 1 || kf[i + 1] != kf[i];
                if (first || last)
                    lmk_time_next(first ? ev[2 * r] : NULL, last ? ev[2 * r + 1] : NULL);
                rc = enqueue_kernel(m, B, kf[i], kl[i], NULL);
                r += last;
            }
        if (waits) rc = handoff_leave(m, rc);
        if (rc == LM_OK && hipStreamSynchronize(m->stream) != hipSuccess) rc = LM_ERR_HIP;
        for (int t = 0, r = 0; t < nst && rc == LM_OK; t++)
            for (int i = 0, len = 0; i < nk && rc == LM_OK; i++) {
                len++;
                if (!(i == nk - 1 || kf[i + 1] != kf[i])) continue;
                float ms = 0.f;
                if (hipEventElapsedTime(&ms, ev[2 * r], ev[2 * r + 1]) != hipSuccess) rc = LM_ERR_HIP;
                if (st0 + t > 0) {
                    sum[kf[i]] += ms;
                    cnt[kf[i]] += len;
                }
                r++;
                len = 0;
            }
    }
    for (int f = 0; f < LM_KERN_COUNT; f++) {
        us_per_launch[f] = cnt[f] ? (float)(sum[f] * 1e3 / cnt[f]) : 0.f;
        if (launches_per_step)
            launches_per_step[f] = fam_inside(f, lvl)                            ? 0
                                   : f == LM_KERN_CLS || f == LM_KERN_ARGMAX ? 1
                                                                             : m->L;
    }
    for (size_t i = 0; ev && i < nev; i++)
        if (ev[i]) hipEventDestroy(ev[i]);
    free(ev);
    free(kf);
    free(kl);
    if (rc == LM_OK)
        HIPCHK(hipMemcpyAsync(m->d_pos, hio + B, B * 4, hipMemcpyHostToDevice, m->stream));
    if (rc == LM_OK) rc = queue_err_read(m);
    HIPCHK(hipStreamSynchronize(m->stream));
    if (rc == LM_OK) rc = check_err(m);
    return rc;
}

/* Diagnostics: one MFMA GEMM C = A W^T on caller data (plain store epilogue
 * with argmax partials).  A is fp16 bits [M, K] (a_f32 == 0) or fp32 [M, K];
 * W fp16 bits [N, K]; C fp32 [M, N]; part (may be NULL) [M, ceil(N/32)]. */
int lm_selftest_gemm(int M, int N, int K, int a_f32, const void *A, const uint16_t *W, float *C,
                     LMArgPartHost *part)
{
    if (M < 1 || N < 1 || K < 64 || K % 64 || !A || !W || !C) return LM_ERR_INVALID;
    int rc = lm_init();
    if (rc) return rc;
    const size_t asz = (size_t)M * K * 2, wsz = (size_t)N * K * 2;
    const size_t csz = (size_t)M * N * 4, np = (size_t)M * ((N + 31) / 32);
    uint16_t *a16 = NULL;
    if (a_f32) {   /* the kernels take fp16 operands: round on the host (RNE) */
        a16 = (uint16_t *)malloc(asz);
        if (!a16) return LM_ERR_OOM;
        lm_f32_to_f16((const float *)A, a16, (size_t)M * K);
        A = a16;
    }
    void *dA = NULL, *dW = NULL, *dC = NULL, *dP = NULL;
    hipError_t e = hipMalloc(&dA, asz);
    if (e == hipSuccess) e = hipMalloc(&dW, wsz);
    if (e == hipSuccess) e = hipMalloc(&dC, csz);
    if (e == hipSuccess) e = hipMalloc(&dP, np * sizeof(LMArgPart));
    if (e == hipSuccess) e = hipMemcpy(dA, A, asz, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dW, W, wsz, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(dC, 0xFF, csz);
    if (e == hipSuccess) {
        LMEpilogue ep;
        memset(&ep, 0, sizeof(ep));
        ep.out = (float *)dC; ep.ldc = N; ep.part = (LMArgPart *)dP;
        e = (hipError_t)lmk_gemm(0, (const uint16_t *)dA, K, (const uint16_t *)dW, M, N, K,
                                 LMK_EPI_ARGMAX, &ep);
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(C, dC, csz, hipMemcpyDeviceToHost);
    if (e == hipSuccess && part) e = hipMemcpy(part, dP, np * sizeof(LMArgPart), hipMemcpyDeviceToHost);
    hipFree(dA); hipFree(dW); hipFree(dC); hipFree(dP);
    free(a16);
    HIPCHK(e);
    return LM_OK;
}

int lm_selftest_gemm_split(int M, int N, int K, int nsplit, const uint16_t *A, const uint16_t *W,
                           float *parts)
{
    if (M < 1 || M > 4096 || N < 1 || K < 64 || K % 64 || !A || !W || !parts) return LM_ERR_INVALID;
    if (nsplit == 0) nsplit = lmk_pick_split(M, N, K);
    if (nsplit < 1 || nsplit > LMK_MAX_SPLIT || K % (64 * nsplit)) return LM_ERR_INVALID;
    int rc = lm_init();
    if (rc) return rc;
    const size_t asz = (size_t)M * K * 2, wsz = (size_t)N * K * 2;
    const size_t psz = (size_t)nsplit * M * N * 4;
    void *dA = NULL, *dW = NULL, *dP = NULL;
    hipError_t e = hipMalloc(&dA, asz);
    if (e == hipSuccess) e = hipMalloc(&dW, wsz);
    if (e == hipSuccess) e = hipMalloc(&dP, psz);
    if (e == hipSuccess) e = hipMemcpy(dA, A, asz, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dW, W, wsz, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(dP, 0xFF, psz);
    if (e == hipSuccess)
        e = (hipError_t)lmk_gemm_split(0, (const uint16_t *)dA, K, (const uint16_t *)dW, M, N, K,
                                       nsplit, (float *)dP);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(parts, dP, psz, hipMemcpyDeviceToHost);
    hipFree(dA); hipFree(dW); hipFree(dP);
    HIPCHK(e);
    return nsplit;
}

int lm_selftest_gemm_gate(int M, int N, int K, const uint16_t *A, const uint16_t *W, uint16_t *g)
{
    if (M < 1 || N < 2 * LMK_GATE_BLOCK || N % (2 * LMK_GATE_BLOCK) || K < 64 || K % 64 || !A || !W || !g)
        return LM_ERR_INVALID;
    int rc = lm_init();
    if (rc) return rc;
    const int F = N / 2;
    const size_t asz = (size_t)M * K * 2, wsz = (size_t)N * K * 2, gsz = (size_t)M * F * 2;
    void *dA = NULL, *dW = NULL, *dG = NULL;
    hipError_t e = hipMalloc(&dA, asz);
    if (e == hipSuccess) e = hipMalloc(&dW, wsz);
    if (e == hipSuccess) e = hipMalloc(&dG, gsz);
    if (e == hipSuccess) e = hipMemcpy(dA, A, asz, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dW, W, wsz, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(dG, 0xFF, gsz);
    if (e == hipSuccess) {
        LMEpilogue ep;
        memset(&ep, 0, sizeof(ep));
        ep.g = (uint16_t *)dG; ep.F = F;
        e = (hipError_t)lmk_gemm(0, (const uint16_t *)dA, K, (const uint16_t *)dW, M, N, K, LMK_EPI_GATE, &ep);
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(g, dG, gsz, hipMemcpyDeviceToHost);
    hipFree(dA); hipFree(dW); hipFree(dG);
    HIPCHK(e);
    return LM_OK;
}

int lm_gemm_split_count(int M, int N, int K)
{
    if (M < 1 || N < 1 || K < 64 || K % 64) return LM_ERR_INVALID;
    return lmk_pick_split(M, N, K);
}
