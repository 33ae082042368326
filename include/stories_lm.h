/*
 * stories_lm.h — C ABI of the MI355X (gfx950) Stories / Llama-2 token loop.
 *
 * Plain C types only: no HIP, no torch, no C++ in any signature.  One opaque
 * handle (LMModel) owns every device buffer, one HIP stream and the captured
 * per-step graphs.  Conventions follow libane's C ABI (libane/ane.h:95-231):
 * opaque handle, NULL on failed creation with a status code, negative int
 * status on failure, caller-owned host buffers, a message on stderr for every
 * failure.  A handle is single-threaded and not re-entrant; distinct handles
 * may be used from distinct threads.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   Config                  training/model.h:19-21 (= Llama2Config,
 *                           training/stories_config.h:107-110)
 *   LMWeights               weight members of Model, training/model.h:27-39,
 *                           one contiguous block per tensor (llama2.c file order)
 *   LMLayerWeights          the same members as per-layer pointer arrays, as
 *                           Model holds them (float *wq[N_LAYERS], model.h:27-39;
 *                           LayerWeights, training_dynamic/config.h:39-43)
 *   lm_init                 ane_init, libane/ane.h:97-100
 *   lm_create               model_load_weights + model_compile_kernels,
 *                           training/model.h:78-205; compile_fwd_kernels +
 *                           weight staging, training/training_dynamic/generate.m:251-277,386-392
 *   lm_create_layers        model_compile_kernels(Model *) over an already
 *                           loaded Model, training/model.h:169-205
 *   lm_load_llama2c         model_load_weights, training/model.h:78-164
 *   lm_forward              the per-token body of generate.m:437-487 (KV-cache
 *                           form of training/dashboard.py:205-267)
 *   lm_forward_batch        the same step for B independent sequences
 *   lm_prefill(_batch)      model_forward, training/forward.h:104-170
 *   lm_generate_greedy      the greedy token loop, generate.m:427-516 with
 *                           sample_argmax generate.m:129-136
 *   lm_free                 ane_free, libane/ane.h:230-231
 */
#ifndef STORIES_LM_H
#define STORIES_LM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * Model configuration — the llama2.c file header, same field order
 * (training/model.h:19-21).  In a llama2.c file a negative vocab_size marks an
 * untied classifier that follows rms_final (training/model.h:85-86,155-160).
 * ------------------------------------------------------------------------- */
typedef struct {
    int dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
} Config;

typedef enum { LM_DTYPE_F32 = 0, LM_DTYPE_F16 = 1 } LMDType;

/* Host weight buffers, one element type for all (fp32, or IEEE binary16 bit
 * patterns stored as uint16).  Per-layer tensors are contiguous over layers in
 * the llama2.c file order (training/model.h:94-160):
 *   token_embedding [vocab, dim]          rms_att_w [L, dim]
 *   wq [L, n_heads*hd, dim]               wk, wv [L, n_kv_heads*hd, dim]
 *   wo [L, dim, n_heads*hd]               rms_ffn_w [L, dim]
 *   w1 [L, hidden, dim]  w2 [L, dim, hidden]  w3 [L, hidden, dim]
 *   rms_final_w [dim]                     wcls [vocab, dim] (NULL = tied)
 * Every matrix is W[out, in] row-major: y = W x (training/forward.h:35-44).
 * fp32 input is rounded to fp16 (round-to-nearest-even) on upload. */
typedef struct {
    LMDType dtype;
    const void *token_embedding;
    const void *rms_att_w;
    const void *wq, *wk, *wv, *wo;
    const void *rms_ffn_w;
    const void *w1, *w2, *w3;
    const void *rms_final_w;
    const void *wcls;
} LMWeights;

/* The same weights as per-layer pointers, the way the reference's Model holds
 * them (training/model.h:27-39: float *wq[N_LAYERS] ..., each layer's tensor
 * malloc'd on its own by model_load_weights, model.h:129-147): every per-layer
 * member points at an array of n_layers pointers, entry l at layer l's tensor
 * (rms_att_w[l] [dim], wq[l] [n_heads*hd, dim], wk[l] and wv[l]
 * [n_kv_heads*hd, dim], wo[l] [dim, n_heads*hd], rms_ffn_w[l] [dim], w1[l] and
 * w3[l] [hidden, dim], w2[l] [dim, hidden]), all of one element type. */
typedef struct {
    LMDType dtype;
    const void *token_embedding;              /* [vocab, dim]            */
    const void *const *rms_att_w;             /* [n_layers] -> [dim]     */
    const void *const *wq, *const *wk, *const *wv, *const *wo;
    const void *const *rms_ffn_w;
    const void *const *w1, *const *w2, *const *w3;
    const void *rms_final_w;                  /* [dim]                   */
    const void *wcls;                         /* [vocab, dim]; NULL = tied */
} LMLayerWeights;

typedef struct LMModel LMModel;

/* Status codes.  0 / -1 / -2 keep ane_init's meaning (libane/ane.h:99). */
#define LM_OK               0
#define LM_ERR_NO_DEVICE   (-1)   /* no HIP device visible                        */
#define LM_ERR_NOT_GFX950  (-2)   /* device present but not gfx950 (CDNA4)        */
#define LM_ERR_INVALID     (-3)   /* NULL handle / pointer, bad count             */
#define LM_ERR_OOM         (-4)   /* host or device allocation failed             */
#define LM_ERR_HIP         (-5)   /* a HIP runtime call failed                    */
#define LM_ERR_IO          (-6)   /* file open / read / write failed              */
#define LM_ERR_FORMAT      (-7)   /* truncated or inconsistent weight file        */
#define LM_ERR_RANGE       (-8)   /* token, position, slot or length out of range */
#define LM_ERR_UNSUPPORTED (-9)   /* shape outside what the kernels are built for */
#define LM_ERR_NOT_INIT    (-10)  /* lm_init was not called or failed             */

/* Human-readable text for a status code (static storage). */
const char *lm_strerror(int status);

/* ---------------------------------------------------------------------------
 * Device
 * ------------------------------------------------------------------------- */

/* Select device 0 and check it is gfx950.  0 on success, LM_ERR_NO_DEVICE,
 * LM_ERR_NOT_GFX950.  Idempotent.  Replaces ane_init (libane/ane.h:97-100). */
int lm_init(void);

typedef struct {
    char name[64];          /* marketing name from the runtime         */
    char arch[32];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int  compute_units;
    int  clock_khz;
    int  l2_bytes;
    size_t total_mem;
} LMDeviceInfo;

/* Fill *out for device 0.  Replaces ane_device_info (libane/ane.h:108-109). */
int lm_device_info(LMDeviceInfo *out);

/* ---------------------------------------------------------------------------
 * Model lifetime
 * ------------------------------------------------------------------------- */

/* Build a device model from host weights.  The weights are copied (fp16 on
 * device); the caller keeps ownership of *w.  max_batch sequences ("slots") of
 * up to max_seq positions each get an fp16 KV cache.  Requires dim % 64 == 0,
 * head_dim in {64, 128}, hidden_dim % 64 == 0, n_heads % n_kv_heads == 0.
 * Returns NULL and sets *status (if non-NULL) on failure. */
LMModel *lm_create(const Config *cfg, const LMWeights *w, int max_batch,
                   int max_seq, int *status);

/* lm_create from per-layer weight pointers (LMLayerWeights): a caller holding
 * a loaded Model passes its pointer arrays as they are, with no repacking.
 * The result is identical to lm_create on the same values.  A NULL array or a
 * NULL entry fails with LM_ERR_INVALID (checked before any device call). */
LMModel *lm_create_layers(const Config *cfg, const LMLayerWeights *w, int max_batch,
                          int max_seq, int *status);

/* Read a llama2.c model file (fp32 values, header as Config, file order of
 * training/model.h:78-164, negative vocab_size = untied) and lm_create it.
 * Truncated files and inconsistent headers fail with LM_ERR_FORMAT. */
LMModel *lm_load_llama2c(const char *path, int max_batch, int max_seq,
                         int *status);

/* Read a BLZT version 4 training checkpoint (the reference's format:
 * load_gen_checkpoint, training/training_dynamic/generate.m:212-248; header
 * config.h:78-86) and lm_create it: the weights are read, the Adam state is
 * skipped, the classifier is the embedding.  Shapes with q_dim != dim fail
 * with LM_ERR_FORMAT. */
LMModel *lm_load_blzt(const char *path, int max_batch, int max_seq, int *status);

/* Host only: rewrite a BLZT v4 checkpoint's weights as a llama2.c file (tied
 * classifier). */
int lm_blzt_to_llama2c(const char *blzt_path, const char *out_path);

/* Release every host and device resource of the handle.  NULL is a no-op. */
void lm_free(LMModel *m);

/* Copy the model's Config (vocab_size always positive) into *out. */
int lm_get_config(const LMModel *m, Config *out);

/* ---------------------------------------------------------------------------
 * Forward
 * ------------------------------------------------------------------------- */

/* One decode step of slot 0: embed `token` at position `pos`, append its K/V
 * to the cache, attend over positions 0..pos, return the vocab_size fp32
 * logits.  The pointer is an internal host buffer valid until the next call on
 * the handle; NULL on error (message on stderr).  Positions 0..pos-1 of slot 0
 * must have been filled by earlier steps or by lm_prefill. */
const float *lm_forward(LMModel *m, int token, int pos);

/* One decode step for B sequences: row b uses KV slot b, token tokens[b] at
 * position pos[b].  logits (B x vocab, may be NULL) and argmax (B, may be NULL;
 * lowest index on ties, generate.m:129-136) are host buffers. */
int lm_forward_batch(LMModel *m, const int *tokens, const int *pos, int B,
                     float *logits, int *argmax);

/* Causal forward of S tokens of one sequence at positions pos0..pos0+S-1 into
 * KV slot `slot` (positions < pos0 must already be cached).  Writes the S x
 * vocab_size fp32 logits to `logits` when non-NULL; they always stay readable
 * on the device through lm_read_logits until the next forward call. */
int lm_prefill(LMModel *m, int slot, int pos0, const int *tokens, int S,
               float *logits);

/* nseq independent sequences of S tokens each from position 0, sequence i
 * into KV slot slots[i] (slots NULL = 0..nseq-1); tokens is nseq x S row-major.
 * logits_mode LM_LOGITS_ALL computes all nseq*S logit rows (the training-shape
 * forward, training/forward.h:104-170); LM_LOGITS_LAST only the last row of
 * each sequence (what a decode that follows needs).  `logits` (host, may be
 * NULL) receives nseq*S or nseq rows.  Rows go through the GEMMs together, in
 * chunks of whole sequences when nseq*S exceeds the handle's row capacity; the
 * device keeps the last chunk's logits for lm_read_logits. */
#define LM_LOGITS_ALL  0
#define LM_LOGITS_LAST 1
int lm_prefill_batch(LMModel *m, int nseq, const int *slots, const int *tokens,
                     int S, int logits_mode, float *logits);

/* model_forward with its loss (training/forward.h:104-184; train.m:64 is its
 * caller): the causal forward of nseq sequences of S >= 2 tokens from position
 * 0, as lm_prefill_batch with LM_LOGITS_ALL, and the mean next-token
 * cross-entropy of each sequence, loss[i] = -(1/(S-1)) sum_{t<S-1}
 * log softmax(logits[i, t])[tokens[i, t+1]].  The log-probabilities are taken
 * on the device from the device logits, one fp32 value per row comes back, and
 * the host sums them per sequence in the reference's order; `logits` (host,
 * may be NULL) also receives all nseq*S rows.  loss: nseq floats.
 * LM_ERR_UNSUPPORTED when vocab_size is not a multiple of 4. */
int lm_prefill_loss(LMModel *m, int nseq, const int *slots, const int *tokens,
                    int S, float *logits, float *loss);

/* Copy rows [row0, row0+nrows) of the last forward's device logits to dst. */
int lm_read_logits(LMModel *m, int row0, int nrows, float *dst);

/* Greedy decode of n_steps tokens for B sequences (slot b), entirely on the
 * device: step t feeds the argmax of step t-1 back as the next token without
 * a host round trip (one captured graph replayed per step).  Sequence b starts
 * from first_tokens[b] at position pos0[b] (earlier positions already cached);
 * out_tokens (n_steps x B, row-major by step) receives the generated ids.
 * EOS is not a stop condition here (every step is run); callers that want
 * generate.m's EOS break (generate.m:501) scan out_tokens. */
int lm_generate_greedy(LMModel *m, int B, const int *first_tokens,
                       const int *pos0, int n_steps, int *out_tokens);

/* ---------------------------------------------------------------------------
 * Timing on the model's stream (hipEvents), for benchmarks
 * ------------------------------------------------------------------------- */

/* Block until all work queued on the handle's stream is done. */
int lm_sync(LMModel *m);

/* Record a start event on the handle's stream. */
int lm_timer_begin(LMModel *m);

/* Record a stop event, wait for it, return elapsed ms since lm_timer_begin. */
int lm_timer_end(LMModel *m, float *ms);

/* Execution knobs.  LM_OPT_USE_GRAPH: 1 (default) replays captured hipGraphs,
 * 0 launches kernels directly (debugging / per-kernel timing). */
#define LM_OPT_USE_GRAPH   2
/* LM_OPT_KV_F32: 1 stores the K/V cache in fp32 (the reference forward keeps
 * K and V in fp32, training/forward.h:118-128), 0 (default) in binary16.
 * Changing it reallocates and clears the cache of every slot. */
#define LM_OPT_KV_F32      3
/* LM_OPT_FUSE_QKV_ATTN: 3 (default) runs each layer of the batch-1 decode
 * chain as one launch: QKV GEMV, the attention of every head, Wo + residual,
 * W1/W3 + gate and W2 + residual, each set of work-groups handing its
 * results to the next through tagged words in memory, and folds the argmax
 * into the classifier's launch; batches of 2-4 run level 2 (faster there).
 * 4 takes the whole-layer launch for every batch of 1-4.  Where the
 * whole-layer form is not built for the model's widths and batch, level 2
 * runs.  2 runs QKV, attention and Wo as one launch and the FFN as two; 1
 * also launches Wo apart; 0 launches all five apart. */
#define LM_OPT_FUSE_QKV_ATTN 5
/* LM_OPT_HANDOFF_US: microseconds (the device's real-time counter) after
 * which a wait for a tagged hand-off word inside a fused launch gives up
 * (default 100000); every other wait of the call then ends at once, the
 * kernels run to their end and the call returns LM_ERR_HIP.  >= 1. */
#define LM_OPT_HANDOFF_US  6
/* LM_OPT_HANDOFF_ABORT: value 1 raises the give-up flag from the host, so
 * that every hand-off wait of the next decode call ends at once and that call
 * returns LM_ERR_HIP (the flag is then cleared).  For tests of that path. */
#define LM_OPT_HANDOFF_ABORT 7
/* LM_OPT_LAYER_WGS: at most this many work-groups of the whole-layer launch
 * (LM_OPT_FUSE_QKV_ATTN 3/4) share a CU (1-4, default 2; 0 = as many as
 * registers and LDS allow).  The launch holds more work-groups than the
 * device runs at once; with the cap, the W1/W3 and W2 work-groups are
 * dispatched as the QKV ones finish, so their weight loads do not compete
 * with the first roles'. */
#define LM_OPT_LAYER_WGS   8
/* LM_OPT_PREFILL_FOLD: 1 (default) folds the row norm after an unsplit Wo or
 * W2 of a prefill chunk into the GEMMs on either side (the GEMM writes
 * fp16(x * gain) and the row's sums of squares; the next GEMM scales its
 * product rows), 0 keeps the row norm a launch of its own.  The folded operand
 * is rounded before the row is normalised; a chunk in which it overflows
 * fp16 is redone with the norm apart, so both give finite results. */
#define LM_OPT_PREFILL_FOLD 9
int lm_set_option(LMModel *m, int option, int value);

/* ---------------------------------------------------------------------------
 * Weight utilities (host only, no device needed)
 * ------------------------------------------------------------------------- */

/* Number of scalars in the llama2.c-ordered weight set of cfg (untied adds a
 * classifier of vocab x dim).  Uses |vocab_size|. */
size_t lm_weights_numel(const Config *cfg, int untied);

/* Point *out at the tensors of a contiguous llama2.c-ordered buffer `base` of
 * element type dtype (fp32 or fp16 bits).  untied=0 makes wcls NULL (tied). */
int lm_weights_view(const Config *cfg, LMDType dtype, const void *base,
                    int untied, LMWeights *out);

/* Fill a contiguous fp16 buffer (lm_weights_numel(cfg, untied) elements, file
 * order) with seeded weights: every matrix entry is round-to-nearest-even fp16
 * of std * N(0,1), the normal drawn by Box-Muller from SplitMix64 counters keyed
 * by (seed, tensor index, element index); norm gains are exactly 1.0.  The
 * result is identical for any thread count. */
int lm_synth_weights_f16(const Config *cfg, uint64_t seed, float std,
                         int untied, uint16_t *out);

/* Write a llama2.c file (fp32 values; vocab_size written negative when
 * w->wcls is non-NULL and distinct from the embedding). */
int lm_write_llama2c(const char *path, const Config *cfg, const LMWeights *w);

/* IEEE binary16 <-> binary32 (round to nearest, ties to even). */
void lm_f32_to_f16(const float *src, uint16_t *dst, size_t n);
void lm_f16_to_f32(const uint16_t *src, float *dst, size_t n);

/* The fp32 RoPE rotation table used on the device, built on the host with the
 * reference's expressions (training/forward.h:58-61): for position p and pair
 * i (i = 0..head_dim/2-1), freq = 1/powf(10000, 2i/head_dim), angle = p*freq,
 * cos_out[p*(hd/2)+i] = cosf(angle), sin_out[...] = sinf(angle). */
int lm_rope_table(int max_seq, int head_dim, float *cos_out, float *sin_out);

/* ---------------------------------------------------------------------------
 * Diagnostics (no counterpart in the reference)
 * ------------------------------------------------------------------------- */

/* Run the device wave-reduction self-test on 64 inputs: out4 = {sum of lanes
 * 0..31, sum of lanes 32..63, wave sum (DPP), wave sum (shuffles)}. */
int lm_selftest_reduce(const float *in64, float *out4);

/* Argmax partial as the kernels write it: best value and its column. */
typedef struct { float val; int idx; } LMArgPartHost;

/* Run one MFMA GEMM C = A W^T (fp32 accumulation) on caller data through the
 * LDS-tiled kernel the prefill and batched decode use (the tile the runtime
 * picks for M rows): A [M, K] fp16 bits (a_f32 = 0) or fp32 (a_f32 = 1,
 * rounded to fp16 on load), W [N, K] fp16 bits, C [M, N] fp32, part (may be
 * NULL) [M, ceil(N/32)] per-32-column argmax partials.  K % 64 == 0. */
int lm_selftest_gemm(int M, int N, int K, int a_f32, const void *A, const uint16_t *W,
                     float *C, LMArgPartHost *part);

/* Run the K-split GEMM the forward uses for narrow projections (the tiled
 * kernel, up to 4096 rows; K a multiple of 64*nsplit): parts[s] [M, N] fp32 = A[:, s*K/n .. (s+1)*K/n)
 * W[:, same]^T for s < n, n = nsplit, or the runtime's own choice when
 * nsplit == 0.  A [M, K] and W [N, K] fp16 bits; parts holds n*M*N floats (size
 * it with lm_gemm_split_count).  Returns n (> 0) or a negative status. */
int lm_selftest_gemm_split(int M, int N, int K, int nsplit, const uint16_t *A, const uint16_t *W,
                           float *parts);

/* Run the W1/W3 GEMM with the SiLU-gate epilogue the forward uses (the tile
 * the runtime picks for M rows): W [N, K] holds W1 and W3 rows interleaved in
 * blocks of 16 (block j: W1 rows 16j .. 16j+15, then W3 rows 16j .. 16j+15),
 * h = A W^T in fp32, and g[m, 16j + c] = fp16(silu(h[m, 32j + c]) *
 * h[m, 32j + 16 + c]) for c < 16.  A [M, K] fp16 bits, g [M, N/2] fp16 bits;
 * N a multiple of 32, K of 64. */
int lm_selftest_gemm_gate(int M, int N, int K, const uint16_t *A, const uint16_t *W, uint16_t *g);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): the GEMM and argmax of lm_selftest_gemm on the caller's device
 * buffers, allocating nothing.  C = A W^T (fp32 accumulation; A [M, K] and W
 * [N, K] fp16 bits, C [M, N] fp32, all device pointers; C may be NULL) and
 * ids[m] = the lowest column of row m's maximum (device int[M]), queued on
 * `stream` (a hipStream_t; NULL = the null stream) without waiting.  The
 * argmax partials live in a static 512 KiB device array per GPU, so M *
 * ceil(N / 32) may not exceed 65536 (LM_ERR_RANGE beyond, nothing queued);
 * K % 64 == 0.  Calls that overlap on one GPU share that array and race.
 * lm_init must have succeeded (LM_ERR_NOT_INIT otherwise). */
int lm_gemm_argmax_noalloc(int M, int N, int K, const uint16_t *A, const uint16_t *W, float *C,
                           int *ids, void *stream);

/* The split count the runtime uses for an [M, K] x [N, K]^T GEMM (1: unsplit). */
int lm_gemm_split_count(int M, int N, int K);

/* Kernel families of a decode step (index into lm_profile_chain's output). */
#define LM_KERN_QKV    0   /* rmsnorm + QKV GEMV + RoPE + KV append          */
#define LM_KERN_ATTN   1   /* causal attention over the KV cache              */
#define LM_KERN_WO     2   /* Wo GEMV + residual                            */
#define LM_KERN_W13    3   /* rmsnorm + W1/W3 GEMV + SiLU gate              */
#define LM_KERN_W2     4   /* W2 GEMV + residual                            */
#define LM_KERN_CLS    5   /* final rmsnorm + classifier + argmax partials   */
#define LM_KERN_ARGMAX 6   /* argmax reduction + greedy loop state          */
#define LM_KERN_COUNT  7

/* Mean device microseconds per launch of each decode kernel family inside the
 * real decode chain: `steps` greedy decode steps of B rows from tokens[b] at
 * positions pos[b] (advancing as a decode does), launched directly and queued
 * back to back in runs of 16 steps as the greedy loop's graphs run them.
 * Each run of consecutive launches of one family (at the default fusion level
 * the n_layers whole-layer launches of a step, then the classifier) is timed
 * by events at its first dispatch's device start and its last one's end, with
 * no event between them, and its time shared equally among its launches.
 * One untimed step runs first.  launches_per_step[k] (may
 * be NULL) = launches of family k in one decode step.  Needs pos[b] + steps +
 * 1 <= max_seq; leaves the KV cache at those positions and the activations
 * overwritten. */
int lm_profile_chain(LMModel *m, int B, const int *tokens, const int *pos, int steps,
                     float *us_per_launch, int *launches_per_step);

/* ---------------------------------------------------------------------------
 * Text: tokenizer, random stream, samplers (host only, no device needed)
 * ------------------------------------------------------------------------- */

/* llama2.c tokenizer.bin: int max_token_length, then per token {float score,
 * int len, len bytes} (replaces tokenizer_load, generate.m:37-56).  NULL on
 * failure with *status = LM_ERR_IO / LM_ERR_FORMAT / LM_ERR_OOM. */
typedef struct LMTokenizer LMTokenizer;
LMTokenizer *lm_tokenizer_load(const char *path, int vocab_size, int *status);
void lm_tokenizer_free(LMTokenizer *t);
int lm_tokenizer_vocab_size(const LMTokenizer *t);

/* The token's string, "" when out of range (tokenizer_decode, generate.m:58-65). */
const char *lm_tokenizer_decode(const LMTokenizer *t, int token);

/* Greedy BPE of text into at most max_tokens ids, returned count (or a
 * negative status): every byte becomes its single-byte token (bytes without
 * one are skipped), then the adjacent pair whose concatenation is the
 * highest-scoring token is merged until none is (tokenizer_encode,
 * generate.m:68-126; no BOS, no leading space). */
int lm_tokenizer_encode(const LMTokenizer *t, const char *text, int *tokens, int max_tokens);

/* Random stream with the drand48 recurrence and srand48 seeding (the
 * reference's sampler draws, generate.m:153,197), with explicit state. */
typedef struct { uint64_t x; } LMRng;
void lm_rng_seed(LMRng *r, uint64_t seed);
double lm_rng_next(LMRng *r);

/* Mean next-token cross-entropy over S logit rows [S, V] (host, e.g. from
 * lm_prefill): *loss = -(1/(S-1)) sum_{t<S-1} log softmax(logits[t])[tokens[t+1]],
 * with the reference's arithmetic (model_forward's loss, training/forward.h:
 * 174-183).  LM_ERR_INVALID for S < 2, LM_ERR_RANGE for a token outside [0, V). */
int lm_mean_ce(const float *logits, const int *tokens, int S, int V, float *loss);

/* Samplers over n host logits (generate.m:129-209): argmax (lowest index on
 * ties); temperature softmax then one draw; nucleus (top-p) over the
 * temperature softmax.  Return the token, or a negative status. */
int lm_sample_argmax(const float *logits, int n);
int lm_sample_temperature(const float *logits, int n, float temp, LMRng *r);
int lm_sample_topp(const float *logits, int n, float temp, float topp, LMRng *r);

#ifdef __cplusplus
}
#endif

#endif /* STORIES_LM_H */
