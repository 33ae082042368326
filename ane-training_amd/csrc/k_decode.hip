/*
 * k_decode.hip — decode kernels for gfx950: the small-batch (B <= 4) chain, and
 * the attention of decode rows for every batch size (k_attn_decode; after a
 * K-split QKV GEMM of 5..64 rows, k_attn_decode_part, which first sums q, k, v
 * from the GEMM's partials, rotates and appends them).
 *
 * One decode step of one layer is five stages, shaped after the reference's
 * fused forward programs (training/training_dynamic/mil_dynamic.h:56-288) and
 * cut only where every output needs the whole of the previous vector.  They
 * run as five launches, or (k_qkv_attn) as roles of the work-groups of one
 * launch that hand their results on through tagged words in memory:
 *   qkv_rope   rmsnorm prologue (forward.h:46-53) + [Wq;Wk;Wv] GEMV
 *              (forward.h:122-124) + interleaved RoPE (forward.h:55-70) + KV
 *              append; layer 0 also gathers the embedding row (forward.h:108-110)
 *   attn       causal attention of one (sequence, head) per work-group over the
 *              cached positions 0..pos (forward.h:72-99)
 *   wo         Wo GEMV + residual (forward.h:134-136)
 *   ffn13      rmsnorm prologue + W1/W3 GEMV + SiLU gate (forward.h:139-151)
 *   w2         W2 GEMV + residual (forward.h:157-159)
 * and per token the classifier (forward.h:163-170) with per-work-group argmax
 * partials, and their reduction (generate.m:129-136, 474-493).
 *
 * GEMV mapping: a wave owns a pair of weight rows, each 32-lane half one row;
 * a lane streams 16-byte (8 x fp16) chunks (c*32 + lane) of its row.  Every
 * kernel issues its weight loads first, before it reads the activation vector
 * that the previous launch produced, so the HBM latency of the weights overlaps
 * the prologue.  The fp32 activation vector is staged in LDS and the half-wave
 * sums are formed with DPP.  Pairs line up with RoPE pairs (rows 2i, 2i+1) and
 * with the gate pairs (row i of W1 in half 0, row i of W3 in half 1).
 */
#include "k_common.h"
#include "lm_internal.h"
#include <hip/hip_ext.h>

#include <atomic>

/* Launch-timing slot for lm_profile_chain: when armed, the next decode-chain
 * kernel launch of this host thread goes through hipExtLaunchKernelGGL with the
 * two events (either may be NULL), which the device timestamps at that
 * dispatch's start and end; a start armed on one launch and a stop on a later
 * one time the run of launches between them with no event in between. */
static thread_local hipEvent_t t_ev0, t_ev1;
static thread_local int t_armed;

extern "C" void lmk_time_next(hipEvent_t start, hipEvent_t stop)
{
    t_ev0 = start;
    t_ev1 = stop;
    t_armed = 1;
}

#define DLAUNCH(K, grid, block, shm, s, ...)                                          \
    do {                                                                             \
        if (t_armed) {                                                               \
            t_armed = 0;                                                             \
            hipExtLaunchKernelGGL(K, grid, block, shm, s, t_ev0, t_ev1, 0, __VA_ARGS__); \
        } else {                                                                     \
            hipLaunchKernelGGL(K, grid, block, shm, s, __VA_ARGS__);                 \
        }                                                                            \
    } while (0)

#define WG 256
#define NWAVE (WG / 64)

/* ---- prologues ---------------------------------------------------------- */

/* Every global load of a prologue is issued up front (K / WG is a compile-time
 * trip count), so a prologue costs one memory latency, which the weight loads
 * issued before it also cover. */

/* Raw input rows of a normalising prologue, loaded into registers: src_b is
 * x[b*K ..] (fp32) or, when emb != NULL, the fp16 embedding row emb[tok[b]*K ..];
 * rows B <= b < NB are zero.  wv holds the gain w[i] of this thread's columns. */
template <int K, int NB>
struct NormIn {
    float v[NB][K / WG];
    float w[K / WG];
};

template <int K, int NB>
__device__ __forceinline__ void norm_load(const float *__restrict__ x, const u16 *__restrict__ emb,
                                          const int *__restrict__ tok, const float *__restrict__ w,
                                          int B, NormIn<K, NB> &in)
{
    constexpr int PER = K / WG;
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < PER; j++) in.w[j] = w[tid + j * WG];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (b < B) {
            if (emb) {
                const u16 *er = emb + (size_t)tok[b] * K;
#pragma unroll
                for (int j = 0; j < PER; j++) in.v[b][j] = h2f(er[tid + j * WG]);
            } else {
#pragma unroll
                for (int j = 0; j < PER; j++) in.v[b][j] = x[(size_t)b * K + tid + j * WG];
            }
        } else {
#pragma unroll
            for (int j = 0; j < PER; j++) in.v[b][j] = 0.f;
        }
    }
}

/* The normalising prologue with the row scale left to the caller:
 * xs[b*K + i] = src_b[i] * w[i] and scale[b] = 1/sqrt(mean(src_b^2) + 1e-5)
 * (forward.h:46-53).  The norm is one factor per row, so it distributes over
 * the caller's dot products, which it multiplies in after their sums: one
 * barrier instead of two (one before the scale is known, one after the
 * normalised rows are written), and the scale's reduction overlaps the LDS
 * writes.  With store_x, work-group 0 also writes the raw rows to x. */
template <int K, int NB>
__device__ __forceinline__ void norm_to_lds_unscaled(const NormIn<K, NB> &in, int B,
                                                     float *__restrict__ x, bool store_x,
                                                     float *xs, float scale[NB])
{
    constexpr int PER = K / WG;
    __shared__ float red[NB][NWAVE];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            ss = fmaf(in.v[b][j], in.v[b][j], ss);
            xs[b * K + tid + j * WG] = in.v[b][j] * in.w[j];
        }
        ss = wave_sum(ss);
        if (lane == 0) red[b][wv] = ss;
    }
    if (store_x && blockIdx.x == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++)
            if (b < B) {
#pragma unroll
                for (int j = 0; j < PER; j++) x[(size_t)b * K + tid + j * WG] = in.v[b][j];
            }
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < NWAVE; i++) tot += red[b][i];
        scale[b] = 1.0f / sqrtf(tot / K + 1e-5f);
    }
}

/* NB rows of K fp32 from src (rows >= B zero), loaded into registers. */
template <int K, int NB>
struct RowsIn {
    float v[NB][K / WG];
};

template <int K, int NB>
__device__ __forceinline__ void rows_load(const float *__restrict__ src, int B, RowsIn<K, NB> &in)
{
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < K / WG; j++)
            in.v[b][j] = b < B ? src[(size_t)b * K + threadIdx.x + j * WG] : 0.f;
}

template <int K, int NB>
__device__ __forceinline__ void rows_to_lds(const RowsIn<K, NB> &in, float *xs)
{
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < K / WG; j++) xs[b * K + threadIdx.x + j * WG] = in.v[b][j];
    __syncthreads();
}

/* ---- GEMV core ------------------------------------------------------------ */

/* Issue the loads of one fp16 row (length K) for half-wave lane hl. */
template <int K>
__device__ __forceinline__ void hw_load(const u16 *__restrict__ wrow, int hl, uint4 wv[K / 256])
{
#pragma unroll
    for (int c = 0; c < K / 256; c++)
        wv[c] = *(const uint4 *)(wrow + (size_t)(c * 32 + hl) * 8);
}

/* Half-wave partial dot products of a prefetched row with NB fp32 LDS rows. */
template <int K, int NB>
__device__ __forceinline__ void hw_dot(const uint4 wv[K / 256], const float *xs, int hl,
                                       float acc[NB])
{
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = 0.f;
#pragma unroll
    for (int c = 0; c < K / 256; c++) {
        float w[8];
        unpack8(wv[c], w);
        const int k0 = (c * 32 + hl) * 8;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float4 xa = *(const float4 *)(xs + b * K + k0);
            const float4 xb = *(const float4 *)(xs + b * K + k0 + 4);
            float a = acc[b];
            a = fmaf(w[0], xa.x, a); a = fmaf(w[1], xa.y, a);
            a = fmaf(w[2], xa.z, a); a = fmaf(w[3], xa.w, a);
            a = fmaf(w[4], xb.x, a); a = fmaf(w[5], xb.y, a);
            a = fmaf(w[6], xb.z, a); a = fmaf(w[7], xb.w, a);
            acc[b] = a;
        }
    }
}

/* Reduce per-half partials; r0[b] = row of half 0, r1[b] = row of half 1
 * (uniform across the wave). */
template <int NB>
__device__ __forceinline__ void pair_reduce(const float acc[NB], float r0[NB], float r1[NB])
{
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float s = half_wave_sum(acc[b]);
        r0[b] = readlane_f(s, 31);
        r1[b] = readlane_f(s, 63);
    }
}

/* ---- QKV + RoPE + KV append ------------------------------------------------ */

/* Hand-off words of the fused QKV + attention kernel: 64-bit words {value
 * bits, tag}, stored and loaded as relaxed agent-scope atomics, so a reader
 * that sees the current tag sees that launch's value (each word carries its
 * own proof of freshness; no ordering between words is assumed).  q, k and v
 * of row b: tq[b*NQ + i], tk[b*NKV + i], tv[b*NKV + i] (k and v as the cache
 * stores them).  The tag of a launch is epoch * n_layers + layer + 1, epoch the
 * decode-step count the argmax kernel advances: never 0 (the buffers' initial
 * contents) and never repeated within 2^32 launches. */
struct QkvTagged {
    unsigned long long *tq, *tk, *tv;
    unsigned long long *ta;         /* head outputs [b*NQ + h*hd + d] (Wo in the launch), in
                                     * LM_TA_COPIES copies LM_TAG_B*NQ words apart */
    unsigned long long *tx;         /* x after Wo [b*D + i] (FFN in the launch), in
                                     * LM_TX_COPIES copies LM_TAG_B*D apart */
    unsigned long long *tgt;        /* gate g [b*F + i] (FFN in the launch), copies
                                     * LM_TAG_B*F apart */
    const unsigned *epoch;
    int layer, n_layers;
    int *err;                       /* set when a hand-off wait gives up */
};

__device__ __forceinline__ unsigned qkv_tag(const QkvTagged &t)
{
    return *t.epoch * (unsigned)t.n_layers + (unsigned)t.layer + 1u;
}

__device__ __forceinline__ void tag_store(unsigned long long *w, float v, unsigned tag)
{
    const unsigned long long word =
        ((unsigned long long)tag << 32) | (unsigned long long)__builtin_bit_cast(unsigned, v);
    __hip_atomic_store(w, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Poll one tagged word until it carries `tag`.  The wait is bounded in real
 * time: err[1] is its limit in microseconds of the 100 MHz real-time counter
 * (s_memrealtime), so it ends however slowly polls return (a profiler's
 * counter pass, a busy memory system); one that gives up sets err[0] and
 * returns the word's value as it is.  A wait also stops at once when err[0]
 * is set (checked before the first sleep and every 256 polls after), so that
 * after one wait has given up, or after the host has raised the flag, the
 * rest of the launch and the launches queued behind it end within
 * microseconds; the host reads the flag with the call's results and reports
 * the failure. */
__device__ __forceinline__ float tag_wait(const unsigned long long *w, unsigned tag, int *err)
{
    unsigned long long v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((unsigned)(v >> 32) == tag) return __builtin_bit_cast(float, (unsigned)v);
    const unsigned long long lim = 100ull * (unsigned)err[1];   /* us -> 10 ns ticks */
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    for (int spin = 0; (unsigned)(v >> 32) != tag; spin++) {
        if ((spin & 255) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
            break;
        if ((spin & 15) == 15 && __builtin_amdgcn_s_memrealtime() - t0 > lim) {
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return __builtin_bit_cast(float, (unsigned)v);
}

__device__ __forceinline__ unsigned long long tag_peek(const unsigned long long *w)
{
    return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* The value of a word already read as v, or, when v carries another tag, of
 * the wait on it: a thread reads all its words first and waits only on those
 * not yet written, so its reads overlap instead of following one another. */
__device__ __forceinline__ float tag_take(unsigned long long v, const unsigned long long *w,
                                          unsigned tag, int *err)
{
    return (unsigned)(v >> 32) == tag ? __builtin_bit_cast(float, (unsigned)v) : tag_wait(w, tag, err);
}

/* Before a work-group reads a span of words (the doorbell): one thread polls
 * one word of the span while the others wait at the barrier, so that a waiting
 * work-group keeps one poll in flight instead of one per thread; the k-th
 * reader of a copy polls the last word of the copy's k-th 128-byte line
 * (wrapping), so that the readers of one copy poll different lines.  A hint
 * only: each word is still checked by its reader. */
__device__ __forceinline__ void tag_doorbell(const unsigned long long *w, int n, int k, unsigned tag,
                                             int *err)
{
    if (threadIdx.x == 0) (void)tag_wait(w + (k * 16 + 15) % n, tag, err);
    __syncthreads();
}

/* dst[i] = value of w[i] for i < n, this work-group's threads taking
 * i = threadIdx.x + j * WG, eight reads in flight per thread. */
__device__ __forceinline__ void tag_wait_span(const unsigned long long *w, int n, unsigned tag,
                                              int *err, float *dst)
{
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * WG) {
        unsigned long long v[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            v[j] = i0 + j * WG < n ? tag_peek(w + i0 + j * WG) : 0ull;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (i0 + j * WG < n) dst[i0 + j * WG] = tag_take(v[j], w + i0 + j * WG, tag, err);
    }
}

/* Rows of [Wq; Wk; Wv] . rmsnorm(x[b]) for the row pairs of this work-group,
 * RoPE'd and stored (q fp32, k/v into the cache); with tg, also as tagged
 * hand-off words. */
template <int D, int NB, typename KT>
__device__ __forceinline__ void qkv_rows(
    float *__restrict__ x, const u16 *__restrict__ emb, const int *__restrict__ tok,
    const float *__restrict__ rms_w, const u16 *__restrict__ W, int NQ, int NKV, int hd,
    const float *__restrict__ rc, const float *__restrict__ rs, const int *__restrict__ pos,
    int B, float *__restrict__ q, KT *__restrict__ kc, KT *__restrict__ vc, int max_seq,
    int npairs, const QkvTagged *tg, bool store_x = true)
{
    __shared__ __attribute__((aligned(16))) float xs[NB * D];
    const int p = blockIdx.x * NWAVE + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int r = 2 * min(p, npairs - 1);
    uint4 wv[D / 256];
    hw_load<D>(W + (size_t)(r + half) * D, hl, wv);
    NormIn<D, NB> in;
    norm_load<D, NB>(x, emb, tok, rms_w, B, in);
    /* epilogue operands: position and rotation of this row pair per sequence */
    const int half_hd = hd >> 1;
    const bool rot = r < NQ + NKV;
    const int rr = r < NQ ? r : (rot ? r - NQ : r - NQ - NKV);
    int ps[NB];
    float cr[NB], sr[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        ps[b] = b < B ? pos[b] : 0;
        const int ti = ps[b] * half_hd + ((rr & (hd - 1)) >> 1);
        cr[b] = rot ? rc[ti] : 1.f;
        sr[b] = rot ? rs[ti] : 0.f;
    }
    float scale[NB];
    norm_to_lds_unscaled<D, NB>(in, B, x, emb != nullptr && store_x, xs, scale);
    if (p >= npairs) return;
    float acc[NB], r0[NB], r1[NB];
    hw_dot<D, NB>(wv, xs, hl, acc);
    pair_reduce<NB>(acc, r0, r1);
    if (lane != 0) return;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        r0[b] *= scale[b];
        r1[b] *= scale[b];
    }
    /* hd is a power of two (64 or 128) */
    const int lg = __builtin_ctz((unsigned)hd);
    const int Hkv = NKV >> lg;
    const int h = rr >> lg, d = rr & (hd - 1);
    const unsigned tag = tg ? qkv_tag(*tg) : 0u;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (b >= B) break;
        if (rot) {
            const float a = r0[b], e = r1[b], c = cr[b], sn = sr[b];
            const float o0 = fmaf(a, c, -(e * sn));  /* forward.h:64 */
            const float o1 = fmaf(a, sn, e * c);     /* forward.h:65 */
            if (r < NQ) {
                if (tg) {
                    tag_store(tg->tq + (size_t)b * NQ + r, o0, tag);
                    tag_store(tg->tq + (size_t)b * NQ + r + 1, o1, tag);
                } else {
                    *(float2 *)(q + (size_t)b * NQ + r) = make_float2(o0, o1);
                }
            } else {
                KT *dst = kc + (((size_t)b * Hkv + h) * max_seq + ps[b]) * hd + d;
                dst[0] = kv_pack<KT>(o0);
                dst[1] = kv_pack<KT>(o1);
                if (tg) {
                    tag_store(tg->tk + (size_t)b * NKV + rr, kv_round<KT>(o0), tag);
                    tag_store(tg->tk + (size_t)b * NKV + rr + 1, kv_round<KT>(o1), tag);
                }
            }
        } else {
            KT *dst = vc + (((size_t)b * Hkv + h) * max_seq + ps[b]) * hd + d;
            dst[0] = kv_pack<KT>(r0[b]);
            dst[1] = kv_pack<KT>(r1[b]);
            if (tg) {
                tag_store(tg->tv + (size_t)b * NKV + rr, kv_round<KT>(r0[b]), tag);
                tag_store(tg->tv + (size_t)b * NKV + rr + 1, kv_round<KT>(r1[b]), tag);
            }
        }
    }
}

template <int D, int NB, typename KT>
__global__ void __launch_bounds__(WG) k_qkv_rope(
    float *__restrict__ x, const u16 *__restrict__ emb, const int *__restrict__ tok,
    const float *__restrict__ rms_w, const u16 *__restrict__ W, int NQ, int NKV, int hd,
    const float *__restrict__ rc, const float *__restrict__ rs, const int *__restrict__ pos,
    int B, float *__restrict__ q, KT *__restrict__ kc, KT *__restrict__ vc, int max_seq,
    int npairs)
{
    qkv_rows<D, NB, KT>(x, emb, tok, rms_w, W, NQ, NKV, hd, rc, rs, pos, B, q, kc, vc, max_seq, npairs,
                        nullptr);
}

/* ---- decode attention ------------------------------------------------------- */

/* Materialise a float4 in registers at this point of the program (an empty
 * asm that reads and writes each element), so the compiler cannot sink the
 * code that computed it past later code. */
__device__ __forceinline__ void pin4(float4 &v)
{
    float x = v.x, y = v.y, z = v.z, w = v.w;
    asm volatile("" : "+v"(x), "+v"(y), "+v"(z), "+v"(w));
    v = make_float4(x, y, z, w);
}

/* 8 cache elements at p as raw bits (fp16: one 16-byte load; fp32: two). */
struct KV8h { uint4 a; };
struct KV8f { float4 a, b; };
template <typename KT> struct KVRaw;
template <> struct KVRaw<u16> { typedef KV8h T; };
template <> struct KVRaw<float> { typedef KV8f T; };

__device__ __forceinline__ void kv_raw_load(const u16 *p, KV8h &r) { r.a = *(const uint4 *)p; }
__device__ __forceinline__ void kv_raw_load(const float *p, KV8f &r)
{
    r.a = *(const float4 *)p;
    r.b = *(const float4 *)(p + 4);
}
__device__ __forceinline__ void kv_raw_unpack(const KV8h &r, float f[8]) { unpack8(r.a, f); }
__device__ __forceinline__ void kv_raw_unpack(const KV8f &r, float f[8])
{
    f[0] = r.a.x; f[1] = r.a.y; f[2] = r.a.z; f[3] = r.a.w;
    f[4] = r.b.x; f[5] = r.b.y; f[6] = r.b.z; f[7] = r.b.w;
}

/* Work-group (h, b), 4 waves: query row b (q[b], cache slot slot[b] or b when
 * slot is NULL) attends to positions 0..pos[b].  The positions are cut in tiles;
 * wave w takes tiles w, w+4, ...  Within a tile a group of HD/8 lanes holds one
 * position (8 dims per lane): K and V of the tile are loaded together, scores
 * are q.k * (1/sqrt(hd)) (forward.h:84), then an online softmax keeps the
 * running (max, sum, weighted V).  The four waves merge through LDS and the
 * normalised head output (forward.h:95-97) goes to out[b, h*HD ..] (fp32), or
 * in fp16 to out16 when that is given (the operand of the Wo GEMM). */
/* Decode rows straight from a K-split QKV GEMM: part holds ns partials
 * [M, NQ + 2*NKV] (sstride floats apart); the row's q, k, v are their sums in
 * split order, q and k RoPE'd at pos[b] with the host tables (forward.h:55-70).
 * The first query head of each kv group appends k, v to the cache
 * (forward.h:118-128); every work-group takes the current position from its own
 * copy (rounded to the cache's element type), as one more term of the softmax
 * merge, so none waits for another's append. */
template <typename KT>
struct QkvPart {
    const float *part;
    size_t sstride;
    int ns, NQ, NKV;
    const float *rc, *rs;   /* RoPE cos / sin [max_seq][hd/2] */
    KT *kc, *vc;            /* the cache, written at the current position */
};

template <int HD, typename KT>
__device__ __forceinline__ void attn_head(
    const float *__restrict__ q, const KT *__restrict__ kc, const KT *__restrict__ vc,
    const int *__restrict__ pos, const int *__restrict__ slot, int H, int Hkv, int max_seq,
    float *oh, int h, int b, const QkvPart<KT> *qp = nullptr, const QkvTagged *qt = nullptr)
{
    /* positions per tile: 32 (measured against 64: the four waves share short
     * contexts more evenly).  Two tiles fit the registers except at hd 128 with
     * an fp32 cache, so the next tile's K/V loads are in flight while the
     * current one computes (DB) */
    constexpr int TILE = 32;
    constexpr bool DB = !(HD == 128 && sizeof(KT) == 4);
    constexpr int G = HD / 8;        /* lanes per position            */
    constexpr int PP = 64 / G;       /* positions per pass            */
    constexpr int NP = TILE / PP;    /* passes per tile               */
    typedef typename KVRaw<KT>::T Raw;
    __shared__ float sm[NWAVE], sl[NWAVE];
    __shared__ __attribute__((aligned(16))) float so[NWAVE][HD];
    __shared__ __attribute__((aligned(16))) float sqkv[3][HD];   /* q, k, v of a split QKV */
    __shared__ float scur;                                        /* its current score */
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int ctx = pos[b] + 1;
    /* positions read from the cache: all of them, or with qp / qt all but the
     * current one, which is added from LDS at the end */
    const bool cur = qp || qt;
    const int vis = cur ? ctx - 1 : ctx;
    const int ntiles = (vis + TILE - 1) / TILE;
    const int dq = lane % G, pp = lane / G;
    const int cs = slot ? slot[b] : b;
    const size_t base = ((size_t)cs * Hkv + small_div(h, small_div(H, Hkv))) * max_seq * HD + dq * 8;
    const KT *K = kc + base;
    const KT *V = vc + base;
    /* scores in log2 units: exp(x) = exp2(x * log2 e), the hardware exp2 */
    const float scale = 1.4426950408889634f / sqrtf((float)HD);
    float qf[8];
    if (!cur) {
        const float *qr = q + (size_t)b * H * HD + h * HD + dq * 8;
        const float4 a = *(const float4 *)qr, c = *(const float4 *)(qr + 4);
        qf[0] = a.x; qf[1] = a.y; qf[2] = a.z; qf[3] = a.w;
        qf[4] = c.x; qf[5] = c.y; qf[6] = c.z; qf[7] = c.w;
    }
    float m = -INFINITY, l = 0.f, o[8];
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = 0.f;
    /* hd 64: the wave's first tile is loaded before pos[b] has arrived
     * (positions clamped into the cache, masked below; the cache is zeroed at
     * allocation, so every value read is finite), so the K/V fetch does not
     * wait for it.  (Loading the second tile that early as well was 3% slower
     * for 64 rows at 192-255 positions: the waves with one tile then read a
     * whole tile of unused cache rows.) */
    constexpr bool EARLY = HD == 64;
    Raw kr[NP], vr[NP];
    Raw kr1[NP], vr1[NP];            /* the wave's next tile (DB) */
    /* split partials (qp): thread t < 3*HD/4 owns 4 columns of q, k or v; at
     * hd 64 (whose first tile is loaded early) the first PE partials and the
     * RoPE factors are loaded before the tile's loads, so that the sum that
     * every score waits for does not queue behind the tile (C2 1.2% faster;
     * at hd 128 the registers cost more than the order gains) */
    constexpr int PE = EARLY ? 8 : 0;
    float4 pt[PE > 0 ? PE : 1];
    float2 pc = make_float2(1.f, 1.f), psn = make_float2(0.f, 0.f);
    const bool pown = qp && (int)threadIdx.x < 3 * HD / 4;
    const int pvec = threadIdx.x / (HD / 4), pe4 = (threadIdx.x % (HD / 4)) * 4;
    const int pg = small_div(h, small_div(H, Hkv));
    const float *psrc = nullptr;
    if (pown) {
        const int col = pvec == 0 ? h * HD : (pvec == 1 ? qp->NQ + pg * HD : qp->NQ + qp->NKV + pg * HD);
        psrc = qp->part + (size_t)b * (qp->NQ + 2 * qp->NKV) + col + pe4;
    }
    if (PE > 0 && pown) {
#pragma unroll
        for (int u = 0; u < PE; u++)
            pt[u] = u < qp->ns ? *(const float4 *)(psrc + (size_t)u * qp->sstride)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
        const int ti = (ctx - 1) * (HD / 2) + (pe4 >> 1);
        pc = *(const float2 *)(qp->rc + ti);
        psn = *(const float2 *)(qp->rs + ti);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (EARLY || qt) {   /* also at hd 128 when q waits for the QKV work-groups */
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int p = min(wv * TILE + pp + PP * i, max_seq - 1);
            kv_raw_load(K + (size_t)p * HD, kr[i]);
            kv_raw_load(V + (size_t)p * HD, vr[i]);
        }
        if constexpr (DB) {
            /* waiting for the QKV work-groups of the same launch: the second
             * tile too, so that no tile load follows the wait (a wave with one
             * tile reads one tile of unused rows) */
            if (qt) {
#pragma unroll
                for (int i = 0; i < NP; i++) {
                    const int p = min((wv + NWAVE) * TILE + pp + PP * i, max_seq - 1);
                    kv_raw_load(K + (size_t)p * HD, kr1[i]);
                    kv_raw_load(V + (size_t)p * HD, vr1[i]);
                }
            }
        }
        /* keeps the tile's loads ahead of the partials' (the scheduler would
         * otherwise issue them after the partials' sum, a second round trip) */
        __builtin_amdgcn_sched_barrier(0);
    }
    if (qp) {
        /* q, k, v from the split partials: the owning threads sum their 4
         * columns over the partials (in split order; past the first PE, groups
         * of four loaded at once), rotate q and k (forward.h:62-68), append k, v
         * to the cache from the first query head of the kv group
         * (forward.h:118-128) and leave them in LDS */
        if (pown) {
            const int vec = pvec, e4 = pe4, g = pg;
            const float *src = psrc;
            const int ns = qp->ns;
            float2 c = pc, sn = psn;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (PE > 0) {
#pragma unroll
                for (int u = 0; u < PE; u++) {
                    acc.x += pt[u].x; acc.y += pt[u].y; acc.z += pt[u].z; acc.w += pt[u].w;
                }
            } else {
                const int ti = (ctx - 1) * (HD / 2) + (e4 >> 1);
                c = *(const float2 *)(qp->rc + ti);
                sn = *(const float2 *)(qp->rs + ti);
            }
            for (int s0 = PE; s0 < ns; s0 += 4) {
                float4 tt[4];
#pragma unroll
                for (int u = 0; u < 4; u++) tt[u] = *(const float4 *)(src + (size_t)min(s0 + u, ns - 1) * qp->sstride);
#pragma unroll
                for (int u = 0; u < 4; u++) {   /* past the last partial: add zero */
                    const float4 z = s0 + u < ns ? tt[u] : make_float4(0.f, 0.f, 0.f, 0.f);
                    acc.x += z.x; acc.y += z.y; acc.z += z.z; acc.w += z.w;
                }
            }
            if (vec < 2) {
                const float a0 = acc.x, b0 = acc.y, a1 = acc.z, b1 = acc.w;
                acc.x = fmaf(a0, c.x, -(b0 * sn.x));
                acc.y = fmaf(a0, sn.x, b0 * c.x);
                acc.z = fmaf(a1, c.y, -(b1 * sn.y));
                acc.w = fmaf(a1, sn.y, b1 * c.y);
            }
            *(float4 *)(&sqkv[vec][e4]) = acc;
            if (vec > 0 && h % (H / Hkv) == 0) {
                KT *dst = (vec == 1 ? qp->kc : qp->vc) + ((size_t)cs * Hkv + g) * max_seq * HD +
                          (size_t)(ctx - 1) * HD + e4;
                dst[0] = kv_pack<KT>(acc.x);
                dst[1] = kv_pack<KT>(acc.y);
                dst[2] = kv_pack<KT>(acc.z);
                dst[3] = kv_pack<KT>(acc.w);
            }
        }
    }
    /* Binary16 cache in the fused launch: the two tiles loaded above are
     * converted to fp32 here, before the wait for q, k, v, so that the
     * conversions (16 per position per lane) are off the path from the
     * words' arrival to the head output; the empty asm keeps the compiler from
     * sinking them past the wait.  (The fp32 cache needs no conversion; with
     * two whole-layer work-groups per CU the registers are there at head dim
     * 64: 164 VGPRs.  At 128 two converted tiles take 256 registers.) */
    constexpr bool PRECVT = DB && sizeof(KT) == 2 && HD == 64;
    KV8f ck[PRECVT ? 2 : 1][NP], cv[PRECVT ? 2 : 1][NP];
    if constexpr (PRECVT) {
        if (qt) {
#pragma unroll
            for (int i = 0; i < NP; i++) {
                float f[8];
                kv_raw_unpack(kr[i], f);
                ck[0][i] = KV8f{make_float4(f[0], f[1], f[2], f[3]), make_float4(f[4], f[5], f[6], f[7])};
                kv_raw_unpack(vr[i], f);
                cv[0][i] = KV8f{make_float4(f[0], f[1], f[2], f[3]), make_float4(f[4], f[5], f[6], f[7])};
                kv_raw_unpack(kr1[i], f);
                ck[1][i] = KV8f{make_float4(f[0], f[1], f[2], f[3]), make_float4(f[4], f[5], f[6], f[7])};
                kv_raw_unpack(vr1[i], f);
                cv[1][i] = KV8f{make_float4(f[0], f[1], f[2], f[3]), make_float4(f[4], f[5], f[6], f[7])};
            }
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int i = 0; i < NP; i++) {
                    pin4(ck[u][i].a); pin4(ck[u][i].b);
                    pin4(cv[u][i].a); pin4(cv[u][i].b);
                }
        }
    }
    if (qt) {
        /* q, k, v of the current position from the tagged hand-off words the
         * QKV work-groups of this launch store (k, v as the cache holds
         * them), after the first K/V tile's loads are in flight: each thread
         * polls its words until they carry this launch's tag (bounded: a wait
         * that gives up sets qt->err, and the kernel still ends) */
        const unsigned tag = qkv_tag(*qt);
        const int g = small_div(h, small_div(H, Hkv));
        constexpr int NT = (3 * HD + WG - 1) / WG;
        const unsigned long long *wp[NT];
        unsigned long long v[NT];
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int t = threadIdx.x + j * WG, vec = t / HD, e = t % HD;
            wp[j] = vec == 0 ? qt->tq + (size_t)b * H * HD + h * HD + e
                             : (vec == 1 ? qt->tk : qt->tv) + (size_t)b * Hkv * HD + g * HD + e;
            v[j] = t < 3 * HD ? tag_peek(wp[j]) : 0ull;
        }
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int t = threadIdx.x + j * WG;
            if (t < 3 * HD) sqkv[t / HD][t % HD] = tag_take(v[j], wp[j], tag, qt->err);
        }
    }
    if (cur) {
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; j++) qf[j] = sqkv[0][dq * 8 + j];
        /* the current position's score, its k rounded as the cache would, by
         * the last wave (tiles go to the waves in turn, so it has the fewest);
         * it is read only at the merge, after the barrier */
        if (wv == NWAVE - 1) {
            float d = 0.f;
#pragma unroll
            for (int j = lane; j < HD; j += 64) d = fmaf(sqkv[0][j], kv_round<KT>(sqkv[1][j]), d);
            d = wave_sum(d);
            if (lane == 0) scur = d * scale;
        }
    }
    /* Sum over each aligned group of G lanes, in every lane of the group: the
     * xor-1/2/4(/8) butterfly as DPP moves (after each step the value is
     * uniform over quads, then octets, so the half-row and row mirrors pair the
     * lanes exactly as xor 4 and xor 8 would).  The same pairing as shuffles,
     * so the same sums, without LDS permutes. */
    auto gsum = [](float d) {
        d += dpp_f<DPP_QUAD_XOR1>(d);
        d += dpp_f<DPP_QUAD_XOR2>(d);
        d += dpp_f<DPP_ROW_HALF_MIRROR>(d);
        if constexpr (G == 16) d += dpp_f<DPP_ROW_MIRROR>(d);
        return d;
    };
    /* Combine the lanes with the same l % G (the same dims) across the 64/G
     * groups: xor 8 as a DPP rotate of each 16-lane row by 8 (G = 8), then xor
     * 16 and xor 32 as permlane swaps. */
    auto across = [](float v, auto op) {
        if constexpr (G == 8) v = op(v, dpp_f<DPP_ROW_ROR8>(v));
        v = op(v, xor16_f(v));
        return op(v, xor32_f(v));
    };
    auto fadd = [](float a, float b) { return a + b; };
    /* online softmax update with tile t (forward.h:82-97), held in kr/vr */
    auto consume = [&](int t, const auto (&tk)[NP], const auto (&tv)[NP]) {
        float s[NP];
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < NP; i++) {
            float kf[8];
            kv_raw_unpack(tk[i], kf);
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < 8; j++) d = fmaf(qf[j], kf[j], d);
            d = gsum(d);
            const int p = t * TILE + pp + PP * i;
            s[i] = p < vis ? d * scale : -INFINITY;
            tmax = fmaxf(tmax, s[i]);
        }
        tmax = across(tmax, [](float a, float b) { return fmaxf(a, b); });
        const float mn = fmaxf(m, tmax);
        const float corr = __builtin_amdgcn_exp2f(m - mn);   /* 0 on the first tile */
        l *= corr;
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] *= corr;
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const float e = __builtin_amdgcn_exp2f(s[i] - mn);   /* 0 for masked positions */
            l += e;
            float vf[8];
            kv_raw_unpack(tv[i], vf);
#pragma unroll
            for (int j = 0; j < 8; j++) o[j] = fmaf(e, vf[j], o[j]);
        }
        m = mn;
    };
    {
        /* later tiles: positions past the visible ones load the last visible
         * position again (masked in consume), so every load is unconditional
         * and the wait for a tile never covers the next tile's loads */
        const int plast = max(vis - 1, 0);
        auto fetch = [&](int t, Raw (&tk)[NP], Raw (&tv)[NP]) {
#pragma unroll
            for (int i = 0; i < NP; i++) {
                const int p = min(t * TILE + pp + PP * i, plast);
                kv_raw_load(K + (size_t)p * HD, tk[i]);
                kv_raw_load(V + (size_t)p * HD, tv[i]);
            }
        };
        if (!EARLY && !qt) fetch(wv, kr, vr);
        if (PRECVT && qt) {
            /* the converted first two tiles, then any later ones one at a
             * time (contexts past 8 tiles) */
            if (wv < ntiles) {                                   /* wave-uniform */
                consume(wv, ck[0], cv[0]);
                if (wv + NWAVE < ntiles) consume(wv + NWAVE, ck[PRECVT ? 1 : 0], cv[PRECVT ? 1 : 0]);
                for (int t = wv + 2 * NWAVE; t < ntiles; t += NWAVE) {
                    fetch(t, kr, vr);
                    consume(t, kr, vr);
                }
            }
        } else if constexpr (DB) {
            /* kr holds the wave's first tile and kr1 its second (both in
             * flight); the first tile is consumed outside the loop, which keeps
             * the loop's registers at two tiles (143 -> 109 VGPRs at hd 64).
             * The scheduling barriers keep each fetch ahead of the compute it
             * overlaps (the compiler would sink the loads to their first use). */
            if (!qt) fetch(wv + NWAVE, kr1, vr1);
            __builtin_amdgcn_sched_barrier(0);
            if (wv < ntiles) {                                   /* wave-uniform */
                consume(wv, kr, vr);
                for (int t = wv + NWAVE; t < ntiles; t += 2 * NWAVE) {   /* kr1: tile t */
                    fetch(t + NWAVE, kr, vr);
                    __builtin_amdgcn_sched_barrier(0);
                    consume(t, kr1, vr1);
                    if (t + NWAVE >= ntiles) break;
                    fetch(t + 2 * NWAVE, kr1, vr1);
                    __builtin_amdgcn_sched_barrier(0);
                    consume(t + NWAVE, kr, vr);
                }
            }
        } else {
            for (int t = wv; t < ntiles; t += NWAVE) {      /* wave-uniform */
                if (t != wv) fetch(t, kr, vr);
                consume(t, kr, vr);
            }
        }
    }
    l = across(l, fadd);
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = across(o[j], fadd);
    if (lane < G) {
#pragma unroll
        for (int j = 0; j < 8; j++) so[wv][dq * 8 + j] = o[j];
    }
    if (lane == 0) { sm[wv] = m; sl[wv] = l; }
    __syncthreads();
    if (threadIdx.x < HD) {
        const int d = threadIdx.x;
        float M = cur ? scur : -INFINITY;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) M = fmaxf(M, sm[w]);
        float L = 0.f, acc = 0.f;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) {
            const float f = sm[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sm[w] - M);
            L = fmaf(sl[w], f, L);
            acc = fmaf(so[w][d], f, acc);
        }
        if (cur) {   /* the current position, after the cached ones */
            const float f = __builtin_amdgcn_exp2f(scur - M);
            L += f;
            acc = fmaf(kv_round<KT>(sqkv[2][d]), f, acc);
        }
        oh[d] = acc / L;
    }
    __syncthreads();
}

/* Work-group (h, b): the head output to out[b, h*HD ..] (fp32), or in fp16 to
 * out16 when that is given (the operand of the Wo GEMM). */
template <int HD, typename KT>
__global__ void __launch_bounds__(WG) k_attn_decode(
    const float *__restrict__ q, const KT *__restrict__ kc, const KT *__restrict__ vc,
    const int *__restrict__ pos, const int *__restrict__ slot, int H, int Hkv, int max_seq,
    float *__restrict__ out, u16 *__restrict__ out16)
{
    __shared__ float oh[HD];
    attn_head<HD, KT>(q, kc, vc, pos, slot, H, Hkv, max_seq, oh, blockIdx.x, blockIdx.y);
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    if (d < HD) {
        if (out16) out16[(size_t)b * H * HD + h * HD + d] = f2h(oh[d]);
        else out[(size_t)b * H * HD + h * HD + d] = oh[d];
    }
}

/* Work-group (h, b) for decode rows of the MFMA path whose QKV GEMM ran
 * K-split: q, k, v come from the partials (QkvPart), the head output goes to
 * out16[b, h*HD ..] in fp16 (the Wo GEMM operand). */
template <int HD, typename KT>
__global__ void __launch_bounds__(WG) k_attn_decode_part(
    const float *__restrict__ part, size_t sstride, int ns, int NQ, int NKV,
    const int *__restrict__ pos, const int *__restrict__ slot, int H, int Hkv, int max_seq,
    const float *__restrict__ rc, const float *__restrict__ rs, KT *__restrict__ kc,
    KT *__restrict__ vc, u16 *__restrict__ out16)
{
    __shared__ float oh[HD];
    const QkvPart<KT> qp = {part, sstride, ns, NQ, NKV, rc, rs, kc, vc};
    attn_head<HD, KT>(nullptr, kc, vc, pos, slot, H, Hkv, max_seq, oh, blockIdx.x, blockIdx.y, &qp);
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    if (d < HD) out16[(size_t)b * H * HD + h * HD + d] = f2h(oh[d]);
}

/* ---- QKV + attention in one launch (batch 1-4 decode) ----------------------- */

/* Wo role of k_qkv_attn, work-group a of the role, a row pair per wave:
 * x'[b, r..r+1] = (layer 0: the embedding row, else x) + Wo[r..r+1, :] . attn[b],
 * the head outputs taken from copy a % LM_TA_COPIES of their tagged words.
 * Without the FFN in the launch (F == 0) x' goes to x; with it, to every copy
 * of the tagged words tx (x is then written by the W2 role). */
template <int D, int NB, int F>
__device__ __forceinline__ void wo_role(float *__restrict__ x, const u16 *__restrict__ emb,
                                        const int *__restrict__ tok, const u16 *__restrict__ Wo,
                                        int B, int NQ, const QkvTagged &tg, int a, float *xs)
{
    const int p = a * NWAVE + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int wpairs = D / 2;
    const int r = 2 * min(p, wpairs - 1);
    uint4 wv[D / 256];
    hw_load<D>(Wo + (size_t)(r + half) * D, hl, wv);
    float2 xo[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (b >= B) {
            xo[b] = make_float2(0.f, 0.f);
        } else if (emb) {
            const u16 *er = emb + (size_t)tok[b] * D + r;
            xo[b] = make_float2(h2f(er[0]), h2f(er[1]));
        } else {
            xo[b] = *(const float2 *)(x + (size_t)b * D + r);
        }
    }
    const unsigned tag = qkv_tag(tg);
    const unsigned long long *tac = tg.ta + (size_t)(a % LM_TA_COPIES) * LM_TAG_B * NQ;
    tag_doorbell(tac, B * D, a / LM_TA_COPIES, tag, tg.err);
    tag_wait_span(tac, B * D, tag, tg.err, xs);
    __syncthreads();
    if (p >= wpairs) return;
    float acc[NB], r0[NB], r1[NB];
    hw_dot<D, NB>(wv, xs, hl, acc);
    pair_reduce<NB>(acc, r0, r1);
    if constexpr (F == 0) {
        if (lane == 0) {
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if (b >= B) break;
                *(float2 *)(x + (size_t)b * D + r) = make_float2(xo[b].x + r0[b], xo[b].y + r1[b]);
            }
        }
    } else if (lane < LM_TX_COPIES) {
        unsigned long long *dst = tg.tx + (size_t)lane * LM_TAG_B * D + r;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            tag_store(dst + (size_t)b * D, xo[b].x + r0[b], tag);
            tag_store(dst + (size_t)b * D + 1, xo[b].y + r1[b], tag);
        }
    }
}

/* W1/W3 role of k_qkv_attn (the FFN in the launch), work-group a of the role,
 * one hidden unit i per wave as in k_ffn13: x' from copy a % LM_TX_COPIES of
 * its tagged words, normalised as norm_to_lds_unscaled does (the row scale
 * applied to the dot products), then
 * g[b, i] = silu(W1[i] . xn) * (W3[i] . xn) stored to every copy of the tagged
 * words tgt.  (One unit per wave measured faster than two or four: more
 * work-groups load the weights.) */
template <int D, int NB, int F>
__device__ __forceinline__ void w13_role(const float *__restrict__ rms_w, const u16 *__restrict__ W13,
                                         int B, const QkvTagged &tg, int a, float *xs)
{
    constexpr int PER = D / WG;
    __shared__ float red[NB][NWAVE];
    const int tid = threadIdx.x, wv_ = tid >> 6;
    const int i0 = a * NWAVE + wv_;
    const int i = min(i0, F - 1);
    const int lane = tid & 63, half = lane >> 5, hl = lane & 31;
    constexpr int GB = LMK_GATE_BLOCK;
    const size_t row = (size_t)(i / GB) * (2 * GB) + half * GB + (i % GB);
    uint4 wv[D / 256];
    hw_load<D>(W13 + row * D, hl, wv);
    float w[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) w[j] = rms_w[tid + j * WG];
    const unsigned tag = qkv_tag(tg);
    /* each thread's words are the elements tid + j*WG of each row, which are
     * also the ones it normalises: no barrier between the two */
    const unsigned long long *txc = tg.tx + (size_t)(a % LM_TX_COPIES) * LM_TAG_B * D;
    tag_doorbell(txc, B * D, a / LM_TX_COPIES, tag, tg.err);
    tag_wait_span(txc, B * D, tag, tg.err, xs);
    /* the row scale is applied to the dot products (it distributes over
     * them), so xs takes x' * gain at once: one barrier */
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            float *e = xs + b * D + tid + j * WG;
            const float v = b < B ? *e : 0.f;
            ss = fmaf(v, v, ss);
            *e = v * w[j];
        }
        ss = wave_sum(ss);
        if (lane == 0) red[b][wv_] = ss;
    }
    __syncthreads();
    if (i0 >= F) return;
    float scale[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float tot = 0.f;
#pragma unroll
        for (int k = 0; k < NWAVE; k++) tot += red[b][k];
        scale[b] = 1.0f / sqrtf(tot / D + 1e-5f);
    }
    float acc[NB], h1[NB], h3[NB];
    hw_dot<D, NB>(wv, xs, hl, acc);
    pair_reduce<NB>(acc, h1, h3);
    if (lane < LM_TG_COPIES) {
        unsigned long long *dst = tg.tgt + (size_t)lane * LM_TAG_B * F + i;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            h1[b] *= scale[b];
            h3[b] *= scale[b];
            const float silu = h1[b] / (1.0f + expf(-h1[b]));  /* forward.h:101 */
            tag_store(dst + (size_t)b * F, silu * h3[b], tag);  /* forward.h:151 */
        }
    }
}

/* W2 role of k_qkv_attn (the FFN in the launch), work-group a of the role, a
 * row pair per wave as in k_w2_residual: x[b, r..r+1] = x'[b, r..r+1] +
 * W2[r..r+1, :] . g[b], g from copy a % LM_TG_COPIES of its tagged words. */
template <int D, int NB, int F>
__device__ __forceinline__ void w2_role(float *__restrict__ x, const u16 *__restrict__ W2, int B,
                                        const QkvTagged &tg, int a, float *xs)
{
    const int p = a * NWAVE + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int wpairs = D / 2;
    const int r = 2 * min(p, wpairs - 1);
    uint4 wv[F / 256];
    hw_load<F>(W2 + (size_t)(r + half) * F, hl, wv);
    const unsigned tag = qkv_tag(tg);
    const unsigned long long *txc = tg.tx + (size_t)(a % LM_TX_COPIES) * LM_TAG_B * D + r;
    const unsigned long long *tgc = tg.tgt + (size_t)(a % LM_TG_COPIES) * LM_TAG_B * F;
    tag_doorbell(tgc, B * F, a / LM_TG_COPIES, tag, tg.err);
    /* x' of this row pair (written before any gate word) with the gate */
    unsigned long long v0[NB], v1[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        v0[b] = b < B ? tag_peek(txc + (size_t)b * D) : 0ull;
        v1[b] = b < B ? tag_peek(txc + (size_t)b * D + 1) : 0ull;
    }
    tag_wait_span(tgc, B * F, tag, tg.err, xs);
    for (int k = B * F + threadIdx.x; k < NB * F; k += WG) xs[k] = 0.f;
    float2 xo[NB];
#pragma unroll
    for (int b = 0; b < NB; b++)
        xo[b] = b < B ? make_float2(tag_take(v0[b], txc + (size_t)b * D, tag, tg.err),
                                    tag_take(v1[b], txc + (size_t)b * D + 1, tag, tg.err))
                      : make_float2(0.f, 0.f);
    __syncthreads();
    if (p >= wpairs) return;
    float acc[NB], r0[NB], r1[NB];
    hw_dot<F, NB>(wv, xs, hl, acc);
    pair_reduce<NB>(acc, r0, r1);
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            *(float2 *)(x + (size_t)b * D + r) = make_float2(xo[b].x + r0[b], xo[b].y + r1[b]);
        }
    }
}

/* The FFN operands of a layer run inside k_qkv_attn. */
struct FfnArgs {
    const float *rms_w;   /* rms_ffn gains [D] */
    const u16 *w13;       /* W1/W3 rows interleaved in LMK_GATE_BLOCK blocks [2F, D] */
    const u16 *w2;        /* [D, F] */
};

/* One launch of the batch 1-4 decode chain per layer; its work-groups take
 * roles in this order, each role waiting only on roles before it:
 *  - 0 .. nprod-1: the QKV GEMV of k_qkv_rope, also storing q, k, v as tagged
 *    hand-off words;
 *  - then one per (row b, head h): the attention of head h, row b, which loads
 *    its first cached K/V tile, waits for the current position's q, k, v words
 *    and hands the head output on (fp32 to out[b, h*HD ..] without WO, else
 *    as tagged words, in LM_TA_COPIES copies);
 *  - with WO, D/(2*NWAVE) work-groups of the Wo GEMV + residual (wo_role);
 *  - with F > 0 (the layer's FFN in the launch too), F/NWAVE work-groups of the
 *    W1/W3 gate (w13_role), then D/(2*NWAVE) of the W2 GEMV + residual
 *    (w2_role).
 * A role's work-groups come after every work-group it waits for in dispatch
 * order, so the waits end however many work-groups the device holds at once.
 * In layer 0 (emb) the residual starts from the embedding row and the QKV
 * work-groups leave x alone, so each element of x has one writer in the
 * launch; the QKV and Wo work-groups read x before they store any word, and x
 * is written only after every word of every head, so no read of x in the
 * launch sees the value written in it. */
template <int D, int NB, typename KT, int HD, bool WO, int F>
__global__ void __launch_bounds__(WG) k_qkv_attn(
    float *__restrict__ x, const u16 *__restrict__ emb, const int *__restrict__ tok,
    const float *__restrict__ rms_w, const u16 *__restrict__ W, int NQ, int NKV,
    const float *__restrict__ rc, const float *__restrict__ rs, const int *__restrict__ pos,
    int B, KT *__restrict__ kc, KT *__restrict__ vc, int max_seq, int npairs, int nprod, int H,
    QkvTagged tg, float *__restrict__ out, const u16 *__restrict__ Wo, FfnArgs ffn)
{
    static_assert(F == 0 || WO, "the FFN roles take x' from the Wo role");
    static_assert(LM_TA_COPIES <= 64 && LM_TX_COPIES <= 64 && LM_TG_COPIES <= 64, "a wave's lanes store the copies");
    if ((int)blockIdx.x < nprod) {
        qkv_rows<D, NB, KT>(x, emb, tok, rms_w, W, NQ, NKV, HD, rc, rs, pos, B, nullptr, kc, vc,
                            max_seq, npairs, &tg, !WO);
        return;
    }
    int a = blockIdx.x - nprod;
    if (!WO || a < H * B) {
        __shared__ float oh[HD];
        const int h = a % H, b = a / H;
        attn_head<HD, KT>(nullptr, kc, vc, pos, nullptr, H, NKV / HD, max_seq, oh, h, b, nullptr, &tg);
        if constexpr (WO) {
            /* every copy of the head output, the work-group's threads taking
             * (element, copy) pairs */
            const unsigned tag = qkv_tag(tg);
            for (int t = threadIdx.x; t < HD * LM_TA_COPIES; t += WG) {
                const int e = t % HD, c = t / HD;
                tag_store(tg.ta + (size_t)c * LM_TAG_B * NQ + (size_t)b * NQ + h * HD + e, oh[e], tag);
            }
        } else if ((int)threadIdx.x < HD) {
            out[(size_t)b * H * HD + h * HD + threadIdx.x] = oh[threadIdx.x];
        }
        return;
    }
    if constexpr (WO) {
        /* the LDS rows of whichever of the Wo, W1/W3 and W2 roles this
         * work-group takes */
        constexpr int ROW = F > D ? F : D;
        __shared__ __attribute__((aligned(16))) float xs[NB * ROW];
        constexpr int NWO = (D / 2 + NWAVE - 1) / NWAVE;
        a -= H * B;
        if (F == 0 || a < NWO) {
            wo_role<D, NB, F>(x, emb, tok, Wo, B, NQ, tg, a, xs);
            return;
        }
        if constexpr (F > 0) {
            constexpr int N13 = (F + NWAVE - 1) / NWAVE;
            a -= NWO;
            if (a < N13) w13_role<D, NB, F>(ffn.rms_w, ffn.w13, B, tg, a, xs);
            else w2_role<D, NB, F>(x, ffn.w2, B, tg, a - N13, xs);
        }
    }
}

/* ---- Wo + residual ---------------------------------------------------------- */

template <int D, int NB>
__global__ void __launch_bounds__(WG) k_wo_residual(
    const float *__restrict__ attn, const u16 *__restrict__ W, int B, float *__restrict__ x,
    int npairs)
{
    __shared__ __attribute__((aligned(16))) float xs[NB * D];
    const int p = blockIdx.x * NWAVE + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int r = 2 * min(p, npairs - 1);
    uint4 wv[D / 256];
    hw_load<D>(W + (size_t)(r + half) * D, hl, wv);
    RowsIn<D, NB> in;
    rows_load<D, NB>(attn, B, in);
    float2 xo[NB];
#pragma unroll
    for (int b = 0; b < NB; b++)
        xo[b] = b < B ? *(const float2 *)(x + (size_t)b * D + r) : make_float2(0.f, 0.f);
    rows_to_lds<D, NB>(in, xs);
    if (p >= npairs) return;
    float acc[NB], r0[NB], r1[NB];
    hw_dot<D, NB>(wv, xs, hl, acc);
    pair_reduce<NB>(acc, r0, r1);
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            *(float2 *)(x + (size_t)b * D + r) = make_float2(xo[b].x + r0[b], xo[b].y + r1[b]);
        }
    }
}

/* ---- W1/W3 + SiLU gate ------------------------------------------------------ */

template <int D, int NB>
__global__ void __launch_bounds__(WG) k_ffn13(
    float *__restrict__ x, const float *__restrict__ rms_w, const u16 *__restrict__ W13,
    int F, int B, float *__restrict__ g)
{
    __shared__ __attribute__((aligned(16))) float xs[NB * D];
    const int i0 = blockIdx.x * NWAVE + (threadIdx.x >> 6);
    const int i = min(i0, F - 1);
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    constexpr int GB = LMK_GATE_BLOCK;
    const size_t row = (size_t)(i / GB) * (2 * GB) + half * GB + (i % GB);
    uint4 wv[D / 256];
    hw_load<D>(W13 + row * D, hl, wv);
    NormIn<D, NB> in;
    norm_load<D, NB>(x, nullptr, nullptr, rms_w, B, in);
    float scale[NB];
    norm_to_lds_unscaled<D, NB>(in, B, x, false, xs, scale);
    if (i0 >= F) return;
    float acc[NB], h1[NB], h3[NB];
    hw_dot<D, NB>(wv, xs, hl, acc);
    pair_reduce<NB>(acc, h1, h3);
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            h1[b] *= scale[b];
            h3[b] *= scale[b];
            const float silu = h1[b] / (1.0f + expf(-h1[b]));  /* forward.h:101 */
            g[(size_t)b * F + i] = silu * h3[b];                /* forward.h:151 */
        }
    }
}

/* ---- W2 + residual ------------------------------------------------------------ */

template <int F, int NB>
__global__ void __launch_bounds__(WG) k_w2_residual(
    const float *__restrict__ g, const u16 *__restrict__ W, int D, int B,
    float *__restrict__ x, int npairs)
{
    __shared__ __attribute__((aligned(16))) float xs[NB * F];
    const int p = blockIdx.x * NWAVE + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int r = 2 * min(p, npairs - 1);
    uint4 wv[F / 256];
    hw_load<F>(W + (size_t)(r + half) * F, hl, wv);
    RowsIn<F, NB> in;
    rows_load<F, NB>(g, B, in);
    float2 xo[NB];
#pragma unroll
    for (int b = 0; b < NB; b++)
        xo[b] = b < B ? *(const float2 *)(x + (size_t)b * D + r) : make_float2(0.f, 0.f);
    rows_to_lds<F, NB>(in, xs);
    if (p >= npairs) return;
    float acc[NB], r0[NB], r1[NB];
    hw_dot<F, NB>(wv, xs, hl, acc);
    pair_reduce<NB>(acc, r0, r1);
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            *(float2 *)(x + (size_t)b * D + r) = make_float2(xo[b].x + r0[b], xo[b].y + r1[b]);
        }
    }
}

/* ---- classifier + argmax ----------------------------------------------------- */

#ifndef CLS_PAIRS_PER_WAVE
#define CLS_PAIRS_PER_WAVE 4
#endif
#define CLS_ROWS_PER_WG (2 * CLS_PAIRS_PER_WAVE * NWAVE)

/* The argmax reduction inside the classifier launch (k_cls with fold.tw): the
 * classifier work-groups store the partial of row b, blk as two tagged words
 * (value bits; index), tw[b*nblk + blk] and tw[(LM_TAG_B + b)*nblk + blk],
 * tagged *epoch + 1; one more work-group, last in dispatch order, waits for
 * them and does k_argmax_final's work. */
struct ArgFold {
    unsigned long long *tw;     /* 2 * LM_TAG_B * nblk words, zero at allocation */
    unsigned *epoch;
    int *tok, *pos, *hist;
    int hist_stride;
    int *err;
};

/* The reducer of k_cls with fold: rows 0..B-1 over nblk partials (lowest index
 * on ties, the combine being commutative and associative, so any order gives
 * k_argmax_final's result). */
__device__ __forceinline__ void cls_argmax_fold(const ArgFold &f, int nblk, int B)
{
    __shared__ float sv[NWAVE];
    __shared__ int si[NWAVE];
    const unsigned tag = *f.epoch + 1u;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int b = 0; b < B; b++) {
        const unsigned long long *wv_ = f.tw + (size_t)b * nblk;
        const unsigned long long *wi_ = f.tw + (size_t)(LM_TAG_B + b) * nblk;
        if (threadIdx.x == 0) (void)tag_wait(wi_ + nblk - 1, tag, f.err);   /* doorbell */
        __syncthreads();
        float v = -INFINITY;
        int id = 0x7FFFFFFF;
        for (int i0 = threadIdx.x; i0 < nblk; i0 += 4 * WG) {
            unsigned long long pv[4], pi[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = i0 + j * WG;
                pv[j] = i < nblk ? tag_peek(wv_ + i) : 0ull;
                pi[j] = i < nblk ? tag_peek(wi_ + i) : 0ull;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = i0 + j * WG;
                if (i < nblk) {
                    const float pval = tag_take(pv[j], wv_ + i, tag, f.err);
                    const int pidx = __builtin_bit_cast(int, tag_take(pi[j], wi_ + i, tag, f.err));
                    argmax_combine(v, id, pval, pidx);
                }
            }
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(v, off, 64);
            const int oi = __shfl_xor(id, off, 64);
            argmax_combine(v, id, ov, oi);
        }
        if (lane == 0) { sv[wv] = v; si[wv] = id; }
        __syncthreads();
        if (threadIdx.x == 0) {
            v = sv[0];
            id = si[0];
            for (int w = 1; w < NWAVE; w++) argmax_combine(v, id, sv[w], si[w]);
            if (id == 0x7FFFFFFF) id = 0;
            f.tok[b] = id;
            if (f.hist) {
                const int p = f.pos[b];
                f.hist[(size_t)b * f.hist_stride + p + 1] = id;
                f.pos[b] = p + 1;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) *f.epoch += 1u;   /* the next step's hand-off tags */
}

template <int D, int NB>
__global__ void __launch_bounds__(WG) k_cls(
    const float *__restrict__ x, const float *__restrict__ rms_w, const u16 *__restrict__ W,
    int V, int B, float *__restrict__ logits, LMArgPart *__restrict__ part, ArgFold fold)
{
    if (fold.tw && blockIdx.x == gridDim.x - 1) {
        cls_argmax_fold(fold, gridDim.x - 1, B);
        return;
    }
    const unsigned ftag = fold.tw ? *fold.epoch + 1u : 0u;
    __shared__ __attribute__((aligned(16))) float xs[NB * D];
    __shared__ float bvs[NB][NWAVE];
    __shared__ int bis[NB][NWAVE];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, half = lane >> 5, hl = lane & 31;
    const int row0 = blockIdx.x * CLS_ROWS_PER_WG + wv * 2 * CLS_PAIRS_PER_WAVE;
    /* x and the gain first: the norm's sums and barrier then run while the
     * weight rows are still arriving */
    NormIn<D, NB> in;
    norm_load<D, NB>(x, nullptr, nullptr, rms_w, B, in);
    __builtin_amdgcn_sched_barrier(0);
    uint4 wr[CLS_PAIRS_PER_WAVE][D / 256];
#pragma unroll
    for (int pp = 0; pp < CLS_PAIRS_PER_WAVE; pp++) {
        const int rl = min(row0 + 2 * pp + half, V - 1);
        hw_load<D>(W + (size_t)rl * D, hl, wr[pp]);
    }
    __builtin_amdgcn_sched_barrier(0);
    float scale[NB];
    norm_to_lds_unscaled<D, NB>(in, B, nullptr, false, xs, scale);
    float bv[NB];
    int bi[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) { bv[b] = -INFINITY; bi[b] = 0x7FFFFFFF; }
#pragma unroll
    for (int pp = 0; pp < CLS_PAIRS_PER_WAVE; pp++) {
        const int r = row0 + 2 * pp;
        float acc[NB], r0[NB], r1[NB];
        hw_dot<D, NB>(wr[pp], xs, hl, acc);
        pair_reduce<NB>(acc, r0, r1);
#pragma unroll
        for (int b = 0; b < NB; b++) {
            r0[b] *= scale[b];
            r1[b] *= scale[b];
        }
        if (r < V) {
            const bool has1 = r + 1 < V;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                argmax_combine(bv[b], bi[b], r0[b], r);
                if (has1) argmax_combine(bv[b], bi[b], r1[b], r + 1);
            }
            if (logits && lane == 0) {
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    if (b >= B) break;
                    if (has1)
                        *(float2 *)(logits + (size_t)b * V + r) = make_float2(r0[b], r1[b]);
                    else
                        logits[(size_t)b * V + r] = r0[b];
                }
            }
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) { bvs[b][wv] = bv[b]; bis[b][wv] = bi[b]; }
    }
    __syncthreads();
    if (threadIdx.x < NB && (int)threadIdx.x < B) {
        const int b = threadIdx.x;
        float v = bvs[b][0];
        int id = bis[b][0];
        for (int w = 1; w < NWAVE; w++) argmax_combine(v, id, bvs[b][w], bis[b][w]);
        if (fold.tw) {
            const int nblk = gridDim.x - 1;
            tag_store(fold.tw + (size_t)b * nblk + blockIdx.x, v, ftag);
            tag_store(fold.tw + (size_t)(LM_TAG_B + b) * nblk + blockIdx.x,
                      __builtin_bit_cast(float, id), ftag);
        } else {
            part[(size_t)b * gridDim.x + blockIdx.x] = LMArgPart{v, id};
        }
    }
}

/* Work-group b reduces the nblk argmax partials of row b: tok[b] = argmax
 * (lowest index on ties); with hist, also hist[b*stride + pos[b] + 1] = tok[b]
 * and pos[b] += 1 (device-resident greedy loop state). */
__global__ void __launch_bounds__(WG) k_argmax_final(
    const LMArgPart *__restrict__ part, int nblk, int *__restrict__ tok, int *__restrict__ pos,
    int *__restrict__ hist, int hist_stride, unsigned *__restrict__ epoch)
{
    __shared__ float sv[NWAVE];
    __shared__ int si[NWAVE];
    const int b = blockIdx.x;
    float v = -INFINITY;
    int id = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < nblk; i += WG) {
        const LMArgPart pt = part[(size_t)b * nblk + i];
        argmax_combine(v, id, pt.val, pt.idx);
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(id, off, 64);
        argmax_combine(v, id, ov, oi);
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (lane == 0) { sv[wv] = v; si[wv] = id; }
    __syncthreads();
    if (threadIdx.x == 0) {
        v = sv[0];
        id = si[0];
        for (int w = 1; w < NWAVE; w++) argmax_combine(v, id, sv[w], si[w]);
        if (id == 0x7FFFFFFF) id = 0;
        tok[b] = id;
        if (hist) {
            const int p = pos[b];
            hist[(size_t)b * hist_stride + p + 1] = id;
            pos[b] = p + 1;
        }
        if (epoch && b == 0) *epoch += 1u;   /* the next step's hand-off tags */
    }
}

/* ---- self-test of the DPP reductions ------------------------------------------ */

__global__ void k_selftest_reduce(const float *in, float *out)
{
    const int lane = threadIdx.x;
    const float v = in[lane];
    const float hs = half_wave_sum(v);
    const float h0 = readlane_f(hs, 31), h1 = readlane_f(hs, 63);
    const float ws = wave_sum(v);
    const float ss = wave_sum_shfl(v);
    if (lane == 0) { out[0] = h0; out[1] = h1; out[2] = ws; out[3] = ss; }
}

/* ============================== launchers =================================== */

#define DISPATCH_NB(B, ...)                                   \
    switch ((B) <= 1 ? 1 : (B) <= 2 ? 2 : 4) {                \
    case 1: { constexpr int NB_ = 1; __VA_ARGS__; } break;    \
    case 2: { constexpr int NB_ = 2; __VA_ARGS__; } break;    \
    default: { constexpr int NB_ = 4; __VA_ARGS__; } break;   \
    }

#define DISPATCH_K(K, ...)                                            \
    switch (K) {                                                      \
    case 256: { constexpr int K_ = 256; __VA_ARGS__; } break;         \
    case 512: { constexpr int K_ = 512; __VA_ARGS__; } break;         \
    case 768: { constexpr int K_ = 768; __VA_ARGS__; } break;         \
    case 1024: { constexpr int K_ = 1024; __VA_ARGS__; } break;       \
    case 2048: { constexpr int K_ = 2048; __VA_ARGS__; } break;       \
    case 5632: { constexpr int K_ = 5632; __VA_ARGS__; } break;       \
    default: return hipErrorInvalidValue;                             \
    }

/* Model widths (dim) the kernels are instantiated for; hidden widths add 5632. */
#define DISPATCH_D(K, ...)                                            \
    switch (K) {                                                      \
    case 256: { constexpr int K_ = 256; __VA_ARGS__; } break;         \
    case 512: { constexpr int K_ = 512; __VA_ARGS__; } break;         \
    case 768: { constexpr int K_ = 768; __VA_ARGS__; } break;         \
    case 1024: { constexpr int K_ = 1024; __VA_ARGS__; } break;       \
    case 2048: { constexpr int K_ = 2048; __VA_ARGS__; } break;       \
    default: return hipErrorInvalidValue;                             \
    }

/* LDS budget of the GEMV kernels: NB rows of K fp32 within the 160 KB a
 * gfx950 work-group may hold (the compiler checks each kernel's whole static
 * LDS against the same limit). */
#define GEMV_LDS_OK(K_, NB_) ((size_t)(K_) * (NB_) * 4 <= 163840)

extern "C" int lmk_qkv_rope(hipStream_t s, float *x, const uint16_t *emb, const int *tok,
                            const float *rms_w, const uint16_t *wqkv, int D, int NQ, int NKV,
                            int hd, const float *rope_cos, const float *rope_sin, const int *pos,
                            int B, float *q, void *kc, void *vc, int kv_f32, int max_seq)
{
    if (B < 1 || B > 4 || NQ != D || (hd & 1) || NKV % hd || (emb && !tok))
        return hipErrorInvalidValue;
    const int npairs = (NQ + 2 * NKV) / 2;
    dim3 grid((npairs + NWAVE - 1) / NWAVE);
    DISPATCH_D(D, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        if (kv_f32)
            DLAUNCH((k_qkv_rope<K_, NB_, float>), grid, dim3(WG), 0, s, x, emb, tok,
                               rms_w, wqkv, NQ, NKV, hd, rope_cos, rope_sin, pos, B, q,
                               (float *)kc, (float *)vc, max_seq, npairs);
        else
            DLAUNCH((k_qkv_rope<K_, NB_, u16>), grid, dim3(WG), 0, s, x, emb, tok,
                               rms_w, wqkv, NQ, NKV, hd, rope_cos, rope_sin, pos, B, q,
                               (u16 *)kc, (u16 *)vc, max_seq, npairs);
    }));
    return hipGetLastError();
}

/* (model width, hidden width) pairs the whole-layer launch is instantiated
 * for; K_ and F_ name them in the body. */
#define DISPATCH_DF(D, F, ...)                                                          \
    do {                                                                                \
        if ((D) == 256 && (F) == 512) { constexpr int K_ = 256, F_ = 512; __VA_ARGS__; }     \
        else if ((D) == 512 && (F) == 1024) { constexpr int K_ = 512, F_ = 1024; __VA_ARGS__; } \
        else if ((D) == 768 && (F) == 2048) { constexpr int K_ = 768, F_ = 2048; __VA_ARGS__; } \
        else if ((D) == 1024 && (F) == 1024) { constexpr int K_ = 1024, F_ = 1024; __VA_ARGS__; } \
        else if ((D) == 2048 && (F) == 5632) { constexpr int K_ = 2048, F_ = 5632; __VA_ARGS__; } \
        else return hipErrorInvalidValue;                                               \
    } while (0)

extern "C" int lmk_layer_fusable(int D, int F, int B)
{
    if (B < 1 || B > 4) return 0;
    DISPATCH_DF(D, F, DISPATCH_NB(B, {
        return GEMV_LDS_OK(K_, NB_) && GEMV_LDS_OK(F_, NB_);
    }));
    return 0;
}

/* Dynamic LDS for a launch of kernel KERN that leaves room for at most `cap`
 * of its work-groups on one CU (160 KiB of LDS per CU on gfx950): enough that
 * cap + 1 no longer fit, never so much that cap do not, and never past one
 * CU's LDS.  0 when cap < 1, when the static LDS already does it, or when the
 * attributes cannot be read.  Memoised per kernel instantiation (KERN is a
 * template argument, so each instantiation has its own memo) and cap. */
template <auto KERN>
static size_t lds_cap_pad(int cap)
{
    constexpr size_t PER_CU = 160 * 1024, GRAIN = 512;
    static std::atomic<long> memo[5] = {{-1}, {-1}, {-1}, {-1}, {-1}};
    if (cap < 1 || cap > 4) return 0;
    long v = memo[cap].load(std::memory_order_relaxed);
    if (v >= 0) return (size_t)v;
    hipFuncAttributes a;
    size_t pad = 0;
    if (hipFuncGetAttributes(&a, (const void *)KERN) == hipSuccess) {
        const size_t stat = a.sharedSizeBytes, need = PER_CU / (cap + 1) + 1;
        if (stat < need) {
            pad = (need - stat + GRAIN - 1) / GRAIN * GRAIN;
            if (stat + pad > PER_CU / cap || stat + pad > PER_CU) pad = 0;
        }
    }
    memo[cap].store((long)pad, std::memory_order_relaxed);
    return pad;
}

extern "C" int lmk_qkv_attn(hipStream_t s, float *x, const uint16_t *emb, const int *tok,
                            const float *rms_w, const uint16_t *wqkv, int D, int NQ, int NKV, int hd,
                            const float *rope_cos, const float *rope_sin, const int *pos, int B,
                            void *kc, void *vc, int kv_f32, int max_seq, int H,
                            unsigned long long *tagged, const unsigned *epoch, int layer,
                            int n_layers, int *err, float *out, const uint16_t *wo,
                            const float *rms_ffn, const uint16_t *w13, const uint16_t *w2, int F,
                            int wgs_per_cu)
{
    if (B < 1 || B > 4 || NQ != D || H < 1 || NQ != H * hd || NKV % hd || H % (NKV / hd) ||
        (emb && !tok) || !tagged || !epoch || !err || (!out && !wo) || (hd != 64 && hd != 128) ||
        (w13 && (!wo || !w2 || !rms_ffn || F < 1 || F % LMK_GATE_BLOCK || !lmk_layer_fusable(D, F, B))))
        return hipErrorInvalidValue;
    const int npairs = (NQ + 2 * NKV) / 2;
    const int nprod = (npairs + NWAVE - 1) / NWAVE;
    const int nwo = wo ? (D / 2 + NWAVE - 1) / NWAVE : 0;
    dim3 grid(nprod + H * B + nwo);   /* with the FFN: + its roles' work-groups, below */
    unsigned long long *ta = tagged + (size_t)LM_TAG_B * (NQ + 2 * NKV);
    unsigned long long *tx = ta + (size_t)LM_TA_COPIES * LM_TAG_B * NQ;
    unsigned long long *tgt = tx + (size_t)LM_TX_COPIES * LM_TAG_B * D;
    const QkvTagged tg = {tagged, tagged + (size_t)LM_TAG_B * NQ, tagged + (size_t)LM_TAG_B * (NQ + NKV),
                          ta, tx, tgt, epoch, layer, n_layers, err};
    const FfnArgs ffn = {rms_ffn, (const u16 *)w13, (const u16 *)w2};
#define LAUNCH_QA(HD_, KT_, WO_, F_)                                                                 \
    do {                                                                                             \
        const size_t shm_ = F_ ? lds_cap_pad<k_qkv_attn<K_, NB_, KT_, HD_, WO_, F_>>(wgs_per_cu) : 0; \
        DLAUNCH((k_qkv_attn<K_, NB_, KT_, HD_, WO_, F_>), grid, dim3(WG), shm_, s, x, emb, tok, rms_w, \
                wqkv, NQ, NKV, rope_cos, rope_sin, pos, B, (KT_ *)kc, (KT_ *)vc, max_seq, npairs,      \
                nprod, H, tg, out, (const u16 *)wo, ffn);                                            \
    } while (0)
#define LAUNCH_QA_KV(WO_, F_)                                    \
    do {                                                         \
        if (hd == 64 && kv_f32) LAUNCH_QA(64, float, WO_, F_);   \
        else if (hd == 64) LAUNCH_QA(64, u16, WO_, F_);          \
        else if (kv_f32) LAUNCH_QA(128, float, WO_, F_);         \
        else LAUNCH_QA(128, u16, WO_, F_);                       \
    } while (0)
    if (w13) {
        DISPATCH_DF(D, F, DISPATCH_NB(B, {
            grid.x += (F_ + NWAVE - 1) / NWAVE + (K_ / 2 + NWAVE - 1) / NWAVE;
            LAUNCH_QA_KV(true, F_);
        }));
    } else {
        DISPATCH_D(D, DISPATCH_NB(B, {
            if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
            if (wo) LAUNCH_QA_KV(true, 0);
            else LAUNCH_QA_KV(false, 0);
        }));
    }
#undef LAUNCH_QA_KV
#undef LAUNCH_QA
    return hipGetLastError();
}

extern "C" int lmk_attn_decode(hipStream_t s, const float *q, const void *kc, const void *vc,
                               int kv_f32, const int *pos, const int *slot, int B, int H, int Hkv,
                               int hd, int max_seq, float *out, uint16_t *out16)
{
    if (B < 1 || B > 65535 || H < 1 || Hkv < 1 || H % Hkv) return hipErrorInvalidValue;
    dim3 grid(H, B);
#define LAUNCH_ATTN(HD_, KT_)                                                                  \
    DLAUNCH((k_attn_decode<HD_, KT_>), grid, dim3(WG), 0, s, q, (const KT_ *)kc,   \
                       (const KT_ *)vc, pos, slot, H, Hkv, max_seq, out, (u16 *)out16)
    if (hd == 64 && kv_f32) LAUNCH_ATTN(64, float);
    else if (hd == 64) LAUNCH_ATTN(64, u16);
    else if (hd == 128 && kv_f32) LAUNCH_ATTN(128, float);
    else if (hd == 128) LAUNCH_ATTN(128, u16);
    else return hipErrorInvalidValue;
#undef LAUNCH_ATTN
    return hipGetLastError();
}

extern "C" int lmk_attn_decode_part(hipStream_t s, const float *part, size_t sstride, int ns, int NQ,
                                    int NKV, const int *pos, const int *slot, int B, int H, int Hkv,
                                    int hd, int max_seq, const float *rope_cos, const float *rope_sin,
                                    void *kc, void *vc, int kv_f32, uint16_t *out16)
{
    if (B < 1 || B > 65535 || H < 1 || Hkv < 1 || H % Hkv || ns < 1 || NQ != H * hd ||
        NKV != Hkv * hd || !part || !pos || !slot || !kc || !vc || !out16 || !rope_cos || !rope_sin)
        return hipErrorInvalidValue;
    dim3 grid(H, B);
#define LAUNCH_ADP(HD_, KT_)                                                                      \
    hipLaunchKernelGGL((k_attn_decode_part<HD_, KT_>), grid, dim3(WG), 0, s, part, sstride, ns, NQ, \
                       NKV, pos, slot, H, Hkv, max_seq, rope_cos, rope_sin, (KT_ *)kc, (KT_ *)vc,  \
                       (u16 *)out16)
    if (hd == 64 && kv_f32) LAUNCH_ADP(64, float);
    else if (hd == 64) LAUNCH_ADP(64, u16);
    else if (hd == 128 && kv_f32) LAUNCH_ADP(128, float);
    else if (hd == 128) LAUNCH_ADP(128, u16);
    else return hipErrorInvalidValue;
#undef LAUNCH_ADP
    return hipGetLastError();
}

extern "C" int lmk_wo_residual(hipStream_t s, const float *attn, const uint16_t *wo, int D, int B,
                               float *x)
{
    if (B < 1 || B > 4 || (D & 1)) return hipErrorInvalidValue;
    const int npairs = D / 2;
    dim3 grid((npairs + NWAVE - 1) / NWAVE);
    DISPATCH_D(D, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        DLAUNCH((k_wo_residual<K_, NB_>), grid, dim3(WG), 0, s, attn, wo, B, x, npairs);
    }));
    return hipGetLastError();
}

extern "C" int lmk_ffn13(hipStream_t s, float *x, const float *rms_w, const uint16_t *w13, int D,
                         int F, int B, float *g)
{
    if (B < 1 || B > 4 || F % LMK_GATE_BLOCK) return hipErrorInvalidValue;
    dim3 grid((F + NWAVE - 1) / NWAVE);
    DISPATCH_D(D, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        DLAUNCH((k_ffn13<K_, NB_>), grid, dim3(WG), 0, s, x, rms_w, w13, F, B, g);
    }));
    return hipGetLastError();
}

extern "C" int lmk_w2_residual(hipStream_t s, const float *g, const uint16_t *w2, int D, int F, int B,
                               float *x)
{
    if (B < 1 || B > 4 || (D & 1)) return hipErrorInvalidValue;
    const int npairs = D / 2;
    dim3 grid((npairs + NWAVE - 1) / NWAVE);
    DISPATCH_K(F, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        DLAUNCH((k_w2_residual<K_, NB_>), grid, dim3(WG), 0, s, g, w2, D, B, x, npairs);
    }));
    return hipGetLastError();
}


extern "C" int lmk_cls_nblk(int V) { return (V + CLS_ROWS_PER_WG - 1) / CLS_ROWS_PER_WG; }

extern "C" int lmk_cls(hipStream_t s, const float *x, const float *rms_w, const uint16_t *wcls, int D,
                       int V, int B, float *logits, LMArgPart *part, unsigned long long *fold_tw,
                       unsigned *epoch, int *tok, int *pos, int *hist, int hist_stride, int *err)
{
    if (B < 1 || B > 4 || V < 1 || (!part && !fold_tw) ||
        (fold_tw && (!epoch || !tok || !err || (hist && !pos))))
        return hipErrorInvalidValue;
    dim3 grid(lmk_cls_nblk(V) + (fold_tw ? 1 : 0));
    const ArgFold fold = {fold_tw, epoch, tok, pos, hist, hist_stride, err};
    DISPATCH_D(D, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        DLAUNCH((k_cls<K_, NB_>), grid, dim3(WG), 0, s, x, rms_w, wcls, V, B, logits,
                           part, fold);
    }));
    return hipGetLastError();
}

extern "C" int lmk_argmax_final(hipStream_t s, const LMArgPart *part, int nblk, int B, int *tok,
                                int *pos, int *hist, int hist_stride, unsigned *epoch)
{
    if (B < 1 || nblk < 1 || !tok || (hist && !pos)) return hipErrorInvalidValue;
    DLAUNCH(k_argmax_final, dim3(B), dim3(WG), 0, s, part, nblk, tok, pos, hist,
                       hist_stride, epoch);
    return hipGetLastError();
}

extern "C" int lmk_selftest_reduce(hipStream_t s, const float *in, float *out)
{
    hipLaunchKernelGGL(k_selftest_reduce, dim3(1), dim3(64), 0, s, in, out);
    return hipGetLastError();
}
