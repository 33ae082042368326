/*
 * k_decode.hip — per-op decode kernels for small batches (B <= 4), gfx950.
 *
 * One decode step of one layer is five launches, shaped after the reference's
 * fused forward programs (training/training_dynamic/mil_dynamic.h:56-288) but
 * cut where a full-vector dependency forces a grid-wide boundary:
 *   qkv_rope   rmsnorm prologue (forward.h:46-53) + [Wq;Wk;Wv] GEMV
 *              (forward.h:122-124) + interleaved RoPE (forward.h:55-70) + KV append
 *   attn       split-KV causal attention over the fp16 cache (forward.h:72-99)
 *   wo         split merge + Wo GEMV + residual (forward.h:134-136)
 *   ffn13      rmsnorm prologue + W1/W3 GEMV + SiLU gate (forward.h:139-151)
 *   w2         W2 GEMV + residual (forward.h:157-159)
 * and per token embed (forward.h:108-110), classifier + argmax partials
 * (forward.h:163-170, generate.m:474-493) and the argmax merge.
 *
 * GEMV mapping: a wave owns a pair of weight rows, each 32-lane half one row;
 * a lane streams 16-byte (8 x fp16) chunks (c*32 + lane) of its row, multiplies
 * against the fp32 activation held in LDS and the half-wave sum is formed with
 * DPP.  Pairs line up with RoPE pairs (rows 2i, 2i+1) and with the gate pairs
 * (row i of W1 in half 0, row i of W3 in half 1).
 */
#include "k_common.h"
#include "lm_internal.h"

#define WG 256
#define NWAVE (WG / 64)

/* ---- prologues ---------------------------------------------------------- */

/* xs[b*K + i] = x[b*K + i] * (1/sqrt(mean(x_b^2) + 1e-5)) * w[i] for b < B,
 * zero rows for B <= b < NB (forward.h:46-53). */
template <int K, int NB>
__device__ __forceinline__ void rmsnorm_to_lds(const float *__restrict__ x,
                                               const float *__restrict__ w, int B,
                                               float *xs)
{
    __shared__ float red[NB][NWAVE];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float ss = 0.f;
        for (int i = tid; i < K; i += WG) {
            float v = b < B ? x[(size_t)b * K + i] : 0.f;
            xs[b * K + i] = v;
            ss = fmaf(v, v, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[b][wv] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < NWAVE; i++) tot += red[b][i];
        float scale = 1.0f / sqrtf(tot / K + 1e-5f);
        for (int i = tid; i < K; i += WG) xs[b * K + i] = xs[b * K + i] * scale * w[i];
    }
    __syncthreads();
}

template <int K, int NB>
__device__ __forceinline__ void rows_to_lds(const float *__restrict__ src, int B, float *xs)
{
    for (int i = threadIdx.x; i < NB * K; i += WG) xs[i] = (i / K) < B ? src[i] : 0.f;
    __syncthreads();
}

/* ---- GEMV core ------------------------------------------------------------ */

/* Half-wave dot products of one fp16 row (length K) with NB fp32 vectors in
 * LDS.  hl = lane within the half (0..31); acc[b] is this lane's partial. */
template <int K, int NB>
__device__ __forceinline__ void hw_dot(const u16 *__restrict__ wrow, const float *xs, int hl,
                                       float acc[NB])
{
    constexpr int CPL = K / 256;
    uint4 wv[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++)
        wv[c] = *(const uint4 *)(wrow + (size_t)(c * 32 + hl) * 8);
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
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

/* ---- embed ----------------------------------------------------------------- */

__global__ void __launch_bounds__(WG) k_embed(const u16 *__restrict__ E, const int *__restrict__ tok,
                                              float *__restrict__ x, int D)
{
    const int b = blockIdx.y;
    const int t = tok[b];
    for (int i = blockIdx.x * WG + threadIdx.x; i < D; i += gridDim.x * WG)
        x[(size_t)b * D + i] = h2f(E[(size_t)t * D + i]);
}

/* ---- QKV + RoPE + KV append ------------------------------------------------ */

template <int D, int NB, typename KT>
__global__ void __launch_bounds__(WG) k_qkv_rope(
    const float *__restrict__ x, const float *__restrict__ rms_w, const u16 *__restrict__ W,
    int NQ, int NKV, int hd, const float *__restrict__ rc, const float *__restrict__ rs,
    const int *__restrict__ pos, int B, float *__restrict__ q, KT *__restrict__ kc,
    KT *__restrict__ vc, int max_seq, int npairs)
{
    __shared__ __attribute__((aligned(16))) float xs[NB * D];
    rmsnorm_to_lds<D, NB>(x, rms_w, B, xs);
    const int p = blockIdx.x * NWAVE + (threadIdx.x >> 6);
    if (p >= npairs) return;
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int r = 2 * p;
    float acc[NB], r0[NB], r1[NB];
    hw_dot<D, NB>(W + (size_t)(r + half) * D, xs, hl, acc);
    pair_reduce<NB>(acc, r0, r1);
    if (lane != 0) return;
    const int half_hd = hd >> 1;
    const int Hkv = NKV / hd;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (b >= B) break;
        const int ps = pos[b];
        if (r < NQ + NKV) {
            const int rr = r < NQ ? r : r - NQ;
            const int i = (rr % hd) >> 1;
            const float c = rc[ps * half_hd + i], s = rs[ps * half_hd + i];
            const float a = r0[b], e = r1[b];
            const float o0 = fmaf(a, c, -(e * s));   /* forward.h:64 */
            const float o1 = fmaf(a, s, e * c);      /* forward.h:65 */
            if (r < NQ) {
                q[(size_t)b * NQ + r] = o0;
                q[(size_t)b * NQ + r + 1] = o1;
            } else {
                const int h = rr / hd, d = rr % hd;
                KT *dst = kc + (((size_t)b * Hkv + h) * max_seq + ps) * hd + d;
                dst[0] = kv_pack<KT>(o0);
                dst[1] = kv_pack<KT>(o1);
            }
        } else {
            const int rr = r - NQ - NKV;
            const int h = rr / hd, d = rr % hd;
            KT *dst = vc + (((size_t)b * Hkv + h) * max_seq + ps) * hd + d;
            dst[0] = kv_pack<KT>(r0[b]);
            dst[1] = kv_pack<KT>(r1[b]);
        }
    }
}

/* ---- split-KV decode attention --------------------------------------------- */

template <int HD, typename KT>
__global__ void __launch_bounds__(64) k_attn_decode(
    const float *__restrict__ q, const KT *__restrict__ kc, const KT *__restrict__ vc,
    const int *__restrict__ pos, int H, int Hkv, int max_seq, int nsplit,
    float *__restrict__ part)
{
    constexpr int CH = LMK_ATTN_CHUNK;
    constexpr int G = HD / 8;        /* lanes per position            */
    constexpr int PP = 64 / G;       /* positions per pass            */
    constexpr int NPASS = CH / PP;
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x;
    const int ctx = pos[b] + 1;
    const int p0 = split * CH;
    float *out = part + ((size_t)(b * H + h) * nsplit + split) * (HD + 2);
    if (p0 >= ctx) {
        for (int i = lane; i < HD + 2; i += 64) out[i] = i == 0 ? -INFINITY : 0.f;
        return;
    }
    const int p1 = min(ctx, p0 + CH);
    const int dq = lane % G, pp = lane / G;
    const int kvh = h / (H / Hkv);
    const size_t base = ((size_t)b * Hkv + kvh) * max_seq * HD;
    const KT *K = kc + base;
    const KT *V = vc + base;
    const float scale = 1.0f / sqrtf((float)HD);
    float qf[8];
    {
        const float *qp = q + (size_t)b * H * HD + h * HD + dq * 8;
        const float4 a = *(const float4 *)qp, c = *(const float4 *)(qp + 4);
        qf[0] = a.x; qf[1] = a.y; qf[2] = a.z; qf[3] = a.w;
        qf[4] = c.x; qf[5] = c.y; qf[6] = c.z; qf[7] = c.w;
    }
    float s[NPASS];
#pragma unroll
    for (int i = 0; i < NPASS; i++) {
        const int p = p0 + pp + PP * i;
        float d = 0.f;
        if (p < p1) {
            float kf[8];
            kv_load8(K + (size_t)p * HD + dq * 8, kf);
#pragma unroll
            for (int j = 0; j < 8; j++) d = fmaf(qf[j], kf[j], d);
        }
#pragma unroll
        for (int off = 1; off < G; off <<= 1) d += __shfl_xor(d, off, 64);
        s[i] = p < p1 ? d * scale : -INFINITY;
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPASS; i++) m = fmaxf(m, s[i]);
#pragma unroll
    for (int off = G; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float l = 0.f, o[8];
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = 0.f;
#pragma unroll
    for (int i = 0; i < NPASS; i++) {
        const int p = p0 + pp + PP * i;
        if (p < p1) {
            const float e = expf(s[i] - m);
            l += e;
            float vf[8];
            kv_load8(V + (size_t)p * HD + dq * 8, vf);
#pragma unroll
            for (int j = 0; j < 8; j++) o[j] = fmaf(e, vf[j], o[j]);
        }
    }
#pragma unroll
    for (int off = G; off < 64; off <<= 1) {
        l += __shfl_xor(l, off, 64);
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] += __shfl_xor(o[j], off, 64);
    }
    if (lane < G) {
#pragma unroll
        for (int j = 0; j < 8; j++) out[2 + dq * 8 + j] = o[j];
    }
    if (lane == 0) { out[0] = m; out[1] = l; }
}

/* ---- Wo + residual ---------------------------------------------------------- */

/* attn[b, h*hd + d] from the split partials of (b, h). */
template <int D, int NB>
__device__ __forceinline__ void merge_attn_to_lds(const float *__restrict__ part, int nsplit,
                                                  int H, int hd, int B, float *xs)
{
    const int HDp = hd + 2;
    for (int e = threadIdx.x; e < NB * D; e += WG) {
        const int b = e / D, c = e % D;
        float v = 0.f;
        if (b < B) {
            const int h = c / hd, d = c % hd;
            const float *pb = part + (size_t)(b * H + h) * nsplit * HDp;
            float M = -INFINITY;
            for (int s = 0; s < nsplit; s++) M = fmaxf(M, pb[s * HDp]);
            float L = 0.f, acc = 0.f;
            for (int s = 0; s < nsplit; s++) {
                const float w = expf(pb[s * HDp] - M);
                L = fmaf(pb[s * HDp + 1], w, L);
                acc = fmaf(pb[s * HDp + 2 + d], w, acc);
            }
            v = acc / L;
        }
        xs[e] = v;
    }
    __syncthreads();
}

template <int D, int NB>
__global__ void __launch_bounds__(WG) k_wo_residual(
    const float *__restrict__ part, int nsplit, const u16 *__restrict__ W, int H, int hd,
    int B, float *__restrict__ x, int npairs)
{
    __shared__ __attribute__((aligned(16))) float xs[NB * D];
    merge_attn_to_lds<D, NB>(part, nsplit, H, hd, B, xs);
    const int p = blockIdx.x * NWAVE + (threadIdx.x >> 6);
    if (p >= npairs) return;
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int r = 2 * p;
    float acc[NB], r0[NB], r1[NB];
    hw_dot<D, NB>(W + (size_t)(r + half) * D, xs, hl, acc);
    pair_reduce<NB>(acc, r0, r1);
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            x[(size_t)b * D + r] += r0[b];
            x[(size_t)b * D + r + 1] += r1[b];
        }
    }
}

/* ---- W1/W3 + SiLU gate ------------------------------------------------------ */

template <int D, int NB>
__global__ void __launch_bounds__(WG) k_ffn13(
    const float *__restrict__ x, const float *__restrict__ rms_w, const u16 *__restrict__ W13,
    int F, int B, float *__restrict__ g)
{
    __shared__ __attribute__((aligned(16))) float xs[NB * D];
    rmsnorm_to_lds<D, NB>(x, rms_w, B, xs);
    const int i = blockIdx.x * NWAVE + (threadIdx.x >> 6);
    if (i >= F) return;
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    constexpr int GB = LMK_GATE_BLOCK;
    const size_t row = (size_t)(i / GB) * (2 * GB) + half * GB + (i % GB);
    float acc[NB], h1[NB], h3[NB];
    hw_dot<D, NB>(W13 + row * D, xs, hl, acc);
    pair_reduce<NB>(acc, h1, h3);
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
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
    rows_to_lds<F, NB>(g, B, xs);
    const int p = blockIdx.x * NWAVE + (threadIdx.x >> 6);
    if (p >= npairs) return;
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int r = 2 * p;
    float acc[NB], r0[NB], r1[NB];
    hw_dot<F, NB>(W + (size_t)(r + half) * F, xs, hl, acc);
    pair_reduce<NB>(acc, r0, r1);
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            x[(size_t)b * D + r] += r0[b];
            x[(size_t)b * D + r + 1] += r1[b];
        }
    }
}

/* ---- classifier + argmax partials ------------------------------------------ */

#define CLS_PAIRS_PER_WAVE 16
#define CLS_ROWS_PER_WG (2 * CLS_PAIRS_PER_WAVE * NWAVE)

template <int D, int NB>
__global__ void __launch_bounds__(WG) k_cls(
    const float *__restrict__ x, const float *__restrict__ rms_w, const u16 *__restrict__ W,
    int V, int B, float *__restrict__ logits, LMArgPart *__restrict__ part)
{
    __shared__ __attribute__((aligned(16))) float xs[NB * D];
    __shared__ float bvs[NB][NWAVE];
    __shared__ int bis[NB][NWAVE];
    rmsnorm_to_lds<D, NB>(x, rms_w, B, xs);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, half = lane >> 5, hl = lane & 31;
    float bv[NB];
    int bi[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) { bv[b] = -INFINITY; bi[b] = 0x7FFFFFFF; }
    const int row0 = blockIdx.x * CLS_ROWS_PER_WG + wv * 2 * CLS_PAIRS_PER_WAVE;
    for (int pp = 0; pp < CLS_PAIRS_PER_WAVE; pp++) {
        const int r = row0 + 2 * pp;
        if (r >= V) break;
        const int rl = min(r + half, V - 1);
        float acc[NB], r0[NB], r1[NB];
        hw_dot<D, NB>(W + (size_t)rl * D, xs, hl, acc);
        pair_reduce<NB>(acc, r0, r1);
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
                logits[(size_t)b * V + r] = r0[b];
                if (has1) logits[(size_t)b * V + r + 1] = r1[b];
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
        part[(size_t)b * gridDim.x + blockIdx.x] = LMArgPart{v, id};
    }
}

/* ---- argmax merge + greedy loop state ---------------------------------------- */

__global__ void __launch_bounds__(WG) k_argmax_final(
    const LMArgPart *__restrict__ part, int nblk, int *__restrict__ tok, int *__restrict__ pos,
    int *__restrict__ hist, int hist_stride)
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

/* LDS budget of the GEMV kernels: NB rows of K fp32. */
#define GEMV_LDS_OK(K_, NB_) ((size_t)(K_) * (NB_) * 4 <= 65536)

extern "C" int lmk_embed(hipStream_t s, const uint16_t *embed, const int *tok, float *x, int B, int D)
{
    if (B <= 0 || D <= 0) return hipErrorInvalidValue;
    dim3 grid((D + WG - 1) / WG, B);
    hipLaunchKernelGGL(k_embed, grid, dim3(WG), 0, s, embed, tok, x, D);
    return hipGetLastError();
}

extern "C" int lmk_qkv_rope(hipStream_t s, const float *x, const float *rms_w, const uint16_t *wqkv,
                            int D, int NQ, int NKV, int hd, const float *rope_cos,
                            const float *rope_sin, const int *pos, int B, float *q, void *kc,
                            void *vc, int kv_f32, int max_seq)
{
    if (B < 1 || B > 4 || NQ != D || (hd & 1) || NKV % hd) return hipErrorInvalidValue;
    const int npairs = (NQ + 2 * NKV) / 2;
    dim3 grid((npairs + NWAVE - 1) / NWAVE);
    DISPATCH_K(D, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        if (kv_f32)
            hipLaunchKernelGGL((k_qkv_rope<K_, NB_, float>), grid, dim3(WG), 0, s, x, rms_w, wqkv, NQ,
                               NKV, hd, rope_cos, rope_sin, pos, B, q, (float *)kc, (float *)vc,
                               max_seq, npairs);
        else
            hipLaunchKernelGGL((k_qkv_rope<K_, NB_, u16>), grid, dim3(WG), 0, s, x, rms_w, wqkv, NQ,
                               NKV, hd, rope_cos, rope_sin, pos, B, q, (u16 *)kc, (u16 *)vc,
                               max_seq, npairs);
    }));
    return hipGetLastError();
}

template <int HD, typename KT>
static void launch_attn_decode(hipStream_t s, dim3 grid, const float *q, const void *kc,
                               const void *vc, const int *pos, int H, int Hkv, int max_seq,
                               int nsplit, float *part)
{
    hipLaunchKernelGGL((k_attn_decode<HD, KT>), grid, dim3(64), 0, s, q, (const KT *)kc,
                       (const KT *)vc, pos, H, Hkv, max_seq, nsplit, part);
}

extern "C" int lmk_attn_decode(hipStream_t s, const float *q, const void *kc, const void *vc,
                               int kv_f32, const int *pos, int B, int H, int Hkv, int hd,
                               int max_seq, int nsplit, float *part)
{
    if (B < 1 || H < 1 || Hkv < 1 || H % Hkv || nsplit < 1 ||
        nsplit * LMK_ATTN_CHUNK < max_seq)
        return hipErrorInvalidValue;
    dim3 grid(nsplit, H, B);
    if (hd == 64 && kv_f32)
        launch_attn_decode<64, float>(s, grid, q, kc, vc, pos, H, Hkv, max_seq, nsplit, part);
    else if (hd == 64)
        launch_attn_decode<64, u16>(s, grid, q, kc, vc, pos, H, Hkv, max_seq, nsplit, part);
    else if (hd == 128 && kv_f32)
        launch_attn_decode<128, float>(s, grid, q, kc, vc, pos, H, Hkv, max_seq, nsplit, part);
    else if (hd == 128)
        launch_attn_decode<128, u16>(s, grid, q, kc, vc, pos, H, Hkv, max_seq, nsplit, part);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" int lmk_wo_residual(hipStream_t s, const float *part, int nsplit, const uint16_t *wo, int D,
                               int H, int hd, int B, float *x)
{
    if (B < 1 || B > 4 || H * hd != D) return hipErrorInvalidValue;
    const int npairs = D / 2;
    dim3 grid((npairs + NWAVE - 1) / NWAVE);
    DISPATCH_K(D, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        hipLaunchKernelGGL((k_wo_residual<K_, NB_>), grid, dim3(WG), 0, s, part, nsplit, wo, H, hd, B, x, npairs);
    }));
    return hipGetLastError();
}

extern "C" int lmk_ffn13(hipStream_t s, const float *x, const float *rms_w, const uint16_t *w13, int D,
                         int F, int B, float *g)
{
    if (B < 1 || B > 4 || F % LMK_GATE_BLOCK) return hipErrorInvalidValue;
    dim3 grid((F + NWAVE - 1) / NWAVE);
    DISPATCH_K(D, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        hipLaunchKernelGGL((k_ffn13<K_, NB_>), grid, dim3(WG), 0, s, x, rms_w, w13, F, B, g);
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
        hipLaunchKernelGGL((k_w2_residual<K_, NB_>), grid, dim3(WG), 0, s, g, w2, D, B, x, npairs);
    }));
    return hipGetLastError();
}

extern "C" int lmk_cls_nblk(int V) { return (V + CLS_ROWS_PER_WG - 1) / CLS_ROWS_PER_WG; }

extern "C" int lmk_cls(hipStream_t s, const float *x, const float *rms_w, const uint16_t *wcls, int D,
                       int V, int B, float *logits, LMArgPart *part)
{
    if (B < 1 || B > 4 || V < 1) return hipErrorInvalidValue;
    dim3 grid(lmk_cls_nblk(V));
    DISPATCH_K(D, DISPATCH_NB(B, {
        if (!GEMV_LDS_OK(K_, NB_)) return hipErrorInvalidValue;
        hipLaunchKernelGGL((k_cls<K_, NB_>), grid, dim3(WG), 0, s, x, rms_w, wcls, V, B, logits, part);
    }));
    return hipGetLastError();
}

extern "C" int lmk_argmax_final(hipStream_t s, const LMArgPart *part, int nblk, int B, int *tok, int *pos,
                                int *hist, int hist_stride)
{
    if (B < 1 || nblk < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax_final, dim3(B), dim3(WG), 0, s, part, nblk, tok, pos, hist, hist_stride);
    return hipGetLastError();
}

extern "C" int lmk_selftest_reduce(hipStream_t s, const float *in, float *out)
{
    hipLaunchKernelGGL(k_selftest_reduce, dim3(1), dim3(64), 0, s, in, out);
    return hipGetLastError();
}
