/*
 * k_persist.hip — batch-1 greedy decode as one persistent kernel (gfx950).
 *
 * One cooperative launch runs n decode steps (training/training_dynamic/
 * generate.m:427-516 with a KV cache, as training/dashboard.py:205-276) with the
 * argmax fed back on the device.  Every work-group (one per CU) walks the same
 * phase sequence per token:
 *   per layer  QKV   rmsnorm (forward.h:46-53) + [Wq;Wk;Wv] rows + RoPE
 *                    (forward.h:55-70) + K/V append
 *              ATTN  causal attention of one (head, position chunk) on the
 *                    work-groups that own one (forward.h:72-99)
 *              WO    merge of the chunks + Wo rows + residual (forward.h:134-136)
 *              W13   rmsnorm + W1/W3 rows + SiLU gate (forward.h:139-151)
 *              W2    W2 rows + residual (forward.h:157-159)
 *   per token  CLS   final rmsnorm + classifier rows + argmax partial
 *                    (forward.h:163-170), then every work-group reduces the
 *                    partials to the next token (generate.m:129-136)
 *
 * Phase hand-off: every value a phase publishes is a 64-bit word {fp32 value,
 * 32-bit tag} written with one agent-scope atomic store; the consumer polls the
 * words themselves with agent-scope atomic loads until their tag is the
 * current step's.  The data is its own ready flag, so a hand-off costs one
 * store-to-load latency and no barrier, fence or cache flush.  Each buffer is
 * rewritten once per step: a producer can only reach the next step's write
 * after every work-group has produced rows of a later phase, which each does
 * only after consuming the buffer, so no word is overwritten before it is read.
 *
 * K/V cache entries written inside the kernel use agent-scope stores and are
 * read with agent-scope loads (the per-XCD L2s are not coherent with each
 * other); the current position's K/V also travel as tagged words.
 *
 * Weights (read-only) use plain 16-byte loads, issued one phase ahead into
 * registers so their HBM latency hides behind the previous hand-off.
 *
 * Every wait is bounded: on a time-out the work-group raises *err and all
 * work-groups leave at their next wait, so the grid always drains.
 */
#include "k_common.h"
#include "lm_internal.h"

typedef unsigned long long u64;

#define PT 512                 /* threads per work-group */
#define PW (PT / 64)           /* waves per work-group   */
#define SPIN_MAX (1 << 21)     /* polls before a wait gives up (about a second) */

/* ---- tagged words ----------------------------------------------------------- */

__device__ __forceinline__ u64 ll_load(const u64 *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void ll_store(u64 *p, float v, unsigned tag)
{
    __hip_atomic_store(p, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool ll_ready(u64 w, unsigned tag) { return (unsigned)(w >> 32) == tag; }
__device__ __forceinline__ float ll_val(u64 w) { return __uint_as_float((unsigned)w); }

/* Poll one word until its tag is `tag` and return it; on time-out, or when
 * another work-group has raised *err, return a word whose tag differs. */
__device__ __noinline__ u64 ll_spin(const u64 *p, unsigned tag, int *err)
{
    u64 w = ll_load(p);
    for (int spin = 1; !ll_ready(w, tag); spin++) {
        if ((spin & 255) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
            break;
        if (spin > SPIN_MAX) {
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        w = ll_load(p);
    }
    return w;
}

/* Make w[...] ready: re-poll when its first load was early. */
#define LL_WAIT(ok, word, ptr, tag, err)                          \
    do {                                                          \
        if ((ok) && !ll_ready(word, tag)) {                       \
            (word) = ll_spin(ptr, tag, err);                      \
            (ok) = ll_ready(word, tag);                           \
        }                                                         \
    } while (0)

/* Wait for words [0, n) of buf (this thread: i = tid + k*PT) and store their
 * values to dst[i].  All of this thread's loads are issued before the first
 * check; dst is written only after every thread of the work-group has its
 * words (so earlier readers of dst are done).  Returns false (for the whole
 * work-group) on time-out. */
template <int MAXPER>
__device__ __forceinline__ bool ll_fetch(const u64 *__restrict__ buf, int n, unsigned tag,
                                         float *dst, int *err)
{
    u64 w[MAXPER];
#pragma unroll
    for (int k = 0; k < MAXPER; k++) {
        const int i = threadIdx.x + k * PT;
        w[k] = i < n ? ll_load(buf + i) : ((u64)tag << 32);
    }
    bool ok = true;
#pragma unroll
    for (int k = 0; k < MAXPER; k++) {
        const int i = threadIdx.x + k * PT;
        if (i < n) LL_WAIT(ok, w[k], buf + i, tag, err);
    }
    if (__syncthreads_or(!ok)) return false;
#pragma unroll
    for (int k = 0; k < MAXPER; k++) {
        const int i = threadIdx.x + k * PT;
        if (i < n) dst[i] = ll_val(w[k]);
    }
    __syncthreads();
    return true;
}

/* ---- coherent K/V cache access ---------------------------------------------------- */

template <typename KT> struct KVT;
template <> struct KVT<float> {
    /* 8 fp32 = 4 x 64-bit */
    static __device__ __forceinline__ void load8(const float *p, float f[8])
    {
        const u64 *q = (const u64 *)p;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u64 w = ll_load(q + i);
            f[2 * i] = __uint_as_float((unsigned)w);
            f[2 * i + 1] = __uint_as_float((unsigned)(w >> 32));
        }
    }
    static __device__ __forceinline__ void store2(float *p, float a, float b)
    {
        const u64 w = ((u64)__float_as_uint(b) << 32) | (u64)__float_as_uint(a);
        __hip_atomic_store((u64 *)p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    static __device__ __forceinline__ float round(float v) { return v; }
};
template <> struct KVT<u16> {
    /* 8 binary16 = 2 x 64-bit */
    static __device__ __forceinline__ void load8(const u16 *p, float f[8])
    {
        const u64 *q = (const u64 *)p;
        const u64 a = ll_load(q), b = ll_load(q + 1);
        uint4 v;
        v.x = (unsigned)a; v.y = (unsigned)(a >> 32); v.z = (unsigned)b; v.w = (unsigned)(b >> 32);
        unpack8(v, f);
    }
    static __device__ __forceinline__ void store2(u16 *p, float a, float b)
    {
        const unsigned w = (unsigned)f2h(a) | ((unsigned)f2h(b) << 16);
        __hip_atomic_store((unsigned *)p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    static __device__ __forceinline__ float round(float v) { return h2f(f2h(v)); }
};

/* ---- kernel arguments ------------------------------------------------------------- */

struct PDArgs {
    const u16 *layers;
    size_t layer_elems, off_wo, off_w13, off_w2;
    const u16 *embed, *wcls;
    const float *rms_att, *rms_ffn, *rms_final, *rope_cos, *rope_sin;
    void *kc, *vc;
    size_t kv_layer_elems;
    u64 *ll;                   /* tagged-word buffers, lmk_persist_ll_words() words */
    float *logits;             /* V floats or NULL */
    int *out_tok;              /* n_steps greedy ids */
    int *state_tok, *state_pos;
    int *err;
    int V, L, H, Hkv, max_seq;
    int tok0, pos0, n_steps;
    unsigned tag0;
};

/* Vectors that every work-group reads are published in NREP copies; work-group
 * w reads copy w % NREP, which spreads the polling over NREP times as many
 * memory lines (one copy polled by all 256 work-groups is a hot spot).
 * Tagged-word layout: per layer q[NQ] | kvnew[2*NKV] | NREP x attn partials
 * [H*SMAX*(HD+2)] | NREP x x_wo[D] | NREP x g[F] | NREP x x_w2[D]; then NREP x
 * cls partials [2*grid]. */
#define SMAX 2
#define NREP 8

__host__ __device__ __forceinline__ size_t ll_layer_words(int D, int F, int H, int Hkv, int hd)
{
    return (size_t)H * hd + 2 * (size_t)Hkv * hd +
           NREP * ((size_t)H * SMAX * (hd + 2) + 2 * (size_t)D + F);
}

/* Publish word i of a replicated vector of n words. */
__device__ __forceinline__ void ll_store_rep(u64 *buf, int n, int i, float v, unsigned tag)
{
#pragma unroll
    for (int r = 0; r < NREP; r++) ll_store(buf + (size_t)r * n + i, v, tag);
}

/* ---- the kernel ------------------------------------------------------------------- */

/* Half-wave dot product of a prefetched fp16 row (K/256 chunks per lane) with an
 * fp32 LDS vector; result valid in every lane of the half after the reduction. */
template <int K>
__device__ __forceinline__ float hrow_dot(const uint4 *wv, const float *xs, int hl)
{
    float a = 0.f;
#pragma unroll
    for (int c = 0; c < K / 256; c++) {
        float w[8];
        unpack8(wv[c], w);
        const int k0 = (c * 32 + hl) * 8;
        const float4 xa = *(const float4 *)(xs + k0);
        const float4 xb = *(const float4 *)(xs + k0 + 4);
        a = fmaf(w[0], xa.x, a); a = fmaf(w[1], xa.y, a);
        a = fmaf(w[2], xa.z, a); a = fmaf(w[3], xa.w, a);
        a = fmaf(w[4], xb.x, a); a = fmaf(w[5], xb.y, a);
        a = fmaf(w[6], xb.z, a); a = fmaf(w[7], xb.w, a);
    }
    return a;
}

template <int K>
__device__ __forceinline__ void hrow_load(const u16 *row, int hl, uint4 *wv)
{
#pragma unroll
    for (int c = 0; c < K / 256; c++) wv[c] = *(const uint4 *)(row + (size_t)(c * 32 + hl) * 8);
}

/* Full-wave row (K/512 chunks per lane). */
template <int K>
__device__ __forceinline__ void wrow_load(const u16 *row, int lane, uint4 *wv)
{
#pragma unroll
    for (int c = 0; c < K / 512; c++) wv[c] = *(const uint4 *)(row + (size_t)(c * 64 + lane) * 8);
}

template <int K>
__device__ __forceinline__ float wrow_dot(const uint4 *wv, const float *xs, int lane)
{
    float a = 0.f;
#pragma unroll
    for (int c = 0; c < K / 512; c++) {
        float w[8];
        unpack8(wv[c], w);
        const int k0 = (c * 64 + lane) * 8;
        const float4 xa = *(const float4 *)(xs + k0);
        const float4 xb = *(const float4 *)(xs + k0 + 4);
        a = fmaf(w[0], xa.x, a); a = fmaf(w[1], xa.y, a);
        a = fmaf(w[2], xa.z, a); a = fmaf(w[3], xa.w, a);
        a = fmaf(w[4], xb.x, a); a = fmaf(w[5], xb.y, a);
        a = fmaf(w[6], xb.z, a); a = fmaf(w[7], xb.w, a);
    }
    return a;
}

/* In-place rmsnorm of the LDS vector raw[D] into out[D] with gain g (this
 * thread's gains prefetched in gr[]): out = raw * (1/sqrt(mean(raw^2) + 1e-5)) * g. */
template <int D>
__device__ __forceinline__ void lds_rmsnorm(const float *raw, const float *gr, float *out, float *red)
{
    constexpr int PER = (D + PT - 1) / PT;
    const int tid = threadIdx.x;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = tid + k * PT;
        if (i < D) ss = fmaf(raw[i], raw[i], ss);
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < PW; i++) tot += red[i];
    const float scale = 1.0f / sqrtf(tot / D + 1e-5f);
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = tid + k * PT;
        if (i < D) out[i] = raw[i] * scale * gr[k];
    }
    __syncthreads();
}

template <int D>
__device__ __forceinline__ void gains_load(const float *g, float gr[(D + PT - 1) / PT])
{
#pragma unroll
    for (int k = 0; k < (D + PT - 1) / PT; k++) {
        const int i = threadIdx.x + k * PT;
        gr[k] = i < D ? g[i] : 0.f;
    }
}

template <int D, int F, int HD, typename KT>
__global__ void __launch_bounds__(PT) k_decode_persist(PDArgs a)
{
    constexpr int NQ_MAX = D;                    /* H*HD == D */
    constexpr int CD = D / 256;                  /* uint4 per lane, half-wave row of D */
    constexpr int CF = F / 512;                  /* uint4 per lane, full-wave row of F */
    constexpr int G = HD / 8;                    /* attention lanes per position */
    constexpr int PPW = 64 / G;                  /* positions per wave pass */
    constexpr int PASS = PW * PPW;               /* positions per work-group pass */
    constexpr int DPER = (D + PT - 1) / PT;
    constexpr int FPER = (F + PT - 1) / PT;
    constexpr int PART = SMAX * (HD + 2);        /* partial words per head */
    typedef KVT<KT> kv;

    __shared__ __attribute__((aligned(16))) float x_in[D];    /* residual input of the layer */
    __shared__ __attribute__((aligned(16))) float x_mid[D];   /* residual after Wo          */
    __shared__ __attribute__((aligned(16))) float xs[D > F ? D : F]; /* normalised / gate / attn */
    __shared__ __attribute__((aligned(16))) float part[NQ_MAX / HD * PART];
    __shared__ float red[PW];
    __shared__ float so[PW][HD];
    __shared__ float sm[PW], sl[PW];
    __shared__ float cls_v[PW * 2];
    __shared__ int cls_i[PW * 2];

    const int NWG = gridDim.x, w = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, hl = lane & 31;
    const int H = a.H, Hkv = a.Hkv, L = a.L, V = a.V;
    const int NQ = H * HD, NKV = Hkv * HD;
    const int qkv_pairs = (NQ + 2 * NKV) / 2;
    const size_t LLW = ll_layer_words(D, F, H, Hkv, HD);
    u64 *const cls_ll = a.ll + (size_t)L * LLW;
    const int half_hd = HD / 2;
    /* attention work: (head, split) -> work-group h*SMAX+s spread over the grid */
    const int att_stride = NWG / (H * SMAX);
    const int my_att = (w % att_stride == 0 && w / att_stride < H * SMAX) ? w / att_stride : -1;

    uint4 wq[CD], wo[CD], w13[CD], w2[CF > 0 ? CF : 1];
    float gq[DPER], gf[DPER];
    int tok = a.tok0;
    bool alive = true;

    /* this work-group's rows of each phase (wave-level) */
    const int qp = w + wave * NWG;                 /* QKV row pair       */
    const bool has_qp = qp < qkv_pairs;
    const int op = w + wave * NWG;                 /* Wo row pair        */
    const bool has_op = op < D / 2;
    const int gi = w + wave * NWG;                 /* gate index         */
    const bool has_gi = gi < F;
    const int r2 = w + wave * NWG;                 /* W2 row (full wave) */
    const bool has_r2 = r2 < D;

    auto load_qkv = [&](int l) {
        const u16 *lw = a.layers + (size_t)l * a.layer_elems;
        if (has_qp) hrow_load<D>(lw + (size_t)(2 * qp + half) * D, hl, wq);
        gains_load<D>(a.rms_att + (size_t)l * D, gq);
    };
    auto load_wo = [&](int l) {
        const u16 *lw = a.layers + (size_t)l * a.layer_elems + a.off_wo;
        if (has_op) hrow_load<D>(lw + (size_t)(2 * op + half) * D, hl, wo);
    };
    auto load_w13 = [&](int l) {
        const u16 *lw = a.layers + (size_t)l * a.layer_elems + a.off_w13;
        constexpr int GB = LMK_GATE_BLOCK;
        if (has_gi) {
            const size_t row = (size_t)(gi / GB) * (2 * GB) + half * GB + (gi % GB);
            hrow_load<D>(lw + row * D, hl, w13);
        }
        gains_load<D>(a.rms_ffn + (size_t)l * D, gf);
    };
    auto load_w2 = [&](int l) {
        const u16 *lw = a.layers + (size_t)l * a.layer_elems + a.off_w2;
        if (has_r2) wrow_load<F>(lw + (size_t)r2 * F, lane, w2);
    };

    load_qkv(0);
    load_wo(0);
    for (int step = 0; step < a.n_steps && alive; step++) {
        const unsigned tag = a.tag0 + (unsigned)step;
        const int pos = a.pos0 + step;
        const int ctx = pos + 1;
        /* attention split of this step: S chunks of CH positions (CH a multiple
         * of the work-group pass) */
        const int CH = PASS * ((ctx + PASS * SMAX - 1) / (PASS * SMAX));
        const int S = (ctx + CH - 1) / CH;
        /* the embedding row of this step's token starts the residual stream */
        for (int i = tid; i < D; i += PT) x_in[i] = h2f(a.embed[(size_t)tok * D + i]);
        __syncthreads();

        for (int l = 0; l < L && alive; l++) {
            u64 *ll = a.ll + (size_t)l * LLW;
            u64 *ll_q = ll, *ll_kv = ll + NQ, *ll_part = ll_kv + 2 * NKV;
            u64 *ll_xwo = ll_part + (size_t)NREP * H * PART, *ll_g = ll_xwo + (size_t)NREP * D;
            u64 *ll_xw2 = ll_g + (size_t)NREP * F;
            const int rep = w % NREP;
            const size_t kvo = (size_t)l * a.kv_layer_elems;
            KT *kc = (KT *)a.kc + kvo, *vc = (KT *)a.vc + kvo;

            /* ---------------- QKV ---------------- */
            load_w13(l);
            if (l > 0) {
                alive = ll_fetch<DPER>(a.ll + (size_t)(l - 1) * LLW + (LLW - (size_t)NREP * D) +
                                           (size_t)rep * D, D, tag, x_in, a.err);
                if (!alive) break;
            }
            /* attention work-groups prefetch the cached K/V of their chunk's first
             * pass (positions < pos are final; pos itself arrives as tagged words) */
            float kf[8], vf[8];
            const int ah = my_att >= 0 ? my_att / SMAX : 0, as = my_att >= 0 ? my_att % SMAX : 0;
            const int akvh = ah / (H / Hkv);
#pragma unroll
            for (int j = 0; j < 8; j++) { kf[j] = 0.f; vf[j] = 0.f; }
            if (my_att >= 0 && as < S) {
                const int p = as * CH + wave * PPW + lane / G;
                if (p < pos) {
                    const size_t off = (((size_t)akvh) * a.max_seq + p) * HD + (lane % G) * 8;
                    kv::load8(kc + off, kf);
                    kv::load8(vc + off, vf);
                }
            }
            __syncthreads();
            lds_rmsnorm<D>(x_in, gq, xs, red);
            if (has_qp) {
                float acc = hrow_dot<D>(wq, xs, hl);
                acc = half_wave_sum(acc);
                const float r0 = readlane_f(acc, 31), r1 = readlane_f(acc, 63);
                const int r = 2 * qp;
                if (lane == 0) {
                    if (r < NQ + NKV) {
                        const int rr = r < NQ ? r : r - NQ;
                        const int ti = pos * half_hd + ((rr % HD) >> 1);
                        const float c = a.rope_cos[ti], sn = a.rope_sin[ti];
                        const float o0 = fmaf(r0, c, -(r1 * sn));   /* forward.h:64 */
                        const float o1 = fmaf(r0, sn, r1 * c);      /* forward.h:65 */
                        if (r < NQ) {
                            ll_store(ll_q + r, o0, tag);
                            ll_store(ll_q + r + 1, o1, tag);
                        } else {
                            const int h = rr / HD, d = rr % HD;
                            kv::store2(kc + (((size_t)h) * a.max_seq + pos) * HD + d, o0, o1);
                            ll_store(ll_kv + rr, kv::round(o0), tag);
                            ll_store(ll_kv + rr + 1, kv::round(o1), tag);
                        }
                    } else {
                        const int rr = r - NQ - NKV;
                        const int h = rr / HD, d = rr % HD;
                        kv::store2(vc + (((size_t)h) * a.max_seq + pos) * HD + d, r0, r1);
                        ll_store(ll_kv + NKV + rr, kv::round(r0), tag);
                        ll_store(ll_kv + NKV + rr + 1, kv::round(r1), tag);
                    }
                }
            }

            /* ---------------- ATTN ---------------- */
            if (my_att >= 0 && as < S) {
                const int h = ah, kvh = akvh;
                const int dq = lane % G;
                const int p0 = as * CH, p1 = min(ctx, p0 + CH);
                const int npass = (p1 - p0 + PASS - 1) / PASS;   /* uniform over the group */
                const float scale = 1.0f / sqrtf((float)HD);
                /* q of this head: 8 dims per lane */
                float qf[8];
                bool ok = true;
                {
                    u64 qw[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) qw[j] = ll_load(ll_q + h * HD + dq * 8 + j);
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        LL_WAIT(ok, qw[j], ll_q + h * HD + dq * 8 + j, tag, a.err);
                        qf[j] = ll_val(qw[j]);
                    }
                }
                float m = -INFINITY, lsum = 0.f, o[8];
#pragma unroll
                for (int j = 0; j < 8; j++) o[j] = 0.f;
                for (int pass = 0; pass < npass; pass++) {
                    const int p = p0 + pass * PASS + wave * PPW + lane / G;
                    if (pass > 0) {
#pragma unroll
                        for (int j = 0; j < 8; j++) { kf[j] = 0.f; vf[j] = 0.f; }
                        if (p < pos) {
                            const size_t off = (((size_t)kvh) * a.max_seq + p) * HD + dq * 8;
                            kv::load8(kc + off, kf);
                            kv::load8(vc + off, vf);
                        }
                    }
                    if (p == pos) {
                        /* current position: K/V from this step's tagged words */
                        u64 kw[8], vw[8];
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            kw[j] = ll_load(ll_kv + kvh * HD + dq * 8 + j);
                            vw[j] = ll_load(ll_kv + NKV + kvh * HD + dq * 8 + j);
                        }
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            LL_WAIT(ok, kw[j], ll_kv + kvh * HD + dq * 8 + j, tag, a.err);
                            LL_WAIT(ok, vw[j], ll_kv + NKV + kvh * HD + dq * 8 + j, tag, a.err);
                            kf[j] = ll_val(kw[j]);
                            vf[j] = ll_val(vw[j]);
                        }
                    }
                    const bool valid = p < p1;
                    float d = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; j++) d = fmaf(qf[j], kf[j], d);
#pragma unroll
                    for (int off = 1; off < G; off <<= 1) d += __shfl_xor(d, off, 64);
                    const float sc = valid ? d * scale : -INFINITY;   /* forward.h:84 */
                    float tmax = sc;
#pragma unroll
                    for (int off = G; off < 64; off <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, off, 64));
                    const float mn = fmaxf(m, tmax);               /* uniform over the wave */
                    if (mn != -INFINITY) {
                        const float corr = expf(m - mn);
                        const float e = valid ? expf(sc - mn) : 0.f;
                        lsum = lsum * corr + e;
#pragma unroll
                        for (int j = 0; j < 8; j++) o[j] = fmaf(e, vf[j], o[j] * corr);
                        m = mn;
                    }
                }
#pragma unroll
                for (int off = G; off < 64; off <<= 1) {
                    lsum += __shfl_xor(lsum, off, 64);
#pragma unroll
                    for (int j = 0; j < 8; j++) o[j] += __shfl_xor(o[j], off, 64);
                }
                if (lane < G) {
#pragma unroll
                    for (int j = 0; j < 8; j++) so[wave][dq * 8 + j] = o[j];
                }
                if (lane == 0) { sm[wave] = m; sl[wave] = lsum; }
                alive = !__syncthreads_or(!ok);
                if (!alive) break;
                if (tid < HD) {
                    float M = sm[0];
#pragma unroll
                    for (int i = 1; i < PW; i++) M = fmaxf(M, sm[i]);
                    float Ls = 0.f, acc = 0.f;
#pragma unroll
                    for (int i = 0; i < PW; i++) {
                        const float f = sm[i] == -INFINITY ? 0.f : expf(sm[i] - M);
                        Ls = fmaf(sl[i], f, Ls);
                        acc = fmaf(so[i][tid], f, acc);
                    }
                    const int i0 = h * PART + as * (HD + 2);
                    ll_store_rep(ll_part, H * PART, i0 + 2 + tid, acc, tag);
                    if (tid == 0) {
                        ll_store_rep(ll_part, H * PART, i0, M, tag);
                        ll_store_rep(ll_part, H * PART, i0 + 1, Ls, tag);
                    }
                }
            }

            /* ---------------- WO ---------------- */
            load_w2(l);
            {
                /* partial words of every head's first S chunks */
                const int n = H * PART;
                const u64 *pr = ll_part + (size_t)rep * n;
                bool ok = true;
                constexpr int PPER = (NQ_MAX / HD * PART + PT - 1) / PT;
                u64 pw[PPER];
#pragma unroll
                for (int k = 0; k < PPER; k++) {
                    const int i = tid + k * PT;
                    const bool need = i < n && (i % PART) / (HD + 2) < S;
                    pw[k] = need ? ll_load(pr + i) : ((u64)tag << 32);
                }
#pragma unroll
                for (int k = 0; k < PPER; k++) {
                    const int i = tid + k * PT;
                    if (i < n && (i % PART) / (HD + 2) < S) {
                        LL_WAIT(ok, pw[k], pr + i, tag, a.err);
                        part[i] = ll_val(pw[k]);
                    }
                }
                alive = !__syncthreads_or(!ok);
                if (!alive) break;
                /* merge the chunks of each head: attn[h*HD+d] */
                for (int e = tid; e < NQ; e += PT) {
                    const int h = e / HD, d = e % HD;
                    const float *ph = part + (size_t)h * PART;
                    float M = -INFINITY;
                    for (int s = 0; s < S; s++) M = fmaxf(M, ph[s * (HD + 2)]);
                    float Ls = 0.f, acc = 0.f;
                    for (int s = 0; s < S; s++) {
                        const float f = expf(ph[s * (HD + 2)] - M);
                        Ls = fmaf(ph[s * (HD + 2) + 1], f, Ls);
                        acc = fmaf(ph[s * (HD + 2) + 2 + d], f, acc);
                    }
                    xs[e] = acc / Ls;
                }
                __syncthreads();
                if (has_op) {
                    float acc = hrow_dot<D>(wo, xs, hl);
                    acc = half_wave_sum(acc);
                    const float r0 = readlane_f(acc, 31), r1 = readlane_f(acc, 63);
                    const int r = 2 * op;
                    if (lane == 0) {
                        ll_store_rep(ll_xwo, D, r, x_in[r] + r0, tag);
                        ll_store_rep(ll_xwo, D, r + 1, x_in[r + 1] + r1, tag);
                    }
                }
            }

            /* ---------------- W13 ---------------- */
            if (l + 1 < L) load_qkv(l + 1);
            alive = ll_fetch<DPER>(ll_xwo + (size_t)rep * D, D, tag, x_mid, a.err);
            if (!alive) break;
            lds_rmsnorm<D>(x_mid, gf, xs, red);
            if (has_gi) {
                float acc = hrow_dot<D>(w13, xs, hl);
                acc = half_wave_sum(acc);
                const float h1 = readlane_f(acc, 31), h3 = readlane_f(acc, 63);
                if (lane == 0) {
                    const float silu = h1 / (1.0f + expf(-h1));   /* forward.h:101 */
                    ll_store_rep(ll_g, F, gi, silu * h3, tag);    /* forward.h:151 */
                }
            }

            /* ---------------- W2 ---------------- */
            if (l + 1 < L) load_wo(l + 1);
            alive = ll_fetch<FPER>(ll_g + (size_t)rep * F, F, tag, xs, a.err);
            if (!alive) break;
            if (has_r2) {
                float acc = wrow_dot<F>(w2, xs, lane);
                acc = wave_sum(acc);
                if (lane == 0) ll_store_rep(ll_xw2, D, r2, x_mid[r2] + acc, tag);
            }
        }
        if (!alive) break;

        /* ---------------- CLS ---------------- */
        {
            constexpr int RPR = 2 * PW;                       /* rows per round (half-waves) */
            const int rows = (V - w + NWG - 1) / NWG;         /* rows r = w + k*NWG          */
            const int rounds = (rows + RPR - 1) / RPR;
            uint4 c0[CD], c1[CD];
            auto cls_load = [&](int rd, uint4 *dst) {
                const int k = rd * RPR + wave * 2 + half;
                const int r = min(w + k * NWG, V - 1);
                hrow_load<D>(a.wcls + (size_t)r * D, hl, dst);
            };
            float bv = -INFINITY;
            int bi = 0x7FFFFFFF;
            auto cls_row = [&](int rd, const uint4 *src) {
                float acc = hrow_dot<D>(src, xs, hl);
                acc = half_wave_sum(acc);
                const int k = rd * RPR + wave * 2 + half;
                const int r = w + k * NWG;
                const float v0 = readlane_f(acc, 31), v1 = readlane_f(acc, 63);
                const float mine = half ? v1 : v0;
                if (k < rows) {
                    argmax_combine(bv, bi, mine, r);
                    if (a.logits && hl == 0) a.logits[r] = mine;
                }
            };
            cls_load(0, c0);
            float gfin[DPER];
            gains_load<D>(a.rms_final, gfin);
            alive = ll_fetch<DPER>(a.ll + (size_t)(L - 1) * LLW + (LLW - (size_t)NREP * D) +
                                       (size_t)(w % NREP) * D, D, tag, x_in, a.err);
            if (!alive) break;
            lds_rmsnorm<D>(x_in, gfin, xs, red);
            for (int rd = 0; rd < rounds; rd += 2) {
                if (rd + 1 < rounds) cls_load(rd + 1, c1);
                cls_row(rd, c0);
                if (rd + 1 < rounds) {
                    if (rd + 2 < rounds) cls_load(rd + 2, c0);
                    cls_row(rd + 1, c1);
                }
            }
            /* work-group argmax: lanes 0 and 32 hold their half's best */
            if (hl == 0) { cls_v[wave * 2 + half] = bv; cls_i[wave * 2 + half] = bi; }
            __syncthreads();
            if (tid == 0) {
                float v = cls_v[0];
                int id = cls_i[0];
                for (int i = 1; i < 2 * PW; i++) argmax_combine(v, id, cls_v[i], cls_i[i]);
                ll_store_rep(cls_ll, 2 * NWG, 2 * w, v, tag);
                ll_store_rep(cls_ll, 2 * NWG, 2 * w + 1, __int_as_float(id), tag);
            }
            /* next step's first weights, then every work-group reduces the partials */
            load_qkv(0);
            load_wo(0);
            alive = ll_fetch<(2 * 256 + PT - 1) / PT>(cls_ll + (size_t)(w % NREP) * 2 * NWG, 2 * NWG,
                                                      tag, xs, a.err);
            if (!alive) break;
            float v = -INFINITY;
            int id = 0x7FFFFFFF;
            for (int i = tid; i < NWG; i += PT) argmax_combine(v, id, xs[2 * i], __float_as_int(xs[2 * i + 1]));
            for (int off = 32; off > 0; off >>= 1) {
                const float ov = __shfl_xor(v, off, 64);
                const int oi = __shfl_xor(id, off, 64);
                argmax_combine(v, id, ov, oi);
            }
            if (lane == 0) { cls_v[wave] = v; cls_i[wave] = id; }
            __syncthreads();
            v = cls_v[0];
            id = cls_i[0];
            for (int i = 1; i < PW; i++) argmax_combine(v, id, cls_v[i], cls_i[i]);
            if (id == 0x7FFFFFFF) id = 0;
            tok = id;
            if (w == 0 && tid == 0) a.out_tok[step] = tok;
            __syncthreads();
        }
    }
    if (w == 0 && tid == 0) {
        *a.state_tok = tok;
        *a.state_pos = a.pos0 + a.n_steps;
    }
}

/* ============================== launcher =================================== */

extern "C" size_t lmk_persist_ll_words(int D, int F, int L, int H, int Hkv, int hd, int grid)
{
    return (size_t)L * ll_layer_words(D, F, H, Hkv, hd) + (size_t)NREP * 2 * grid;
}

extern "C" int lmk_persist_grid(void)
{
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return ncu < 256 ? ncu : 256;
}

extern "C" int lmk_persist_supported(int D, int F, int hd, int H)
{
    const bool shape = (D == 768 && F == 2048 && hd == 64) || (D == 256 && F == 512 && hd == 64) ||
                       (D == 512 && F == 1024 && hd == 128);
    return shape && H * SMAX <= lmk_persist_grid() && D <= 2 * lmk_persist_grid() * PW;
}

extern "C" int lmk_decode_persist(hipStream_t s, const LMPersistArgs *p)
{
    PDArgs a;
    a.layers = p->layers; a.layer_elems = p->layer_elems; a.off_wo = p->off_wo;
    a.off_w13 = p->off_w13; a.off_w2 = p->off_w2;
    a.embed = p->embed; a.wcls = p->wcls;
    a.rms_att = p->rms_att; a.rms_ffn = p->rms_ffn; a.rms_final = p->rms_final;
    a.rope_cos = p->rope_cos; a.rope_sin = p->rope_sin;
    a.kc = p->kc; a.vc = p->vc; a.kv_layer_elems = p->kv_layer_elems;
    a.ll = (u64 *)p->ll; a.logits = p->logits; a.out_tok = p->out_tok;
    a.state_tok = p->state_tok; a.state_pos = p->state_pos; a.err = p->err;
    a.V = p->V; a.L = p->L; a.H = p->H; a.Hkv = p->Hkv; a.max_seq = p->max_seq;
    a.tok0 = p->tok0; a.pos0 = p->pos0; a.n_steps = p->n_steps; a.tag0 = p->tag0;
    const int grid = p->grid;
    if (grid < 1 || grid > lmk_persist_grid() || a.H * SMAX > grid || a.n_steps < 1 ||
        a.pos0 < 0 || a.pos0 + a.n_steps > a.max_seq || a.tok0 < 0 || a.tok0 >= a.V ||
        a.H % a.Hkv || a.max_seq > 64 * SMAX * 16)
        return hipErrorInvalidValue;
    void *args[] = {&a};
#define LAUNCH_PD(D_, F_, HD_)                                                                  \
    do {                                                                                        \
        if (p->kv_f32)                                                                          \
            return hipLaunchCooperativeKernel((const void *)k_decode_persist<D_, F_, HD_, float>, \
                                              dim3(grid), dim3(PT), args, 0, s);                \
        return hipLaunchCooperativeKernel((const void *)k_decode_persist<D_, F_, HD_, u16>,     \
                                          dim3(grid), dim3(PT), args, 0, s);                    \
    } while (0)
    const int D = p->D, F = p->F, hd = p->hd;
    if (a.H * hd != D) return hipErrorInvalidValue;
    if (D == 768 && F == 2048 && hd == 64) LAUNCH_PD(768, 2048, 64);
    if (D == 256 && F == 512 && hd == 64) LAUNCH_PD(256, 512, 64);
    if (D == 512 && F == 1024 && hd == 128) LAUNCH_PD(512, 1024, 128);
#undef LAUNCH_PD
    return hipErrorInvalidValue;
}
