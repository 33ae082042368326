/*
 * k_gemm.hip — fp16 MFMA GEMMs with fused epilogues for prefill and batched
 * decode (gfx950, v_mfma_f32_32x32x16_f16, fp32 accumulation).
 *
 *   C[m, n] = sum_k A[m, k] * W[n, k]      (y = W x per row, forward.h:36-44)
 *
 * W is an fp16 weight matrix [N, K] (row-major, K contiguous), A the
 * activations [M, lda]: fp16, or fp32 converted to fp16 while staging, with the
 * RMSNorm of forward.h:46-53 applied on the way (A * rstd[m] * gain[k]) so a
 * normalised copy of x is never written.  Epilogues (one per call site of
 * forward.h:104-170):
 *   EPI_STORE  logits [M, ldc] fp32 (optional) and per-32-column argmax partials
 *   EPI_RESID  x[m, n] += C                          (forward.h:136, 159)
 *   EPI_GATE   g[m, i] = silu(h1) * h3 in fp16; W1/W3 rows interleaved in
 *              blocks of 16, so h3 sits 16 columns right of h1 (forward.h:149-151)
 *   EPI_QKV    RoPE on q/k column pairs (forward.h:55-70); q -> fp32 [M, NQ];
 *              k, v -> the K/V cache at (slot[m], pos[m])
 *
 * MFMA lane layout (checked on the device): for a 32x32x16 step lane l holds
 * A[l%32][8*(l/32) .. +8], B[8*(l/32) .. +8][l%32] (= W[n0 + l%32][k ..]), and
 * accumulator i holds C[8*(i/4) + 4*(l/32) + i%4][l%32].
 *
 * Two tilings:
 *   k_gemm_tile    M > 64 rows: work-group tile BM x BN, four waves 2 x 2, K
 *                  staged through double-buffered LDS in steps of 64
 *   k_gemm_skinny  M <= 64 rows (decode batches): a work-group owns 32 columns
 *                  and all rows; its four waves split K, stream their weight
 *                  fragments straight from HBM into registers (each weight byte
 *                  read once) and add their partial tiles through LDS.
 */
#include <type_traits>

#include "k_common.h"
#include "lm_internal.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));

/* Compile-time loop: f(std::integral_constant<int, i>) for i in [I, N), so
 * register arrays are only ever indexed by constants. */
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

#define GT 256                    /* threads per work-group */

/* ---- operand staging ------------------------------------------------------- */

/* 8 consecutive A elements of row m from k0 as fp16 bits (uint4). */
template <typename AT, bool NORM>
__device__ __forceinline__ uint4 load_a8(const AT *__restrict__ A, int lda, int m, int k0,
                                         const float *__restrict__ rstd,
                                         const float *__restrict__ gain);

template <>
__device__ __forceinline__ uint4 load_a8<u16, false>(const u16 *__restrict__ A, int lda, int m,
                                                     int k0, const float *, const float *)
{
    return *(const uint4 *)(A + (size_t)m * lda + k0);
}

template <bool NORM>
__device__ __forceinline__ uint4 cvt_a8(const float f[8], float rs, const float *__restrict__ gain,
                                        int k0)
{
    f16x8 h;
    if (NORM) {
        const float4 g0 = *(const float4 *)(gain + k0), g1 = *(const float4 *)(gain + k0 + 4);
        h[0] = (_Float16)(f[0] * rs * g0.x); h[1] = (_Float16)(f[1] * rs * g0.y);
        h[2] = (_Float16)(f[2] * rs * g0.z); h[3] = (_Float16)(f[3] * rs * g0.w);
        h[4] = (_Float16)(f[4] * rs * g1.x); h[5] = (_Float16)(f[5] * rs * g1.y);
        h[6] = (_Float16)(f[6] * rs * g1.z); h[7] = (_Float16)(f[7] * rs * g1.w);
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) h[j] = (_Float16)f[j];
    }
    return __builtin_bit_cast(uint4, h);
}

template <>
__device__ __forceinline__ uint4 load_a8<float, false>(const float *__restrict__ A, int lda, int m,
                                                       int k0, const float *, const float *)
{
    const float *p = A + (size_t)m * lda + k0;
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    return cvt_a8<false>(f, 1.f, nullptr, k0);
}

template <>
__device__ __forceinline__ uint4 load_a8<float, true>(const float *__restrict__ A, int lda, int m,
                                                      int k0, const float *__restrict__ rstd,
                                                      const float *__restrict__ gain)
{
    const float *p = A + (size_t)m * lda + k0;
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    return cvt_a8<true>(f, rstd[m], gain, k0);
}

__device__ __forceinline__ f32x16 mfma32(uint4 a, uint4 b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

/* ---- epilogues ------------------------------------------------------------- */

struct EpiArgs {
    int M, N;
    float *out;             /* STORE: logits [M, ldc] (may be NULL); RESID: x [M, ldc] */
    int ldc;
    LMArgPart *part;        /* STORE: argmax partial per (row, 32-col tile), may be NULL */
    int nparts;             /* partials per row (N / 32 rounded up)                      */
    u16 *g;                 /* GATE: gate [M, F] fp16 */
    int F;
    float *q;               /* QKV */
    void *kc, *vc;
    int kv_f32, NQ, NKV, hd, Hkv, max_seq;
    const int *slot, *pos;
    const float *rope_cos, *rope_sin;
};

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_GATE = 2, EPI_QKV = 3 };

/* Apply epilogue E to one 32x32 accumulator tile at (m0, n0). */
template <int E>
__device__ __forceinline__ void epilogue_tile(const f32x16 &acc, int m0, int n0, const EpiArgs &e)
{
    const int lane = threadIdx.x & 63;
    const int n = n0 + (lane & 31);
    const int rbase = m0 + 4 * (lane >> 5);
    if (E == EPI_STORE) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = rbase + 8 * (i >> 2) + (i & 3);
            float v = acc[i];
            const bool ok = r < e.M && n < e.N;
            if (ok && e.out) e.out[(size_t)r * e.ldc + n] = v;
            if (e.part) {
                /* argmax over the 32 columns of this row (lanes of one half) */
                float bv = ok ? v : -INFINITY;
                int bi = ok ? n : 0x7FFFFFFF;
#pragma unroll
                for (int off = 16; off > 0; off >>= 1) {
                    const float ov = __shfl_xor(bv, off, 64);
                    const int oi = __shfl_xor(bi, off, 64);
                    argmax_combine(bv, bi, ov, oi);
                }
                if ((lane & 31) == 0 && r < e.M && n0 < e.N)
                    e.part[(size_t)r * e.nparts + n0 / 32] = LMArgPart{bv, bi};
            }
        }
    } else if (E == EPI_RESID) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = rbase + 8 * (i >> 2) + (i & 3);
            if (r < e.M && n < e.N) e.out[(size_t)r * e.ldc + n] += acc[i];
        }
    } else if (E == EPI_GATE) {
        /* tile columns 0..15 hold W1 rows 16j.., columns 16..31 the W3 rows */
        const int c = lane & 31;
        const int gi = (n0 / 32) * 16 + (c & 15);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = rbase + 8 * (i >> 2) + (i & 3);
            const float h3 = __shfl_xor(acc[i], 16, 64);
            if (c < 16 && r < e.M && n < e.N) {
                const float h1 = acc[i];
                const float silu = h1 / (1.0f + expf(-h1));        /* forward.h:101 */
                e.g[(size_t)r * e.F + gi] = f2h(silu * h3);         /* forward.h:151 */
            }
        }
    } else {  /* EPI_QKV */
        const bool odd = n & 1;
        const bool rot = n < e.NQ + e.NKV;
        const int nn = n < e.NQ ? n : (rot ? n - e.NQ : n - e.NQ - e.NKV);
        const int h = nn / e.hd, d = nn % e.hd;
        const int half_hd = e.hd >> 1;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = rbase + 8 * (i >> 2) + (i & 3);
            const float other = __shfl_xor(acc[i], 1, 64);
            if (r >= e.M || n >= e.N) continue;
            const int p = e.pos[r];
            float v = acc[i];
            if (rot) {
                const int ti = p * half_hd + (d >> 1);
                const float c = e.rope_cos[ti], s = e.rope_sin[ti];
                /* pair (a, b) = (even column, odd column), forward.h:62-68 */
                v = odd ? fmaf(other, s, v * c) : fmaf(v, c, -(other * s));
            }
            if (n < e.NQ) {
                e.q[(size_t)r * e.NQ + n] = v;
            } else {
                const size_t off = (((size_t)e.slot[r] * e.Hkv + h) * e.max_seq + p) * e.hd + d;
                void *dst = rot ? e.kc : e.vc;
                if (e.kv_f32) ((float *)dst)[off] = v;
                else ((u16 *)dst)[off] = f2h(v);
            }
        }
    }
}

/* ---- tiled GEMM (prefill) ------------------------------------------------- */

#define BK 64        /* K per LDS stage */
#define LDS_PAD 8    /* halves of padding per LDS row (16 bytes) */

/* Three-stage pipeline: while the waves multiply stage k out of one LDS
 * buffer, stage k+1 sits in registers on its way to the other buffer and
 * stage k+2 is being fetched from memory, so a global load has two stages of
 * MFMA work to arrive. */
template <int BM, int BN, typename AT, bool NORM, int E>
__global__ void __launch_bounds__(GT) k_gemm_tile(const AT *__restrict__ A, int lda,
                                                  const float *__restrict__ rstd,
                                                  const float *__restrict__ gain,
                                                  const u16 *__restrict__ W, int K, EpiArgs e)
{
    constexpr int WM = BM / 2, WN = BN / 2;     /* wave tile */
    constexpr int TM = WM / 32, TN = WN / 32;   /* MFMA tiles per wave */
    constexpr int LR = BK + LDS_PAD;            /* LDS row stride (halves) */
    constexpr int CPR = BK / 8;                 /* 16-byte chunks per tile row */
    constexpr int ACH = BM * CPR / GT;          /* A chunks per thread */
    constexpr int BCH = BN * CPR / GT;
    static_assert(ACH >= 1 && BCH >= 1 && TM >= 1 && TN >= 1, "tile too small");
    __shared__ __attribute__((aligned(16))) u16 sa[2][BM * LR];
    __shared__ __attribute__((aligned(16))) u16 sb[2][BN * LR];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int M = e.M, N = e.N;

    uint4 ra0[ACH], rb0[BCH], ra1[ACH], rb1[BCH];
    /* register stages are named, not passed by pointer, so they stay in VGPRs */
#define GLOAD(k0_, RA, RB)                                                                 \
    do {                                                                                   \
        const int k0v_ = (k0_);                                                            \
        static_for<0, ACH>([&](auto c) {                                                   \
            const int idx = tid + c * GT;                                                  \
            const int r = min(m0 + idx / CPR, M - 1);                                      \
            RA[c] = load_a8<AT, NORM>(A, lda, r, k0v_ + (idx % CPR) * 8, rstd, gain);      \
        });                                                                                \
        static_for<0, BCH>([&](auto c) {                                                   \
            const int idx = tid + c * GT;                                                  \
            const int r = min(n0 + idx / CPR, N - 1);                                      \
            RB[c] = *(const uint4 *)(W + (size_t)r * K + k0v_ + (idx % CPR) * 8);          \
        });                                                                                \
    } while (0)
#define SSTORE(buf_, RA, RB)                                                               \
    do {                                                                                   \
        static_for<0, ACH>([&](auto c) {                                                   \
            const int idx = tid + c * GT;                                                  \
            *(uint4 *)(&sa[buf_][(idx / CPR) * LR + (idx % CPR) * 8]) = RA[c];             \
        });                                                                                \
        static_for<0, BCH>([&](auto c) {                                                   \
            const int idx = tid + c * GT;                                                  \
            *(uint4 *)(&sb[buf_][(idx / CPR) * LR + (idx % CPR) * 8]) = RB[c];             \
        });                                                                                \
    } while (0)

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (f32x16){};
    auto compute = [&](int buf) {
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            uint4 fa[TM], fb[TN];
            const int kk = ks * 16 + (lane >> 5) * 8;
#pragma unroll
            for (int i = 0; i < TM; i++)
                fa[i] = *(const uint4 *)(&sa[buf][(wm * WM + i * 32 + (lane & 31)) * LR + kk]);
#pragma unroll
            for (int j = 0; j < TN; j++)
                fb[j] = *(const uint4 *)(&sb[buf][(wn * WN + j * 32 + (lane & 31)) * LR + kk]);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = mfma32(fa[i], fb[j], acc[i][j]);
        }
    };

    const int nk = K / BK;
    GLOAD(0, ra0, rb0);
    SSTORE(0, ra0, rb0);
    if (nk > 1) GLOAD(BK, ra1, rb1);
    __syncthreads();
    for (int kt = 0; kt < nk; kt += 2) {
        /* stage kt from buffer 0; registers 1 hold stage kt+1 */
        if (kt + 2 < nk) GLOAD((kt + 2) * BK, ra0, rb0);
        compute(0);
        if (kt + 1 < nk) {
            SSTORE(1, ra1, rb1);
            __syncthreads();
            /* stage kt+1 from buffer 1; registers 0 hold stage kt+2 */
            if (kt + 3 < nk) GLOAD((kt + 3) * BK, ra1, rb1);
            compute(1);
            if (kt + 2 < nk) {
                SSTORE(0, ra0, rb0);
                __syncthreads();
            }
        }
    }
#undef GLOAD
#undef SSTORE
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            epilogue_tile<E>(acc[i][j], m0 + wm * WM + i * 32, n0 + wn * WN + j * 32, e);
}

/* ---- skinny GEMM (decode batches, M <= 64) ---------------------------------- */

#define SK_STEPS 8   /* k-steps of 16 fetched per pipeline stage */

template <int MT, typename AT, bool NORM, int E>
__global__ void __launch_bounds__(GT) k_gemm_skinny(const AT *__restrict__ A, int lda,
                                                    const float *__restrict__ rstd,
                                                    const float *__restrict__ gain,
                                                    const u16 *__restrict__ W, int K, EpiArgs e)
{
    __shared__ float red[3][MT * 16][64];
    /* MFMA instructions execute whatever the EXEC mask says, so every branch
     * around them must be wave-uniform in the compiler's eyes: the wave index
     * goes through readfirstlane and all K-range tests become scalar branches */
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * 32;
    const int M = e.M, N = e.N;
    const int nsteps = K / 16;                    /* k-steps of the whole row      */
    const int per = (nsteps + 3) / 4;             /* k-steps of this wave's slice  */
    const int s0 = wave * per, s1 = min(nsteps, s0 + per);
    const int wrow = min(n0 + (lane & 31), N - 1);
    const int koff = (lane >> 5) * 8;
    const u16 *wp = W + (size_t)wrow * K + koff;
    int arow[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) arow[i] = min(i * 32 + (lane & 31), M - 1);

    f32x16 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i] = (f32x16){};

    uint4 fb[2][SK_STEPS], fa[2][SK_STEPS][MT];
    auto fetch = [&](int st, int b) {
#pragma unroll
        for (int j = 0; j < SK_STEPS; j++) {
            const int s = st + j;
            if (s < s1) {
                fb[b][j] = *(const uint4 *)(wp + s * 16);
#pragma unroll
                for (int i = 0; i < MT; i++)
                    fa[b][j][i] = load_a8<AT, NORM>(A, lda, arow[i], s * 16 + koff, rstd, gain);
            }
        }
    };
    auto consume = [&](int st, int b) {
#pragma unroll
        for (int j = 0; j < SK_STEPS; j++)
            if (st + j < s1)
#pragma unroll
                for (int i = 0; i < MT; i++) acc[i] = mfma32(fa[b][j][i], fb[b][j], acc[i]);
    };
    if (s0 < s1) {
        fetch(s0, 0);
        for (int st = s0; st < s1; st += 2 * SK_STEPS) {
            if (st + SK_STEPS < s1) fetch(st + SK_STEPS, 1);
            consume(st, 0);
            if (st + SK_STEPS < s1) {
                if (st + 2 * SK_STEPS < s1) fetch(st + 2 * SK_STEPS, 0);
                consume(st + SK_STEPS, 1);
            }
        }
    }
    /* sum the four waves' partial tiles */
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int v = 0; v < 16; v++) red[wave - 1][i * 16 + v][lane] = acc[i][v];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < MT; i++) {
#pragma unroll
            for (int v = 0; v < 16; v++)
                acc[i][v] += red[0][i * 16 + v][lane] + red[1][i * 16 + v][lane] +
                             red[2][i * 16 + v][lane];
            epilogue_tile<E>(acc[i], i * 32, n0, e);
        }
    }
}

/* ---- per-row RMSNorm ------------------------------------------------------------ */

/* One wave per row m (forward.h:46-53): with emb != NULL the row is first set
 * to the fp16 embedding row emb[tok[m]] (forward.h:108-110); then
 * xn[m, k] = fp16(x[m, k] * (1/sqrt(mean(x[m]^2) + 1e-5)) * gain[k]), the GEMM
 * operand of the projection that follows.  The row stays in registers
 * (D/64 values per lane). */
template <int D>
__global__ void __launch_bounds__(GT) k_rownorm(float *__restrict__ x, int M,
                                                const u16 *__restrict__ emb,
                                                const int *__restrict__ tok,
                                                const float *__restrict__ gain,
                                                u16 *__restrict__ xn)
{
    constexpr int PER = D / 64;              /* values per lane, in chunks of 4 */
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * (GT / 64) + (threadIdx.x >> 6);
    if (m >= M) return;
    float *xr = x + (size_t)m * D;
    float v[PER];
    if (emb) {
        const u16 *er = emb + (size_t)tok[m] * D;
#pragma unroll
        for (int c = 0; c < PER / 4; c++) {
            const uint2 h = *(const uint2 *)(er + c * 256 + lane * 4);
            const f16x2 a = __builtin_bit_cast(f16x2, h.x), b = __builtin_bit_cast(f16x2, h.y);
            v[4 * c] = (float)a.x; v[4 * c + 1] = (float)a.y;
            v[4 * c + 2] = (float)b.x; v[4 * c + 3] = (float)b.y;
            *(float4 *)(xr + c * 256 + lane * 4) = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2],
                                                               v[4 * c + 3]);
        }
    } else {
#pragma unroll
        for (int c = 0; c < PER / 4; c++) {
            const float4 t = *(const float4 *)(xr + c * 256 + lane * 4);
            v[4 * c] = t.x; v[4 * c + 1] = t.y; v[4 * c + 2] = t.z; v[4 * c + 3] = t.w;
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; i++) ss = fmaf(v[i], v[i], ss);
    ss = wave_sum(ss);
    const float rs = 1.0f / sqrtf(ss / D + 1e-5f);
    u16 *xo = xn + (size_t)m * D;
#pragma unroll
    for (int c = 0; c < PER / 4; c++) {
        const float4 g = *(const float4 *)(gain + c * 256 + lane * 4);
        const unsigned lo = (unsigned)f2h(v[4 * c] * rs * g.x) | ((unsigned)f2h(v[4 * c + 1] * rs * g.y) << 16);
        const unsigned hi = (unsigned)f2h(v[4 * c + 2] * rs * g.z) | ((unsigned)f2h(v[4 * c + 3] * rs * g.w) << 16);
        *(uint2 *)(xo + c * 256 + lane * 4) = make_uint2(lo, hi);
    }
}

/* ============================== launchers =================================== */

extern "C" int lmk_rownorm(hipStream_t s, float *x, int D, int M, const uint16_t *emb, const int *tok,
                           const float *gain, uint16_t *xn)
{
    if (M < 1 || (emb && !tok) || !gain || !xn) return hipErrorInvalidValue;
    dim3 grid((M + 3) / 4);
    switch (D) {
    case 256: hipLaunchKernelGGL(k_rownorm<256>, grid, dim3(GT), 0, s, x, M, emb, tok, gain, xn); break;
    case 512: hipLaunchKernelGGL(k_rownorm<512>, grid, dim3(GT), 0, s, x, M, emb, tok, gain, xn); break;
    case 768: hipLaunchKernelGGL(k_rownorm<768>, grid, dim3(GT), 0, s, x, M, emb, tok, gain, xn); break;
    case 1024: hipLaunchKernelGGL(k_rownorm<1024>, grid, dim3(GT), 0, s, x, M, emb, tok, gain, xn); break;
    case 2048: hipLaunchKernelGGL(k_rownorm<2048>, grid, dim3(GT), 0, s, x, M, emb, tok, gain, xn); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

static EpiArgs to_epi(const LMEpilogue *p, int M, int N)
{
    EpiArgs e;
    e.M = M; e.N = N;
    e.out = p->out; e.ldc = p->ldc; e.part = p->part; e.nparts = (N + 31) / 32;
    e.g = (u16 *)p->g; e.F = p->F;
    e.q = p->q; e.kc = p->kc; e.vc = p->vc; e.kv_f32 = p->kv_f32;
    e.NQ = p->NQ; e.NKV = p->NKV; e.hd = p->hd; e.Hkv = p->Hkv; e.max_seq = p->max_seq;
    e.slot = p->slot; e.pos = p->pos; e.rope_cos = p->rope_cos; e.rope_sin = p->rope_sin;
    return e;
}

template <typename AT, bool NORM, int E>
static int launch_gemm(hipStream_t s, const void *A, int lda, const float *rstd, const float *gain,
                       const uint16_t *W, int M, int N, int K, const EpiArgs &e)
{
    if (M <= 64) {
        dim3 grid((N + 31) / 32);
        if (M <= 32)
            hipLaunchKernelGGL((k_gemm_skinny<1, AT, NORM, E>), grid, dim3(GT), 0, s, (const AT *)A,
                               lda, rstd, gain, W, K, e);
        else
            hipLaunchKernelGGL((k_gemm_skinny<2, AT, NORM, E>), grid, dim3(GT), 0, s, (const AT *)A,
                               lda, rstd, gain, W, K, e);
        return hipGetLastError();
    }
    /* prefill tiles: the largest of 128x128, 128x64, 64x64 that still gives
     * the 256 CUs a work-group each (small M or narrow N take smaller tiles) */
    const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    const long t12864 = (long)((M + 127) / 128) * ((N + 63) / 64);
    if (t128 >= 256 || (K % BK)) {
        if (K % BK) return hipErrorInvalidValue;
        dim3 grid((M + 127) / 128, (N + 127) / 128);
        hipLaunchKernelGGL((k_gemm_tile<128, 128, AT, NORM, E>), grid, dim3(GT), 0, s,
                           (const AT *)A, lda, rstd, gain, W, K, e);
    } else if (t12864 >= 256) {
        dim3 grid((M + 127) / 128, (N + 63) / 64);
        hipLaunchKernelGGL((k_gemm_tile<128, 64, AT, NORM, E>), grid, dim3(GT), 0, s,
                           (const AT *)A, lda, rstd, gain, W, K, e);
    } else {
        dim3 grid((M + 63) / 64, (N + 63) / 64);
        hipLaunchKernelGGL((k_gemm_tile<64, 64, AT, NORM, E>), grid, dim3(GT), 0, s,
                           (const AT *)A, lda, rstd, gain, W, K, e);
    }
    return hipGetLastError();
}

extern "C" int lmk_gemm(hipStream_t s, int a_kind, const void *A, int lda, const float *rstd,
                        const float *gain, const uint16_t *W, int M, int N, int K, int epi,
                        const LMEpilogue *ep)
{
    if (M < 1 || N < 1 || K < 32 || K % 32 || lda < K || !A || !W || !ep) return hipErrorInvalidValue;
    if (a_kind == LMK_A_F32_NORM && (!rstd || !gain)) return hipErrorInvalidValue;
    if (epi == EPI_GATE && (N % 32 || !ep->g)) return hipErrorInvalidValue;
    if (epi == EPI_QKV && (!ep->q || !ep->kc || !ep->vc || !ep->slot || !ep->pos || (ep->hd & 1) ||
                           N != ep->NQ + 2 * ep->NKV))
        return hipErrorInvalidValue;
    if (epi == EPI_RESID && (!ep->out || ep->ldc < N)) return hipErrorInvalidValue;
    if (epi == EPI_STORE && ep->out && ep->ldc < N) return hipErrorInvalidValue;
    const EpiArgs e = to_epi(ep, M, N);
#define BY_EPI(AT_, NORM_)                                                                        \
    switch (epi) {                                                                                \
    case EPI_STORE: return launch_gemm<AT_, NORM_, EPI_STORE>(s, A, lda, rstd, gain, W, M, N, K, e); \
    case EPI_RESID: return launch_gemm<AT_, NORM_, EPI_RESID>(s, A, lda, rstd, gain, W, M, N, K, e); \
    case EPI_GATE: return launch_gemm<AT_, NORM_, EPI_GATE>(s, A, lda, rstd, gain, W, M, N, K, e);   \
    case EPI_QKV: return launch_gemm<AT_, NORM_, EPI_QKV>(s, A, lda, rstd, gain, W, M, N, K, e);     \
    default: return hipErrorInvalidValue;                                                         \
    }
    switch (a_kind) {
    case LMK_A_F16: BY_EPI(u16, false);
    case LMK_A_F32: BY_EPI(float, false);
    case LMK_A_F32_NORM: BY_EPI(float, true);
    default: return hipErrorInvalidValue;
    }
#undef BY_EPI
}
