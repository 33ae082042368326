/*
 * k_gemm.hip — fp16 MFMA GEMMs with fused epilogues for prefill and batched
 * decode (gfx950, v_mfma_f32_32x32x16_f16, fp32 accumulation).
 *
 *   C[m, n] = sum_k A[m, k] * W[n, k]      (y = W x per row, forward.h:36-44)
 *
 * W is an fp16 weight matrix [N, K] (row-major, K contiguous), A the fp16
 * activations [M, lda] (normalised rows, attention output or gate, each written
 * once by the kernel that produces it).  Epilogues (one per call site of
 * forward.h:104-170):
 *   EPI_STORE  logits [M, ldc] fp32
 *   EPI_ARGMAX logits (optional) and per-32-column argmax partials (greedy decode)
 *   EPI_RESID  x[m, n] += C                          (forward.h:136, 159)
 *   EPI_GATE   g[m, i] = silu(h1) * h3 in fp16; W1/W3 rows interleaved in
 *              blocks of 16, so h3 sits 16 columns right of h1 (forward.h:149-151)
 *   EPI_QKV    RoPE on q/k column pairs (forward.h:55-70); q -> fp32 [M, NQ];
 *              k, v -> the K/V cache at (slot[m], pos[m])
 *   EPI_RESNORM x[m, n] += C (forward.h:136, 159), u[m, n] = fp16(x[m, n] *
 *              gain[n]) and the sum of x[m, n]^2 over each row's 32 columns:
 *              the RMSNorm of x (forward.h:46-53) finished by the GEMM that
 *              reads u, which scales its product row m by 1/sqrt(mean + 1e-5)
 *              (rs_ss) before its own epilogue
 *
 * MFMA lane layout (checked on the device): for a 32x32x16 step lane l holds
 * A[l%32][8*(l/32) .. +8], B[8*(l/32) .. +8][l%32] (= W[n0 + l%32][k ..]), and
 * accumulator i holds C[8*(i/4) + 4*(l/32) + i%4][l%32].
 *
 * Kernels:
 *   k_gemm_tile    work-group tile BM x BN: 64 x 64 for most shapes (four waves
 *                  2 x 2), 256 x 128 for the largest (eight waves 4 x 2), 128 x 128
 *                  (eight waves) K-split in 2 for long-K narrow GEMMs of 1024+
 *                  rows, 64 x 64 also for decode-row classifiers, 32 x 64 for up to
 *                  32 rows (two waves), 32 x 32 (one wave) for decode-row gate
 *                  GEMMs of few tiles; K streamed by direct global->LDS loads into a ring of
 *                  64-wide stages (3 deep for prefill, 4 for decode rows, 6 for
 *                  32-row gate tiles); XCD-aware tile order; an optional K-split
 *                  over blockIdx.y (fp32 partials, summed by the kernel that
 *                  next reads them)
 *   k_rownorm      row norm with the residual add of pending partials, one wave
 *                  per row (from 512 rows); k_rownorm_blk, one work-group per
 *                  row, below that
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
    int lghd;               /* QKV: log2(hd) (hd is a power of two) */
    const int *slot, *pos;
    const float *rope_cos, *rope_sin;
    size_t sstride;         /* STORE of a K-split GEMM: out of split s is out + s*sstride */
    int nt;                 /* STORE / ARGMAX: non-temporal stores of out */
    const float *gain;      /* RESNORM: gain [N]; u [M, N] fp16; ss [M, nss] */
    u16 *u;
    float *ss;
    int *ovf;               /* RESNORM: set when a u value overflows fp16 (may be NULL) */
    const float *rs_ss;     /* STORE / GATE / QKV: row sums of squares [M, nss] of the
                             * RESNORM that wrote A, or NULL */
    int nss;
};

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_GATE = 2, EPI_QKV = 3, EPI_ARGMAX = 4, EPI_RESNORM = 5 };

/* Apply epilogue E to one 32x32 accumulator tile at (m0, n0).  Every operand
 * the epilogue reads (residual, positions, rotation angles) is loaded for the
 * whole tile before the first store: stores the compiler cannot prove disjoint
 * from those loads would otherwise serialise one memory round trip per element.
 * xpre: the tile's residual values (RESID, RESNORM) and, after them, the
 * lane's gain (RESNORM), loaded before the main loop, or nullptr to load them
 * here. */
template <int E>
__device__ __forceinline__ void epilogue_tile(const f32x16 &acc, int m0, int n0, const EpiArgs &e,
                                              const float *xpre = nullptr)
{
    const int lane = threadIdx.x & 63;
    const int n = n0 + (lane & 31);
    const int rbase = m0 + 4 * (lane >> 5);
    int rr[16];
    bool ok[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        rr[i] = rbase + 8 * (i >> 2) + (i & 3);
        ok[i] = rr[i] < e.M && n < e.N;
    }
    if (E == EPI_STORE || E == EPI_ARGMAX) {
        if (e.out && e.nt) {   /* logits: streamed past the caches */
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (ok[i]) __builtin_nontemporal_store(acc[i], &e.out[(size_t)rr[i] * e.ldc + n]);
        } else if (e.out) {
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (ok[i]) e.out[(size_t)rr[i] * e.ldc + n] = acc[i];
        }
        if (E == EPI_ARGMAX) {
            /* argmax over the 32 columns of each row (the lanes of one half),
             * with DPP moves: lanes 31 and 63 end up with their half's result */
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float bv = ok[i] ? acc[i] : -INFINITY;
                int bi = ok[i] ? n : 0x7FFFFFFF;
                half_wave_argmax(bv, bi);
                if ((lane & 31) == 31 && rr[i] < e.M && n0 < e.N)
                    e.part[(size_t)rr[i] * e.nparts + n0 / 32] = LMArgPart{bv, bi};
            }
        }
    } else if (E == EPI_RESID) {
        float xv[16];
#pragma unroll
        for (int i = 0; i < 16; i++) xv[i] = xpre ? xpre[i] : ok[i] ? e.out[(size_t)rr[i] * e.ldc + n] : 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (ok[i]) e.out[(size_t)rr[i] * e.ldc + n] = xv[i] + acc[i];
    } else if (E == EPI_RESNORM) {
        /* the residual add, the gained fp16 row for the next GEMM, and each
         * row's sum of squares over this tile's 32 columns (N is a multiple
         * of 32) */
        float xv[16];
#pragma unroll
        for (int i = 0; i < 16; i++) xv[i] = xpre ? xpre[i] : ok[i] ? e.out[(size_t)rr[i] * e.ldc + n] : 0.f;
        const float gn = xpre ? xpre[16] : n < e.N ? e.gain[n] : 0.f;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = xv[i] + acc[i];
        /* u is rounded before the row is normalised: a |x * gain| that fp16
         * cannot hold (65520 and up round to infinity; NaN too) is reported,
         * and the caller redoes the rows with the row norm apart */
        bool big = false;
#pragma unroll
        for (int i = 0; i < 16; i++) big |= ok[i] && !(fabsf(v[i] * gn) < 65520.f);
        if (big && e.ovf) *e.ovf = 1;
        if (m0 + 32 <= e.M && n0 + 32 <= e.N) {   /* whole tile: no per-element masks */
#pragma unroll
            for (int i = 0; i < 16; i++) {
                e.out[(size_t)rr[i] * e.ldc + n] = v[i];
                e.u[(size_t)rr[i] * e.N + n] = f2h(v[i] * gn);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (ok[i]) {
                    e.out[(size_t)rr[i] * e.ldc + n] = v[i];
                    e.u[(size_t)rr[i] * e.N + n] = f2h(v[i] * gn);
                }
        }
        /* Row sums over the 32 lanes of each half by reduce-scatter: at the
         * stage of offset o each lane keeps half of its remaining sums (the
         * upper half where lane & o) and adds the partner's copy of them, so
         * after the offsets 16, 8, 4, 2 and a last add over offset 1, lane l
         * holds the sum of row index (l & 31) >> 1 of its half. */
        float q[16];
#pragma unroll
        for (int i = 0; i < 16; i++) q[i] = ok[i] ? v[i] * v[i] : 0.f;
        static_for<0, 4>([&](auto S) {
            constexpr int o = 16 >> decltype(S)::value, c = 8 >> decltype(S)::value;
            const bool hi = lane & o;
#pragma unroll
            for (int j = 0; j < c; j++) {
                const float keep = hi ? q[j + c] : q[j], give = hi ? q[j] : q[j + c];
                q[j] = keep + __shfl_xor(give, o, 64);
            }
        });
        q[0] += __shfl_xor(q[0], 1, 64);
        const int ri = (lane & 31) >> 1;
        const int row = rbase + 8 * (ri >> 2) + (ri & 3);
        if (!(lane & 1) && row < e.M && n0 < e.N) e.ss[(size_t)row * e.nss + n0 / 32] = q[0];
    } else if (E == EPI_GATE) {
        /* tile columns 0..15 hold W1 rows 16j.., columns 16..31 the W3 rows */
        /* rows rr[i], rr[i+1] (i even) of gate index gi: lane c < 16 takes row
         * rr[i] (h1 its own, h3 from lane c + 16), lane c + 16 takes row rr[i+1]
         * (h3 its own, h1 from lane c), so every lane evaluates one gate per pair.
         * sigmoid(h1) = 1/(1 + e^-h1) with the hardware exp2 and reciprocal
         * (about 1 ulp each in fp32); the gate is rounded to fp16 afterwards. */
        const int c = lane & 31;
        const bool lo = c < 16;
        const int gi = (n0 / 32) * 16 + (c & 15);
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            /* the empty asm keeps a lane-dependent select between the two
             * elements from becoming a 16-way select over the vector */
            float a0 = acc[i], a1 = acc[i + 1];
            asm("" : "+v"(a0), "+v"(a1));
            const float other = xor16_f(lo ? a1 : a0);
            const float h1 = lo ? a0 : other;
            const float h3 = lo ? other : a1;
            const int r = lo ? rr[i] : rr[i + 1];
            const bool okr = lo ? ok[i] : ok[i + 1];
            const float ex = __builtin_amdgcn_exp2f(-h1 * 1.4426950408889634f);
            const float silu = h1 * __builtin_amdgcn_rcpf(1.0f + ex);   /* forward.h:101 */
            if (okr) e.g[(size_t)r * e.F + gi] = f2h(silu * h3);        /* forward.h:151 */
        }
    } else {  /* EPI_QKV */
        const bool odd = n & 1;
        const bool rot = n < e.NQ + e.NKV;
        const bool isq = n < e.NQ;
        const int nn = isq ? n : (rot ? n - e.NQ : n - e.NQ - e.NKV);
        const int h = nn >> e.lghd, d = nn & (e.hd - 1);
        const int half_hd = e.hd >> 1;
        int pr[16], sr[16];
        float cr[16], sn[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = ok[i] ? rr[i] : 0;
            pr[i] = e.pos[r];
            sr[i] = isq ? 0 : e.slot[r];
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int ti = pr[i] * half_hd + (d >> 1);
            cr[i] = rot ? e.rope_cos[ti] : 1.f;
            sn[i] = rot ? e.rope_sin[ti] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float other = dpp_f<DPP_QUAD_XOR1>(acc[i]);   /* column n ^ 1 */
            if (!ok[i]) continue;
            float v = acc[i];
            if (rot)   /* pair (a, b) = (even column, odd column), forward.h:62-68 */
                v = odd ? fmaf(other, sn[i], v * cr[i]) : fmaf(v, cr[i], -(other * sn[i]));
            if (isq) {
                e.q[(size_t)rr[i] * e.NQ + n] = v;
            } else {
                const size_t off = (((size_t)sr[i] * e.Hkv + h) * e.max_seq + pr[i]) * e.hd + d;
                void *dst = rot ? e.kc : e.vc;
                if (e.kv_f32) ((float *)dst)[off] = v;
                else ((u16 *)dst)[off] = f2h(v);
            }
        }
    }
}

/* ---- tiled GEMM (prefill) ------------------------------------------------- */

#define BKH 64                 /* K (halves) per LDS stage: one 128-byte row per tile row */
#ifndef LMK_GATE_KS
#define LMK_GATE_KS 2          /* wave groups splitting K in a decode-row gate tile */
#endif
#ifndef DEC_RING
#define DEC_RING 4             /* LDS ring depth of decode-row (M <= 64) tiles (measured: 4 beats 3, 6 and 8) */
#endif

/* vmcnt(n) with the other counters left alone (gfx9 s_waitcnt encoding). */
#define WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 0xF) | ((((n) >> 4) & 3) << 14))

/* Tile rows (A rows, then W rows) live in LDS as 128-byte rows of 8 chunks of
 * 8 halves; chunk c of row r sits at slot c ^ ((r >> 1) & 7), so the 32 rows a
 * fragment read touches hit distinct banks.  Direct global->LDS loads write
 * 64 lanes x 16 bytes = 8 consecutive rows per wave instruction, lane l at
 * slot l % 8 of row l / 8: the swizzle is applied to the source address. */
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

/* 16-byte LDS reads issued as inline assembly, together with the wait for
 * them in the same statement.  The compiler cannot tell which LDS buffer its
 * own ds_reads touch relative to the direct global->LDS loads in flight, and
 * would wait for all of those loads before every read; these reads are
 * invisible to it, so the kernel orders them explicitly (vmcnt + barrier before
 * a stage's reads).  The lgkmcnt(0) wait sits inside the statement: were it a
 * statement of its own, the compiler could schedule a use of a read's result
 * (an MFMA, a register copy) between the read and the wait. */
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned lds_off(const u16 *p)
{
    return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) u16 *)p;
}
__device__ __forceinline__ void lds_read_wait(u32x4 (&v)[2], const unsigned (&a)[2])
{
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1])
                 : "v"(a[0]), "v"(a[1])
                 : "memory");
}
__device__ __forceinline__ void lds_read_wait(u32x4 (&v)[3], const unsigned (&a)[3])
{
    asm volatile("ds_read_b128 %0, %3\n\tds_read_b128 %1, %4\n\tds_read_b128 %2, %5\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2])
                 : "memory");
}
__device__ __forceinline__ void lds_read_wait(u32x4 (&v)[4], const unsigned (&a)[4])
{
    asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\t"
                 "ds_read_b128 %3, %7\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
                 : "memory");
}
__device__ __forceinline__ void lds_read_wait(u32x4 (&v)[6], const unsigned (&a)[6])
{
    asm volatile("ds_read_b128 %0, %6\n\tds_read_b128 %1, %7\n\tds_read_b128 %2, %8\n\t"
                 "ds_read_b128 %3, %9\n\tds_read_b128 %4, %10\n\tds_read_b128 %5, %11\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5])
                 : "memory");
}

/* Split form for software pipelining: lds_read_issue starts the reads, and
 * lds_wait_regs waits for them while naming their destination registers as
 * in/out operands, so no use of the results can be scheduled before the wait.
 * (A register copy of a pending result between the two statements would still
 * be wrong; the build checks the generated code for that.) */
template <int N>
__device__ __forceinline__ void lds_read_issue(u32x4 (&v)[N], const unsigned (&a)[N])
{
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("ds_read_b128 %0, %1" : "=&v"(v[i]) : "v"(a[i]) : "memory");
}
__device__ __forceinline__ void lds_wait_regs(u32x4 (&v)[2])
{
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]) : : "memory");
}
__device__ __forceinline__ void lds_wait_regs(u32x4 (&v)[3])
{
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]) : : "memory");
}
__device__ __forceinline__ void lds_wait_regs(u32x4 (&v)[4])
{
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : : "memory");
}
__device__ __forceinline__ void lds_wait_regs(u32x4 (&v)[6])
{
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5])
                 :
                 : "memory");
}

/* GATE epilogue of a BM x BN work-group tile through LDS: the gates (computed
 * in the accumulator layout, as epilogue_tile does) are staged as fp16 rows of
 * BN/2 gates, then written with one 16-byte store per 8 gates instead of one
 * 2-byte store per gate.  sg: LDS of at least BM * (BN/2 + 8) halves, no longer
 * read by any wave's main loop. */
template <int BM, int BN, int TM, int TN, int WVM, int WVN, int KG = 1>
__device__ __forceinline__ void gate_tile_lds(const f32x16 (&acc)[TM][TN], u16 *sg, int m0, int n0,
                                              int wm, int wn, const EpiArgs &e, bool own = true)
{
    constexpr int NT = 64 * WVM * WVN * KG;   /* threads: KG groups of WVM x WVN waves */
    constexpr int GW = BN / 2, GLD = GW + 8;
    const int lane = threadIdx.x & 63, c = lane & 31;
    const bool lo = c < 16;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if (!own) continue;   /* another K group's wave: the tile is group 0's */
            const int rl = wm * (BM / WVM) + i * 32 + 4 * (lane >> 5);
            const int gl = (wn * (BN / WVN) + j * 32) / 2 + (c & 15);
#pragma unroll
            for (int k = 0; k < 16; k += 2) {
                /* lane c < 16: row of element k (h1 own, h3 from lane c + 16);
                 * lane c + 16: row of element k + 1 (h3 own, h1 from lane c).
                 * The empty asm keeps the two elements separate values: a
                 * select between them would otherwise become an element read at
                 * a lane-dependent index, i.e. a 16-way select chain. */
                float a0 = acc[i][j][k], a1 = acc[i][j][k + 1];
                asm("" : "+v"(a0), "+v"(a1));
                const float other = xor16_f(lo ? a1 : a0);
                const float h1 = lo ? a0 : other;
                const float h3 = lo ? other : a1;
                const int r = rl + 8 * (k >> 2) + (k & 3) + (lo ? 0 : 1);
                const float ex = __builtin_amdgcn_exp2f(-h1 * 1.4426950408889634f);
                const float silu = h1 * __builtin_amdgcn_rcpf(1.0f + ex);   /* forward.h:101 */
                sg[r * GLD + gl] = f2h(silu * h3);                          /* forward.h:151 */
            }
        }
    __syncthreads();
    constexpr int CPR = GW / 8;   /* 16-byte chunks per row */
#pragma unroll
    for (int idx = threadIdx.x; idx < BM * CPR; idx += NT) {
        const int r = idx / CPR, ch = idx % CPR;
        const int row = m0 + r, gi = n0 / 2 + ch * 8;
        if (row < e.M && gi < e.F)
            *(uint4 *)(e.g + (size_t)row * e.F + gi) = *(const uint4 *)(sg + r * GLD + ch * 8);
    }
}

/* Per-item operands of the QKV epilogue (item: 4 consecutive columns of one
 * row, two RoPE pairs): position, cache slot and the pairs' rotation. */
struct QkvItem {
    int p, sl;
    float2 c, sn;
};

/* Position and slot of this thread's items of round `round` (item k: tile row
 * (tid + k*GT) / (BN/4), columns 4 * ((tid + k*GT) % (BN/4)) ..). */
template <int BM, int BN, int NI>
__device__ __forceinline__ void qkv_item_rows(QkvItem (&it)[NI], int round, int m0, const EpiArgs &e)
{
    constexpr int WM = BM / 2, C4 = BN / 4;
#pragma unroll
    for (int k = 0; k < NI; k++) {
        const int r = (threadIdx.x + k * GT) / C4;
        const int row = min(m0 + (r >> 5) * WM + round * 32 + (r & 31), e.M - 1);
        it[k].p = e.pos[row];
        it[k].sl = e.slot[row];
    }
}

/* The items' rotations (clamped indices: the loads stay unconditional). */
template <int BN, int NI>
__device__ __forceinline__ void qkv_item_rope(QkvItem (&it)[NI], int n0, const EpiArgs &e)
{
#pragma unroll
    for (int k = 0; k < NI; k++) {
        const int n = n0 + 4 * ((threadIdx.x + k * GT) % (BN / 4));
        const bool rot = n < e.NQ + e.NKV;
        const int nn = n < e.NQ ? n : n - e.NQ;
        const int ti = rot ? it[k].p * (e.hd >> 1) + ((nn & (e.hd - 1)) >> 1) : 0;
        it[k].c = *(const float2 *)(e.rope_cos + ti);
        it[k].sn = *(const float2 *)(e.rope_sin + ti);
    }
}

/* QKV epilogue of a BM x BN work-group tile through LDS: in rounds of 64 rows
 * (row tile i of both wave rows), the fp32 products are staged in LDS, then
 * each thread takes 4 consecutive columns of a row (two RoPE pairs,
 * forward.h:55-70): q columns go to q [M, NQ] with one 16-byte store, k and v
 * columns to the cache at (slot[row], pos[row]) with one 16- or 8-byte store.
 * pre: positions and slots of round 0's items, loaded before the main loop
 * (TM = 1), or NULL.  b0, b1:
 * LDS of at least 64 * BN floats each, no longer read by any wave's main loop. */
template <int BM, int BN, int TM, int TN, int NI>
__device__ __forceinline__ void qkv_tile_lds(const f32x16 (&acc)[TM][TN], float *b0, float *b1,
                                             int m0, int n0, int wm, int wn, const EpiArgs &e,
                                             const QkvItem (*pre)[NI], bool own = true)
{
    constexpr int WM = BM / 2, WN = BN / 2, C4 = BN / 4;
    static_assert(NI * GT == 64 * C4, "items per thread");
    const int lane = threadIdx.x & 63;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; i++) {
        float *buf = (i & 1) ? b1 : b0;
        /* buf row wm*32 + r holds tile row m0 + wm*WM + i*32 + r; the waves
         * of other K groups (own false) only keep the barriers */
        QkvItem its[NI];
        if (own) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    const int r = wm * 32 + 8 * (k >> 2) + 4 * (lane >> 5) + (k & 3);
                    buf[r * BN + wn * WN + j * 32 + (lane & 31)] = acc[i][j][k];
                }
            if (i == 0 && pre) {
#pragma unroll
                for (int k = 0; k < NI; k++) its[k] = (*pre)[k];
            } else {
                qkv_item_rows<BM, BN, NI>(its, i, m0, e);
            }
            qkv_item_rope<BN, NI>(its, n0, e);
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < NI; k++) {
            if (!own) break;
            const int idx = threadIdx.x + k * GT, r = idx / C4, c4 = idx % C4;
            const int row = m0 + (r >> 5) * WM + i * 32 + (r & 31);
            const int n = n0 + 4 * c4;
            if (row >= e.M || n >= e.N) continue;
            const float4 v = *(const float4 *)(buf + r * BN + 4 * c4);
            const int p = its[k].p;
            const bool isq = n < e.NQ, rot = n < e.NQ + e.NKV;
            const int nn = isq ? n : (rot ? n - e.NQ : n - e.NQ - e.NKV);
            const int d = nn & (e.hd - 1);
            float o[4] = {v.x, v.y, v.z, v.w};
            if (rot) {
                const float2 c = its[k].c, sn = its[k].sn;
                o[0] = fmaf(v.x, c.x, -(v.y * sn.x));   /* forward.h:64 */
                o[1] = fmaf(v.x, sn.x, v.y * c.x);      /* forward.h:65 */
                o[2] = fmaf(v.z, c.y, -(v.w * sn.y));
                o[3] = fmaf(v.z, sn.y, v.w * c.y);
            }
            if (isq) {
                *(float4 *)(e.q + (size_t)row * e.NQ + n) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
                const size_t off =
                    (((size_t)its[k].sl * e.Hkv + (nn >> e.lghd)) * e.max_seq + p) * e.hd + d;
                void *dst = rot ? e.kc : e.vc;
                if (e.kv_f32)
                    *(float4 *)((float *)dst + off) = make_float4(o[0], o[1], o[2], o[3]);
                else
                    *(uint2 *)((u16 *)dst + off) =
                        make_uint2((unsigned)f2h(o[0]) | ((unsigned)f2h(o[1]) << 16),
                                   (unsigned)f2h(o[2]) | ((unsigned)f2h(o[3]) << 16));
            }
        }
    }
}

template <int BM, int BN, int E, int NS, int WVM, bool RS = false, int WVN = 2, int KG = 1>
__global__ void __launch_bounds__(64 * WVM * WVN * KG) k_gemm_tile(const u16 *__restrict__ A, int lda,
                                                         const u16 *__restrict__ W, int K, int kc,
                                                         EpiArgs e, int tm, int tn)
{
    constexpr int NWV = WVM * WVN;                /* waves: WVM along M x WVN along N, */
                                                  /* in each of KG groups along K        */
    constexpr int WM = BM / WVM, WN = BN / WVN;   /* wave tile */
    constexpr int TM = WM / 32, TN = WN / 32;   /* MFMA tiles per wave */
    constexpr int ROWS = BM + BN;               /* tile rows per stage */
    constexpr int STAGE = ROWS * 64;            /* halves per stage (128 B per row) */
    constexpr int LDW = ROWS / 8 / NWV;         /* load instructions per wave per stage */
    static_assert(TM >= 1 && TN >= 1 && LDW >= 1 && ROWS % (8 * NWV) == 0, "tile shape");
    /* the LDS-staged QKV epilogue is written for four waves */
    static_assert((WVM == 2 && WVN == 2) || E != EPI_QKV, "wave layout");
    static_assert(WVN == 1 || WVN == 2, "one or two waves along N");
    static_assert(NS >= 3 && NS <= 8 && LDW * (NS - 2) <= 63, "ring depth (vmcnt holds 63)");
    static_assert(KG == 1 || ((E == EPI_GATE || E == EPI_STORE || E == EPI_QKV) && !RS),
                  "K groups: gate, store or QKV epilogue");
    /* the NS stage buffers are separate arrays (not one indexed ring) so that
     * the compiler can tell a stage's LDS reads from the direct loads in flight
     * into the others and does not wait for those loads */
#define RING_BUF(i) __shared__ __attribute__((aligned(NS > i ? 1024 : 16))) u16 lds##i[NS > i ? KG * STAGE : 8]
    RING_BUF(0); RING_BUF(1); RING_BUF(2); RING_BUF(3);
    RING_BUF(4); RING_BUF(5); RING_BUF(6); RING_BUF(7);
#undef RING_BUF
    auto ring = [&](auto I) -> u16 * {
        constexpr int i = decltype(I)::value % NS;
        if constexpr (i == 0) return lds0;
        else if constexpr (i == 1) return lds1;
        else if constexpr (i == 2) return lds2;
        else if constexpr (i == 3) return lds3;
        else if constexpr (i == 4) return lds4;
        else if constexpr (i == 5) return lds5;
        else if constexpr (i == 6) return lds6;
        else return lds7;
    };

    const int tid = threadIdx.x, lane = tid & 63;
    /* wave within its K group, and the group (KG > 1: group kg takes the
     * kg-th of KG equal K chunks through its own stage buffers) */
    const int wall = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = KG > 1 ? wall / NWV : 0;
    const int wave = KG > 1 ? wall % NWV : wall;
    auto gbuf = [&](auto I) -> u16 * { return ring(I) + (KG > 1 ? kg * STAGE : 0); };
    const int wm = WVN == 2 ? wave >> 1 : wave, wn = WVN == 2 ? wave & 1 : 0;
    /* XCD-aware tile order: work-group id goes to XCD id % 8; give each XCD a
     * contiguous run of tiles (M fastest), i.e. a slice of N, so the W rows of
     * its tiles stay in its own L2. */
    const int T = tm * tn, id = blockIdx.x;
    const int g = (T % 8 == 0) ? (id % 8) * (T / 8) + id / 8 : id;
    const int m0 = (g % tm) * BM, n0 = (g / tm) * BN;
    const int M = e.M, N = e.N;

    /* per-lane source rows of this wave's load instructions (fixed over k);
     * work-group split y takes k = y*kc .. y*kc + kc - 1 (kc = K unsplit) */
    const int k0 = blockIdx.y * kc + kg * (kc / KG);
    const u16 *src[LDW];
#pragma unroll
    for (int i = 0; i < LDW; i++) {
        const int row = (wave * LDW + i) * 8 + lane / 8;
        const int chunk = swz(row, lane % 8);
        if (row < BM)
            src[i] = A + (size_t)min(m0 + row, M - 1) * lda + k0 + chunk * 8;
        else
            src[i] = W + (size_t)min(n0 + row - BM, N - 1) * K + k0 + chunk * 8;
    }
    /* load instructions [I0, I1) of this wave's share of stage kt into buf */
    auto issue_range = [&](u16 *buf, int kt, auto I0, auto I1) {
        u16 *dst = buf + wave * LDW * 8 * 64;
        static_for<decltype(I0)::value, decltype(I1)::value>([&](auto I) {
            __builtin_amdgcn_global_load_lds((const void *)(src[I] + kt * BKH),
                                             (__attribute__((address_space(3))) void *)(dst + I * 8 * 64),
                                             16, 0, 0);
        });
    };
    auto issue = [&](u16 *buf, int kt) {
        issue_range(buf, kt, std::integral_constant<int, 0>{}, std::integral_constant<int, LDW>{});
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (f32x16){};

    /* fragments of k-step ks: A rows (TM), then W rows (TN); the reads of step
     * ks+1 are issued after the MFMAs of step ks, into the other register set */
    constexpr int NF = TM + TN;
    auto frag_addr = [&](const u16 *st, int ks, unsigned (&ad)[NF]) {
        const int c = ks * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int row = wm * WM + i * 32 + (lane & 31);
            ad[i] = lds_off(st + row * 64 + swz(row, c) * 8);
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int row = BM + wn * WN + j * 32 + (lane & 31);
            ad[TM + j] = lds_off(st + row * 64 + swz(row, c) * 8);
        }
    };
    /* k-steps of one stage; the loads of stage kt2 (when ld) are issued a
     * quarter before each step's MFMAs, so they queue behind the matrix work
     * instead of holding the wave after the barrier */
    auto compute = [&](const u16 *st, u16 *ahead, int kt2, bool ld) {
        u32x4 f[2][NF];
        unsigned ad[NF];
        frag_addr(st, 0, ad);
        lds_read_wait(f[0], ad);
        /* The scheduling barriers pin the order reads(ks+1), loads, MFMAs(ks),
         * wait(ks+1): the MFMAs do not depend on the wait, and without them the
         * scheduler hoists the wait above the MFMAs, exposing the LDS latency
         * at every step. */
        static_for<0, BKH / 16>([&](auto KS) {
            constexpr int ks = decltype(KS)::value;
            if (ks + 1 < BKH / 16) {      /* next step's reads run under this step's MFMAs */
                frag_addr(st, ks + 1, ad);
                lds_read_issue<NF>(f[(ks + 1) & 1], ad);
            }
            if (ld)
                issue_range(ahead, kt2, std::integral_constant<int, ks * LDW / 4>{},
                            std::integral_constant<int, (ks + 1) * LDW / 4>{});
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = mfma32(__builtin_bit_cast(uint4, f[ks & 1][i]),
                                       __builtin_bit_cast(uint4, f[ks & 1][TM + j]), acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
            if (ks + 1 < BKH / 16) lds_wait_regs(f[(ks + 1) & 1]);
        });
    };
    /* one k-stage: wait for this wave's loads of stage kt (those of the up to
     * NS-2 later stages in flight may still be outstanding), then a bare
     * barrier (a fenced __syncthreads would wait for every outstanding load) so
     * all waves' loads of stage kt have landed and stage kt-1's buffer is free
     * for stage kt+NS-1 */
    const int nk = kc / KG / BKH;
    auto wait_stage = [&](int kt) {
        const int later = min(NS - 2, nk - 1 - kt);   /* stages issued after kt */
        static_for<0, NS - 1>([&](auto J) {
            constexpr int j = decltype(J)::value;
            if (later == NS - 2 - j) WAIT_VMCNT(LDW * (NS - 2 - j));
        });
    };
    auto step = [&](int kt, const u16 *cur, u16 *ahead) {
        wait_stage(kt);
        __builtin_amdgcn_s_barrier();
        compute(cur, ahead, kt + NS - 1, kt + NS - 1 < nk);
    };
    /* positions and slots of a one-round tile's QKV epilogue, loaded first so
     * that they arrive during the main loop */
    constexpr bool QKV_LDS = E == EPI_QKV && 64 * BN * 2 <= STAGE;
    constexpr int QNI = 64 * BN / 4 / GT;
    QkvItem qpre[QKV_LDS ? QNI : 1];
    if constexpr (QKV_LDS && TM == 1) {
#pragma unroll
        for (int k = 0; k < QNI; k++) {
            if (KG > 1 && kg > 0) break;
            const int r = (threadIdx.x + k * GT) / (BN / 4);
            const int row = min(m0 + (r >> 5) * WM + (r & 31), M - 1);
            qpre[k].p = e.pos[row];
            qpre[k].sl = e.slot[row];
        }
    }
    /* the residual a one-tile wave adds (RESID, RESNORM) and the gain
     * (RESNORM), loaded before the ring so that they arrive during the main
     * loop instead of after it */
    constexpr bool XPRE = (E == EPI_RESID || E == EPI_RESNORM) && TM * TN == 1;
    float xpre[XPRE ? 17 : 1];
    if constexpr (XPRE) {
        const int n = n0 + wn * WN + (lane & 31);
        const int rb = m0 + wm * WM + 4 * (lane >> 5);
        if constexpr (E == EPI_RESNORM) xpre[16] = n < N ? e.gain[n] : 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = rb + 8 * (i >> 2) + (i & 3);
            xpre[i] = r < M && n < N ? e.out[(size_t)r * e.ldc + n] : 0.f;
        }
    }
    /* Row scale after a RESNORM GEMM (RS, e.rs_ss set): thread r < BM loads
     * the nss sums of squares of tile row r (float4s, a uniform count) before
     * the ring's first loads, and adds them once those are issued (the wait
     * then covers only these older loads), leaving the row's scale in LDS; no
     * register stays live through the main loop.  A separate instantiation:
     * in the unscaled kernels the extra arguments and branches delayed the
     * start of every tile (C1's GEMMs 5% slower with the scale unused). */
    static_assert(!RS || E == EPI_GATE || E == EPI_QKV, "row scale before a gate or QKV epilogue");
    static_assert(!RS || BM <= 64 * NWV, "a thread per tile row");
    constexpr int MAXV = RS ? 16 : 1;   /* float4s per row: nss <= 64 */
    __shared__ float rs_sh[RS ? BM : 1];
    float4 ssv[MAXV];
    if constexpr (RS) {
        if (tid < BM) {
            const float4 *src = (const float4 *)(e.rs_ss + (size_t)min(m0 + tid, M - 1) * e.nss);
            const int nv = e.nss >> 2;
#pragma unroll
            for (int j = 0; j < MAXV; j++) ssv[j] = j < nv ? src[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    issue(gbuf(std::integral_constant<int, 0>{}), 0);
    static_for<1, NS - 1>([&](auto I) {
        if (decltype(I)::value < nk) issue(gbuf(I), decltype(I)::value);
    });
    if constexpr (RS) {
        __builtin_amdgcn_sched_barrier(0);
        if (tid < BM) {
            /* 1/sqrt(mean(x^2) + 1e-5) of the row (forward.h:46-53), the
             * partials added in a fixed order */
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < MAXV; j++) sum += (ssv[j].x + ssv[j].y) + (ssv[j].z + ssv[j].w);
            rs_sh[tid] = 1.0f / sqrtf(sum / (float)(32 * e.nss) + 1e-5f);
        }
    }
    for (int kt = 0; kt < nk; kt += NS) {
        static_for<0, NS>([&](auto I) {
            constexpr int i = decltype(I)::value;
            if (kt + i < nk)
                step(kt + i, gbuf(std::integral_constant<int, i>{}),
                     gbuf(std::integral_constant<int, i + NS - 1>{}));
        });
    }
    if constexpr (RS) {   /* the product rows scaled by their row's scale */
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int k = 0; k < 16; k++)
                    acc[i][j][k] *= rs_sh[wm * WM + i * 32 + 8 * (k >> 2) + 4 * (lane >> 5) + (k & 3)];
    }
    if constexpr (KG > 1) {
        /* the K groups' partial tiles summed in group 0, in group order: groups
         * 1.. store theirs to LDS (lane fastest), group 0 adds them */
        static_assert((KG - 1) * NWV * TM * TN * 16 * 64 * 4 <= KG * STAGE * 2, "partials fit lds0");
        float *red = (float *)lds0;
        __syncthreads();   /* every group's last LDS reads are done */
        if (kg > 0) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int k = 0; k < 16; k++)
                        red[((((kg - 1) * NWV + wave) * TM + i) * TN * 16 + j * 16 + k) * 64 + lane] = acc[i][j][k];
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int q = 1; q < KG; q++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int k = 0; k < 16; k++)
                            acc[i][j][k] += red[((((q - 1) * NWV + wave) * TM + i) * TN * 16 + j * 16 + k) * 64 + lane];
        }
    }
    if (E == EPI_STORE) e.out += blockIdx.y * e.sstride;   /* this split's partial */
    if constexpr (E == EPI_GATE) {
        static_assert(BM * (BN / 2 + 8) <= STAGE, "gate staging fits one stage buffer");
        gate_tile_lds<BM, BN, TM, TN, WVM, WVN, KG>(acc, lds0, m0, n0, wm, wn, e, kg == 0);
        return;
    }
    if constexpr (QKV_LDS) {
        qkv_tile_lds<BM, BN, TM, TN, QNI>(acc, (float *)lds0, (float *)lds1, m0, n0, wm, wn, e,
                                          TM == 1 ? &qpre : nullptr, kg == 0);
        return;
    }
    if (KG > 1 && kg > 0) return;   /* (no barrier below for the store epilogue) */
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            epilogue_tile<E>(acc[i][j], m0 + wm * WM + i * 32, n0 + wn * WN + j * 32, e,
                             XPRE ? xpre : nullptr);
}

/* ---- per-row RMSNorm ------------------------------------------------------------ */

/* Row norm, one wave per row m, four rows per work-group (forward.h:46-53): with
 * emb != NULL the row is first set to the fp16 embedding row emb[tok[m]]
 * (forward.h:108-110); with ns > 0 the ns partials of a K-split projection are
 * added to it, in split order (the residual add, forward.h:134-136, 157-159);
 * then xn[m, k] = fp16(x[m, k] * (1/sqrt(mean(x[m]^2) + 1e-5)) * gain[k]), the
 * GEMM operand of the projection that follows.  Lane l holds columns
 * c*256 + 4l .. +3 (c < D/256) as float4 groups, so every access is a 16-byte
 * (x, partials, gain) or 8-byte (embedding, xn) lane segment, and the sum of
 * squares is a wave reduction (no LDS, no barrier).  Partials are loaded four
 * at a time.  RPW rows (waves) per work-group.  Four from 512 rows: 4.5
 * against 6.3 us for a 256-thread work-group per row at 2048 rows with one
 * partial (C3 2-3% faster).  One (a work-group per row, spread over more CUs)
 * for 65-511 rows: C1's 256-token prefill 0.468-0.476 -> 0.465-0.473 ms.  Up
 * to 64 rows the 256-thread work-group per row (k_rownorm_blk) stays, since
 * the one-wave form cost the scaled model's 32 decode rows of 2048 6%. */
template <int D, int RPW = 4>
__global__ void __launch_bounds__(64 * RPW) k_rownorm(float *__restrict__ x, int M,
                                                   const u16 *__restrict__ emb,
                                                   const int *__restrict__ tok,
                                                   const float *__restrict__ sp, int ns,
                                                   size_t sstride,
                                                   const float *__restrict__ gain,
                                                   u16 *__restrict__ xn)
{
    constexpr int C4 = D / 256;
    static_assert(D % 256 == 0, "row width");
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * RPW + (threadIdx.x >> 6);
    if (m >= M) return;                       /* wave-uniform; no barrier below */
    float *xr = x + (size_t)m * D + 4 * lane;
    float4 gv[C4];                            /* gain, loaded first: its latency */
#pragma unroll                                /* overlaps the row's loads        */
    for (int c = 0; c < C4; c++) gv[c] = *(const float4 *)(gain + 4 * lane + c * 256);
    float4 v[C4];
    if (emb) {
        const u16 *er = emb + (size_t)tok[m] * D + 4 * lane;
#pragma unroll
        for (int c = 0; c < C4; c++) {
            const uint2 h = *(const uint2 *)(er + c * 256);
            const f16x2 a = __builtin_bit_cast(f16x2, h.x), b = __builtin_bit_cast(f16x2, h.y);
            v[c] = make_float4((float)a.x, (float)a.y, (float)b.x, (float)b.y);
        }
    } else {
#pragma unroll
        for (int c = 0; c < C4; c++) v[c] = *(const float4 *)(xr + c * 256);
        const float *pr = sp + (size_t)m * D + 4 * lane;
        for (int q = 0; q < ns; q += 4) {
            /* past the last partial a group reloads it and adds zero, so the
             * loads stay unconditional */
            float4 t[4][C4];
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int c = 0; c < C4; c++)
                    t[u][c] = *(const float4 *)(pr + (size_t)min(q + u, ns - 1) * sstride + c * 256);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float z = q + u < ns ? 1.f : 0.f;
#pragma unroll
                for (int c = 0; c < C4; c++) {
                    v[c].x += t[u][c].x * z; v[c].y += t[u][c].y * z;
                    v[c].z += t[u][c].z * z; v[c].w += t[u][c].w * z;
                }
            }
        }
    }
    if (emb || ns > 0) {
#pragma unroll
        for (int c = 0; c < C4; c++) *(float4 *)(xr + c * 256) = v[c];
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < C4; c++) {
        ss = fmaf(v[c].x, v[c].x, ss); ss = fmaf(v[c].y, v[c].y, ss);
        ss = fmaf(v[c].z, v[c].z, ss); ss = fmaf(v[c].w, v[c].w, ss);
    }
    ss = wave_sum(ss);
    const float rs = 1.0f / sqrtf(ss / D + 1e-5f);
    u16 *xo = xn + (size_t)m * D + 4 * lane;
#pragma unroll
    for (int c = 0; c < C4; c++) {
        const float4 g = gv[c];
        const unsigned lo = (unsigned)f2h(v[c].x * rs * g.x) | ((unsigned)f2h(v[c].y * rs * g.y) << 16);
        const unsigned hi = (unsigned)f2h(v[c].z * rs * g.z) | ((unsigned)f2h(v[c].w * rs * g.w) << 16);
        *(uint2 *)(xo + c * 256) = make_uint2(lo, hi);
    }
}

/* The same row norm with one 256-thread work-group per row (four waves share
 * it: thread t owns the D/256 values 4t .. 4t+3 (+1024 ...), so every load of
 * the row is issued at once, and the sum of squares goes through LDS), for
 * fewer than 512 rows. */
template <int D>
__global__ void __launch_bounds__(GT) k_rownorm_blk(float *__restrict__ x, int M,
                                                const u16 *__restrict__ emb,
                                                const int *__restrict__ tok,
                                                const float *__restrict__ sp, int ns,
                                                size_t sstride,
                                                const float *__restrict__ gain,
                                                u16 *__restrict__ xn)
{
    constexpr int PER = D / GT;              /* values per thread */
    constexpr int C4 = (PER + 3) / 4;        /* float4 groups per thread */
    static_assert(D % GT == 0, "row width");
    __shared__ float red[GT / 64];
    const int t = threadIdx.x;
    const int m = blockIdx.x;
    float *xr = x + (size_t)m * D;
    /* value i of this thread is column col(i) = (i/4)*1024 + 4t + i%4 (D >= 1024),
     * or t*PER + i (D < 1024) */
    auto col = [&](int c) { return PER >= 4 ? c * (4 * GT) + 4 * t : t * PER; };
    /* gain, loaded first so its latency overlaps the row's loads (C2 and C4
     * decode steps 0.5% faster than loading it after the reduction) */
    float gl[C4 * 4];
#pragma unroll
    for (int c = 0; c < C4; c++) {
        if (PER >= 4) {
            const float4 g4 = *(const float4 *)(gain + col(c));
            gl[4 * c] = g4.x; gl[4 * c + 1] = g4.y; gl[4 * c + 2] = g4.z; gl[4 * c + 3] = g4.w;
        } else {
#pragma unroll
            for (int i = 0; i < PER; i++) gl[i] = gain[col(0) + i];
        }
    }
    float v[C4 * 4];
    if (emb) {
        const u16 *er = emb + (size_t)tok[m] * D;
#pragma unroll
        for (int c = 0; c < C4; c++) {
            if (PER >= 4) {
                const uint2 h = *(const uint2 *)(er + col(c));
                const f16x2 a = __builtin_bit_cast(f16x2, h.x), b = __builtin_bit_cast(f16x2, h.y);
                v[4 * c] = (float)a.x; v[4 * c + 1] = (float)a.y;
                v[4 * c + 2] = (float)b.x; v[4 * c + 3] = (float)b.y;
            } else {
#pragma unroll
                for (int i = 0; i < PER; i++) v[i] = h2f(er[col(0) + i]);
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < C4; c++) {
            if (PER >= 4) {
                const float4 q4 = *(const float4 *)(xr + col(c));
                v[4 * c] = q4.x; v[4 * c + 1] = q4.y; v[4 * c + 2] = q4.z; v[4 * c + 3] = q4.w;
            } else {
#pragma unroll
                for (int i = 0; i < PER; i++) v[i] = xr[col(0) + i];
            }
        }
        if (ns > 0) {
            /* partials in groups of four: the group's loads are all issued before
             * its adds (the adds stay in split order) */
            auto add_part = [&](const float (&t)[C4 * 4]) {
#pragma unroll
                for (int i = 0; i < PER; i++) v[i] += t[i];
            };
            auto load_part = [&](int q, float (&t)[C4 * 4]) {
                const float *pr = sp + q * sstride + (size_t)m * D;
#pragma unroll
                for (int c = 0; c < C4; c++) {
                    if (PER >= 4) {
                        const float4 q4 = *(const float4 *)(pr + col(c));
                        t[4 * c] = q4.x; t[4 * c + 1] = q4.y; t[4 * c + 2] = q4.z; t[4 * c + 3] = q4.w;
                    } else {
#pragma unroll
                        for (int i = 0; i < PER; i++) t[i] = pr[col(0) + i];
                    }
                }
            };
            /* groups of eight partials: all loads of a group are issued before
             * its adds (in split order); past the last partial the group reloads
             * it and adds zero, so the loads stay unconditional */
            for (int q = 0; q < ns; q += 8) {
                float t[8][C4 * 4];
#pragma unroll
                for (int u = 0; u < 8; u++) load_part(min(q + u, ns - 1), t[u]);
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    if (q + u >= ns) {
#pragma unroll
                        for (int i = 0; i < PER; i++) t[u][i] = 0.f;
                    }
                    add_part(t[u]);
                }
            }
        }
    }
    if (emb || ns > 0) {
#pragma unroll
        for (int c = 0; c < C4; c++) {
            if (PER >= 4)
                *(float4 *)(xr + col(c)) = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
            else
#pragma unroll
                for (int i = 0; i < PER; i++) xr[col(0) + i] = v[i];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; i++) ss = fmaf(v[i], v[i], ss);
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < GT / 64; w++) tot += red[w];
    const float rs = 1.0f / sqrtf(tot / D + 1e-5f);
    u16 *xo = xn + (size_t)m * D;
#pragma unroll
    for (int c = 0; c < C4; c++) {
        if (PER >= 4) {
            const float *g = gl + 4 * c;
            const unsigned lo = (unsigned)f2h(v[4 * c] * rs * g[0]) | ((unsigned)f2h(v[4 * c + 1] * rs * g[1]) << 16);
            const unsigned hi = (unsigned)f2h(v[4 * c + 2] * rs * g[2]) | ((unsigned)f2h(v[4 * c + 3] * rs * g[3]) << 16);
            *(uint2 *)(xo + col(c)) = make_uint2(lo, hi);
        } else {
#pragma unroll
            for (int i = 0; i < PER; i++) xo[col(0) + i] = f2h(v[i] * rs * gl[i]);
        }
    }
}

/* ============================== launchers =================================== */


extern "C" int lmk_rownorm(hipStream_t s, float *x, int D, int M, const uint16_t *emb, const int *tok,
                           const float *sp, int ns, size_t sstride, const float *gain, uint16_t *xn)
{
    if (M < 1 || (emb && !tok) || !gain || !xn || ns < 0 || (ns && (!sp || emb)))
        return hipErrorInvalidValue;
    if (M > 64 && M < 512) {   /* a one-wave work-group per row */
        dim3 grid(M);
        switch (D) {
        case 256: hipLaunchKernelGGL((k_rownorm<256, 1>), grid, dim3(64), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        case 512: hipLaunchKernelGGL((k_rownorm<512, 1>), grid, dim3(64), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        case 768: hipLaunchKernelGGL((k_rownorm<768, 1>), grid, dim3(64), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        case 1024: hipLaunchKernelGGL((k_rownorm<1024, 1>), grid, dim3(64), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        case 2048: hipLaunchKernelGGL((k_rownorm<2048, 1>), grid, dim3(64), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (M < 512) {   /* a work-group per row */
        dim3 grid(M);
        switch (D) {
        case 256: hipLaunchKernelGGL(k_rownorm_blk<256>, grid, dim3(GT), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        case 512: hipLaunchKernelGGL(k_rownorm_blk<512>, grid, dim3(GT), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        case 768: hipLaunchKernelGGL(k_rownorm_blk<768>, grid, dim3(GT), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        case 1024: hipLaunchKernelGGL(k_rownorm_blk<1024>, grid, dim3(GT), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        case 2048: hipLaunchKernelGGL(k_rownorm_blk<2048>, grid, dim3(GT), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    dim3 grid((M + 3) / 4);
    switch (D) {
    case 256: hipLaunchKernelGGL(k_rownorm<256>, grid, dim3(256), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
    case 512: hipLaunchKernelGGL(k_rownorm<512>, grid, dim3(256), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
    case 768: hipLaunchKernelGGL(k_rownorm<768>, grid, dim3(256), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
    case 1024: hipLaunchKernelGGL(k_rownorm<1024>, grid, dim3(256), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
    case 2048: hipLaunchKernelGGL(k_rownorm<2048>, grid, dim3(256), 0, s, x, M, emb, tok, sp, ns, sstride, gain, xn); break;
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
    e.lghd = p->hd > 0 ? __builtin_ctz((unsigned)p->hd) : 0;
    e.slot = p->slot; e.pos = p->pos; e.rope_cos = p->rope_cos; e.rope_sin = p->rope_sin;
    e.sstride = 0;
    e.nt = p->stream_out;
    e.gain = p->gain; e.u = (u16 *)p->u; e.ss = p->ss; e.ovf = p->ovf;
    e.rs_ss = p->rs_ss; e.nss = p->nss;
    return e;
}

/* LDS ring depth: 3 stages where several work-groups share a CU (prefill),
 * deeper for decode rows (M <= 64), whose few work-groups per CU need more
 * weight bytes in flight each to cover the memory latency. */
template <int BM, int BN>
static constexpr int ring_depth(bool rows64, bool gate = false)
{
    constexpr int fit = 160 * 1024 / ((BM + BN) * 128);   /* stages that fit the LDS */
    /* 32-row gate tiles: 6 stages (W1/W3 of 32 scaled-model rows 12.3 us against 13.3) */
    constexpr int want = BM == 32 && DEC_RING < 6 ? 6 : DEC_RING;
    return BM <= 64 && rows64 ? ((gate ? want : DEC_RING) < fit ? (gate ? want : DEC_RING) : fit) : 3;
}

/* Ring depth of a tile whose K is walked by G wave groups, each with its own
 * stage buffers: at most 6 stages, as many as the LDS holds for G rings. */
template <int BM, int BN, int G>
static constexpr int ks_ring()
{
    constexpr int fit = 160 * 1024 / (G * (BM + BN) * 128);
    return fit < 6 ? fit : 6;
}

template <int BM, int BN, int E, bool RS = false>
static void launch_tile(hipStream_t s, const uint16_t *A, int lda, const uint16_t *W, int M, int N,
                        int K, const EpiArgs &e)
{
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    if constexpr (BM == 256 && E != EPI_QKV) {   /* eight waves (4 x 2): two per SIMD */
        hipLaunchKernelGGL((k_gemm_tile<BM, BN, E, 3, 4, RS>), dim3(tm * tn), dim3(512), 0, s, (const u16 *)A,
                           lda, (const u16 *)W, K, K, e, tm, tn);
    } else if constexpr (BM == 32 && BN == 32) {   /* one wave (per K group) */
        constexpr int G = E == EPI_GATE && !RS ? LMK_GATE_KS : 1;
        if (G > 1 && K % (G * BKH) == 0)
            hipLaunchKernelGGL((k_gemm_tile<BM, BN, E, ks_ring<BM, BN, G>(), 1, RS, 1, G>),
                               dim3(tm * tn), dim3(64 * G), 0, s, (const u16 *)A, lda, (const u16 *)W, K, K, e, tm, tn);
        else
            hipLaunchKernelGGL((k_gemm_tile<BM, BN, E, ring_depth<BM, BN>(true, E == EPI_GATE), 1, RS, 1>),
                               dim3(tm * tn), dim3(64), 0, s, (const u16 *)A, lda, (const u16 *)W, K, K, e, tm, tn);
    } else if constexpr (BM == 32) {               /* two waves (1 x 2) over 32 rows (per K group) */
        constexpr int G = E == EPI_GATE && !RS ? LMK_GATE_KS : 1;
        if (G > 1 && K % (G * BKH) == 0)
            hipLaunchKernelGGL((k_gemm_tile<BM, BN, E, ks_ring<BM, BN, G>(), 1, RS, 2, G>), dim3(tm * tn),
                               dim3(128 * G), 0, s, (const u16 *)A, lda, (const u16 *)W, K, K, e, tm, tn);
        else
            hipLaunchKernelGGL((k_gemm_tile<BM, BN, E, ring_depth<BM, BN>(true, E == EPI_GATE), 1, RS>), dim3(tm * tn),
                               dim3(128), 0, s, (const u16 *)A, lda, (const u16 *)W, K, K, e, tm, tn);
    } else {
        if (M <= 64 && BM == 64)
            hipLaunchKernelGGL((k_gemm_tile<BM, BN, E, ring_depth<BM, BN>(true), 2, RS>), dim3(tm * tn),
                               dim3(GT), 0, s, (const u16 *)A, lda, (const u16 *)W, K, K, e, tm, tn);
        else if ((E == EPI_GATE || E == EPI_QKV) && !RS && BM == 64 && BN == 64 && tm * tn <= 256 &&
                 K % (2 * BKH) == 0) {
            /* prefill-row gate or QKV, one round of tiles: K in two wave
             * groups (eight waves, two per SIMD) */
            if constexpr ((E == EPI_GATE || E == EPI_QKV) && !RS && BM == 64 && BN == 64)
                hipLaunchKernelGGL((k_gemm_tile<BM, BN, E, 3, 2, false, 2, 2>), dim3(tm * tn), dim3(2 * GT), 0, s,
                                   (const u16 *)A, lda, (const u16 *)W, K, K, e, tm, tn);
        } else
            hipLaunchKernelGGL((k_gemm_tile<BM, BN, E, 3, 2, RS>), dim3(tm * tn), dim3(GT), 0, s, (const u16 *)A,
                               lda, (const u16 *)W, K, K, e, tm, tn);
    }
}

/* The tiled kernel over grid (tiles, ns), split y taking k-chunk y*K/ns. */
template <int BM, int BN>
static void launch_tile_split(hipStream_t s, const uint16_t *A, int lda, const uint16_t *W, int M,
                              int N, int K, int ns, const EpiArgs &e)
{
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    if constexpr (BM == 128 && BN == 128)   /* eight waves (4 x 2) */
        hipLaunchKernelGGL((k_gemm_tile<BM, BN, EPI_STORE, 3, 4>), dim3(tm * tn, ns), dim3(512), 0, s,
                           (const u16 *)A, lda, (const u16 *)W, K, K / ns, e, tm, tn);
    else if constexpr (BM == 32)
        hipLaunchKernelGGL((k_gemm_tile<BM, BN, EPI_STORE, ring_depth<BM, BN>(true), 1>), dim3(tm * tn, ns),
                           dim3(128), 0, s, (const u16 *)A, lda, (const u16 *)W, K, K / ns, e, tm, tn);
    else if (M <= 64 && BM == 64)
        hipLaunchKernelGGL((k_gemm_tile<BM, BN, EPI_STORE, ring_depth<BM, BN>(true), 2>), dim3(tm * tn, ns),
                           dim3(GT), 0, s, (const u16 *)A, lda, (const u16 *)W, K, K / ns, e, tm, tn);
    else
        hipLaunchKernelGGL((k_gemm_tile<BM, BN, EPI_STORE, 3, 2>), dim3(tm * tn, ns), dim3(GT), 0, s,
                           (const u16 *)A, lda, (const u16 *)W, K, K / ns, e, tm, tn);
}

/* Tile choice (measured on MI355X over the Stories and scaled-model shapes):
 * 64 x 64 tiles everywhere, since four of them share a CU and hide each
 * other's latency, except for GEMMs big enough to give every CU a 256 x 128
 * tile (classifiers, the 2048-row W1/W3), where the larger tile's lower L2
 * traffic wins; a decode-row classifier (N >= 16384, which cannot be K-split
 * ahead of its argmax) takes 64 x 64 tiles, twice the work-groups of 64 x 128
 * (C2 0.4480 -> 0.4434, C4 1.148 -> 1.142 ms/step; 32 x 64 lost at C2);
 * up to 32 rows take 32 x 64 tiles of two waves (a 64-row tile would stage and
 * multiply half padding: 5% faster on the scaled model's 32-row QKV and W2;
 * the LDS-staged QKV epilogue keeps its four-wave 64-row tile), and so does
 * the gate GEMM of 33-64 decode rows, which cannot be K-split: two row tiles
 * per column tile put 128 work-groups instead of 64 on the 64-row W1/W3 of
 * Stories (C2 0.4690/0.4683 -> 0.4643/0.4641 ms/step, same box).  A gate GEMM
 * of up to 64 rows whose 32 x 64 tiles would leave half the CUs or more
 * without a work-group takes 32 x 32 tiles of one wave instead (twice the
 * work-groups; each 32-column tile is 16 W1 rows and their 16 W3 partners):
 * C2 0.4618-0.4627 -> 0.4580-0.4583 ms/step, while the scaled model's 176
 * gate tiles of 32 rows lost 1.6% as 352 one-wave tiles.  The decode-row gate
 * tiles (32 x 32 and 32 x 64) walk K in LMK_GATE_KS wave groups, each with its
 * own ring over a contiguous K chunk, their partial tiles summed in LDS before
 * the gate epilogue (the gate cannot be split over work-groups): two groups
 * took C2 0.442-0.444 -> 0.437-0.438 ms/step and C4 1.142-1.143 -> 1.137-1.138
 * (same box, two alternating runs each); four were 0.3% faster again at C2 and
 * 1% slower at C4.  The 64 x 64 gate and QKV tiles of prefill rows (not
 * row-scaled), when they fit one round (at most 256 tiles), take two K groups
 * as well, eight waves, two per SIMD: C1 0.474-0.489 -> 0.467-0.479 ms with
 * the gate, -> 0.461-0.468 with both; the K-split Wo and W2 of those rows in
 * two groups as well gave part of it back.  K is a multiple of the 64-wide
 * stage. */
template <int E, bool RS = false>
static int launch_gemm(hipStream_t s, const uint16_t *A, int lda, const uint16_t *W, int M, int N,
                       int K, const EpiArgs &e)
{
    if (K % BKH) return hipErrorInvalidValue;
    if constexpr (RS) {
        /* row-scaled GEMMs (prefill rows): the two prefill tiles, but QKV only
         * on 64 x 64 (its four-wave 256 x 128 tile with the row scale used
         * in-flight LDS read registers early; the assembly check rejects it) */
        if (E == EPI_GATE && (long)((M + 255) / 256) * ((N + 127) / 128) >= 240) {
            if constexpr (E == EPI_GATE) launch_tile<256, 128, E, true>(s, A, lda, W, M, N, K, e);
        } else launch_tile<64, 64, E, true>(s, A, lda, W, M, N, K, e);
    } else if (M <= 64 && N >= 16384) {
        /* decode-row classifiers (and any other wide decode-row GEMM, the
         * QKV epilogue included) on 64 x 64 tiles */
        launch_tile<64, 64, E>(s, A, lda, W, M, N, K, e);
    }
    else if ((long)((M + 255) / 256) * ((N + 127) / 128) >= 240) launch_tile<256, 128, E>(s, A, lda, W, M, N, K, e);
    else if (E == EPI_GATE && M <= 64 && (long)((M + 31) / 32) * ((N + 63) / 64) <= 128) {
        if constexpr (E == EPI_GATE) launch_tile<32, 32, E>(s, A, lda, W, M, N, K, e);
    } else if (E != EPI_QKV && (M <= 32 || (E == EPI_GATE && M <= 64))) {
        if constexpr (E != EPI_QKV) launch_tile<32, 64, E>(s, A, lda, W, M, N, K, e);
    } else launch_tile<64, 64, E>(s, A, lda, W, M, N, K, e);
    return hipGetLastError();
}

extern "C" int lmk_gemm(hipStream_t s, const uint16_t *A, int lda, const uint16_t *W, int M, int N,
                        int K, int epi, const LMEpilogue *ep)
{
    if (M < 1 || N < 1 || K < BKH || K % BKH || lda < K || !A || !W || !ep) return hipErrorInvalidValue;
    if (epi == EPI_GATE && (N % 32 || !ep->g)) return hipErrorInvalidValue;
    if (epi == EPI_QKV && (!ep->q || !ep->kc || !ep->vc || !ep->slot || !ep->pos || ep->hd < 4 ||
                           (ep->hd & (ep->hd - 1)) ||
                           N != ep->NQ + 2 * ep->NKV))
        return hipErrorInvalidValue;
    if (epi == EPI_RESID && (!ep->out || ep->ldc < N)) return hipErrorInvalidValue;
    if (epi == EPI_RESNORM && (!ep->out || ep->ldc < N || !ep->gain || !ep->u || !ep->ss || N % 32 ||
                               ep->nss != N / 32))
        return hipErrorInvalidValue;
    if (ep->rs_ss && ((epi != EPI_GATE && epi != EPI_QKV) || ep->nss < 4 ||
                      ep->nss > 64 || ep->nss % 4 || ((uintptr_t)ep->rs_ss & 15)))
        return hipErrorInvalidValue;
    if ((epi == EPI_STORE || epi == EPI_ARGMAX) && ep->out && ep->ldc < N) return hipErrorInvalidValue;
    if (epi == EPI_ARGMAX && !ep->part) return hipErrorInvalidValue;
    const EpiArgs e = to_epi(ep, M, N);
    switch (epi) {
    case EPI_STORE: return launch_gemm<EPI_STORE>(s, A, lda, W, M, N, K, e);
    case EPI_RESID: return launch_gemm<EPI_RESID>(s, A, lda, W, M, N, K, e);
    case EPI_GATE:
        return ep->rs_ss ? launch_gemm<EPI_GATE, true>(s, A, lda, W, M, N, K, e)
                         : launch_gemm<EPI_GATE>(s, A, lda, W, M, N, K, e);
    case EPI_QKV:
        return ep->rs_ss ? launch_gemm<EPI_QKV, true>(s, A, lda, W, M, N, K, e)
                         : launch_gemm<EPI_QKV>(s, A, lda, W, M, N, K, e);
    case EPI_ARGMAX: return launch_gemm<EPI_ARGMAX>(s, A, lda, W, M, N, K, e);
    case EPI_RESNORM: return launch_gemm<EPI_RESNORM>(s, A, lda, W, M, N, K, e);
    default: return hipErrorInvalidValue;
    }
}

/* K-split count (measured on MI355X): K is cut into the fewest splits whose
 * k-chunks (a multiple of 64) are at most 512 long, for decode rows (M <= 64,
 * up to LMK_MAX_DEC_SPLIT splits) and for prefill GEMMs with fewer than 128
 * tiles of 64 x 64 (up to LMK_MAX_ROW_SPLIT); larger GEMMs are not split.
 * Decode rows stop at 8 splits even where more would give every CU a
 * work-group: each split adds a partial that is written, read back and summed
 * by the row norm, which loads eight partials per memory round trip.  The
 * W2 of 64 Stories rows at 8 splits instead of 16: C2 0.4580-0.4589 ->
 * 0.4482-0.4490 ms/step; the scaled model's 32-row W2 at 8 instead of 11:
 * C4 1.180-1.182 -> 1.146-1.150 ms/step (6 or 4 were slower on both). */
/* Long-K narrow GEMMs of many rows (the 2048-row W2) run 128 x 128 tiles of
 * eight waves K-split in 2: 12.8 us against 14.5 for unsplit 64 x 64 tiles at
 * C3's W2, while the row norm that adds the partials reads the second one for
 * 0.03 us more. */
static bool wide_split(int M, int N, int K) { return M >= 1024 && N <= 1024 && K >= 2048 && K % 128 == 0; }

extern "C" int lmk_pick_split(int M, int N, int K)
{
    int cap = LMK_MAX_DEC_SPLIT;
    if (M > 64) {
        if (wide_split(M, N, K)) return 2;
        if ((long)((M + 63) / 64) * ((N + 63) / 64) >= 128) return 1;
        cap = LMK_MAX_ROW_SPLIT;
    }
    int best = 1;
    for (int ns = 1; ns <= cap; ns++) {
        if (K % (BKH * ns)) continue;
        best = ns;
        if (K / ns <= 512) break;
    }
    if (M <= 64) {
        /* decode rows: more splits (k-chunks of at least 128) until the grid
         * holds a work-group per CU */
        const long tiles = (N + 63) / 64;
        for (int ns = best + 1; ns <= cap && tiles * best < 256; ns++)
            if (K % (BKH * ns) == 0 && K / ns >= 128) best = ns;
    }
    return best;
}

/* The K-split GEMM (grid: tiles x ns); every k-chunk is a multiple of the
 * 64-wide stage. */
extern "C" int lmk_gemm_split(hipStream_t s, const uint16_t *A, int lda, const uint16_t *W, int M,
                              int N, int K, int ns, float *part)
{
    if (M < 1 || N < 1 || ns < 1 || ns > LMK_MAX_SPLIT || K % (BKH * ns) || lda < K || !A || !W ||
        !part)
        return hipErrorInvalidValue;
    EpiArgs e = {};
    e.M = M; e.N = N; e.out = part; e.ldc = N; e.nparts = (N + 31) / 32;
    e.sstride = (size_t)M * N;
    if (ns == 2 && wide_split(M, N, K)) launch_tile_split<128, 128>(s, A, lda, W, M, N, K, ns, e);
    else if (M <= 32) launch_tile_split<32, 64>(s, A, lda, W, M, N, K, ns, e);
    else launch_tile_split<64, 64>(s, A, lda, W, M, N, K, ns, e);
    return hipGetLastError();
}
