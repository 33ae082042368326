/*
 * k_attn.hip — causal prefill attention on MFMA (gfx950).
 *
 * Rows of a prefill chunk come in whole sequences of S consecutive rows with
 * consecutive positions.  Work-group (query block, head) takes 128 query rows of
 * one sequence; each of its four waves owns 32 rows.  Keys are visited in
 * tiles of 64 positions, 0 .. (last query position of the block), and for each
 * tile (forward.h:72-99, restated as an online softmax):
 *   S  = Q K^T * (1/sqrt(hd))   32x32x16 f16 MFMAs, fp32 accumulation; keys
 *                               after the query's position are masked (-inf)
 *   m' = max(m, rowmax S); P = exp(S - m'); l = l*exp(m - m') + rowsum P;
 *   O  = O*exp(m - m') + P V    P and V rounded to fp16 for the MFMA
 * and finally out = O / l, in fp16 (the operand of the Wo GEMM).  K (row-major) and V (transposed) of the tile are
 * staged in LDS once per work-group; P goes from the accumulator layout to the
 * operand layout through a per-wave LDS tile.
 */
#include "k_common.h"
#include "lm_internal.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));

#define AT 256          /* threads per work-group */
#define BQ 128          /* query rows per work-group */
#define BKV 64          /* keys per tile */

__device__ __forceinline__ f32x16 mfma32h(uint4 a, uint4 b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

/* 8 cache elements -> 8 fp16 */
__device__ __forceinline__ uint4 kv8_f16(const u16 *p) { return *(const uint4 *)p; }
__device__ __forceinline__ uint4 kv8_f16(const float *p)
{
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    f16x8 h;
    h[0] = (_Float16)a.x; h[1] = (_Float16)a.y; h[2] = (_Float16)a.z; h[3] = (_Float16)a.w;
    h[4] = (_Float16)b.x; h[5] = (_Float16)b.y; h[6] = (_Float16)b.z; h[7] = (_Float16)b.w;
    return __builtin_bit_cast(uint4, h);
}

template <int HD, typename KT>
__global__ void __launch_bounds__(AT) k_attn_prefill(
    const float *__restrict__ q, const KT *__restrict__ kc, const KT *__restrict__ vc,
    const int *__restrict__ pos, const int *__restrict__ slot, int S, int nqb, int H, int Hkv,
    int max_seq, u16 *__restrict__ out)
{
    constexpr int KLD = HD + 8;          /* K tile row stride (halves)  */
    constexpr int VLD = BKV + 8;         /* V^T tile row stride (halves) */
    constexpr int PLD = BKV + 8;         /* P tile row stride (halves)  */
    constexpr int KS = HD / 16;          /* MFMA k-steps over head dims */
    constexpr int DT = HD / 32;          /* 32-wide output column tiles */
    __shared__ __attribute__((aligned(16))) u16 sk[BKV * KLD];
    __shared__ __attribute__((aligned(16))) u16 svt[HD * VLD];
    __shared__ __attribute__((aligned(16))) u16 sp[4][32 * PLD];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int seq = blockIdx.x / nqb, qb = blockIdx.x % nqb;
    const int h = blockIdx.y;
    const int kvh = h / (H / Hkv);
    const int NQ = H * HD;
    const int row0 = seq * S + qb * BQ;           /* first row of the block       */
    const int nrows = min(BQ, S - qb * BQ);       /* valid rows of the block      */
    const int p0 = pos[row0];                     /* position of the block's row 0 */
    const int cs = slot[row0];
    const size_t cbase = ((size_t)cs * Hkv + kvh) * max_seq * HD;
    const float scale = 1.0f / sqrtf((float)HD);

    /* this wave's query rows: wr0 .. wr0+31 of the block */
    const int wr0 = wave * 32;
    const bool wave_active = wr0 < nrows;
    /* Q fragments (A operand): row l%32, dims ks*16 + 8*(l/32) .. +8 */
    uint4 qa[KS];
    {
        const int r = min(wr0 + (lane & 31), nrows - 1);
        const float *qp = q + (size_t)(row0 + r) * NQ + h * HD + (lane >> 5) * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qa[ks] = kv8_f16(qp + ks * 16);
    }
    f32x16 o[DT];
#pragma unroll
    for (int j = 0; j < DT; j++) o[j] = (f32x16){};
    float mrow[16], lrow[16];
#pragma unroll
    for (int i = 0; i < 16; i++) { mrow[i] = -INFINITY; lrow[i] = 0.f; }

    const int last_pos = p0 + nrows - 1;          /* last query position of the block */
    const int ntiles = last_pos / BKV + 1;
    const int wave_last = p0 + min(wr0 + 31, nrows - 1);
    for (int kt = 0; kt < ntiles; kt++) {
        const int k0 = kt * BKV;
        /* stage K [key][dim] and V^T [dim][key] of positions k0 .. k0+63 */
        __syncthreads();
        for (int c = tid; c < BKV * HD / 8; c += AT) {
            const int key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
            const int p = min(k0 + key, last_pos);
            const uint4 kk = kv8_f16(kc + cbase + (size_t)p * HD + d0);
            const uint4 vv = kv8_f16(vc + cbase + (size_t)p * HD + d0);
            *(uint4 *)(&sk[key * KLD + d0]) = kk;
            const unsigned vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int j = 0; j < 8; j++)
                svt[(d0 + j) * VLD + key] = (u16)(vw[j >> 1] >> (16 * (j & 1)));
        }
        __syncthreads();
        if (!wave_active || k0 > wave_last) continue;   /* wave-uniform */
        /* S = Q K^T for the 2 key column tiles */
        f32x16 sacc[2];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            sacc[nt] = (f32x16){};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const uint4 kb = *(const uint4 *)(&sk[(nt * 32 + (lane & 31)) * KLD + ks * 16 +
                                                      (lane >> 5) * 8]);
                sacc[nt] = mfma32h(qa[ks], kb, sacc[nt]);
            }
        }
        /* mask, online softmax, P to LDS */
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);   /* row within wave */
            const int qp = p0 + wr0 + r;
            float s0 = sacc[0][i] * scale, s1 = sacc[1][i] * scale;
            const int key0 = k0 + (lane & 31), key1 = key0 + 32;
            if (key0 > qp) s0 = -INFINITY;
            if (key1 > qp) s1 = -INFINITY;
            float mx = fmaxf(s0, s1);
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            const float mn = fmaxf(mrow[i], mx);
            /* rows past the sequence end stay fully masked: mn = -inf */
            const float corr = mn == -INFINITY ? 1.f : expf(mrow[i] - mn);
            const float e0 = mn == -INFINITY ? 0.f : expf(s0 - mn);
            const float e1 = mn == -INFINITY ? 0.f : expf(s1 - mn);
            lrow[i] = lrow[i] * corr + e0 + e1;        /* per-lane partial row sum */
            mrow[i] = mn;
#pragma unroll
            for (int j = 0; j < DT; j++) o[j][i] *= corr;
            sp[wave][r * PLD + (lane & 31)] = f2h(e0);
            sp[wave][r * PLD + 32 + (lane & 31)] = f2h(e1);
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);   /* lgkmcnt(0): this wave's P writes landed */
        __builtin_amdgcn_wave_barrier();
        /* O += P V : A = P [row][key], B = V^T [dim][key] */
#pragma unroll
        for (int ks = 0; ks < BKV / 16; ks++) {
            const uint4 pa = *(const uint4 *)(&sp[wave][(lane & 31) * PLD + ks * 16 + (lane >> 5) * 8]);
#pragma unroll
            for (int j = 0; j < DT; j++) {
                const uint4 vb = *(const uint4 *)(&svt[(j * 32 + (lane & 31)) * VLD + ks * 16 +
                                                       (lane >> 5) * 8]);
                o[j] = mfma32h(pa, vb, o[j]);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (!wave_active) return;
    /* finish the row sums across the 32 lanes of each half and write O / l */
#pragma unroll
    for (int i = 0; i < 16; i++) {
        float l = lrow[i];
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
        const int r = wr0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (r < nrows) {
            const float inv = 1.0f / l;
#pragma unroll
            for (int j = 0; j < DT; j++)
                out[(size_t)(row0 + r) * NQ + h * HD + j * 32 + (lane & 31)] = f2h(o[j][i] * inv);
        }
    }
}

extern "C" int lmk_attn_prefill(hipStream_t s, const float *q, const void *kc, const void *vc,
                                int kv_f32, const int *pos, const int *slot, int S, int nseq,
                                int H, int Hkv, int hd, int max_seq, uint16_t *out)
{
    if (S < 1 || nseq < 1 || H < 1 || Hkv < 1 || H % Hkv || !pos || !slot) return hipErrorInvalidValue;
    const int nqb = (S + BQ - 1) / BQ;
    dim3 grid(nqb * nseq, H);
#define LAUNCH_AP(HD_, KT_)                                                                      \
    hipLaunchKernelGGL((k_attn_prefill<HD_, KT_>), grid, dim3(AT), 0, s, q, (const KT_ *)kc,      \
                       (const KT_ *)vc, pos, slot, S, nqb, H, Hkv, max_seq, out)
    if (hd == 64 && kv_f32) LAUNCH_AP(64, float);
    else if (hd == 64) LAUNCH_AP(64, u16);
    else if (hd == 128 && kv_f32) LAUNCH_AP(128, float);
    else if (hd == 128) LAUNCH_AP(128, u16);
    else return hipErrorInvalidValue;
#undef LAUNCH_AP
    return hipGetLastError();
}
