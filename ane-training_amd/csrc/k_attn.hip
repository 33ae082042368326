/*
 * k_attn.hip — causal prefill attention on MFMA (gfx950).
 *
 * Rows of a prefill chunk come in whole sequences of S consecutive rows with
 * consecutive positions.  Work-group (query block, head) takes 128 query rows of
 * one sequence; each of its four waves owns 32 of them.  Keys are visited in
 * tiles of 64 positions, 0 .. (last query position of the block); for each tile
 * (forward.h:72-99, restated as an online softmax):
 *   S^T = K Q^T * (1/sqrt(hd))  32x32x16 f16 MFMAs, fp32 accumulation; keys after
 *                               the query's position are masked (-inf)
 *   m' = max(m, max_key S); P = exp(S - m'); l = l*exp(m - m') + sum_key P;
 *   O^T = O^T*exp(m - m') + V^T P^T   P and V rounded to fp16 for the MFMA
 * and finally out = O / l, in fp16 (the operand of the Wo GEMM).
 *
 * Computing the transposed scores puts one query in each accumulator column, so
 * lane l holds 32 of the tile's 64 scores of query l % 32 (lane l ^ 32 the other
 * 32): the softmax needs one cross-lane exchange per tile, and the accumulator
 * already has the layout of the B operand of the V^T P^T product, up to an order
 * of the 16 keys of each MFMA step.  That order is undone by storing V^T in LDS
 * with bits 2 and 3 of the key index swapped.  K and V^T of tile t+2 are fetched
 * into registers while tile t computes, and tile t+1 is stored into the other of
 * two LDS buffers.
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

/* LDS column of key k of a tile in V^T: bits 2 and 3 swapped, so that the 8 keys
 * lane l contributes to an MFMA step (4 from each of two groups of 8) are
 * contiguous */
__device__ __forceinline__ int vperm(int k) { return (k & ~12) | ((k & 4) << 1) | ((k >> 1) & 4); }

template <int HD, typename KT>
__global__ void __launch_bounds__(AT) k_attn_prefill(
    const float *__restrict__ q, const KT *__restrict__ kc, const KT *__restrict__ vc,
    const int *__restrict__ pos, const int *__restrict__ slot, int S, int nqb, int H, int Hkv,
    int max_seq, u16 *__restrict__ out)
{
    constexpr int KLD = HD + 8;          /* K tile row stride (halves)   */
    constexpr int VLD = BKV + 8;         /* V^T tile row stride (halves) */
    constexpr int KS = HD / 16;          /* MFMA k-steps over head dims  */
    constexpr int DT = HD / 32;          /* 32-dim row tiles of O^T      */
    constexpr int CPT = BKV * HD / 8 / AT;   /* 16-byte chunks per thread per array */
    static_assert(CPT >= 1 && BKV * HD / 8 % AT == 0, "staging shape");
    __shared__ __attribute__((aligned(16))) u16 sk[2][BKV * KLD];
    __shared__ __attribute__((aligned(16))) u16 svt[2][HD * VLD];

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5;
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
    /* scores are kept in log2 units: exp(x) = exp2(x * log2 e) */
    const float scale = 1.4426950408889634f / sqrtf((float)HD);

    const int last_pos = p0 + nrows - 1;          /* last query position of the block */
    const int ntiles = last_pos / BKV + 1;

    /* K / V chunks of one tile: chunk c = tid + i*AT is key c / (HD/8), dims
     * (c % (HD/8))*8 .. +8; keys past the block's last position repeat it (they
     * are masked for every query that reads them) */
    /* two register sets: tile t sits in set t % 2 from its fetch (two tiles
     * ahead of its use) until it is stored to LDS (one tile ahead) */
    uint4 rk0[CPT], rv0[CPT], rk1[CPT], rv1[CPT];
    auto fetch = [&](int kt, uint4 (&rk)[CPT], uint4 (&rv)[CPT]) {
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c = tid + i * AT, key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
            const size_t off = cbase + (size_t)min(kt * BKV + key, last_pos) * HD + d0;
            rk[i] = kv8_f16(kc + off);
            rv[i] = kv8_f16(vc + off);
        }
    };
    auto stash = [&](int b, const uint4 (&rk)[CPT], const uint4 (&rv)[CPT]) {
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c = tid + i * AT, key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
            *(uint4 *)(&sk[b][key * KLD + d0]) = rk[i];
            const unsigned vw[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
            const int pk = vperm(key);
#pragma unroll
            for (int j = 0; j < 8; j++)
                svt[b][(d0 + j) * VLD + pk] = (u16)(vw[j >> 1] >> (16 * (j & 1)));
        }
    };
    fetch(0, rk0, rv0);
    fetch(1, rk1, rv1);   /* past the last tile: the last position again, unused */

    /* this wave's queries: block rows wr0 .. wr0+31; lane l takes row wr0 + l%32 */
    const int wr0 = wave * 32;
    const bool wave_active = wr0 < nrows;
    const int wave_last = p0 + min(wr0 + 31, nrows - 1);
    const int qrow = wr0 + (lane & 31);
    const int qp = p0 + qrow;                     /* this lane's query position */
    /* Q^T fragments (B operand): query l%32, dims ks*16 + 8*(l/32) .. +8 */
    uint4 qb16[KS];
    {
        const float *qs = q + (size_t)(row0 + min(qrow, nrows - 1)) * NQ + h * HD + g * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qb16[ks] = kv8_f16(qs + ks * 16);
    }
    f32x16 o[DT];
#pragma unroll
    for (int j = 0; j < DT; j++) o[j] = (f32x16){};
    float mrow = -INFINITY, lrow = 0.f;

    stash(0, rk0, rv0);
    __syncthreads();
    /* tile kt: fetch tile kt+2 into the set tile kt left (unconditionally, so
     * the compiler waits only for the older set), compute kt, store kt+1 */
    auto body = [&](int kt, uint4 (&rka)[CPT], uint4 (&rva)[CPT], const uint4 (&rkb)[CPT],
                    const uint4 (&rvb)[CPT]) {
        const int b = kt & 1;
        fetch(kt + 2, rka, rva);
        const int k0 = kt * BKV;
        if (wave_active && k0 <= wave_last) {     /* wave-uniform */
            const u16 *K = sk[b], *VT = svt[b];
            /* S^T tiles: rows = keys nt*32 + (0..31), columns = the wave's queries */
            f32x16 sacc[2];
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                sacc[nt] = (f32x16){};
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const uint4 ka = *(const uint4 *)(&K[(nt * 32 + (lane & 31)) * KLD + ks * 16 + g * 8]);
                    sacc[nt] = mfma32h(ka, qb16[ks], sacc[nt]);
                }
            }
            /* element i of tile nt is key k0 + nt*32 + 8*(i/4) + 4*g + i%4 */
            float mx = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = k0 + nt * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                    const float v = key > qp ? -INFINITY : sacc[nt][i] * scale;
                    sacc[nt][i] = v;
                    mx = fmaxf(mx, v);
                }
            mx = fmaxf(mx, xor32_f(mx));
            const float mn = fmaxf(mrow, mx);
            /* a query with every key so far masked keeps m = -inf: nothing to scale */
            const float corr = mn == -INFINITY ? 1.f : exp2f(mrow - mn);
            const float sub = mn == -INFINITY ? 0.f : mn;
            float ls = 0.f;
            uint4 pb[2][2];
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    f16x8 hv;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const float e = exp2f(sacc[nt][8 * hh + j] - sub);
                        ls += e;
                        hv[j] = (_Float16)e;
                    }
                    pb[nt][hh] = __builtin_bit_cast(uint4, hv);
                }
            lrow = lrow * corr + ls;               /* per-lane partial row sum */
            mrow = mn;
#pragma unroll
            for (int j = 0; j < DT; j++) o[j] *= corr;
            /* O^T += V^T P^T over the 4 steps of 16 keys */
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++)
#pragma unroll
                    for (int j = 0; j < DT; j++) {
                        const uint4 va = *(const uint4 *)(&VT[(j * 32 + (lane & 31)) * VLD + nt * 32 +
                                                              hh * 16 + g * 8]);
                        o[j] = mfma32h(va, pb[nt][hh], o[j]);
                    }
        }
        if (kt + 1 < ntiles) stash(b ^ 1, rkb, rvb);
        __syncthreads();
    };
    for (int kt = 0; kt < ntiles; kt += 2) {
        body(kt, rk0, rv0, rk1, rv1);
        if (kt + 1 < ntiles) body(kt + 1, rk1, rv1, rk0, rv0);
    }
    if (!wave_active) return;
    /* finish the row sum across the lane pair and write O / l:
     * element i of o[j] is dim j*32 + 8*(i/4) + 4*g + i%4 of query l%32 */
    const float l = lrow + xor32_f(lrow);
    if (qrow < nrows) {
        const float inv = 1.0f / l;
        u16 *op = out + (size_t)(row0 + qrow) * NQ + h * HD;
#pragma unroll
        for (int j = 0; j < DT; j++)
#pragma unroll
            for (int i4 = 0; i4 < 4; i4++) {
                const unsigned lo = (unsigned)f2h(o[j][4 * i4] * inv) |
                                    ((unsigned)f2h(o[j][4 * i4 + 1] * inv) << 16);
                const unsigned hi = (unsigned)f2h(o[j][4 * i4 + 2] * inv) |
                                    ((unsigned)f2h(o[j][4 * i4 + 3] * inv) << 16);
                *(uint2 *)(op + j * 32 + 8 * i4 + 4 * g) = make_uint2(lo, hi);
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
