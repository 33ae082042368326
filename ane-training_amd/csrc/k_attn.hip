/*
 * k_attn.hip — causal prefill attention on MFMA (gfx950).
 *
 * Rows of a prefill chunk come in whole sequences of S consecutive rows with
 * consecutive positions.  Keys are visited in tiles of 64 positions, 0 ..
 * (last query position of the block); a wave owning 32 queries updates its
 * online softmax with each tile (forward.h:72-99, scores in log2 units):
 *   S^T = K Q^T * (log2 e / sqrt(hd))   32x32x16 f16 MFMAs, fp32 accumulation;
 *                                       keys after the query's position masked
 *   m' = max_key S if it exceeds m by more than 8, else m;
 *   P = 2^(S - m'); l = l*2^(m - m') + sum_key P;
 *   O^T = O^T*2^(m - m') + V^T P^T      P and V rounded to fp16 for the MFMA
 * and out = O / l, in fp16 (the operand of the Wo GEMM).  Any m' at or below
 * the true maximum gives the same O / l; keeping m unless it falls 8 behind
 * bounds P by 2^8 and skips the rescale of O on most tiles.  Only tiles that
 * hold a key after some query of the wave are masked.
 *
 * Computing the transposed scores puts one query in each accumulator column, so
 * lane l holds 32 of the tile's 64 scores of query l % 32 (lane l ^ 32 the other
 * 32): the softmax needs one cross-lane exchange per tile, and the accumulator
 * already has the layout of the B operand of the V^T P^T product, up to an order
 * of the 16 keys of each MFMA step.  That order is undone by storing V^T in LDS
 * with bits 2 and 3 of the key index swapped; V^T rows are XOR-swizzled in
 * 16-byte units so that neither the transposing writes nor the fragment reads
 * conflict in the LDS banks.
 *
 * Two work-group shapes share that per-tile step:
 *   k_attn_prefill_blk    128 queries per work-group, 32 per wave; the four
 *                         waves share each staged tile (K/V of tile t+2 in
 *                         registers while tile t computes, tile t+1 in the other
 *                         LDS buffer).  Least K/V traffic: for many blocks.
 *   k_attn_prefill_split  32 queries per work-group; the four waves split the
 *                         key tiles round-robin, each staging its own, and merge
 *                         their (m, l, O) through LDS.  The last query block waits
 *                         for a quarter of its tiles: for few blocks (short
 *                         prompts), where the work-group count is the limit.
 */
#include "k_common.h"
#include "lm_internal.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));

#define AT 256          /* threads per work-group (4 waves) */
#define NW 4            /* waves per work-group */
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
 * contiguous.  The map is its own inverse. */
__device__ __forceinline__ int vperm(int k) { return (k & ~12) | ((k & 4) << 1) | ((k >> 1) & 4); }

/* V^T tile: row d (a head dim) holds the tile's BKV keys in vperm order as 16-byte
 * units; unit u of row d sits in slot u ^ vswz(d).  The 8 rows that one 16-byte
 * fragment read serves per LDS cycle (d .. d+7) and the 8 rows d0 + j, d0 = 0, 8,
 * .. 56 that one staging write serves then fall in 8 different slots: no bank
 * conflicts on either side. */
__device__ __forceinline__ int vswz(int d) { return (d ^ (d >> 3)) & 7; }
__device__ __forceinline__ int vt_off(int d, int col) { return d * BKV + (((col >> 3) ^ vswz(d)) << 3) + (col & 7); }

/* Staging unit `pr` (0 .. BKV/2 * HD/8 - 1) of a tile: dims d0 .. d0+7 of the keys
 * in V^T columns pk and pk+1 (keys vperm(pk), vperm(pk) + 1: pk is even and vperm
 * keeps bit 0).  Consecutive units take the 8 dim groups of one column pair, then
 * the next pair: one wave's 32-lane half covers 4 pairs of one 16-byte unit. */
template <int HD>
__device__ __forceinline__ void pair_of(int pr, int &pk, int &d0)
{
    pk = ((pr >> 3) & (BKV / 2 - 1)) * 2;
    d0 = ((pr & 7) + (pr / (BKV / 2 * 8)) * 8) * 8;
}

/* Store one staging unit: K rows of KLD halves (two 16-byte writes), V^T in the
 * swizzled layout (8 dword writes, each the two keys of one dim). */
template <int KLD>
__device__ __forceinline__ void stage_pair(u16 *sk, u16 *svt, int pk, int d0, uint4 ka, uint4 kb,
                                           uint4 va, uint4 vb)
{
    const int key = vperm(pk);
    *(uint4 *)(&sk[key * KLD + d0]) = ka;
    *(uint4 *)(&sk[(key + 1) * KLD + d0]) = kb;
    const unsigned wa[4] = {va.x, va.y, va.z, va.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const unsigned a = wa[j >> 1], b = wb[j >> 1];
        const unsigned w = (j & 1) ? (a >> 16) | (b & 0xffff0000u) : (a & 0xffffu) | (b << 16);
        *(unsigned *)(&svt[vt_off(d0 + j, pk)]) = w;
    }
}

/* The running maximum m of a query is raised only when a tile's maximum exceeds
 * it by more than this (log2 units), so P = 2^(S - m) <= 2^8 stays well inside
 * fp16 and the rescale of O and l is skipped for most tiles. */
#define M_SLACK 8.0f

/* Online-softmax update of one wave's 32 queries (lane l: query l % 32 at
 * position qp) with the staged tile of keys k0 .. k0+63 (K rows, V^T).  MASK:
 * the tile holds keys after some query's position (wave-uniform choice). */
template <int HD, int KLD, bool MASK>
__device__ __forceinline__ void tile_update(const u16 *sk, const u16 *svt, const uint4 (&qb16)[HD / 16],
                                            int k0, int qp, float scale, f32x16 (&o)[HD / 32],
                                            float &mrow, float &lrow)
{
    constexpr int KS = HD / 16, DT = HD / 32;
    const int lane = threadIdx.x & 63, g = lane >> 5;
    /* S^T tiles: rows = keys nt*32 + (0..31), columns = the wave's queries */
    f32x16 sacc[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        sacc[nt] = (f32x16){};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const uint4 ka = *(const uint4 *)(&sk[(nt * 32 + (lane & 31)) * KLD + ks * 16 + g * 8]);
            sacc[nt] = mfma32h(ka, qb16[ks], sacc[nt]);
        }
    }
    /* element i of tile nt is key k0 + nt*32 + 8*(i/4) + 4*g + i%4; the maximum
     * is taken over the raw dot products (scale > 0) */
    float mx = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            if constexpr (MASK) {
                const int key = k0 + nt * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                if (key > qp) sacc[nt][i] = -INFINITY;
            }
            mx = fmaxf(mx, sacc[nt][i]);
        }
    mx = fmaxf(mx, xor32_f(mx)) * scale;
    /* a query with every key so far masked keeps m = -inf (and O = l = 0) */
    const bool raise = mx > mrow + M_SLACK;
    if (__builtin_amdgcn_ballot_w64(raise)) {     /* wave-uniform */
        const float mn = raise ? mx : mrow;
        const float corr = __builtin_amdgcn_exp2f(mrow - mn);   /* 0 from m = -inf, 1 if kept */
        lrow *= corr;
#pragma unroll
        for (int j = 0; j < DT; j++) o[j] *= corr;
        mrow = mn;
    }
    const float sub = mrow == -INFINITY ? 0.f : mrow;
    float ls = 0.f;
    uint4 pb[2][2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            f16x8 hv;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float e = __builtin_amdgcn_exp2f(fmaf(sacc[nt][8 * hh + j], scale, -sub));
                ls += e;
                hv[j] = (_Float16)e;
            }
            pb[nt][hh] = __builtin_bit_cast(uint4, hv);
        }
    lrow += ls;                                /* per-lane partial row sum */
    /* O^T += V^T P^T over the 4 steps of 16 keys */
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int j = 0; j < DT; j++) {
                const uint4 va = *(const uint4 *)(&svt[vt_off(j * 32 + (lane & 31), nt * 32 + hh * 16 + g * 8)]);
                o[j] = mfma32h(va, pb[nt][hh], o[j]);
            }
}

/* Q^T fragments (B operand) of a wave: query row `row` (fp32 q [rows, NQ]),
 * dims ks*16 + 8*(l/32) .. +8 of head h */
template <int HD>
__device__ __forceinline__ void load_q(const float *q, size_t row, int NQ, int h, uint4 (&qb16)[HD / 16])
{
    const float *qs = q + row * NQ + h * HD + ((threadIdx.x & 63) >> 5) * 8;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ks++) qb16[ks] = kv8_f16(qs + ks * 16);
}

/* ---- 128-query blocks, shared tiles ---------------------------------------- */

#define BQB 128         /* query rows per work-group */

template <int HD, typename KT>
__global__ void __launch_bounds__(AT) k_attn_prefill_blk(
    const float *__restrict__ q, const KT *__restrict__ kc, const KT *__restrict__ vc,
    const int *__restrict__ pos, const int *__restrict__ slot, int S, int nqb, int H, int Hkv,
    int max_seq, u16 *__restrict__ out)
{
    constexpr int KLD = HD + 8;          /* K tile row stride (halves)   */
    constexpr int DT = HD / 32;          /* 32-dim row tiles of O^T      */
    constexpr int PPT = BKV * HD / 16 / AT;  /* staging units per thread */
    static_assert(PPT >= 1 && BKV * HD / 16 % AT == 0, "staging shape");
    __shared__ __attribute__((aligned(16))) u16 sk[2][BKV * KLD];
    __shared__ __attribute__((aligned(16))) u16 svt[2][HD * BKV];

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int seq = small_div(blockIdx.x, nqb), qb = blockIdx.x - seq * nqb;
    const int h = blockIdx.y;
    const int kvh = small_div(h, small_div(H, Hkv));
    const int NQ = H * HD;
    const int row0 = seq * S + qb * BQB;          /* first row of the block       */
    const int nrows = min(BQB, S - qb * BQB);     /* valid rows of the block      */
    const int p0 = pos[row0];                     /* position of the block's row 0 */
    const int cs = slot[row0];
    const size_t cbase = ((size_t)cs * Hkv + kvh) * max_seq * HD;
    /* scores are kept in log2 units: exp(x) = exp2(x * log2 e) */
    const float scale = 1.4426950408889634f / sqrtf((float)HD);
    const int last_pos = p0 + nrows - 1;          /* last query position of the block */
    const int ntiles = last_pos / BKV + 1;

    /* K / V of one tile: thread t stages units t + i*AT (two keys, 8 dims each:
     * [0] key, [1] key + 1); keys past the block's last position repeat it (they
     * are masked for every query that reads them).  Two register sets: tile t
     * sits in set t % 2 from its fetch (two tiles ahead of its use) until it is
     * stored to LDS (one tile ahead). */
    uint4 rk0[PPT][2], rv0[PPT][2], rk1[PPT][2], rv1[PPT][2];
    auto fetch = [&](int kt, uint4 (&rk)[PPT][2], uint4 (&rv)[PPT][2]) {
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            int pk, d0;
            pair_of<HD>(tid + i * AT, pk, d0);
            const int key = kt * BKV + vperm(pk);
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const size_t off = cbase + (size_t)min(key + e, last_pos) * HD + d0;
                rk[i][e] = kv8_f16(kc + off);
                rv[i][e] = kv8_f16(vc + off);
            }
        }
    };
    auto stash = [&](int b, const uint4 (&rk)[PPT][2], const uint4 (&rv)[PPT][2]) {
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            int pk, d0;
            pair_of<HD>(tid + i * AT, pk, d0);
            stage_pair<KLD>(sk[b], svt[b], pk, d0, rk[i][0], rk[i][1], rv[i][0], rv[i][1]);
        }
    };
    fetch(0, rk0, rv0);
    fetch(1, rk1, rv1);   /* past the last tile: the last position again, unused */

    /* this wave's queries: block rows wr0 .. wr0+31; lane l takes row wr0 + l%32 */
    const int wr0 = wave * 32;
    const bool wave_active = wr0 < nrows;
    const int wave_first = p0 + wr0, wave_last = p0 + min(wr0 + 31, nrows - 1);
    const int qrow = wr0 + (lane & 31);
    const int qp = p0 + qrow;                     /* this lane's query position */
    uint4 qb16[HD / 16];
    load_q<HD>(q, (size_t)(row0 + min(qrow, nrows - 1)), NQ, h, qb16);
    f32x16 o[DT];
#pragma unroll
    for (int j = 0; j < DT; j++) o[j] = (f32x16){};
    float mrow = -INFINITY, lrow = 0.f;

    stash(0, rk0, rv0);
    __syncthreads();
    /* tile kt: fetch tile kt+2 into the set tile kt left (unconditionally, so
     * the compiler waits only for the older set), compute kt, store kt+1 */
    auto body = [&](int kt, uint4 (&rka)[PPT][2], uint4 (&rva)[PPT][2], const uint4 (&rkb)[PPT][2],
                    const uint4 (&rvb)[PPT][2]) {
        const int b = kt & 1;
        fetch(kt + 2, rka, rva);
        const int k0 = kt * BKV;
        if (wave_active && k0 <= wave_last) {     /* wave-uniform */
            if (k0 + BKV - 1 <= wave_first)       /* every key visible to every query */
                tile_update<HD, KLD, false>(sk[b], svt[b], qb16, k0, qp, scale, o, mrow, lrow);
            else
                tile_update<HD, KLD, true>(sk[b], svt[b], qb16, k0, qp, scale, o, mrow, lrow);
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

/* ---- 32-query blocks, key tiles split across the waves ---------------------- */

#define BQS 32          /* query rows per work-group */

template <int HD, typename KT>
__global__ void __launch_bounds__(AT) k_attn_prefill_split(
    const float *__restrict__ q, const KT *__restrict__ kc, const KT *__restrict__ vc,
    const int *__restrict__ pos, const int *__restrict__ slot, int S, int nqb, int H, int Hkv,
    int max_seq, u16 *__restrict__ out)
{
    constexpr int KLD = HD + 8;          /* K tile row stride (halves)   */
    constexpr int KS = HD / 16;          /* MFMA k-steps over head dims  */
    constexpr int DT = HD / 32;          /* 32-dim row tiles of O^T      */
    constexpr int PPL = BKV * HD / 16 / 64;  /* staging units per lane (one wave stages a tile) */
    constexpr bool PREF = HD == 64 && sizeof(KT) == 2;   /* next tile in registers */
    constexpr int STAGE = BKV * KLD + HD * BKV;          /* halves of one wave's K and V^T */
    static_assert(BKV * HD / 8 % 256 == 0, "staging shape");
    constexpr int MLD = HD + 1;                          /* merge row stride (floats) */
    static_assert(NW * STAGE * 2 >= (NW * BQS * MLD + 2 * NW * BQS) * 4, "merge area fits the staging area");
    __shared__ __attribute__((aligned(16))) u16 stg[NW * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int seq = small_div(blockIdx.x, nqb), qb = blockIdx.x - seq * nqb;
    const int h = blockIdx.y;
    const int kvh = small_div(h, small_div(H, Hkv));
    const int NQ = H * HD;
    const int row0 = seq * S + qb * BQS;           /* first row of the block       */
    const int nrows = min(BQS, S - qb * BQS);       /* valid rows of the block      */
    const int p0 = pos[row0];                     /* position of the block's row 0 */
    const int cs = slot[row0];
    const size_t cbase = ((size_t)cs * Hkv + kvh) * max_seq * HD;
    /* scores are kept in log2 units: exp(x) = exp2(x * log2 e) */
    const float scale = 1.4426950408889634f / sqrtf((float)HD);
    const int last_pos = p0 + nrows - 1;          /* last query position of the block */
    const int ntiles = last_pos / BKV + 1;
    u16 *sk = stg + wave * STAGE, *svt = sk + BKV * KLD;

    /* K / V of one tile for this wave: lane l stages units l + i*64 (two keys, 8
     * dims each); keys past the block's last position repeat it (masked for
     * every query that reads them) */
    auto load = [&](int kt, int i, uint4 (&k8)[2], uint4 (&v8)[2]) {
        int pk, d0;
        pair_of<HD>(lane + i * 64, pk, d0);
        const int key = kt * BKV + vperm(pk);
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const size_t off = cbase + (size_t)min(key + e, last_pos) * HD + d0;
            k8[e] = kv8_f16(kc + off);
            v8[e] = kv8_f16(vc + off);
        }
    };
    auto put = [&](int i, const uint4 (&k8)[2], const uint4 (&v8)[2]) {
        int pk, d0;
        pair_of<HD>(lane + i * 64, pk, d0);
        stage_pair<KLD>(sk, svt, pk, d0, k8[0], k8[1], v8[0], v8[1]);
    };
    /* hd 64 with an fp16 cache: the whole next tile is held in registers while
     * the current one computes; otherwise a tile is staged 2 units at a time */
    constexpr int RC = PREF ? PPL : 1;
    uint4 rk[RC][2], rv[RC][2];
    auto fetch = [&](int kt) {
#pragma unroll
        for (int i = 0; i < RC; i++) load(kt, i, rk[i], rv[i]);
    };
    auto stage = [&](int kt) {
        if constexpr (PREF) {
#pragma unroll
            for (int i = 0; i < PPL; i++) put(i, rk[i], rv[i]);
        } else {
#pragma unroll
            for (int i0 = 0; i0 < PPL; i0 += 2) {
                uint4 k4[2][2], v4[2][2];
#pragma unroll
                for (int i = 0; i < 2; i++) load(kt, i0 + i, k4[i], v4[i]);
#pragma unroll
                for (int i = 0; i < 2; i++) put(i0 + i, k4[i], v4[i]);
            }
        }
    };
    if (PREF && wave < ntiles) fetch(wave);       /* wave-uniform */

    /* lane l takes query row l%32 of the block */
    const int qrow = lane & 31;
    const int qp = p0 + qrow;                     /* this lane's query position */
    uint4 qb16[KS];
    load_q<HD>(q, (size_t)(row0 + min(qrow, nrows - 1)), NQ, h, qb16);
    f32x16 o[DT];
#pragma unroll
    for (int j = 0; j < DT; j++) o[j] = (f32x16){};
    float mrow = -INFINITY, lrow = 0.f;

    for (int kt = wave; kt < ntiles; kt += NW) {  /* wave-uniform */
        stage(kt);
        __builtin_amdgcn_s_waitcnt(0xc07f);       /* lgkmcnt(0): the wave's LDS writes landed */
        __builtin_amdgcn_wave_barrier();
        if (PREF && kt + NW < ntiles) fetch(kt + NW);
        if (kt * BKV + BKV - 1 <= p0)             /* wave-uniform: no key after any query */
            tile_update<HD, KLD, false>(sk, svt, qb16, kt * BKV, qp, scale, o, mrow, lrow);
        else
            tile_update<HD, KLD, true>(sk, svt, qb16, kt * BKV, qp, scale, o, mrow, lrow);
        __builtin_amdgcn_wave_barrier();           /* the tile's reads precede the next stash */
    }
    /* merge the four waves: each writes (m, l, O) of its 32 queries; element i of
     * o[j] is dim j*32 + 8*(i/4) + 4*g + i%4 of query l%32 */
    const float lsum = lrow + xor32_f(lrow);
    __syncthreads();                               /* every wave is done with its staging area */
    float *mo = (float *)stg;                      /* [NW][BQS][MLD] outputs */
    float *mm = mo + NW * BQS * MLD, *ml = mm + NW * BQS;
    if (g == 0) {
        mm[wave * BQS + qrow] = mrow;
        ml[wave * BQS + qrow] = lsum;
    }
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            mo[(wave * BQS + qrow) * MLD + j * 32 + 8 * (i >> 2) + 4 * g + (i & 3)] = o[j][i];
    __syncthreads();
    /* thread t: query t / 8, dims (t % 8) * HD/8 .. +HD/8 */
    constexpr int DPT = HD / 8;
    const int r = tid >> 3, d0 = (tid & 7) * DPT;
    if (r < nrows) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, mm[w * BQS + r]);
        float wgt[NW], L = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float mw = mm[w * BQS + r];
            wgt[w] = mw == -INFINITY ? 0.f : exp2f(mw - M);
            L = fmaf(ml[w * BQS + r], wgt[w], L);
        }
        const float inv = 1.0f / L;
        u16 *op = out + (size_t)(row0 + r) * NQ + h * HD + d0;
#pragma unroll
        for (int d = 0; d < DPT; d += 2) {
            float a = 0.f, bsum = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                a = fmaf(mo[(w * BQS + r) * MLD + d0 + d], wgt[w], a);
                bsum = fmaf(mo[(w * BQS + r) * MLD + d0 + d + 1], wgt[w], bsum);
            }
            *(unsigned *)(op + d) = (unsigned)f2h(a * inv) | ((unsigned)f2h(bsum * inv) << 16);
        }
    }
}

/* Work-group count of the 128-query kernel below which the 32-query kernel
 * is used (measured: 24 blocks of 128 (one 256-token prompt, 12 heads) run
 * 1.7x faster split; 192 (eight prompts) 1.3x faster shared). */
#define BLK_MIN_WGS 128

extern "C" int lmk_attn_prefill(hipStream_t s, const float *q, const void *kc, const void *vc,
                                int kv_f32, const int *pos, const int *slot, int S, int nseq,
                                int H, int Hkv, int hd, int max_seq, uint16_t *out)
{
    if (S < 1 || nseq < 1 || H < 1 || Hkv < 1 || H % Hkv || !pos || !slot) return hipErrorInvalidValue;
    if (hd != 64 && hd != 128) return hipErrorInvalidValue;
    const int nqb_blk = (S + BQB - 1) / BQB;
    if ((long)nqb_blk * nseq * H >= BLK_MIN_WGS) {
        dim3 grid(nqb_blk * nseq, H);
#define LAUNCH_AP(HD_, KT_)                                                                      \
    hipLaunchKernelGGL((k_attn_prefill_blk<HD_, KT_>), grid, dim3(AT), 0, s, q, (const KT_ *)kc,  \
                       (const KT_ *)vc, pos, slot, S, nqb_blk, H, Hkv, max_seq, out)
        if (hd == 64 && kv_f32) LAUNCH_AP(64, float);
        else if (hd == 64) LAUNCH_AP(64, u16);
        else if (kv_f32) LAUNCH_AP(128, float);
        else LAUNCH_AP(128, u16);
#undef LAUNCH_AP
    } else {
        const int nqb = (S + BQS - 1) / BQS;
        dim3 grid(nqb * nseq, H);
#define LAUNCH_AP(HD_, KT_)                                                                        \
    hipLaunchKernelGGL((k_attn_prefill_split<HD_, KT_>), grid, dim3(AT), 0, s, q, (const KT_ *)kc, \
                       (const KT_ *)vc, pos, slot, S, nqb, H, Hkv, max_seq, out)
        if (hd == 64 && kv_f32) LAUNCH_AP(64, float);
        else if (hd == 64) LAUNCH_AP(64, u16);
        else if (kv_f32) LAUNCH_AP(128, float);
        else LAUNCH_AP(128, u16);
#undef LAUNCH_AP
    }
    return hipGetLastError();
}
