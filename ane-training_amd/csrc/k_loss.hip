/*
 * k_loss.hip — next-token log-probabilities of prefill logit rows on the
 * device: the terms of model_forward's loss (training/forward.h:174-183), so a
 * caller gets the mean cross-entropy without copying the logits to the host.
 *
 * Row r of a chunk of sequences of S rows is token t = r % S of its sequence;
 * for t < S-1 its target is the next token, tok[r + 1]:
 *     lp[r] = logits[r][tgt] - mx - log(sum_i exp(logits[r][i] - mx)),
 *     mx = max(-1e9, max_i logits[r][i])          (forward.h:175-180)
 * and the last row of each sequence, which has no target, gets 0.  The host
 * sums -lp[r] over each sequence in the reference's order and divides by S-1.
 *
 * One 256-thread work-group per row.  Each thread keeps a running (max, sum of
 * exp) over its float4 groups, rescaling the sum when the max rises, so the
 * row is read once; the per-thread pairs are merged across the wave and then
 * across the four waves.  fp32 throughout.
 */
#include "k_common.h"
#include "lm_internal.h"

#define LT 256   /* threads per work-group */

/* Merge of two running (max, sum exp(v - max)) pairs. */
__device__ __forceinline__ void lse_merge(float &m, float &s, float m2, float s2)
{
    const float mm = fmaxf(m, m2);
    s = s * expf(m - mm) + s2 * expf(m2 - mm);
    m = mm;
}

__device__ __forceinline__ void lse_add(float &m, float &s, float v)
{
    if (v > m) {
        s = s * expf(m - v) + 1.0f;
        m = v;
    } else {
        s += expf(v - m);
    }
}

__global__ void __launch_bounds__(LT) k_row_logprob(const float *__restrict__ logits, int V,
                                                    const int *__restrict__ tok, int S, int M,
                                                    float *__restrict__ lp)
{
    const int r = blockIdx.x;
    const int t = r % S;
    if (t == S - 1) {   /* the sequence's last row: no target (uniform branch) */
        if (threadIdx.x == 0) lp[r] = 0.f;
        return;
    }
    const float *row = logits + (size_t)r * V;
    const int tgt = tok[r + 1];
    float m = -1e9f, s = 0.f;   /* forward.h:175: mx starts at -1e9 */
    const int nv = V >> 2;      /* float4 groups (rows are 16-byte aligned: V % 4 == 0) */
    const float4 *row4 = (const float4 *)row;
    for (int i = threadIdx.x; i < nv; i += LT) {
        const float4 v = row4[i];
        lse_add(m, s, v.x);
        lse_add(m, s, v.y);
        lse_add(m, s, v.z);
        lse_add(m, s, v.w);
    }
    for (int i = (nv << 2) + threadIdx.x; i < V; i += LT) lse_add(m, s, row[i]);
    /* across the wave */
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float m2 = __shfl_xor(m, off), s2 = __shfl_xor(s, off);
        lse_merge(m, s, m2, s2);
    }
    __shared__ float sm_m[LT / 64], sm_s[LT / 64];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sm_m[wave] = m;
        sm_s[wave] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float mm = sm_m[0], ss = sm_s[0];
#pragma unroll
        for (int w = 1; w < LT / 64; w++) lse_merge(mm, ss, sm_m[w], sm_s[w]);
        lp[r] = row[tgt] - mm - logf(ss);   /* forward.h:181 */
    }
}

extern "C" int lmk_row_logprob(hipStream_t s, const float *logits, int V, const int *tok, int S, int M,
                               float *lp)
{
    if (!logits || !tok || !lp || V < 1 || V % 4 || S < 2 || M < 1 || M % S) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_row_logprob, dim3(M), dim3(LT), 0, s, logits, V, tok, S, M, lp);
    return hipGetLastError();
}
