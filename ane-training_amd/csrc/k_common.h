/*
 * k_common.h — device helpers shared by the gfx950 kernels.
 *
 * Wave64 reductions use DPP row operations (quad_perm, row_half_mirror,
 * row_mirror, row_bcast15/31 — the GFX9-family DPP controls that CDNA4 keeps);
 * fp16 weights are read as 128-bit (8 x binary16) vectors and widened to fp32
 * in registers.
 */
#ifndef K_COMMON_H
#define K_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef unsigned short u16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float h2f(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ u16 f2h(float f) { return __builtin_bit_cast(u16, (_Float16)f); }

/* 8 binary16 values packed in a uint4 -> 8 floats. */
__device__ __forceinline__ void unpack8(const uint4 v, float f[8])
{
    f16x2 a = __builtin_bit_cast(f16x2, v.x);
    f16x2 b = __builtin_bit_cast(f16x2, v.y);
    f16x2 c = __builtin_bit_cast(f16x2, v.z);
    f16x2 d = __builtin_bit_cast(f16x2, v.w);
    f[0] = (float)a.x; f[1] = (float)a.y; f[2] = (float)b.x; f[3] = (float)b.y;
    f[4] = (float)c.x; f[5] = (float)c.y; f[6] = (float)d.x; f[7] = (float)d.y;
}

/* KV-cache element access: binary16 (u16 bits) or fp32. */
template <typename KT> __device__ __forceinline__ KT kv_pack(float v);
template <> __device__ __forceinline__ u16 kv_pack<u16>(float v) { return f2h(v); }
template <> __device__ __forceinline__ float kv_pack<float>(float v) { return v; }

/* v as stored in a cache of element type KT, read back as fp32. */
template <typename KT> __device__ __forceinline__ float kv_round(float v);
template <> __device__ __forceinline__ float kv_round<u16>(float v) { return h2f(f2h(v)); }
template <> __device__ __forceinline__ float kv_round<float>(float v) { return v; }

/* 8 consecutive cache elements -> fp32 (one 16-byte or two 16-byte loads). */
__device__ __forceinline__ void kv_load8(const u16 *p, float f[8]) { unpack8(*(const uint4 *)p, f); }
__device__ __forceinline__ void kv_load8(const float *p, float f[8])
{
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

/* DPP move of v; lanes outside row_mask (or reading an invalid lane) get 0. */
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

#define DPP_QUAD_XOR1 0xB1     /* quad_perm [1,0,3,2] */
#define DPP_QUAD_XOR2 0x4E     /* quad_perm [2,3,0,1] */
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_BCAST15 0x142
#define DPP_ROW_BCAST31 0x143
#define DPP_ROW_ROR8 0x128      /* row_ror:8, lane l of a 16-lane row reads lane l ^ 8 */

/* Sum over each 32-lane half: afterwards lanes 16..31 hold the sum of lanes
 * 0..31 and lanes 48..63 the sum of lanes 32..63 (read lanes 31 and 63). */
__device__ __forceinline__ float half_wave_sum(float v)
{
    v += dpp_f<DPP_QUAD_XOR1>(v);
    v += dpp_f<DPP_QUAD_XOR2>(v);
    v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_f<DPP_ROW_MIRROR>(v);
    v += dpp_f<DPP_ROW_BCAST15, 0xA>(v);
    return v;
}

/* Value of lane l ^ 16 (l ^ 32): v_permlane16_swap (v_permlane32_swap), a VALU
 * exchange.  Swapping v with itself gives (v[l & ~16], v[l | 16]) in every lane
 * (checked on the device), so the partner is the element the lane's own bit does
 * not name. */
__device__ __forceinline__ float xor16_f(float v)
{
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32_f(float v)
{
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

/* DPP move of an int that leaves lanes outside row_mask unchanged. */
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_keep_i(int v)
{
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xF, false);
}

/* Sum over the wave, returned uniformly (scalar). */
__device__ __forceinline__ float wave_sum(float v)
{
    v = half_wave_sum(v);
    v += dpp_f<DPP_ROW_BCAST31, 0xC>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

/* n / d for 0 <= n < 2^20 and 1 <= d < 2^12 without the integer-division
 * sequence: the quotient (n + 0.5) / d keeps at least 1/(2d) from an integer,
 * far more than the error of the hardware reciprocal and the product
 * (about n * 2^-22), so truncation gives the exact integer quotient. */
__device__ __forceinline__ int small_div(int n, int d)
{
    return (int)(((float)n + 0.5f) * __builtin_amdgcn_rcpf((float)d));
}

__device__ __forceinline__ float readlane_f(float v, int lane)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

/* Max over the wave via xor shuffles (uniform result). */
__device__ __forceinline__ float wave_max_shfl(float v)
{
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum_shfl(float v)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

/* Argmax combine: larger value wins, lowest index on ties (generate.m:129-136
 * scans upward with a strict '>'), NaN never wins. */
__device__ __forceinline__ void argmax_combine(float &bv, int &bi, float v, int i)
{
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ void argmax_dpp_step(float &bv, int &bi)
{
    const float ov = __builtin_bit_cast(float, dpp_keep_i<CTRL, ROW_MASK>(__builtin_bit_cast(int, bv)));
    const int oi = dpp_keep_i<CTRL, ROW_MASK>(bi);
    argmax_combine(bv, bi, ov, oi);
}

/* (max, index) over each 32-lane half with DPP moves (VALU only): afterwards
 * lanes 16..31 hold the result of lanes 0..31 and lanes 48..63 that of lanes
 * 32..63 (read lanes 31 and 63).  Lowest index on ties. */
__device__ __forceinline__ void half_wave_argmax(float &bv, int &bi)
{
    argmax_dpp_step<DPP_QUAD_XOR1>(bv, bi);
    argmax_dpp_step<DPP_QUAD_XOR2>(bv, bi);
    argmax_dpp_step<DPP_ROW_HALF_MIRROR>(bv, bi);
    argmax_dpp_step<DPP_ROW_MIRROR>(bv, bi);
    argmax_dpp_step<DPP_ROW_BCAST15, 0xA>(bv, bi);
}

#endif /* K_COMMON_H */
