// xt_common.h - device helpers shared by the EVA02-L kernels for gfx950 (CDNA4): E4M3 / bf16 / fp16 codecs, wave64
// reductions and the MFMA operand types. Compiled with -ffp-contract=off: every fused multiply-add is written as
// __builtin_fmaf so host restatements can follow the same rounding steps.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

#define XT_D 1024       // model width
#define XT_T 1025       // tokens per image: cls + 32 x 32 patches
#define XT_NP 1024      // patches per image
#define XT_K0P 592      // patch operand columns (588 + 4 zero)
#define XT_HID 2730     // SwiGLU hidden units
#define XT_HIDP 2816    // hidden padded to 22 blocks of 128
#define XT_NH 16        // heads
#define XT_HD 64        // head dim
#define XT_TP 1088      // attention rows padded to 17 x 64
#define XT_EPS 1e-6f
#define XT_E4MAX 448.0f

// ---- E4M3 (OCP "fn") ----
// Hardware v_cvt_pk_fp8_f32 rounds to nearest even on gfx950; the clamp to +-448 first gives saturation
// (the reference's __NV_SATFINITE, kern_common.cuh:99). NaN inputs are outside the contract.
__device__ __forceinline__ float e4_clamp(float x) { return __builtin_fminf(__builtin_fmaxf(x, -XT_E4MAX), XT_E4MAX); }

// two floats -> bytes 0, 1 of the result
__device__ __forceinline__ uint32_t e4_pack2(float a, float b)
{
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(e4_clamp(a), e4_clamp(b), 0, false) & 0xffffu;
}

// four floats -> one little-endian 32-bit word
__device__ __forceinline__ uint32_t e4_pack4(float a, float b, float c, float d)
{
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(e4_clamp(a), e4_clamp(b), 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(e4_clamp(c), e4_clamp(d), w, true);
}

// e4_pack4 without the clamp, for values x * (1 / s) of a block scaled by the inverse of its block scale
// s = block_scale(|max|): |x| <= |max|, s = |max| / 448 (1 + d1) and 1 / s rounded once (1 + d2), so
// |x * (1 / s)| <= 448 (1 + 2^-22) after the product's own rounding, which rounds to 448 (the next code up, 480, is
// past the format and the midpoint is 464): the clamp cannot change a code.
__device__ __forceinline__ uint32_t e4_pack4_scaled(float a, float b, float c, float d)
{
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
}

// Block scale from a block |max|: amax / 448 correctly rounded, 1 for a zero block (|max| < 2^-116, where 448 / amax
// would leave the normal range). The reference's per-tensor rule sc = amax / 448 (export_eva.py:64-66) applied per
// block. The quotient is formed without the IEEE division sequence: q = amax RN(1/448), r = amax - 448 q (exact, one
// fma), s = RN(q + r RN(1/448)). That is the correctly rounded quotient for every float amax >= 2^-116 (an exhaustive
// check over all of them, eva_k_scale_bits); at +inf, where r is not finite, q itself is the quotient.
__device__ __forceinline__ float block_scale(float amax)
{
    constexpr float c = 0x1.24924ap-9f;  // RN(1 / 448)
    const float q = amax * c;
    const float s = __builtin_fmaf(__builtin_fmaf(-q, XT_E4MAX, amax), c, q);
    return amax < 0x1p-116f ? 1.0f : (q != __builtin_inff() ? s : q);
}
// 1 / s rounded once per block (the reference's qs = 1 / scl, eva.h:408): activations are packed as x * (1 / s). One
// Newton step y0 + y0 (1 - s y0) from the hardware reciprocal y0, which gives the correctly rounded quotient for every
// s that block_scale returns (exhaustive check on gfx950, eva_k_scale_bits); 0 at +inf, where the step is not finite.
__device__ __forceinline__ float block_scale_inv(float s)
{
    const float y0 = __builtin_amdgcn_rcpf(s);
    const float y1 = __builtin_fmaf(__builtin_fmaf(-s, y0, 1.0f), y0, y0);
    return s != __builtin_inff() ? y1 : 0.0f;
}

// ---- bf16 / fp16 (round to nearest even) ----
__device__ __forceinline__ uint16_t f2bf(float x)
{
    uint32_t u = __float_as_uint(x);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f2h(float x)
{
    asm volatile("" : "+v"(x));  // keep x an fp32 value: no fused fp32-op + fp16-round (v_fma_mix*) single rounding
    _Float16 h = (_Float16)x;
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float h2f(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }

// Raw buffer resource (base, stride 0, num_records = bytes): loads past `bytes` return zero and touch no memory,
// stores past it are dropped
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// ---- wave64 reductions (xor butterfly: every lane ends with the same value) ----
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v);
// Sum over the 64 lanes (all active) by the xor butterfly d = 32, 16, 8, 4, 2, 1: at each step lane i adds the
// partial of lane i ^ d. The exchanges are register moves, not LDS round trips: the permlane32 / permlane16 swaps
// hand lane i the value of lane i ^ 32 / i ^ 16, a row rotation by 8 that of i ^ 8, and a row rotation by 4 that of
// lane i - 4 (mod 16), which after the first three steps holds what lane i ^ 4 holds (a partial then depends on the
// lane index mod 8 only); quad permutations do 2 and 1. The same pairs meet at every step as in a shuffle butterfly,
// so the total is the same bit for bit.
__device__ __forceinline__ float wave_sum(float v)
{
    const int lane = __lane_id();
    {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v += __uint_as_float(lane < 32 ? r[1] : r[0]);
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v += __uint_as_float((lane & 16) ? r[0] : r[1]);
    }
    v += dpp_f<0x128>(v);  // row_ror:8
    v += dpp_f<0x124>(v);  // row_ror:4
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    return v;
}
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
// max over aligned groups of G lanes (G a power of two <= 64)
template <int G>
__device__ __forceinline__ float group_max(float v)
{
#pragma unroll
    for (int off = G / 2; off >= 1; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
template <int G>
__device__ __forceinline__ float group_sum(float v)
{
#pragma unroll
    for (int off = G / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// 16-lane (one DPP row) reductions without LDS traffic: quad_perm xor 1, xor 2, then half-row and row mirrors;
// after each step every lane of the group holds the same partial, so all 16 lanes end with the full result.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
}
// the same over aligned groups of 8 lanes (the first three steps)
__device__ __forceinline__ float row8_sum(float v)
{
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v;
}
// maxima of non-negative floats (block |max| values), which order as their bit patterns: an unsigned max folds into
// the DPP move (v_max_u32_dpp), where a float max needs its own instruction after it
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float row8_absmax(float v)
{
    uint32_t u = __float_as_uint(v);
    u = __builtin_elementwise_max(u, dpp_u<0xB1>(u));
    u = __builtin_elementwise_max(u, dpp_u<0x4E>(u));
    u = __builtin_elementwise_max(u, dpp_u<0x141>(u));
    return __uint_as_float(u);
}
// |max| of non-negative v over the 4 lanes that share lane & 15 (lanes i, i ^ 16, i ^ 32, i ^ 48): two lane swaps
__device__ __forceinline__ float col4_absmax(float v)
{
    const int lane = __lane_id();
    uint32_t u = __float_as_uint(v);
    {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        u = __builtin_elementwise_max(u, lane < 32 ? r[1] : r[0]);
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        u = __builtin_elementwise_max(u, (lane & 16) ? r[0] : r[1]);
    }
    return __uint_as_float(u);
}

__device__ __forceinline__ float row16_absmax(float v)
{
    uint32_t u = __float_as_uint(v);
    u = __builtin_elementwise_max(u, dpp_u<0xB1>(u));
    u = __builtin_elementwise_max(u, dpp_u<0x4E>(u));
    u = __builtin_elementwise_max(u, dpp_u<0x141>(u));
    u = __builtin_elementwise_max(u, dpp_u<0x140>(u));
    return __uint_as_float(u);
}

__device__ __forceinline__ v4f mfma_e4m3_16x16x128(v8i a, v8i b)
{
    v4f z = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}
