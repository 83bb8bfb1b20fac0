// common.hpp - shared device helpers for the gfx950 W8A8 MoE-FFN kernels.
//
// Rounding helpers follow the reference operators' narrowing rules:
//   * rint16(v): fp32 -> fp16 (round-half-even) -> int8 (round-half-even, saturating, NaN -> 0),
//     the two-step narrowing of the reference's vector units
//     (operators/dynamicquant/csrc/ops/dynamic_quant/op_kernel/dynamic_quant_kernel.cpp:20-22,
//      operators/groupedmatmulswigluquant/csrc/ops/grouped_matmul_swiglu_quant/op_kernel/gmsq_vec_kernel.cpp:256-257).
//   * fp32 -> bf16 / fp16 outputs round half to even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cannbench_amd.h"

namespace cb {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int u32;

constexpr float kFltMin = 1.1754944e-38f;
constexpr float kInv127 = 1.0f / 127.0f;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((u32)h) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    u32 u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h)
{
    _Float16 x = __builtin_bit_cast(_Float16, h);
    return (float)x;
}

__device__ __forceinline__ uint16_t f32_to_f16(float f)
{
    _Float16 x = (_Float16)f;  // v_cvt_f16_f32, round-half-even
    return __builtin_bit_cast(uint16_t, x);
}

// Hardware fp32 -> bf16 (v_cvt_pk_bf16_f32, round-half-even) for finite values.
__device__ __forceinline__ uint16_t f32_to_bf16_hw(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

template <bool BF16>
__device__ __forceinline__ float ld16(uint16_t h) { return BF16 ? bf16_to_f32(h) : f16_to_f32(h); }

template <bool BF16>
__device__ __forceinline__ uint16_t st16(float f) { return BF16 ? f32_to_bf16(f) : f32_to_f16(f); }

// fp32 -> fp16 -> int8, both steps round-half-even; saturates, NaN -> 0.  The empty asm keeps v a
// rounded fp32 value: the compiler would otherwise fold a product feeding the fp16 conversion into
// one mixed-precision fma (v_fma_mixlo_f16) that rounds once instead of twice.
__device__ __forceinline__ int rint16(float v)
{
    asm volatile("" : "+v"(v));
    float h = __builtin_rintf((float)(_Float16)v);
    h = (h == h) ? h : 0.0f;  // NaN -> 0
    h = fminf(fmaxf(h, -128.0f), 127.0f);
    return (int)h;
}

// rint16 for v already clamped to [-128, 127] (so not NaN): fp16 rounding, fp16 round-half-even,
// exact conversion - three instructions.  The result equals rint16(v): the fp16 value is exact in
// fp32, and both round it half-to-even to the same integer in [-128, 127].
__device__ __forceinline__ int rint16_inrange(float v)
{
    const _Float16 h = __builtin_elementwise_roundeven((_Float16)v);
    return (int)(short)h;
}

__device__ __forceinline__ u32 pack4_i8(int a, int b, int c, int d)
{
    return (u32)(a & 0xff) | ((u32)(b & 0xff) << 8) | ((u32)(c & 0xff) << 16) | ((u32)(d & 0xff) << 24);
}

// Wave64 reductions through cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Raw buffer resource over [base, base + bytes): a load at an offset >= bytes returns zeros and
// touches no memory, so an absent operand (bytes = 0) needs no branch around its load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ v4i row_load(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2 /* nt */);
}

// Stores at offsets >= the resource size are dropped.
__device__ __forceinline__ void row_store(v4i v, __amdgpu_buffer_rsrc_t r, uint32_t off)
{
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 2 /* nt */);
}

constexpr uint32_t kOffNone = 0x80000000u;  // an offset past every row resource

__device__ __forceinline__ int64_t uniform64(int64_t v)
{
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// 4x4 byte transpose: r[i] byte c -> o[c] byte i (v_perm_b32 only).
__device__ __forceinline__ void transpose4x4_b8(u32 r0, u32 r1, u32 r2, u32 r3, u32& o0, u32& o1,
                                                u32& o2, u32& o3)
{
    u32 t0 = __builtin_amdgcn_perm(r1, r0, 0x05010400u);  // r0b0 r1b0 r0b1 r1b1
    u32 t1 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);  // r0b2 r1b2 r0b3 r1b3
    u32 t2 = __builtin_amdgcn_perm(r3, r2, 0x05010400u);
    u32 t3 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
    o0 = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    o1 = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    o2 = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    o3 = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

}  // namespace cb
