// Shared device/host helpers for the gptrig gfx950 kernels.
//
// bf16 storage is the clang `__bf16` type: conversions from float compile to
// gfx950's v_cvt_pk_bf16_f32 (round-to-nearest-even), the same rounding as
// jax's astype(bfloat16).  MFMA operands are 8-wide bf16 vectors.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gptrig.h"

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

#define GPTRIG_LOG2E 1.4426950408889634f
#define GPTRIG_LN2 0.6931471805599453f

#define GPTRIG_CHECK_LAUNCH()                                   \
  do {                                                          \
    if (hipGetLastError() != hipSuccess) return GPTRIG_E_LAUNCH; \
  } while (0)

__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }
__device__ __forceinline__ bf16 f2bf(float x) { return (bf16)x; }

// 32x32x16 bf16 MFMA: A rows = lane%32 (8 k-values per lane), B cols = lane%32,
// C: lane holds column lane%32, rows 8*(i/4) + 4*(lane/32) + (i%4), i = 0..15.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// 16x16x32 bf16 MFMA: A rows = lane%16, B cols = lane%16,
// C: lane holds column lane%16, rows 4*(lane/16) + i, i = 0..3.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// GELU, tanh approximation (jax.nn.gelu(approximate=True)), in fp32, written
// with the logistic function: with u = k (x + c x^3), k = sqrt(2/pi),
// c = 0.044715,
//   0.5 x (1 + tanh u) = x s,      s = 1 / (1 + exp(-2u)),
//   d/dx                = s (1 + x 2u' (1 - s)),   2u' = 2k (1 + 3c x^2).
// exp(-2u) is one v_exp_f32 of x (a + b x^2) with the constants folded, and
// 1 / (1 + e) one v_rcp_f32 (1 ulp, far below the bf16 rounding of every
// caller's result): 5 and 10 full-rate operations plus the two
// transcendentals, against 10 and 18 for the tanh form.  Both saturate like
// the tanh form: e = inf gives s = 0 (gelu -> -0), e = 0 gives s = 1.
__device__ __forceinline__ float gelu_f(float x) {
  constexpr float a = -2.0f * 0.7978845608028654f * GPTRIG_LOG2E;  // -2k log2(e)
  constexpr float b = a * 0.044715f;
  const float e = fast_exp2(x * __builtin_fmaf(x * x, b, a));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}
__device__ __forceinline__ float gelu_grad_f(float x) {
  constexpr float a = -2.0f * 0.7978845608028654f * GPTRIG_LOG2E;
  constexpr float b = a * 0.044715f;
  constexpr float a2 = 2.0f * 0.7978845608028654f;  // 2k
  constexpr float b2 = a2 * 3.0f * 0.044715f;       // 6kc
  const float x2 = x * x;
  const float s = __builtin_amdgcn_rcpf(1.0f + fast_exp2(x * __builtin_fmaf(x2, b, a)));
  const float w = x * __builtin_fmaf(x2, b2, a2);
  return s * __builtin_fmaf(w, 1.0f - s, 1.0f);
}

// Workgroup barrier without the vmcnt(0)/lgkmcnt(0) drain of __syncthreads():
// the caller issues exactly the s_waitcnt it needs first (gfx950 barriers do
// not wait for outstanding memory by themselves).  The empty asm statements
// keep the compiler from moving memory accesses across the barrier, which the
// bare intrinsic does not.
__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// Buffer resource over [base, base + bytes) with raw (stride 0) addressing:
// loads past the end return zeros and stores / atomics past it are dropped,
// and the base lives in scalar registers, so a per-lane 32-bit offset is all
// an access needs.  0x00020000 is dword 3 of a gfx9-family descriptor
// (32-bit data format, no swizzle, no index).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// One interleaved RoPE pair (rig/nn.py:36-52): (e, o) -> (e c - o s, e s + o c)
// in fp32, each result rounded to bf16.  The backward (transposed) rotation is
// the same with -s.  Shared by the RoPE pass and the epilogues that fuse it, so
// both round identically.
__device__ __forceinline__ bf16x2 rope_pair(float e, float o, float c, float s) {
  // Explicit fused forms, so every call site rounds the same way.
  return bf16x2{(bf16)__builtin_fmaf(e, c, -(o * s)), (bf16)__builtin_fmaf(e, s, o * c)};
}

// s_waitcnt lgkmcnt(0) only (vmcnt and expcnt left at their maxima).
#define GPTRIG_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)

// Pack 8 floats into an MFMA bf16 operand.
__device__ __forceinline__ bf16x8 pack8(const float* v) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (bf16)v[j];
  return r;
}

static inline int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }
