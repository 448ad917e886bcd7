// Shared helpers for the gfx950 kernels and their C-ABI wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "vllm_apple_amd.h"

namespace vaa {

typedef _Float16 f16;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

typedef __bf16 bf16;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4v __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- errors --
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
// Status of the most recent launch on this thread.
int check_launch(const char* what);

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// ------------------------------------------------------------ device util --
__device__ __forceinline__ float h2f(f16 x) { return static_cast<float>(x); }
__device__ __forceinline__ f16 f2h(float x) { return static_cast<f16>(x); }

// 2^x on the hardware exp unit (v_exp_f32).
__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// silu(g) * u in fp32: g / (1 + 2^(-g log2 e)) with the hardware exp and
// reciprocal, shared by the SwiGLU pass and the gate/up GEMM epilogue so the
// two round alike.
__device__ __forceinline__ float silu_mul1(float g, float u) {
  const float e = fast_exp2(-g * kLog2e);
  return (g * __builtin_amdgcn_rcpf(1.f + e)) * u;
}

// ------------------------------------------------- 16-bit element types --
// The attention kernels keep K/V/Q/outputs as raw 16-bit storage and are
// templated on the element type only where values are converted or fed to
// the matrix cores: IEEE fp16 (f16) or bfloat16 (bf16), both with fp32
// accumulation.
template <typename T>
struct Elem;

template <>
struct Elem<f16> {
  using x4 = f16x4;
  using x8 = f16x8;
  // Probabilities enter the PV product as one fp16 value (11 significant
  // bits).
  static constexpr bool kSplitP = false;
  static __device__ __forceinline__ float to_f(f16 v) { return static_cast<float>(v); }
  static __device__ __forceinline__ f16 from_f(float v) { return static_cast<f16>(v); }
  // D[16x16] += A[16x32] B[32x16]
  static __device__ __forceinline__ f32x4 mfma16x16x32(x8 a, x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  // D[16x16] += A[16x16] B[16x16]
  static __device__ __forceinline__ f32x4 mfma16x16x16(x4 a, x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  // D[32x32] += A[32x16] B[16x32]
  static __device__ __forceinline__ f32x16 mfma32x32x16(x8 a, x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Elem<bf16> {
  using x4 = bf16x4;
  using x8 = bf16x8;
  // Probabilities enter the PV product as a bf16 pair p = hi + lo (16
  // significant bits) and two MFMAs: one bf16 value (8 bits) puts an error
  // of 2^-9 p_k |v_k| on every term, which on short contexts with values of
  // opposite sign reaches the attention tolerance (measured on MI355X: up to
  // 0.93 of |d| <= 2e-3 + 1e-2 |ref| in decode, 10x the fp16 path's error).
  static constexpr bool kSplitP = true;
  static __device__ __forceinline__ float to_f(bf16 v) { return static_cast<float>(v); }
  // Round to nearest even (v_cvt_pk_bf16_f32).
  static __device__ __forceinline__ bf16 from_f(float v) { return static_cast<bf16>(v); }
  static __device__ __forceinline__ f32x4 mfma16x16x32(x8 a, x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16x16x16(x4 a, x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4v, a),
                                                     __builtin_bit_cast(i16x4v, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32x32x16(x8 a, x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

// Attention head sizes: any multiple of 8 (16-byte rows) up to 128, computed at
// the next multiple of 32 (the MFMA contraction width) with the tail masked.
inline bool head_size_ok(int hd) { return hd >= 8 && hd <= 128 && hd % 8 == 0; }
inline int padded_head(int hd) { return (hd + 31) / 32 * 32; }

// Validates vaa_attn_params.dtype.
inline bool valid_dtype(int32_t dt) { return dt == VAA_DTYPE_F16 || dt == VAA_DTYPE_BF16; }

// NeoX rotation of 8 pairs (x0[e], x1[e]) by angles with cosine c[e] and sine
// s[e], in fp32 (elementwise.py:185-239):
//   y0 = x0 c - x1 s,  y1 = x0 s + x1 c
// evaluated as one rounded product and one fused multiply-add each, and the
// fp32 results materialised (empty asm) before the caller rounds them to 16
// bits.  Written out so the two kernels that share this (the RoPE kernel and
// the fused QKV epilogue) round alike: otherwise the compiler may contract
// them differently, or fold the final fma and the fp16 conversion into one
// mixed-precision fma (v_fma_mixlo_f16, a single rounding) in one kernel and
// not the other.
__device__ __forceinline__ void rope_rotate8(const float* x0, const float* x1, const float* c,
                                             const float* s, float* y0, float* y1) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float t0 = x1[e] * s[e];
    const float t1 = x1[e] * c[e];
    y0[e] = __builtin_fmaf(x0[e], c[e], -t0);
    y1[e] = __builtin_fmaf(x0[e], s[e], t1);
    asm volatile("" : "+v"(y0[e]), "+v"(y1[e]));
  }
}

// 16-byte global load / store through a generic pointer.
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
// 16-byte global load with the nontemporal hint, for data a kernel reads once
// per call (the decode's K/V stream).  Each load instruction of a wave should
// cover whole 64-byte pieces: scattered 16-byte pieces under the hint cost
// more than they save.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

}  // namespace vaa
