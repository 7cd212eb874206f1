// Shared device/host helpers for the gfx950 compressed-cache kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/dynakv_amd.h"

#define DKV_VERSION 111

typedef __attribute__((ext_vector_type(8))) __bf16 dkv_bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 dkv_bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 dkv_bf16x2;
typedef __attribute__((ext_vector_type(8))) _Float16 dkv_f16x8;
typedef __attribute__((ext_vector_type(4))) _Float16 dkv_f16x4;
typedef __attribute__((ext_vector_type(2))) _Float16 dkv_f16x2;
typedef __attribute__((ext_vector_type(4))) float dkv_f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned dkv_u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned dkv_u32x2;
typedef __attribute__((ext_vector_type(2))) unsigned long long dkv_u64x2;
typedef __attribute__((ext_vector_type(4))) int dkv_i32x4;
typedef __attribute__((ext_vector_type(4))) short dkv_i16x4;

#define DKV_HIP_CHECK_LAUNCH()                                  \
  do {                                                          \
    hipError_t e__ = hipGetLastError();                         \
    if (e__ != hipSuccess) return -(DKV_E_HIP_BASE + (int)e__); \
  } while (0)

static inline int dkv_elt_size(int dtype) {
  return dtype == DKV_F32 ? 4 : (dtype == DKV_F16 || dtype == DKV_BF16) ? 2 : 0;
}

// ---------------------------------------------------------------------------
// scalar conversions (device)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float dkv_bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float dkv_f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
// Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN): gfx950's conversion instruction.
__device__ __forceinline__ uint32_t dkv_f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t dkv_f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// Load element i of a dtype-tagged array as fp32.
template <int DT>
__device__ __forceinline__ float dkv_load_f32(const void* p, long long i) {
  if constexpr (DT == DKV_F32) {
    return ((const float*)p)[i];
  } else if constexpr (DT == DKV_F16) {
    return dkv_f16_bits_to_f32(((const uint16_t*)p)[i]);
  } else {
    return dkv_bf16_bits_to_f32(((const uint16_t*)p)[i]);
  }
}
template <int DT>
__device__ __forceinline__ void dkv_store_f32(void* p, long long i, float v) {
  if constexpr (DT == DKV_F32) {
    ((float*)p)[i] = v;
  } else if constexpr (DT == DKV_F16) {
    ((uint16_t*)p)[i] = (uint16_t)dkv_f32_to_f16_bits(v);
  } else {
    ((uint16_t*)p)[i] = (uint16_t)dkv_f32_to_bf16_bits(v);
  }
}
// Round an fp32 value to the precision of dtype DT and return it as fp32.
template <int DT>
__device__ __forceinline__ float dkv_round_to(float v) {
  if constexpr (DT == DKV_F32) {
    return v;
  } else if constexpr (DT == DKV_F16) {
    return (float)(_Float16)v;
  } else {
    return dkv_bf16_bits_to_f32(dkv_f32_to_bf16_bits(v));
  }
}

// Raw buffer resource over [base, base + bytes): loads outside the range return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dkv_make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

// Wave64 reductions via cross-lane xor shuffles.
__device__ __forceinline__ float dkv_wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float dkv_wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ int dkv_wave_max_i(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, 64));
  return v;
}

// inv_freq_i = exp(-(2i/Dh) * ln(theta)) evaluated in fp32 as the reference kernels do
// (reference fused.py:65-66, two_stage.py:36-41).
__device__ __forceinline__ float dkv_inv_freq(int i, int Dh, float log_theta) {
  float f = (float)(2 * i) / (float)Dh;
  return expf(-f * log_theta);
}

// Rotate-half RoPE of the pair (i, i + 64) of one 128-element row in place: angle
// float(pos) * inv_freq_i in fp32, the rotation in fp32, the results rounded to dtype DT.
template <int DT>
__device__ __forceinline__ void dkv_rope_pair(uint16_t* row, int i, int pos, float log_theta) {
  const float inv = dkv_inv_freq(i, 128, log_theta);
  const float ang = (float)pos * inv;
  const float c = cosf(ang), sn = sinf(ang);
  const float a = dkv_load_f32<DT>(row, i), b = dkv_load_f32<DT>(row, i + 64);
  dkv_store_f32<DT>(row, i, a * c - b * sn);
  dkv_store_f32<DT>(row, i + 64, b * c + a * sn);
}
