// Small device helpers shared by the MFMA attention kernels (split kernel, joint-layout kernels):
// 16x16x32 MFMA wrappers, the bf16 hi + lo split, 16-bit element conversions, masked 16-byte
// gathers and wave-level maxima.
#pragma once
#include "dkv_common.h"

namespace {

constexpr int DKV_OOB = 0x7ffffff0;       // buffer offset that reads as zero
constexpr int DKV_DPP_ROW_SHL8 = 0x108;   // DPP row_shl:8: lane i of a 16-lane row reads lane i+8

// 16x16x32 MFMA in the cache dtype (bf16 or fp16), fp32 accumulation.
template <int DT>
__device__ __forceinline__ dkv_f32x4 dkv_mfma32(const dkv_u32x4& a, const dkv_u32x4& b,
                                                dkv_f32x4 c) {
  if constexpr (DT == DKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dkv_bf16x8, a),
                                                   __builtin_bit_cast(dkv_bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dkv_f16x8, a),
                                                  __builtin_bit_cast(dkv_f16x8, b), c, 0, 0, 0);
}

// x ~= hi + lo in bf16 for two values packed per dword: hi = RNE(x), lo = RNE(x - hi). x - hi is
// exact in fp32 (a bf16 value as fp32 is its bits in the upper half of a dword), so the pair
// carries 16 significant bits over fp32's exponent range.
__device__ __forceinline__ void dkv_split_bf16x2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  const uint32_t h =
      __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, dkv_bf16x2));
  const float l0 = x0 - __uint_as_float(h << 16);
  const float l1 = x1 - __uint_as_float(h & 0xffff0000u);
  hi = h;
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{l0, l1}, dkv_bf16x2));
}

__device__ __forceinline__ uint32_t dkv_pack_f16x2(float lo, float hi) {
  dkv_f16x2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

template <int DT>
__device__ __forceinline__ float dkv_elt_to_f32(uint32_t bits16) {
  if constexpr (DT == DKV_BF16)
    return dkv_bf16_bits_to_f32(bits16);
  else
    return dkv_f16_bits_to_f32(bits16);
}

// Keep-mask of dword d (elements 2d, 2d+1) when the first k (0..8) 16-bit elements are kept.
__device__ __forceinline__ uint32_t dkv_prefix_mask_word(int k, int d) {
  return k >= 2 * d + 2 ? 0xffffffffu : (k == 2 * d + 1 ? 0x0000ffffu : 0u);
}

// Element-wise gather of the first nv (1..8) 16-bit values at element offset e, the rest zero
// (for a window that would cross the end of a buffer resource, where a vector access reads as
// zero in full).
__device__ __forceinline__ dkv_u32x4 dkv_gather8_b16(__amdgpu_buffer_rsrc_t r, int e, int nv) {
  uint32_t v[8];
#pragma unroll
  for (int t = 0; t < 8; ++t)
    v[t] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, t < nv ? (e + t) * 2 : DKV_OOB, 0, 0);
  return dkv_u32x4{v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16),
                   v[6] | (v[7] << 16)};
}

// 16 bytes at element offset e of a buffer resource, or zeros (no memory traffic) when cnt <= 0;
// the elements past cnt are not cleared here (dkv_mask8 does that where the value is used, so
// the load need not complete before the next ones are issued).
__device__ __forceinline__ dkv_u32x4 dkv_load8_raw(__amdgpu_buffer_rsrc_t r, int e, int cnt) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, cnt > 0 ? e * 2 : DKV_OOB, 0, 0);
}
// dkv_load8_raw for a resource whose last windows may cross its end (`end` elements): such a
// window is gathered element by element (a vector access that crosses the end reads as zero).
__device__ __forceinline__ dkv_u32x4 dkv_load8_safe(__amdgpu_buffer_rsrc_t r, uint32_t end, int e,
                                                    int cnt) {
  if (cnt > 0 && (uint32_t)(e + 8) > end) return dkv_gather8_b16(r, e, min(cnt, 8));
  return dkv_load8_raw(r, e, cnt);
}
// v with the elements from index cnt on cleared (cnt <= 0: all, cnt >= 8: none).
__device__ __forceinline__ dkv_u32x4 dkv_mask8(dkv_u32x4 v, int cnt) {
  const int k = min(max(cnt, 0), 8);
  return dkv_u32x4{v.x & dkv_prefix_mask_word(k, 0), v.y & dkv_prefix_mask_word(k, 1),
                   v.z & dkv_prefix_mask_word(k, 2), v.w & dkv_prefix_mask_word(k, 3)};
}

// Float maxima without the NaN-quieting the compiler adds around fmaxf (-inf is an ordinary
// operand here; the inputs are never NaN for finite data).
__device__ __forceinline__ float dkv_max2(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float dkv_max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// max(x, x of lane l ^ 32) and max(x, x of lane l ^ 16) by permlane swaps.
__device__ __forceinline__ float dkv_lane_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return dkv_max2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float dkv_lane_max16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return dkv_max2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ uint32_t dkv_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

}  // namespace
