// Shared device/host helpers for the gfx950 compressed-cache kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/dynakv_amd.h"

#define DKV_VERSION 120

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

// Buffer-resource ranges. A raw buffer resource returns zero for a load past its range without
// touching memory, so the range decides which loads may reach memory: it must never extend past
// memory the caller owns. Every range a kernel uses comes from one of these two functions
// (exported for host-side tests as dkv_flat_range_elems / dkv_view_extent_elems).
//
// Elements one flat-buffer resource covers at most (its byte size stays below 2^31).
constexpr int DKV_FLAT_RSRC_CAP = 0x3ffffff0;
// Elements from row `row` of a packed (rows, ld) flat buffer to the buffer's end, at most `cap`.
// The C ABI's contract for flat buffers: rows * ld elements are addressable from the base
// pointer (a whole (rows, capacity) buffer, or a column slice of one whose storage runs to the
// end of its last row; the Python wrappers pass a contiguous copy of any other view).
__host__ __device__ inline long long dkv_flat_tail_elems(long long rows, long long row,
                                                         long long ld, long long cap) {
  const long long n = (rows - row) * ld;
  return n < 0 ? 0 : (n < cap ? n : cap);
}
// One past the last element of a view with non-negative strides: the elements addressable from
// its base pointer (0 for an empty view).
__host__ __device__ inline long long dkv_view_extent(int nd, const long long* shape,
                                                     const long long* stride) {
  long long last = 0;
  for (int i = 0; i < nd; ++i) {
    if (shape[i] <= 0) return 0;
    last += (shape[i] - 1) * stride[i];
  }
  return last + 1;
}

// Split length (a multiple of gran tokens) of a split-and-merge decode launch whose kernel runs
// one workgroup per CU (256 CUs on MI355X): the workgroups run in rounds of 256, and a last
// round that is partly empty idles the rest of the chip. n splits per unit cost about
// ceil(units * n / 256) rounds of (split + fixed_tokens) tokens, fixed_tokens being a
// workgroup's fixed cost in token-equivalents; the cheapest n is taken, splits of at least
// min_split tokens (or the whole cache when shorter), at most four rounds and max_n splits.
inline long long dkv_rounds_split(long long units, long long S, long long fixed_tokens,
                                  long long min_split, long long gran = 64,
                                  long long max_n = 1LL << 30) {
  const long long Sg = (S + gran - 1) / gran * gran;
  if (min_split > Sg) min_split = Sg;
  long long n_max = (4 * 256 + units - 1) / units;
  if (n_max > Sg / gran) n_max = Sg / gran;
  if (n_max > max_n) n_max = max_n;
  if (n_max < 1) n_max = 1;
  long long sl = Sg, best = -1;
  for (long long n = 1; n <= n_max; ++n) {
    long long split = ((S + n - 1) / n + gran - 1) / gran * gran;
    if (split < min_split) split = min_split;
    const long long rounds = (units * ((S + split - 1) / split) + 255) / 256;
    const long long cost = rounds * (split + fixed_tokens);
    if (best < 0 || cost < best) {
      best = cost;
      sl = split;
    }
  }
  return sl;
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

// Wave64 all-reductions and an inclusive scan on DPP and permlane swaps (no LDS round trips):
// quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and row_mirror reduce within rows of 16,
// the permlane16 / permlane32 swaps across them.
template <int CTRL>
__device__ __forceinline__ float dkv_dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dkv_dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float dkv_wave_sum_fast(float v) {
  v += dkv_dpp_f32<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dkv_dpp_f32<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dkv_dpp_f32<0x141>(v);  // row_half_mirror
  v += dkv_dpp_f32<0x140>(v);  // row_mirror
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return v;
}
__device__ __forceinline__ float dkv_wave_max_fast(float v) {
  v = fmaxf(v, dkv_dpp_f32<0xb1>(v));
  v = fmaxf(v, dkv_dpp_f32<0x4e>(v));
  v = fmaxf(v, dkv_dpp_f32<0x141>(v));
  v = fmaxf(v, dkv_dpp_f32<0x140>(v));
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  return v;
}
__device__ __forceinline__ int dkv_wave_sum_fast_i(int v) {
  v += dkv_dpp_i32<0xb1>(v);
  v += dkv_dpp_i32<0x4e>(v);
  v += dkv_dpp_i32<0x141>(v);
  v += dkv_dpp_i32<0x140>(v);
  {
    const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = (int)r[0] + (int)r[1];
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    v = (int)r[0] + (int)r[1];
  }
  return v;
}
// Inclusive prefix sum over the wave's lanes: row_shr 1, 2, 4, 8 within rows of 16 (lanes
// without a source add 0), then each row adds the totals of the rows before it (row_bcast15
// into rows 1 and 3, row_bcast31 into rows 2 and 3).
__device__ __forceinline__ float dkv_wave_scan_fast(float v) {
  v += dkv_dpp_f32<0x111>(v);
  v += dkv_dpp_f32<0x112>(v);
  v += dkv_dpp_f32<0x114>(v);
  v += dkv_dpp_f32<0x118>(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false));
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
