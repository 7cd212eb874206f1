// Fused element-wise stages of the end-to-end Llama decoder around the compressed-cache
// attention: the residual add with the following RMSNorm, and the SwiGLU activation product.
//
// Reference behaviour: HF Llama as the reference runs it (custom_llama.py:93-323 builds on
// transformers' LlamaDecoderLayer): hidden = residual + sublayer(...); LlamaRMSNorm computes
// x.float() * rsqrt(mean(x^2) + eps), rounds to the model dtype and multiplies by the weight
// in that dtype; the MLP is down(silu(gate(h)) * up(h)) with silu and the product each rounded
// to the model dtype. In torch each of these is several kernels per row block (eight for the
// norm); here each stage is one kernel with the same roundings (the sum of squares is
// accumulated in fp32 in a different order than torch's reduction).
#include "dkv_common.h"

namespace {

constexpr int NORM_THREADS = 256;
constexpr int NORM_MAXC = 4;  // 8-element chunks per thread: H <= 8 * 256 * 4 = 8192

template <int DT>
__device__ __forceinline__ float to_dt(float v) {
  return dkv_round_to<DT>(v);
}

template <int DT>
__device__ __forceinline__ void unpack8(const dkv_u32x4& v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if constexpr (DT == DKV_BF16) {
      f[2 * k] = dkv_bf16_bits_to_f32(w[k] & 0xffffu);
      f[2 * k + 1] = dkv_bf16_bits_to_f32(w[k] >> 16);
    } else {
      f[2 * k] = dkv_f16_bits_to_f32(w[k] & 0xffffu);
      f[2 * k + 1] = dkv_f16_bits_to_f32(w[k] >> 16);
    }
  }
}
template <int DT>
__device__ __forceinline__ dkv_u32x4 pack8(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if constexpr (DT == DKV_BF16)
      w[k] = dkv_f32_to_bf16_bits(f[2 * k]) | (dkv_f32_to_bf16_bits(f[2 * k + 1]) << 16);
    else
      w[k] = dkv_f32_to_f16_bits(f[2 * k]) | (dkv_f32_to_f16_bits(f[2 * k + 1]) << 16);
  }
  return dkv_u32x4{w[0], w[1], w[2], w[3]};
}

// One workgroup per row: r = x (+ delta, rounded, stored back to x), out = rmsnorm(r) * w.
template <int DT>
__global__ __launch_bounds__(NORM_THREADS) void add_rmsnorm_kernel(
    uint16_t* __restrict__ x, long long x_ld, const uint16_t* __restrict__ delta,
    long long d_ld, const uint16_t* __restrict__ w, uint16_t* __restrict__ out, long long o_ld,
    int H, float eps) {
  __shared__ float sRed[NORM_THREADS / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  const int nc = H / 8;
  uint16_t* xr = x + (long long)row * x_ld;
  float v[NORM_MAXC][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NORM_MAXC; ++k) {
    const int c = tid + k * NORM_THREADS;
    if (c < nc) {
      unpack8<DT>(*(const dkv_u32x4*)(xr + 8 * c), v[k]);
      if (delta) {
        float d[8];
        unpack8<DT>(*(const dkv_u32x4*)(delta + (long long)row * d_ld + 8 * c), d);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = to_dt<DT>(v[k][e] + d[e]);
        *(dkv_u32x4*)(xr + 8 * c) = pack8<DT>(v[k]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[k][e], v[k][e], ss);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((tid & 63) == 0) sRed[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_THREADS / 64; ++i) tot += sRed[i];
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int k = 0; k < NORM_MAXC; ++k) {
    const int c = tid + k * NORM_THREADS;
    if (c < nc) {
      float wv[8], o[8];
      unpack8<DT>(*(const dkv_u32x4*)(w + 8 * c), wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = to_dt<DT>(v[k][e] * inv) * wv[e];
      *(dkv_u32x4*)(out + (long long)row * o_ld + 8 * c) = pack8<DT>(o);
    }
  }
}

// out[r][j] = silu(g) * u with g = gu[r][j], u = gu[r][F + j] (PAIRS: g = gu[r][2j], u =
// gu[r][2j + 1], the output of a gate/up weight whose rows interleave the two); silu(g) =
// g / (1 + e^-g) is rounded to the dtype before the product, as torch's F.silu(g) * u rounds it.
template <int DT, bool PAIRS>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                       long long gu_ld,
                                                       uint16_t* __restrict__ out,
                                                       long long o_ld, int F) {
  const int row = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (8 * c >= F) return;
  const uint16_t* gr = gu + (long long)row * gu_ld;
  float g[8], u[8], o[8];
  if constexpr (PAIRS) {
    float a[8], b[8];
    unpack8<DT>(*(const dkv_u32x4*)(gr + 16 * c), a);
    unpack8<DT>(*(const dkv_u32x4*)(gr + 16 * c + 8), b);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      g[e] = a[2 * e];
      u[e] = a[2 * e + 1];
      g[4 + e] = b[2 * e];
      u[4 + e] = b[2 * e + 1];
    }
  } else {
    unpack8<DT>(*(const dkv_u32x4*)(gr + 8 * c), g);
    unpack8<DT>(*(const dkv_u32x4*)(gr + F + 8 * c), u);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to_dt<DT>(g[e] / (1.0f + expf(-g[e]))) * u[e];
  *(dkv_u32x4*)(out + (long long)row * o_ld + 8 * c) = pack8<DT>(o);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int dkv_add_rmsnorm(void* stream, int dtype, void* x, long long x_ld,
                               const void* delta, long long delta_ld, const void* w, void* out,
                               long long out_ld, int rows, int H, float eps) {
  if (dtype != DKV_BF16 && dtype != DKV_F16) return DKV_E_UNSUPPORTED;
  if (rows < 0 || H <= 0 || H % 8 != 0 || H > 8 * NORM_THREADS * NORM_MAXC) return DKV_E_ARG;
  if (rows == 0) return DKV_OK;
  if (!x || !w || !out || x_ld < H || out_ld < H || (delta && delta_ld < H)) return DKV_E_ARG;
  if (!aligned16(x) || !aligned16(w) || !aligned16(out) || (delta && !aligned16(delta)) ||
      (x_ld & 7) || (out_ld & 7) || (delta && (delta_ld & 7)))
    return DKV_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DKV_BF16)
    hipLaunchKernelGGL(add_rmsnorm_kernel<DKV_BF16>, dim3(rows), dim3(NORM_THREADS), 0, st,
                       (uint16_t*)x, x_ld, (const uint16_t*)delta, delta_ld,
                       (const uint16_t*)w, (uint16_t*)out, out_ld, H, eps);
  else
    hipLaunchKernelGGL(add_rmsnorm_kernel<DKV_F16>, dim3(rows), dim3(NORM_THREADS), 0, st,
                       (uint16_t*)x, x_ld, (const uint16_t*)delta, delta_ld,
                       (const uint16_t*)w, (uint16_t*)out, out_ld, H, eps);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

namespace {

template <bool PAIRS>
int silu_mul_launch(void* stream, int dtype, const void* gu, long long gu_ld, void* out,
                    long long out_ld, int rows, int F) {
  if (dtype != DKV_BF16 && dtype != DKV_F16) return DKV_E_UNSUPPORTED;
  if (rows < 0 || F <= 0 || F % 8 != 0) return DKV_E_ARG;
  if (rows == 0) return DKV_OK;
  if (!gu || !out || gu_ld < 2LL * F || out_ld < F) return DKV_E_ARG;
  if (!aligned16(gu) || !aligned16(out) || (gu_ld & 7) || (out_ld & 7)) return DKV_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  for (int r0 = 0; r0 < rows; r0 += 65535) {  // grid y is limited to 65535 rows per launch
    const dim3 grid((unsigned)((F / 8 + 255) / 256), (unsigned)min(rows - r0, 65535));
    const uint16_t* g0 = (const uint16_t*)gu + (long long)r0 * gu_ld;
    uint16_t* o0 = (uint16_t*)out + (long long)r0 * out_ld;
    if (dtype == DKV_BF16)
      hipLaunchKernelGGL((silu_mul_kernel<DKV_BF16, PAIRS>), grid, dim3(256), 0, st, g0, gu_ld,
                         o0, out_ld, F);
    else
      hipLaunchKernelGGL((silu_mul_kernel<DKV_F16, PAIRS>), grid, dim3(256), 0, st, g0, gu_ld,
                         o0, out_ld, F);
    DKV_HIP_CHECK_LAUNCH();
  }
  return DKV_OK;
}

}  // namespace

extern "C" int dkv_silu_mul(void* stream, int dtype, const void* gu, long long gu_ld, void* out,
                            long long out_ld, int rows, int F) {
  return silu_mul_launch<false>(stream, dtype, gu, gu_ld, out, out_ld, rows, F);
}

extern "C" int dkv_silu_mul_pairs(void* stream, int dtype, const void* gu, long long gu_ld,
                                  void* out, long long out_ld, int rows, int F) {
  return silu_mul_launch<true>(stream, dtype, gu, gu_ld, out, out_ld, rows, F);
}

// ---------------------------------------------------------------------------------------
// Skinny GEMM for decode: y[m][n] = sum_k x[m][k] W[n][k] (torch's F.linear with the weight
// W (N, K) row-major), M <= 8 rows of x. The weights stream once from HBM. A workgroup of 4
// waves stages x in LDS once (when it fits; else each lane reads x from global memory) and
// takes blocks of ROWS output columns grid-stride; each lane loads 16 contiguous bytes of each
// of the ROWS weight rows per step (one wave: 1 KB per row, coalesced); products on
// v_dot2_f32_{bf16,f16}, lane partial sums reduced per block, y rounded once to the dtype.
// ---------------------------------------------------------------------------------------
namespace {

constexpr int GV_WAVES = 4;
constexpr int GV_ROWS = 4;
constexpr int GV_UNROLL = 4;  // k-steps per batch of loads (K-split instances)

template <int DT>
__device__ __forceinline__ float dot8(const dkv_u32x4& a, const dkv_u32x4& b, float c) {
  const uint32_t aa[4] = {a.x, a.y, a.z, a.w}, bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DT == DKV_BF16)
      c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dkv_bf16x2, aa[i]),
                                          __builtin_bit_cast(dkv_bf16x2, bb[i]), c, false);
    else
      c = __builtin_amdgcn_fdot2(__builtin_bit_cast(dkv_f16x2, aa[i]),
                                 __builtin_bit_cast(dkv_f16x2, bb[i]), c, false);
  }
  return c;
}

// XLDS: x staged in LDS (M * K * 2 bytes); otherwise each lane reads its x pieces from global
// memory (cache hits after the first wave) -- for M * K too large to stage.
// KSPLIT: the 4 waves of a workgroup share each block of ROWS columns, wave w taking the
// quarter w of K, and add their partial sums through LDS -- four times the waves for a small
// N; otherwise each wave owns its blocks.
// The RMSNorm folded into a GEMV's x staging (GemvNorm): x + delta (rounded; workgroup 0
// stores it to r_out, the updated residual), then rmsnorm(.) * w with the roundings and the
// per-thread / per-wave summation order of add_rmsnorm_kernel (same 256 threads, same chunk of
// each row per thread), so the staged operand is bit-identical to that kernel's output.
// silu(g) * u of two fp32 projections, with silu_mul_kernel's roundings
template <int DT>
__device__ __forceinline__ float glu_of(float acc_g, float acc_u) {
  const float g = to_dt<DT>(acc_g), u = to_dt<DT>(acc_u);
  return to_dt<DT>(g / (1.0f + expf(-g))) * u;
}

struct GemvNorm {
  const uint16_t* delta;  // nullptr: no residual add
  long long d_ld;
  const uint16_t* w;      // (K,)
  uint16_t* r_out;        // (M, K) rows, stride r_ld; written by workgroup 0 when delta is set
  long long r_ld;
  float eps;
};

// GLU: W holds gate and up rows interleaved (row 2j gate j, row 2j + 1 up j) and the kernel
// stores h[j] = silu(gate_j) * up_j instead of the 2F projections (y of F columns), each
// projection rounded to the dtype first and silu rounded before the product, as
// silu_mul_kernel computes it from the stored projections.
template <int DT, int M, bool XLDS, bool KSPLIT, bool NORM, bool GLU = false>
__global__ __launch_bounds__(GV_WAVES * 64) void gemv_kernel(
    const uint16_t* __restrict__ x, long long x_ld, const uint16_t* __restrict__ W,
    long long w_ld, uint16_t* __restrict__ y, long long y_ld, int N, int K, GemvNorm nrm) {
  extern __shared__ __attribute__((aligned(16))) uint16_t sx[];  // [M][K] (XLDS)
  __shared__ float sP[GV_WAVES][GV_ROWS][M];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if constexpr (XLDS && NORM) {
    static_assert(GV_WAVES * 64 == NORM_THREADS, "norm summation order of add_rmsnorm_kernel");
    __shared__ float sRed[M][GV_WAVES];
    const int nc = K / 8;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float ss = 0.f;
      for (int c = tid; c < nc; c += NORM_THREADS) {
        float v[8];
        unpack8<DT>(*(const dkv_u32x4*)(x + (long long)m * x_ld + 8 * c), v);
        if (nrm.delta) {
          float d[8];
          unpack8<DT>(*(const dkv_u32x4*)(nrm.delta + (long long)m * nrm.d_ld + 8 * c), d);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = to_dt<DT>(v[e] + d[e]);
          const dkv_u32x4 r = pack8<DT>(v);
          if (blockIdx.x == 0) *(dkv_u32x4*)(nrm.r_out + (long long)m * nrm.r_ld + 8 * c) = r;
          *(dkv_u32x4*)(sx + m * K + 8 * c) = r;
        } else {
          *(dkv_u32x4*)(sx + m * K + 8 * c) = pack8<DT>(v);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
      if (lane == 0) sRed[m][wave] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float tot = 0.f;
#pragma unroll
      for (int i = 0; i < GV_WAVES; ++i) tot += sRed[m][i];
      const float inv = 1.0f / sqrtf(tot / (float)K + nrm.eps);
      for (int c = tid; c < nc; c += NORM_THREADS) {
        float v[8], wv[8], o[8];
        unpack8<DT>(*(const dkv_u32x4*)(sx + m * K + 8 * c), v);
        unpack8<DT>(*(const dkv_u32x4*)(nrm.w + 8 * c), wv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = to_dt<DT>(v[e] * inv) * wv[e];
        *(dkv_u32x4*)(sx + m * K + 8 * c) = pack8<DT>(o);
      }
    }
    __syncthreads();
  } else if constexpr (XLDS) {
    for (int c = tid; c < M * (K / 8); c += GV_WAVES * 64) {
      const int m = c / (K / 8), kk = 8 * (c % (K / 8));
      *(dkv_u32x4*)(sx + m * K + kk) = *(const dkv_u32x4*)(x + (long long)m * x_ld + kk);
    }
    __syncthreads();
  }
  const int nblk = (N + GV_ROWS - 1) / GV_ROWS;
  // K range of this wave (multiples of 8)
  const int kq = KSPLIT ? ((K / 8 + GV_WAVES - 1) / GV_WAVES) * 8 : K;
  const int kb = KSPLIT ? min(wave * kq, K) : 0, ke = KSPLIT ? min(kb + kq, K) : K;
  const int first = KSPLIT ? blockIdx.x : blockIdx.x * GV_WAVES + wave;
  const int step = KSPLIT ? gridDim.x : gridDim.x * GV_WAVES;
  // KSPLIT: every wave of the workgroup runs the same number of iterations (the barriers)
  for (int blk = first; blk < nblk; blk += step) {
    const int n0 = blk * GV_ROWS;
    float acc[GV_ROWS][M];
#pragma unroll
    for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
    const uint16_t* wr[GV_ROWS];
#pragma unroll
    for (int r = 0; r < GV_ROWS; ++r) wr[r] = W + (long long)min(n0 + r, N - 1) * w_ld;
    int k = kb + 8 * lane;
    if constexpr (KSPLIT) {
      // batches of GV_UNROLL k-steps: every weight load of a batch is issued before its first
      // product (the products keep the k order, so results are unchanged). Measured on MI355X
      // with cold weights: the long K-split rows gain (down, K = 14336, at 4 rows: 28.0 ->
      // 25.0 us), the 4096-wide ones are unchanged, and the shapes with a block per wave
      // (gate/up) lose, so only the K-split instances batch.
      for (; k + (GV_UNROLL - 1) * 512 < ke; k += GV_UNROLL * 512) {
        dkv_u32x4 wv[GV_UNROLL][GV_ROWS];
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u)
#pragma unroll
          for (int r = 0; r < GV_ROWS; ++r)
            wv[u][r] = __builtin_nontemporal_load((const dkv_u32x4*)(wr[r] + k + 512 * u));
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u)
#pragma unroll
          for (int m = 0; m < M; ++m) {
            const int kk = k + 512 * u;
            const dkv_u32x4 xv = XLDS ? *(const dkv_u32x4*)(sx + m * K + kk)
                                      : *(const dkv_u32x4*)(x + (long long)m * x_ld + kk);
#pragma unroll
            for (int r = 0; r < GV_ROWS; ++r) acc[r][m] = dot8<DT>(wv[u][r], xv, acc[r][m]);
          }
      }
    }
    for (; k < ke; k += 512) {
      dkv_u32x4 wv[GV_ROWS];
#pragma unroll
      for (int r = 0; r < GV_ROWS; ++r)
        wv[r] = __builtin_nontemporal_load((const dkv_u32x4*)(wr[r] + k));
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const dkv_u32x4 xv = XLDS ? *(const dkv_u32x4*)(sx + m * K + k)
                                  : *(const dkv_u32x4*)(x + (long long)m * x_ld + k);
#pragma unroll
        for (int r = 0; r < GV_ROWS; ++r) acc[r][m] = dot8<DT>(wv[r], xv, acc[r][m]);
      }
    }
#pragma unroll
    for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float v = acc[r][m];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
        acc[r][m] = v;
      }
    if constexpr (KSPLIT) {
      if (lane == 0)
#pragma unroll
        for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m) sP[wave][r][m] = acc[r][m];
      __syncthreads();
      if constexpr (GLU) {
        if (tid < GV_ROWS / 2 * M) {
          const int r = 2 * (tid / M), m = tid % M;
          if (n0 + r + 1 < N) {
            float sg = 0.f, su = 0.f;
#pragma unroll
            for (int w = 0; w < GV_WAVES; ++w) {
              sg += sP[w][r][m];
              su += sP[w][r + 1][m];
            }
            dkv_store_f32<DT>(y, (long long)m * y_ld + (n0 + r) / 2, glu_of<DT>(sg, su));
          }
        }
      } else if (tid < GV_ROWS * M) {
        const int r = tid / M, m = tid % M;
        if (n0 + r < N) {
          float s = 0.f;
#pragma unroll
          for (int w = 0; w < GV_WAVES; ++w) s += sP[w][r][m];
          dkv_store_f32<DT>(y, (long long)m * y_ld + n0 + r, s);
        }
      }
      __syncthreads();  // sP is rewritten by the next block
    } else if constexpr (GLU) {
      if (lane == 0)
#pragma unroll
        for (int r = 0; r < GV_ROWS; r += 2)
#pragma unroll
          for (int m = 0; m < M; ++m)
            if (n0 + r + 1 < N)
              dkv_store_f32<DT>(y, (long long)m * y_ld + (n0 + r) / 2,
                                glu_of<DT>(acc[r][m], acc[r + 1][m]));
    } else {
      if (lane == 0)
#pragma unroll
        for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m)
            if (n0 + r < N) dkv_store_f32<DT>(y, (long long)m * y_ld + n0 + r, acc[r][m]);
    }
  }
}

constexpr long long GV_XLDS_MAX = 64 * 1024;  // largest x staged in LDS (bytes)

template <int DT, int M, bool NORM, bool GLU>
void launch_gemv(const void* x, long long x_ld, const void* W, long long w_ld, void* y,
                 long long y_ld, int N, int K, const GemvNorm& nrm, hipStream_t st) {
  // as many workgroups as can be resident at once (LDS bound, at most 8 per CU on 256 CUs);
  // each stages x once
  const int nblk = (N + GV_ROWS - 1) / GV_ROWS;
  const bool xlds = (long long)M * K * 2 <= GV_XLDS_MAX;
  const int per_cu = xlds ? max(1, min(8, (160 * 1024) / (M * K * 2 + 1024))) : 8;
  // fewer column blocks than twice the chip's wave slots at 8 waves per CU: split K
  const bool ksplit = nblk < 2 * 256 * 8;
  const int wg_blocks = ksplit ? nblk : (nblk + GV_WAVES - 1) / GV_WAVES;
  // with the norm folded in, every workgroup normalises its own copy of x: at most 4 per CU
  // for the K-split shapes (the q/k/v projection: 11.4 against 12.2 us at 8 per CU, measured
  // on MI355X with cold weights)
  const int cap = (NORM && ksplit) ? 4 : 8;
  const dim3 grid((unsigned)min(wg_blocks, 256 * min(per_cu, cap)));
  const size_t lds = xlds ? (size_t)M * K * 2 : 0;
  const uint16_t* xp = (const uint16_t*)x;
  const uint16_t* wp = (const uint16_t*)W;
  uint16_t* yp = (uint16_t*)y;
  if constexpr (NORM) {  // the caller checked that x fits the LDS staging
    if (ksplit)
      hipLaunchKernelGGL((gemv_kernel<DT, M, true, true, true, GLU>), grid, dim3(GV_WAVES * 64), lds,
                         st, xp, x_ld, wp, w_ld, yp, y_ld, N, K, nrm);
    else
      hipLaunchKernelGGL((gemv_kernel<DT, M, true, false, true, GLU>), grid, dim3(GV_WAVES * 64),
                         lds, st, xp, x_ld, wp, w_ld, yp, y_ld, N, K, nrm);
  } else if (xlds && ksplit) {
    hipLaunchKernelGGL((gemv_kernel<DT, M, true, true, false, GLU>), grid, dim3(GV_WAVES * 64), lds,
                       st, xp, x_ld, wp, w_ld, yp, y_ld, N, K, nrm);
  } else if (xlds) {
    hipLaunchKernelGGL((gemv_kernel<DT, M, true, false, false, GLU>), grid, dim3(GV_WAVES * 64), lds,
                       st, xp, x_ld, wp, w_ld, yp, y_ld, N, K, nrm);
  } else if (ksplit) {
    hipLaunchKernelGGL((gemv_kernel<DT, M, false, true, false, GLU>), grid, dim3(GV_WAVES * 64), lds,
                       st, xp, x_ld, wp, w_ld, yp, y_ld, N, K, nrm);
  } else {
    hipLaunchKernelGGL((gemv_kernel<DT, M, false, false, false, GLU>), grid, dim3(GV_WAVES * 64),
                       lds, st, xp, x_ld, wp, w_ld, yp, y_ld, N, K, nrm);
  }
}

template <int DT, bool NORM, bool GLU = false>
void launch_gemv_m(int M, const void* x, long long x_ld, const void* W, long long w_ld,
                   void* y, long long y_ld, int N, int K, const GemvNorm& nrm, hipStream_t st) {
  switch (M) {
    case 1: launch_gemv<DT, 1, NORM, GLU>(x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st); break;
    case 2: launch_gemv<DT, 2, NORM, GLU>(x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st); break;
    case 3: launch_gemv<DT, 3, NORM, GLU>(x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st); break;
    case 4: launch_gemv<DT, 4, NORM, GLU>(x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st); break;
    case 5: launch_gemv<DT, 5, NORM, GLU>(x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st); break;
    case 6: launch_gemv<DT, 6, NORM, GLU>(x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st); break;
    case 7: launch_gemv<DT, 7, NORM, GLU>(x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st); break;
    default: launch_gemv<DT, 8, NORM, GLU>(x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st); break;
  }
}

}  // namespace

extern "C" int dkv_gemv(void* stream, int dtype, const void* x, long long x_ld, const void* W,
                        long long w_ld, void* y, long long y_ld, int M, int N, int K) {
  if (dtype != DKV_BF16 && dtype != DKV_F16) return DKV_E_UNSUPPORTED;
  if (M < 0 || N < 0 || K <= 0) return DKV_E_ARG;
  if (M == 0 || N == 0) return DKV_OK;
  if (M > 8 || K % 8 != 0) return DKV_E_UNSUPPORTED;
  if (!x || !W || !y || x_ld < K || w_ld < K || y_ld < N) return DKV_E_ARG;
  if (!aligned16(x) || !aligned16(W) || (x_ld & 7) || (w_ld & 7)) return DKV_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const GemvNorm none = {nullptr, 0, nullptr, nullptr, 0, 0.f};
  if (dtype == DKV_BF16)
    launch_gemv_m<DKV_BF16, false>(M, x, x_ld, W, w_ld, y, y_ld, N, K, none, st);
  else
    launch_gemv_m<DKV_F16, false>(M, x, x_ld, W, w_ld, y, y_ld, N, K, none, st);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_gemv_rmsnorm(void* stream, int dtype, const void* x, long long x_ld,
                                const void* delta, long long delta_ld, const void* norm_w,
                                float eps, void* r_out, long long r_ld, const void* W,
                                long long w_ld, void* y, long long y_ld, int M, int N, int K) {
  if (dtype != DKV_BF16 && dtype != DKV_F16) return DKV_E_UNSUPPORTED;
  if (M < 0 || N < 0 || K <= 0) return DKV_E_ARG;
  if (M == 0 || N == 0) return DKV_OK;
  if (M > 8 || K % 8 != 0 || (long long)M * K * 2 > GV_XLDS_MAX) return DKV_E_UNSUPPORTED;
  if (!x || !W || !y || !norm_w || x_ld < K || w_ld < K || y_ld < N) return DKV_E_ARG;
  if (delta && (!r_out || delta_ld < K || r_ld < K)) return DKV_E_ARG;
  if (delta && (r_out == x || r_out == delta)) return DKV_E_ARG;  // read while workgroup 0 writes
  if (!aligned16(x) || !aligned16(W) || !aligned16(norm_w) || (x_ld & 7) || (w_ld & 7) ||
      (delta && (!aligned16(delta) || !aligned16(r_out) || (delta_ld & 7) || (r_ld & 7))))
    return DKV_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const GemvNorm nrm = {(const uint16_t*)delta, delta_ld, (const uint16_t*)norm_w,
                        (uint16_t*)r_out, r_ld, eps};
  if (dtype == DKV_BF16)
    launch_gemv_m<DKV_BF16, true>(M, x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st);
  else
    launch_gemv_m<DKV_F16, true>(M, x, x_ld, W, w_ld, y, y_ld, N, K, nrm, st);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_gemv_glu(void* stream, int dtype, const void* x, long long x_ld,
                            const void* delta, long long delta_ld, const void* norm_w, float eps,
                            void* r_out, long long r_ld, const void* W, long long w_ld, void* h,
                            long long h_ld, int M, int F, int K) {
  if (dtype != DKV_BF16 && dtype != DKV_F16) return DKV_E_UNSUPPORTED;
  if (M < 0 || F < 0 || K <= 0) return DKV_E_ARG;
  if (M == 0 || F == 0) return DKV_OK;
  if (M > 8 || K % 8 != 0) return DKV_E_UNSUPPORTED;
  if (norm_w && (long long)M * K * 2 > GV_XLDS_MAX) return DKV_E_UNSUPPORTED;
  if (!x || !W || !h || x_ld < K || w_ld < K || h_ld < F) return DKV_E_ARG;
  if (delta && (!norm_w || !r_out || delta_ld < K || r_ld < K)) return DKV_E_ARG;
  if (delta && (r_out == x || r_out == delta)) return DKV_E_ARG;  // read while workgroup 0 writes
  if (!aligned16(x) || !aligned16(W) || (x_ld & 7) || (w_ld & 7) ||
      (norm_w && !aligned16(norm_w)) ||
      (delta && (!aligned16(delta) || !aligned16(r_out) || (delta_ld & 7) || (r_ld & 7))))
    return DKV_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const GemvNorm nrm = {(const uint16_t*)delta, delta_ld, (const uint16_t*)norm_w,
                        (uint16_t*)r_out, r_ld, eps};
  const int N = 2 * F;
  if (norm_w) {
    if (dtype == DKV_BF16)
      launch_gemv_m<DKV_BF16, true, true>(M, x, x_ld, W, w_ld, h, h_ld, N, K, nrm, st);
    else
      launch_gemv_m<DKV_F16, true, true>(M, x, x_ld, W, w_ld, h, h_ld, N, K, nrm, st);
  } else {
    if (dtype == DKV_BF16)
      launch_gemv_m<DKV_BF16, false, true>(M, x, x_ld, W, w_ld, h, h_ld, N, K, nrm, st);
    else
      launch_gemv_m<DKV_F16, false, true>(M, x, x_ld, W, w_ld, h, h_ld, N, K, nrm, st);
  }
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
