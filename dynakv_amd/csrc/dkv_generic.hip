// Reference-semantics kernels on the vector ALU: any rank R <= 1024, a basis per query head
// (or shared by head groups), fp32/fp16/bf16 caches. They back the API-level entry points
// abx_sparse / avx / fused_attention_dispatch for inputs the MFMA split-K path does not take.
//
// Reference behaviour: src/dynakv/kernels/two_stage.py:48-189 (scores), :207-324 (avx),
// src/dynakv/kernels/fused.py:28-170 (fused = scores with -inf masking + avx without clamp).
#include "dkv_common.h"

namespace {

// One wave per (b, h, token); block = 4 waves = 4 consecutive tokens.
// Lane l owns the rotate-half pair (l, l + Dh/2).
template <int QDT, int CDT, int ODT, int MODE>
__global__ __launch_bounds__(256) void scores_kernel(
    const void* __restrict__ q, long long q_sb, long long q_sh, const void* __restrict__ basis,
    long long basis_sh, long long basis_sr, int hpg, const void* __restrict__ flat,
    long long flat_ld, const int* __restrict__ lens, long long lens_sb, long long lens_ss,
    const int* __restrict__ offs, long long offs_sb, long long offs_ss, void* __restrict__ out,
    long long out_sb, long long out_sh, long long out_ss, int S, int R, int Dh,
    float log_theta) {
  const int s = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  if (s >= S) return;
  const int lane = threadIdx.x & 63;
  const int half = Dh >> 1;
  const bool act = lane < half;
  const int d0 = act ? lane : 0, d1 = d0 + half;

  const int len = lens[(long long)b * lens_sb + (long long)s * lens_ss];
  const int off = offs[(long long)b * offs_sb + (long long)s * offs_ss];
  const int rr = max(0, min(len, R));
  const long long brow = (long long)(h / hpg) * basis_sh;
  const long long xrow = (long long)b * flat_ld + off;

  float k0 = 0.f, k1 = 0.f;
  for (int jb = 0; jb < rr; jb += 64) {
    const int jl = jb + lane;
    const float xv = jl < rr ? dkv_load_f32<CDT>(flat, xrow + jl) : 0.f;
    const int nj = min(64, rr - jb);
    for (int j = 0; j < nj; ++j) {
      const float xj = __shfl(xv, j, 64);
      const long long bi = brow + (long long)(jb + j) * basis_sr;
      k0 = fmaf(xj, dkv_load_f32<CDT>(basis, bi + d0), k0);
      k1 = fmaf(xj, dkv_load_f32<CDT>(basis, bi + d1), k1);
    }
  }
  // rotate-half RoPE at the cache row index s (reference fused.py:97-102, two_stage.py:130-144)
  const float ang = (float)s * dkv_inv_freq(d0, Dh, log_theta);
  float sn, cs;
  sincosf(ang, &sn, &cs);
  const float r0 = k0 * cs - k1 * sn;
  const float r1 = k1 * cs + k0 * sn;
  const long long qo = (long long)b * q_sb + (long long)h * q_sh;
  float part = act ? dkv_load_f32<QDT>(q, qo + d0) * r0 + dkv_load_f32<QDT>(q, qo + d1) * r1 : 0.f;
  const float dot = dkv_wave_sum(part);
  if (lane == 0) {
    const float scale = 1.0f / sqrtf((float)Dh);
    float z;
    if constexpr (MODE == 0) {
      z = (len > 0 ? dot : -1.0e4f) * scale;
    } else {
      z = len > 0 ? dot * scale : -INFINITY;
    }
    dkv_store_f32<ODT>(out, (long long)b * out_sb + (long long)h * out_sh + (long long)s * out_ss,
                       z);
  }
}

// One block (256 threads) per (h, b); serial online softmax over S in chunks of 256 tokens,
// accumulating in coefficient space, then one projection through the V basis.
template <int SDT, int CDT, int ODT, int MODE>
__global__ __launch_bounds__(256) void av_kernel(
    const void* __restrict__ scores, long long sc_sb, long long sc_sh, long long sc_ss,
    const void* __restrict__ basis, long long basis_sh, long long basis_sr, int hpg,
    const void* __restrict__ flat, long long flat_ld, const int* __restrict__ lens,
    long long lens_sb, long long lens_ss, const int* __restrict__ offs, long long offs_sb,
    long long offs_ss, void* __restrict__ out, long long out_sb, long long out_sh, int S, int R,
    int Dh) {
  constexpr int NR = 4;  // ranks per thread: R <= 1024
  __shared__ float s_p[256];
  __shared__ int s_len[256];
  __shared__ int s_off[256];
  __shared__ float s_red[8];
  __shared__ float s_a[1024];
  __shared__ float s_out[2][128];
  const int h = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long long so = (long long)b * sc_sb + (long long)h * sc_sh;
  const long long xrow = (long long)b * flat_ld;

  float acc[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) acc[k] = 0.f;
  float m = -INFINITY, l = 0.f;

  for (int base = 0; base < S; base += 256) {
    const int t = base + tid;
    const bool in = t < S;
    const float z = in ? dkv_load_f32<SDT>(scores, so + (long long)t * sc_ss) : -INFINITY;
    // chunk max
    float cm = dkv_wave_max(z);
    if (lane == 0) s_red[wave] = cm;
    __syncthreads();
    cm = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();
    const float mn = fmaxf(m, cm);
    // exp(-inf - -inf) is NaN in the reference as well (all-masked leading chunk);
    // keep that behaviour only when there is nothing finite at all.
    const float alpha = (mn == -INFINITY) ? 1.f : expf(m - mn);
    const float p = in ? ((mn == -INFINITY) ? 0.f : expf(z - mn)) : 0.f;
    float ps = dkv_wave_sum(p);
    if (lane == 0) s_red[4 + wave] = ps;
    s_p[tid] = p;
    s_len[tid] = in ? lens[(long long)b * lens_sb + (long long)t * lens_ss] : 0;
    s_off[tid] = in ? offs[(long long)b * offs_sb + (long long)t * offs_ss] : 0;
    __syncthreads();
    ps = s_red[4] + s_red[5] + s_red[6] + s_red[7];
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int k = 0; k < NR; ++k) acc[k] *= alpha;
    const int nt = min(256, S - base);
    for (int tt = 0; tt < nt; ++tt) {
      const float pt = s_p[tt];
      const int rv = min(s_len[tt], R);
      const long long xo = xrow + s_off[tt];
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const int j = tid + 256 * k;
        if (j < rv) acc[k] = fmaf(pt, dkv_load_f32<CDT>(flat, xo + j), acc[k]);
      }
    }
    __syncthreads();
  }
  const float den = MODE == 0 ? fmaxf(l, 1e-6f) : l;
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const int j = tid + 256 * k;
    if (j < R) s_a[j] = acc[k] / den;
  }
  __syncthreads();
  // out[d] = sum_j a[j] * basis[j][d]; two halves of the rank range, then add.
  const int d = tid & 127, hh = tid >> 7;
  const long long brow = (long long)(h / hpg) * basis_sh;
  float o = 0.f;
  if (d < Dh) {
    for (int j = hh; j < R; j += 2) o = fmaf(s_a[j], dkv_load_f32<CDT>(basis, brow + (long long)j * basis_sr + d), o);
  }
  s_out[hh][d] = o;
  __syncthreads();
  if (hh == 0 && d < Dh)
    dkv_store_f32<ODT>(out, (long long)b * out_sb + (long long)h * out_sh + d, s_out[0][d] + s_out[1][d]);
}

template <int QDT, int CDT, int ODT, int MODE>
void launch_scores(hipStream_t st, dim3 g, const void* q, long long q_sb, long long q_sh,
                   const void* basis, long long basis_sh, long long basis_sr, int hpg,
                   const void* flat, long long flat_ld, const int* lens, long long lens_sb,
                   long long lens_ss, const int* offs, long long offs_sb, long long offs_ss,
                   void* out, long long out_sb, long long out_sh, long long out_ss, int S, int R,
                   int Dh, float log_theta) {
  hipLaunchKernelGGL((scores_kernel<QDT, CDT, ODT, MODE>), g, dim3(256), 0, st, q, q_sb, q_sh,
                     basis, basis_sh, basis_sr, hpg, flat, flat_ld, lens, lens_sb, lens_ss, offs,
                     offs_sb, offs_ss, out, out_sb, out_sh, out_ss, S, R, Dh, log_theta);
}

template <int SDT, int CDT, int ODT, int MODE>
void launch_av(hipStream_t st, dim3 g, const void* scores, long long sc_sb, long long sc_sh,
               long long sc_ss, const void* basis, long long basis_sh, long long basis_sr,
               int hpg, const void* flat, long long flat_ld, const int* lens, long long lens_sb,
               long long lens_ss, const int* offs, long long offs_sb, long long offs_ss,
               void* out, long long out_sb, long long out_sh, int S, int R, int Dh) {
  hipLaunchKernelGGL((av_kernel<SDT, CDT, ODT, MODE>), g, dim3(256), 0, st, scores, sc_sb, sc_sh,
                     sc_ss, basis, basis_sh, basis_sr, hpg, flat, flat_ld, lens, lens_sb, lens_ss,
                     offs, offs_sb, offs_ss, out, out_sb, out_sh, S, R, Dh);
}

bool valid_dtype(int d) { return d == DKV_F32 || d == DKV_F16 || d == DKV_BF16; }

}  // namespace

// Dispatch helpers over the three dtypes of one template slot.
#define DKV_DT_SWITCH(DT, NAME, ...)                  \
  switch (DT) {                                       \
    case DKV_F32: { constexpr int NAME = DKV_F32; __VA_ARGS__; break; }   \
    case DKV_F16: { constexpr int NAME = DKV_F16; __VA_ARGS__; break; }   \
    default: { constexpr int NAME = DKV_BF16; __VA_ARGS__; break; }       \
  }

extern "C" int dkv_scores(void* stream, int mode, int q_dtype, int cache_dtype, int out_dtype,
                          const void* q, long long q_sb, long long q_sh, const void* basis,
                          long long basis_sh, long long basis_sr, int n_basis, const void* flat,
                          long long flat_ld, const int* lens, long long lens_sb,
                          long long lens_ss, const int* offs, long long offs_sb,
                          long long offs_ss, void* out, long long out_sb, long long out_sh,
                          long long out_ss, int B, int Hq, int S, int R, int Dh,
                          float log_theta) {
  if (B < 0 || Hq < 0 || S < 0 || R < 0 || Dh <= 0) return DKV_E_ARG;
  if (mode != 0 && mode != 1) return DKV_E_ARG;
  if (!valid_dtype(q_dtype) || !valid_dtype(cache_dtype) || !valid_dtype(out_dtype))
    return DKV_E_ARG;
  if (n_basis <= 0 || Hq % n_basis != 0) return DKV_E_ARG;
  if ((Dh & 1) || Dh > 128) return DKV_E_UNSUPPORTED;
  if (mode == 0 && Dh != 128) return DKV_E_UNSUPPORTED;  // reference abx hard-codes 2x64 dims
  if (mode == 1 && out_dtype != DKV_F32) return DKV_E_ARG;
  if (B == 0 || Hq == 0 || S == 0) return DKV_OK;
  if (!q || !basis || !flat || !lens || !offs || !out) return DKV_E_ARG;
  if (Hq > 65535 || B > 65535) return DKV_E_UNSUPPORTED;
  const int hpg = Hq / n_basis;
  dim3 g((S + 3) / 4, Hq, B);
  hipStream_t st = (hipStream_t)stream;
  DKV_DT_SWITCH(q_dtype, QD, DKV_DT_SWITCH(cache_dtype, CD, DKV_DT_SWITCH(out_dtype, OD,
      if (mode == 0) launch_scores<QD, CD, OD, 0>(st, g, q, q_sb, q_sh, basis, basis_sh, basis_sr,
          hpg, flat, flat_ld, lens, lens_sb, lens_ss, offs, offs_sb, offs_ss, out, out_sb, out_sh,
          out_ss, S, R, Dh, log_theta);
      else launch_scores<QD, CD, DKV_F32, 1>(st, g, q, q_sb, q_sh, basis, basis_sh, basis_sr,
          hpg, flat, flat_ld, lens, lens_sb, lens_ss, offs, offs_sb, offs_ss, out, out_sb, out_sh,
          out_ss, S, R, Dh, log_theta);
  )));
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_av(void* stream, int mode, int scores_dtype, int cache_dtype, int out_dtype,
                      const void* scores, long long sc_sb, long long sc_sh, long long sc_ss,
                      const void* basis, long long basis_sh, long long basis_sr, int n_basis,
                      const void* flat, long long flat_ld, const int* lens, long long lens_sb,
                      long long lens_ss, const int* offs, long long offs_sb, long long offs_ss,
                      void* out, long long out_sb, long long out_sh, int B, int Hq, int S, int R,
                      int Dh) {
  if (B < 0 || Hq < 0 || S < 0 || R < 0 || Dh <= 0) return DKV_E_ARG;
  if (mode != 0 && mode != 1) return DKV_E_ARG;
  if (!valid_dtype(scores_dtype) || !valid_dtype(cache_dtype) || !valid_dtype(out_dtype))
    return DKV_E_ARG;
  if (n_basis <= 0 || Hq % n_basis != 0) return DKV_E_ARG;
  if (R > 1024 || Dh > 128) return DKV_E_UNSUPPORTED;
  if (B == 0 || Hq == 0) return DKV_OK;
  if (!scores && S > 0) return DKV_E_ARG;
  if (!basis || !flat || !lens || !offs || !out) return DKV_E_ARG;
  if (B > 65535) return DKV_E_UNSUPPORTED;
  const int hpg = Hq / n_basis;
  dim3 g(Hq, B);
  hipStream_t st = (hipStream_t)stream;
  DKV_DT_SWITCH(scores_dtype, SD, DKV_DT_SWITCH(cache_dtype, CD, DKV_DT_SWITCH(out_dtype, OD,
      if (mode == 0) launch_av<SD, CD, OD, 0>(st, g, scores, sc_sb, sc_sh, sc_ss, basis, basis_sh,
          basis_sr, hpg, flat, flat_ld, lens, lens_sb, lens_ss, offs, offs_sb, offs_ss, out,
          out_sb, out_sh, S, R, Dh);
      else launch_av<SD, CD, OD, 1>(st, g, scores, sc_sb, sc_sh, sc_ss, basis, basis_sh,
          basis_sr, hpg, flat, flat_ld, lens, lens_sb, lens_ss, offs, offs_sb, offs_ss, out,
          out_sb, out_sh, S, R, Dh);
  )));
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
