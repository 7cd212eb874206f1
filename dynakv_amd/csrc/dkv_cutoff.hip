// Cutoff head: the per-token retained-dimension count r and the masked coefficients that feed
// the cache append, for K and V in one call.
//
// Reference behaviour: src/dynakv/kernels/compressed_attention.py:84-119 (kv_process_fused):
//   logits = b + x @ W                      (addmm in the compute dtype, :92-93)
//   mask   = flip(cumsum(softmax(logits)))  (:99)
//   hard   = mask >= 0.1                    (:100; 0.1 compared in the compute dtype)
//   hard[..., low_rank:] = 0                (:106-107)
//   len    = sum(hard) (int32), out = x * hard (:113-117)
// Here every group g of a row (G groups of D dims; G = 1 is the reference's joint 1024-d head,
// G = 8 with D = 128 its per-head form) has its own W_g and b_g.
//
// Because cumsum of the non-negative softmax is non-decreasing, flip(cumsum) >= thr is a prefix
// mask: its length is the number of positions m whose prefix sum c_m reaches thr, and
// out = x on the first len dims (min(len, low_rank)), x * 0 after them.
//
// Two kernels on the caller's stream:
//   cutoff_logits_kernel  16 rows x 64 logits per workgroup (4 waves, 16x16x32 MFMA over D),
//                         bias added in fp32, rounded to the compute dtype (addmm's output),
//                         written to the caller's workspace;
//   cutoff_rows_kernel    one wave per (row, group, K|V): softmax in fp32 of the rounded
//                         logits (probabilities rounded to the compute dtype, as torch.softmax
//                         returns them), prefix sums accumulated in fp32 and rounded to the
//                         compute dtype, the count against the threshold rounded to the
//                         compute dtype, the masked copy and the int32 length.
// W is taken transposed, Wt[g][n][k] = W_g[k][n] (the input dimension contiguous), so both MFMA
// operands are 16-byte row loads; the Python layer prepares that copy once per weight.
#include "dkv_internal.h"

namespace {

constexpr int CT_ROWS = 16;   // rows per logits workgroup
constexpr int CT_COLS = 64;   // logits per workgroup (16 per wave)

struct CutoffMat {
  const uint16_t* x;   // (M, G*D) rows, stride x_ld
  const uint16_t* wt;  // (G, D, D): wt[g][n][k]
  const uint16_t* b;   // (G, D)
  uint16_t* out;       // (M, G*D) rows, stride out_ld
  int* lens;           // (M, G) rows, stride len_ld
  uint16_t* logits;    // workspace (M, G, D)
};

struct CutoffParams {
  CutoffMat mat[2];
  long long x_ld, out_ld, len_ld;
  int M, G, D, low_rank;
  float threshold;     // already rounded to the compute dtype
};

template <int DT>
__device__ __forceinline__ dkv_f32x4 mfma_16x16x32(const dkv_u32x4& a, const dkv_u32x4& b,
                                                   dkv_f32x4 c) {
  if constexpr (DT == DKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dkv_bf16x8, a),
                                                   __builtin_bit_cast(dkv_bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dkv_f16x8, a),
                                                  __builtin_bit_cast(dkv_f16x8, b), c, 0, 0, 0);
}

template <int DT>
__device__ __forceinline__ float elt_f32(uint16_t v) {
  if constexpr (DT == DKV_BF16)
    return dkv_bf16_bits_to_f32(v);
  else
    return dkv_f16_bits_to_f32(v);
}
template <int DT>
__device__ __forceinline__ uint16_t f32_elt(float v) {
  if constexpr (DT == DKV_BF16)
    return (uint16_t)dkv_f32_to_bf16_bits(v);
  else
    return (uint16_t)dkv_f32_to_f16_bits(v);
}

// grid: (D / 64, ceil(M / 16), 2 * G); wave w computes logits n0 + 16w .. +16 of 16 rows.
// MFMA operands: A = x rows (lane: row i = lane % 16, inputs 8*(lane/16) .. +8 of the k-step),
// B = Wt rows (lane: output n = lane % 16, the same inputs); the result lane holds rows
// 4*(lane/16) + u of output column lane % 16.
template <int DT>
__device__ __forceinline__ void logits_tile(const CutoffParams& p, int mat, int g, int row0,
                                            int n0, int lane) {
  const int i = lane & 15, kg = lane >> 4;
  const CutoffMat& cm = p.mat[mat];
  const int D = p.D;
  const int xrow = min(row0 + i, p.M - 1);  // rows past M compute a copy of the last row
  const uint16_t* xa = cm.x + (long long)xrow * p.x_ld + (long long)g * D + 8 * kg;
  const uint16_t* wb = cm.wt + ((long long)g * D + n0 + i) * D + 8 * kg;
  dkv_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int k = 0;
  for (; k + 128 <= D; k += 128) {
    dkv_u32x4 a[4], b[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      a[s] = *(const dkv_u32x4*)(xa + k + 32 * s);
      b[s] = *(const dkv_u32x4*)(wb + k + 32 * s);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma_16x16x32<DT>(a[s], b[s], acc);
  }
  for (; k < D; k += 32)
    acc = mfma_16x16x32<DT>(*(const dkv_u32x4*)(xa + k), *(const dkv_u32x4*)(wb + k), acc);
  const float bias = elt_f32<DT>(cm.b[(long long)g * D + n0 + i]);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int m = row0 + 4 * kg + u;
    if (m < p.M)
      cm.logits[((long long)m * p.G + g) * D + n0 + i] = f32_elt<DT>(acc[u] + bias);
  }
}
template <int DT>
__global__ __launch_bounds__(256) void cutoff_logits_kernel(CutoffParams p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  logits_tile<DT>(p, blockIdx.z & 1, blockIdx.z >> 1, blockIdx.y * CT_ROWS,
                  blockIdx.x * CT_COLS + wave * 16, lane);
}

// Split-K logits for wide heads (D = 128 * STEPS, the joint 1024-d head: STEPS = 8): grid
// (D / 16, ceil(M / 16), 2 * G), one workgroup per 16 logits of 16 rows; wave w takes the
// quarter w of the input dimension, issues every operand load of its STEPS k-steps before the
// first product, and the four partial sums are added in wave order through LDS (one memory
// round trip per workgroup instead of one per k-step, four times the workgroups of
// cutoff_logits_kernel).
template <int DT, int STEPS>
__global__ __launch_bounds__(256) void cutoff_logits_ks_kernel(CutoffParams p) {
  __shared__ dkv_f32x4 sP[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int mat = blockIdx.z & 1, g = blockIdx.z >> 1;
  const int row0 = blockIdx.y * CT_ROWS, n0 = blockIdx.x * 16;
  const int i = lane & 15, kg = lane >> 4;
  const CutoffMat& cm = p.mat[mat];
  const int D = p.D;
  const int k0 = wave * STEPS * 32;
  const int xrow = min(row0 + i, p.M - 1);  // rows past M compute a copy of the last row
  const uint16_t* xa = cm.x + (long long)xrow * p.x_ld + (long long)g * D + k0 + 8 * kg;
  const uint16_t* wb = cm.wt + ((long long)g * D + n0 + i) * D + k0 + 8 * kg;
  dkv_u32x4 a[STEPS], b[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    a[s] = *(const dkv_u32x4*)(xa + 32 * s);
    b[s] = *(const dkv_u32x4*)(wb + 32 * s);
  }
  dkv_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < STEPS; ++s) acc = mfma_16x16x32<DT>(a[s], b[s], acc);
  sP[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    dkv_f32x4 t = sP[0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) t += sP[w][lane];
    const float bias = elt_f32<DT>(cm.b[(long long)g * D + n0 + i]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int m = row0 + 4 * kg + u;
      if (m < p.M) cm.logits[((long long)m * p.G + g) * D + n0 + i] = f32_elt<DT>(t[u] + bias);
    }
  }
}

// The retained count of one (row m, group g) of a matrix, computed by one wave from the
// row's rounded logits (global workspace or LDS). Lane l owns the E = D / 64 consecutive
// positions l*E .. l*E + E - 1 of the row.
template <int DT, int E>
__device__ __forceinline__ int cutoff_row_len(const CutoffParams& p, const uint16_t* row,
                                              int lane) {
  const uint16_t* lg = row + lane * E;

  float x[E];
  if constexpr (E >= 8) {
    // 16-byte loads (the row and each lane's E elements are 16-byte aligned)
#pragma unroll
    for (int v = 0; v < E / 8; ++v) {
      const dkv_u32x4 w = *(const dkv_u32x4*)(lg + 8 * v);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        x[8 * v + e] = elt_f32<DT>((uint16_t)(ww[e >> 1] >> (16 * (e & 1))));
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = elt_f32<DT>(lg[e]);
  }
  float mx = x[0];
#pragma unroll
  for (int e = 1; e < E; ++e) mx = fmaxf(mx, x[e]);
  mx = dkv_wave_max_fast(mx);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    x[e] = expf(x[e] - mx);
    s += x[e];
  }
  s = dkv_wave_sum_fast(s);
  // probabilities in the compute dtype, then their prefix sums accumulated in fp32
  float run = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    run += dkv_round_to<DT>(x[e] / s);
    x[e] = run;  // inclusive prefix within the lane
  }
  const float inc = dkv_wave_scan_fast(run);  // inclusive scan of the lane totals
  const float excl = inc - run;
  int cnt = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) cnt += dkv_round_to<DT>(excl + x[e]) >= p.threshold ? 1 : 0;
  cnt = dkv_wave_sum_fast_i(cnt);
  return min(cnt, max(p.low_rank, 0));
}

// One wave per (row m, group g, K|V): the count and the masked copy of the row.
template <int DT, int E>
__device__ __forceinline__ void row_task(const CutoffParams& p, int mat, long long rg, int lane) {
  const int m = (int)(rg / p.G), g = (int)(rg % p.G);
  const CutoffMat& cm = p.mat[mat];
  const int D = p.D;
  const int len = cutoff_row_len<DT, E>(p, cm.logits + rg * D, lane);

  const uint16_t* xs = cm.x + (long long)m * p.x_ld + (long long)g * D + lane * E;
  uint16_t* xo = cm.out + (long long)m * p.out_ld + (long long)g * D + lane * E;
  uint16_t xv[E];
  if constexpr (E >= 8) {
    // 16-byte loads of the input (x rows are 16-byte aligned: checked by the host)
#pragma unroll
    for (int v = 0; v < E / 8; ++v) {
      const dkv_u32x4 w = *(const dkv_u32x4*)(xs + 8 * v);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[8 * v + e] = (uint16_t)(ww[e >> 1] >> (16 * (e & 1)));
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) xv[e] = xs[e];
  }
  // x * 1 or x * 0 in the compute dtype, written out bitwise: x * 0 is a zero with x's sign,
  // or NaN for an infinite or NaN x (a multiply would do the same, but the compiler may turn
  // it into an fma with a +0 addend, which loses the sign of -0)
  constexpr uint16_t EXP = DT == DKV_BF16 ? 0x7f80 : 0x7c00;
  constexpr uint16_t QNAN = DT == DKV_BF16 ? 0x7fc0 : 0x7e00;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint16_t xb = xv[e];
    const uint16_t zb = (xb & EXP) == EXP ? QNAN : (uint16_t)(xb & 0x8000);
    xo[e] = lane * E + e < len ? xb : zb;
  }
  if (lane == 0) cm.lens[(long long)m * p.len_ld + g] = len;
}
template <int DT, int E>
__global__ __launch_bounds__(256) void cutoff_rows_kernel(CutoffParams p) {
  const int lane = threadIdx.x & 63;
  const long long task = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long long n_rows = (long long)p.M * p.G;
  if (task >= 2 * n_rows) return;
  row_task<DT, E>(p, (int)(task / n_rows), task % n_rows, lane);
}

// Few rows (M <= 16, D <= 128: a decode step) in one launch of 8 waves per (group, K|V): the
// logits of the rows go to LDS (wave w: output columns 16w .. 16w+15; every operand load issued
// before the first product, the masked copies' inputs loaded ahead as well), then wave w takes
// rows w and w + 8: count, masked copy, length. One memory round trip before the stores.
constexpr int CS_WAVES = 8;

template <int DT>
__device__ __forceinline__ void small_logits(const CutoffParams& p, int mat, int g, int wave,
                                             int lane, uint16_t (*sLog)[128], int row0 = 0) {
  const int n0 = 16 * wave;
  if (n0 >= p.D) return;
  const int i = lane & 15, kg = lane >> 4;
  const CutoffMat& cm = p.mat[mat];
  const int D = p.D;
  const uint16_t* xa =
      cm.x + (long long)min(row0 + i, p.M - 1) * p.x_ld + (long long)g * D + 8 * kg;
  const uint16_t* wb = cm.wt + ((long long)g * D + n0 + i) * D + 8 * kg;
  dkv_u32x4 a[4], b[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int k = min(32 * s, D - 32);  // D = 64: the last two steps are loaded but not used
    a[s] = *(const dkv_u32x4*)(xa + k);
    b[s] = *(const dkv_u32x4*)(wb + k);
  }
  const float bias = elt_f32<DT>(cm.b[(long long)g * D + n0 + i]);
  dkv_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s)
    if (32 * s < D) acc = mfma_16x16x32<DT>(a[s], b[s], acc);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int m = row0 + 4 * kg + u;
    if (m < p.M) {
      const uint16_t v = f32_elt<DT>(acc[u] + bias);
      sLog[m - row0][n0 + i] = v;
      cm.logits[((long long)m * p.G + g) * D + n0 + i] = v;  // the workspace copy, as the
                                                               // two-kernel path leaves it
    }
  }
}

template <int DT, int E>
__global__ __launch_bounds__(64 * CS_WAVES) void cutoff_small_kernel(CutoffParams p) {
  __shared__ uint16_t sLog[CT_ROWS][128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int mat = blockIdx.x & 1, g = blockIdx.x >> 1;
  const CutoffMat& cm = p.mat[mat];
  const int D = p.D;
  uint16_t xr[2][E];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int m = min(wave + CS_WAVES * r, p.M - 1);
    const uint16_t* xs = cm.x + (long long)m * p.x_ld + (long long)g * D + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) xr[r][e] = xs[e];
  }
  small_logits<DT>(p, mat, g, wave, lane, sLog);
  __syncthreads();
  constexpr uint16_t EXP = DT == DKV_BF16 ? 0x7f80 : 0x7c00;
  constexpr uint16_t QNAN = DT == DKV_BF16 ? 0x7fc0 : 0x7e00;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int m = wave + CS_WAVES * r;
    if (m >= p.M) break;
    const int len = cutoff_row_len<DT, E>(p, &sLog[m][0], lane);
    uint16_t* xo = cm.out + (long long)m * p.out_ld + (long long)g * D + lane * E;
    // x * 1 or x * 0 written bitwise, as row_task writes them
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint16_t xb = xr[r][e];
      const uint16_t zb = (xb & EXP) == EXP ? QNAN : (uint16_t)(xb & 0x8000);
      xo[e] = lane * E + e < len ? xb : zb;
    }
    if (lane == 0) cm.lens[(long long)m * p.len_ld + g] = len;
  }
}

// Decode step of the per-head layout, after the logits: for each (batch b, group g, K|V) the
// count, then the decode append of that token to cache row b*G + g at position seq (the first
// len coefficients -- exactly what the masked copy followed by the append stores); waves past
// those tasks rotate the query rows (RoPE at position pos).
struct TailParams {
  CutoffParams cp;
  void* flat[2];
  long long flat_ld[2];
  int* lens[2];
  int* offs[2];
  long long tab_sb[2], tab_ss[2];
  int* ptr[2];
  int seq;
  uint16_t* q;
  long long q_sb;  // elements between batch rows of q (heads are contiguous 128-element rows)
  int q_rows, Hq;
  int pos;
  float log_theta;
};

// count, table entries and append of cache row rg = b*G + g of matrix mat (one wave). pre:
// the row's pointer (lane 0) and this lane's E coefficients when the caller loaded them
// ahead (have_pre), else they are loaded here.
template <int DT, int E>
__device__ __forceinline__ void append_row(const TailParams& t, int mat, long long rg, int lane,
                                           bool have_pre = false, int pre_off = 0,
                                           const uint16_t* pre_x = nullptr) {
  const CutoffParams& p = t.cp;
  const int m = (int)(rg / p.G), g = (int)(rg % p.G);
  const int len = cutoff_row_len<DT, E>(p, p.mat[mat].logits + rg * p.D, lane);
  int off = 0;
  if (lane == 0) {
    off = have_pre ? pre_off : t.ptr[mat][rg];
    t.ptr[mat][rg] = off + len;
    t.lens[mat][rg * t.tab_sb[mat] + (long long)t.seq * t.tab_ss[mat]] = len;
    t.offs[mat][rg * t.tab_sb[mat] + (long long)t.seq * t.tab_ss[mat]] = off;
  }
  off = __shfl(off, 0, 64);
  const uint16_t* xs = p.mat[mat].x + (long long)m * p.x_ld + (long long)g * p.D + lane * E;
  uint16_t* dst = (uint16_t*)t.flat[mat] + rg * t.flat_ld[mat] + off + lane * E;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (lane * E + e < len) dst[e] = have_pre ? pre_x[e] : xs[e];
}

// One launch for the whole tail of a decode step's cutoff head: workgroup 2g + mat computes the
// logits of group g of matrix mat (K or V) for 16 rows at a time (wave w: columns 16w + 64c, as
// cutoff_logits_kernel computes them), then its waves take those rows' counts and appends;
// the workgroups past 2G rotate the query rows (RoPE at position pos), one per wave.
template <int DT, int E>
__global__ __launch_bounds__(256) void cutoff_layer_kernel(TailParams t) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const CutoffParams& p = t.cp;
  const int n_cut = 2 * p.G;
  if ((int)blockIdx.x < n_cut) {
    const int mat = blockIdx.x & 1, g = blockIdx.x >> 1;
    // the first row of each wave: its pointer and coefficients loaded before the logits, so
    // that their latency overlaps the products
    int off0 = 0;
    uint16_t x0[E];
    if (wave < p.M) {
      const long long rg = (long long)wave * p.G + g;
      if (lane == 0) off0 = t.ptr[mat][rg];
      const uint16_t* xs = p.mat[mat].x + (long long)wave * p.x_ld + (long long)g * p.D + lane * E;
#pragma unroll
      for (int e = 0; e < E; ++e) x0[e] = xs[e];
    }
    for (int row0 = 0; row0 < p.M; row0 += CT_ROWS) {
      for (int c0 = 0; c0 < p.D; c0 += CT_COLS) logits_tile<DT>(p, mat, g, row0, c0 + 16 * wave, lane);
      __syncthreads();  // the rows' logits (global workspace) are visible to the workgroup
      for (int m = row0 + wave; m < min(row0 + CT_ROWS, p.M); m += 4)
        append_row<DT, E>(t, mat, (long long)m * p.G + g, lane, m == wave, off0, x0);
    }
    return;
  }
  const long long qr = (long long)(blockIdx.x - n_cut) * 4 + wave;
  if (qr < t.q_rows)
    dkv_rope_pair<DT>(t.q + (qr / t.Hq) * t.q_sb + (qr % t.Hq) * 128, lane, t.pos, t.log_theta);
}

// cutoff_layer_kernel for a decode step of the per-head layout (D <= 128), in one memory round
// trip before the stores: workgroup (16-row tile rt, 2g + mat) of 8 waves loads its rows' append
// pointers and inputs, computes the rows' logits into LDS as cutoff_small_kernel does, then wave
// w appends rows 16 rt + w and 16 rt + w + 8; the workgroups past the 2G x tiles rotate the
// query rows, one per wave.
template <int DT, int E>
__global__ __launch_bounds__(64 * CS_WAVES) void cutoff_layer_small_kernel(TailParams t) {
  __shared__ uint16_t sLog[CT_ROWS][128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const CutoffParams& p = t.cp;
  const int n_cut = 2 * p.G * ((p.M + CT_ROWS - 1) / CT_ROWS);
  if ((int)blockIdx.x < n_cut) {
    const int rt = blockIdx.x / (2 * p.G), id = blockIdx.x % (2 * p.G);
    const int mat = id & 1, g = id >> 1;
    const int row0 = rt * CT_ROWS;
    const int D = p.D;
    int off[2];
    uint16_t xr[2][E];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int m = min(row0 + wave + CS_WAVES * r, p.M - 1);
      off[r] = t.ptr[mat][(long long)m * p.G + g];
      const uint16_t* xs = p.mat[mat].x + (long long)m * p.x_ld + (long long)g * D + lane * E;
#pragma unroll
      for (int e = 0; e < E; ++e) xr[r][e] = xs[e];
    }
    small_logits<DT>(p, mat, g, wave, lane, sLog, row0);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int m = row0 + wave + CS_WAVES * r;
      if (m >= p.M) break;
      const long long rg = (long long)m * p.G + g;
      const int len = cutoff_row_len<DT, E>(p, &sLog[m - row0][0], lane);
      if (lane == 0) {
        t.ptr[mat][rg] = off[r] + len;
        t.lens[mat][rg * t.tab_sb[mat] + (long long)t.seq * t.tab_ss[mat]] = len;
        t.offs[mat][rg * t.tab_sb[mat] + (long long)t.seq * t.tab_ss[mat]] = off[r];
      }
      uint16_t* dst = (uint16_t*)t.flat[mat] + rg * t.flat_ld[mat] + off[r] + lane * E;
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (lane * E + e < len) dst[e] = xr[r][e];
    }
    return;
  }
  const long long qr = (long long)(blockIdx.x - n_cut) * CS_WAVES + wave;
  if (qr < t.q_rows)
    dkv_rope_pair<DT>(t.q + (qr / t.Hq) * t.q_sb + (qr % t.Hq) * 128, lane, t.pos, t.log_theta);
}

// the logits of every (row, group, K|V) into the workspace: split-K for D of 256 and more
void launch_logits(const CutoffParams& p, int dtype, hipStream_t st) {
  const int D = p.D, M = p.M, G = p.G;
  const unsigned gy = (unsigned)((M + CT_ROWS - 1) / CT_ROWS), gz = (unsigned)(2 * G);
#define DKV_LKS(STEPS_)                                                                        \
  do {                                                                                         \
    if (dtype == DKV_BF16)                                                                     \
      hipLaunchKernelGGL((cutoff_logits_ks_kernel<DKV_BF16, STEPS_>), dim3(D / 16, gy, gz),    \
                         dim3(256), 0, st, p);                                                 \
    else                                                                                       \
      hipLaunchKernelGGL((cutoff_logits_ks_kernel<DKV_F16, STEPS_>), dim3(D / 16, gy, gz),     \
                         dim3(256), 0, st, p);                                                 \
  } while (0)
  if (D == 1024)
    DKV_LKS(8);
  else if (D == 512)
    DKV_LKS(4);
  else if (D == 256)
    DKV_LKS(2);
  else if (dtype == DKV_BF16)
    hipLaunchKernelGGL(cutoff_logits_kernel<DKV_BF16>, dim3(D / CT_COLS, gy, gz), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(cutoff_logits_kernel<DKV_F16>, dim3(D / CT_COLS, gy, gz), dim3(256), 0, st, p);
#undef DKV_LKS
}

template <int DT, int E>
void launch_rows(const CutoffParams& p, hipStream_t st) {
  const long long tasks = 2LL * p.M * p.G;
  hipLaunchKernelGGL((cutoff_rows_kernel<DT, E>), dim3((unsigned)((tasks + 3) / 4)), dim3(256), 0,
                     st, p);
}

}  // namespace

extern "C" long long dkv_cutoff_workspace_bytes(int M, int G, int D) {
  if (M < 0 || G <= 0 || D <= 0) return -1;
  return 2LL * M * G * D * 2;
}

extern "C" int dkv_cutoff_kv(void* stream, int dtype, const void* xk, const void* xv,
                             long long x_ld, const void* wt_k, const void* wt_v, const void* b_k,
                             const void* b_v, float threshold, int low_rank, void* out_k,
                             void* out_v, long long out_ld, int* len_k, int* len_v,
                             long long len_ld, void* workspace, long long workspace_bytes, int M,
                             int G, int D) {
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (M < 0 || G <= 0 || D <= 0) return DKV_E_ARG;
  if (M == 0) return DKV_OK;
  if (!xk || !xv || !wt_k || !wt_v || !b_k || !b_v || !out_k || !out_v || !len_k || !len_v ||
      !workspace)
    return DKV_E_ARG;
  if (D % 64 != 0 || D > 1024) return DKV_E_UNSUPPORTED;
  if (x_ld < (long long)G * D || out_ld < (long long)G * D || len_ld < G) return DKV_E_ARG;
  if (x_ld % 8 != 0 || ((uintptr_t)xk | (uintptr_t)xv | (uintptr_t)wt_k | (uintptr_t)wt_v) % 16)
    return DKV_E_UNSUPPORTED;  // 16-byte operand loads
  if (workspace_bytes < dkv_cutoff_workspace_bytes(M, G, D)) return DKV_E_WORKSPACE;
  if ((long long)M * G * D >= (1LL << 31) / 2) return DKV_E_UNSUPPORTED;
  CutoffParams p;
  const void* xs[2] = {xk, xv};
  const void* ws[2] = {wt_k, wt_v};
  const void* bs[2] = {b_k, b_v};
  void* os[2] = {out_k, out_v};
  int* ls[2] = {len_k, len_v};
  for (int t = 0; t < 2; ++t) {
    p.mat[t].x = (const uint16_t*)xs[t];
    p.mat[t].wt = (const uint16_t*)ws[t];
    p.mat[t].b = (const uint16_t*)bs[t];
    p.mat[t].out = (uint16_t*)os[t];
    p.mat[t].lens = ls[t];
    p.mat[t].logits = (uint16_t*)workspace + (long long)t * M * G * D;
  }
  p.x_ld = x_ld;
  p.out_ld = out_ld;
  p.len_ld = len_ld;
  p.M = M;
  p.G = G;
  p.D = D;
  p.low_rank = low_rank < 0 ? D : min(low_rank, D);
  // the reference compares against 0.1 in the compute dtype
  p.threshold = dtype == DKV_BF16 ? (float)(__bf16)threshold : (float)(_Float16)threshold;
  const int E = D / 64;
  if (E != 1 && E != 2 && E != 4 && E != 8 && E != 16) return DKV_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  if (M <= CT_ROWS && D <= 128) {
    if (dtype == DKV_BF16) {
      if (E == 1)
        hipLaunchKernelGGL((cutoff_small_kernel<DKV_BF16, 1>), dim3(2 * G), dim3(64 * CS_WAVES), 0, st, p);
      else
        hipLaunchKernelGGL((cutoff_small_kernel<DKV_BF16, 2>), dim3(2 * G), dim3(64 * CS_WAVES), 0, st, p);
    } else {
      if (E == 1)
        hipLaunchKernelGGL((cutoff_small_kernel<DKV_F16, 1>), dim3(2 * G), dim3(64 * CS_WAVES), 0, st, p);
      else
        hipLaunchKernelGGL((cutoff_small_kernel<DKV_F16, 2>), dim3(2 * G), dim3(64 * CS_WAVES), 0, st, p);
    }
    DKV_HIP_CHECK_LAUNCH();
    return DKV_OK;
  }
  launch_logits(p, dtype, st);
  DKV_HIP_CHECK_LAUNCH();
#define DKV_ROWS_CASE(e)                                        \
  case e:                                                       \
    if (dtype == DKV_BF16)                                      \
      launch_rows<DKV_BF16, e>(p, st);                          \
    else                                                        \
      launch_rows<DKV_F16, e>(p, st);                           \
    break;
  switch (E) {
    DKV_ROWS_CASE(1)
    DKV_ROWS_CASE(2)
    DKV_ROWS_CASE(4)
    DKV_ROWS_CASE(8)
    DKV_ROWS_CASE(16)
    default:
      return DKV_E_UNSUPPORTED;
  }
#undef DKV_ROWS_CASE
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

// The decode step's cutoff head, K+V append and query RoPE in one launch
// (cutoff_layer_kernel). Used by dkv_decode_layer; same checks as
// dkv_cutoff_kv for the cutoff part. The per-row scratch (coef_k/v, len_k/v) of the layer's
// argument block is not used.
int dkv_layer_cutoff_append_rope(void* stream, const DkvDecodeLayer* L, const void* k_coef,
                                 const void* v_coef, void* q, int seq, int pos) {
  const int dtype = L->dtype, M = L->B, G = L->G, D = L->R;
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (M < 0 || G <= 0 || D <= 0 || L->Hq <= 0 || L->Dh != 128) return DKV_E_ARG;
  if (M == 0) return DKV_OK;
  if (!L->wt_k || !L->wt_v || !L->b_k || !L->b_v || !L->cut_ws || !L->flat_k || !L->flat_v ||
      !L->lens_k || !L->offs_k || !L->lens_v || !L->offs_v || !L->ptr_k || !L->ptr_v)
    return DKV_E_ARG;
  if (D % 64 != 0 || D > 1024) return DKV_E_UNSUPPORTED;
  const long long x_ld = L->coef_ld ? L->coef_ld : (long long)G * D;
  const long long q_sb = L->q_sb ? L->q_sb : (long long)L->Hq * 128;
  if (x_ld < (long long)G * D || q_sb < (long long)L->Hq * 128) return DKV_E_ARG;
  if (x_ld % 8 != 0 || ((uintptr_t)k_coef | (uintptr_t)v_coef | (uintptr_t)L->wt_k |
                        (uintptr_t)L->wt_v) % 16)
    return DKV_E_UNSUPPORTED;
  if (L->cut_ws_bytes < dkv_cutoff_workspace_bytes(M, G, D)) return DKV_E_WORKSPACE;
  if ((long long)M * G * D >= (1LL << 31) / 2) return DKV_E_UNSUPPORTED;
  const int E = D / 64;
  if (E != 1 && E != 2 && E != 4 && E != 8 && E != 16) return DKV_E_UNSUPPORTED;
  TailParams t;
  CutoffParams& p = t.cp;
  const void* xs[2] = {k_coef, v_coef};
  const void* ws[2] = {L->wt_k, L->wt_v};
  const void* bs[2] = {L->b_k, L->b_v};
  for (int m = 0; m < 2; ++m) {
    p.mat[m].x = (const uint16_t*)xs[m];
    p.mat[m].wt = (const uint16_t*)ws[m];
    p.mat[m].b = (const uint16_t*)bs[m];
    p.mat[m].out = nullptr;
    p.mat[m].lens = nullptr;
    p.mat[m].logits = (uint16_t*)L->cut_ws + (long long)m * M * G * D;
  }
  p.x_ld = x_ld;
  p.out_ld = x_ld;
  p.len_ld = G;
  p.M = M;
  p.G = G;
  p.D = D;
  p.low_rank = L->low_rank < 0 ? D : min(L->low_rank, D);
  p.threshold = dtype == DKV_BF16 ? (float)(__bf16)L->threshold : (float)(_Float16)L->threshold;
  t.flat[0] = L->flat_k;
  t.flat[1] = L->flat_v;
  t.flat_ld[0] = L->flat_k_ld;
  t.flat_ld[1] = L->flat_v_ld;
  t.lens[0] = L->lens_k;
  t.lens[1] = L->lens_v;
  t.offs[0] = L->offs_k;
  t.offs[1] = L->offs_v;
  t.tab_sb[0] = L->tab_k_sb;
  t.tab_sb[1] = L->tab_v_sb;
  t.tab_ss[0] = L->tab_k_ss;
  t.tab_ss[1] = L->tab_v_ss;
  t.ptr[0] = L->ptr_k;
  t.ptr[1] = L->ptr_v;
  t.seq = seq;
  t.q = (uint16_t*)q;
  t.q_sb = q_sb;
  t.q_rows = pos < 0 ? 0 : M * L->Hq;  // pos < 0: the caller rotated q already
  t.Hq = L->Hq;
  t.pos = pos;
  t.log_theta = L->log_theta;
  hipStream_t st = (hipStream_t)stream;
  if (D <= 128) {
    // every 16-row tile of every (group, K|V) in its own workgroup, then the query rows
    const long long tiles = (M + CT_ROWS - 1) / CT_ROWS;
    const dim3 sgrid((unsigned)(2 * G * tiles + (t.q_rows + CS_WAVES - 1) / CS_WAVES));
    if (E == 1) {
      if (dtype == DKV_BF16)
        hipLaunchKernelGGL((cutoff_layer_small_kernel<DKV_BF16, 1>), sgrid, dim3(64 * CS_WAVES),
                           0, st, t);
      else
        hipLaunchKernelGGL((cutoff_layer_small_kernel<DKV_F16, 1>), sgrid, dim3(64 * CS_WAVES),
                           0, st, t);
    } else {
      if (dtype == DKV_BF16)
        hipLaunchKernelGGL((cutoff_layer_small_kernel<DKV_BF16, 2>), sgrid, dim3(64 * CS_WAVES),
                           0, st, t);
      else
        hipLaunchKernelGGL((cutoff_layer_small_kernel<DKV_F16, 2>), sgrid, dim3(64 * CS_WAVES),
                           0, st, t);
    }
    DKV_HIP_CHECK_LAUNCH();
    return DKV_OK;
  }
  const dim3 grid((unsigned)(2 * G + (t.q_rows + 3) / 4));
#define DKV_TAIL_CASE(e)                                                                 \
  case e:                                                                                \
    if (dtype == DKV_BF16)                                                               \
      hipLaunchKernelGGL((cutoff_layer_kernel<DKV_BF16, e>), grid, dim3(256), 0, st, t);       \
    else                                                                                 \
      hipLaunchKernelGGL((cutoff_layer_kernel<DKV_F16, e>), grid, dim3(256), 0, st, t);        \
    break;
  switch (E) {
    DKV_TAIL_CASE(1)
    DKV_TAIL_CASE(2)
    DKV_TAIL_CASE(4)
    DKV_TAIL_CASE(8)
    DKV_TAIL_CASE(16)
    default:
      return DKV_E_UNSUPPORTED;
  }
#undef DKV_TAIL_CASE
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
