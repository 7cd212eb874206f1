// Split-K compressed decode attention for gfx950 (MFMA), the fast path behind both router
// routes (reference src/dynakv/kernels/fused.py:28-170, two_stage.py:48-324, router.py:20-59).
//
// Work unit: (batch b, KV head k) with hpg query heads sharing K/V basis k; its packed
// coefficients are cache row b*G + k/(Hkv/G). A workgroup (4 waves) owns one unit and one
// contiguous token range ("split"); waves take 16-token tiles round-robin.
//
// Per 16-token tile and wave:
//   1. K^T[128 x 16] = BK^T[128 x R] . X^T[R x 16] on v_mfma_f32_16x16x32_{bf16,f16}.
//      BK^T sits in LDS (staged once per workgroup); X^T is gathered straight from the
//      packed rows with 16-byte buffer loads (one lane = one token x 8 ranks), zero-masked
//      past the token's retained count; rank chunks of 32 stop at the tile's largest count.
//   2. rotate-half RoPE by cache row index on the accumulator registers (lane-local pairs
//      (i, i+64)), cos/sin advanced by an angle-addition recurrence seeded from a table.
//   3. scores[16 tokens x hpg] on one 16x16x32 f16 MFMA chain against the scaled query.
//   4. online softmax in the log2 domain with lazy rescaling (only when the running max grows
//      by more than 2^11.5), then P.X^V on 16x16x16 MFMA in coefficient space (the V basis is
//      applied once per output in the merge kernel).
// Partials (m, l, acc[128]) per (unit, split, head) are LSE-merged and projected through the
// V basis by merge_kernel.
#include "dkv_common.h"

namespace {

constexpr int DH = 128;
constexpr int TILE = 16;
constexpr int WAVES = 4;
constexpr int BK_LD = 136;  // LDS row pitch (elements) of the transposed K basis
constexpr int PREC = DH + 2;  // floats per partial record: m, l, acc[128]
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_THRESH = 11.5f;  // log2 units

struct SplitParams {
  const uint16_t* q;
  long long q_sb, q_sh;
  const uint16_t* k_basis;
  long long k_unit, k_sr;
  const uint16_t* k_flat;
  const uint16_t* v_flat;
  long long k_ld, v_ld;
  const int* lens_k;
  const int* offs_k;
  long long tk_sb, tk_ss;
  const int* lens_v;
  const int* offs_v;
  long long tv_sb, tv_ss;
  const float* rope;  // [n_tb][64] (cos, sin) of tile bases, then [16][64] in-tile deltas,
                      // then [64] per-step (64 positions) rotations
  float* partials;
  int B, Hq, Hkv, G, S, R, hpg, n_splits, split_len, n_tb;
  float q_scale;      // multiplies q before the fp16 cast
  float masked_score; // two-stage: -1e4 * (1/sqrt(Dh)) in fp32
};

template <int DT>
__device__ __forceinline__ dkv_f32x4 mfma_k(const dkv_u32x4& a, const dkv_u32x4& b,
                                            dkv_f32x4 c) {
  if constexpr (DT == DKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dkv_bf16x8, a),
                                                   __builtin_bit_cast(dkv_bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dkv_f16x8, a),
                                                  __builtin_bit_cast(dkv_f16x8, b), c, 0, 0, 0);
}
template <int DT>
__device__ __forceinline__ dkv_f32x4 mfma_pv(const dkv_u32x2& a, const dkv_u32x2& b,
                                             dkv_f32x4 c) {
  if constexpr (DT == DKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(dkv_bf16x4, a),
                                                     __builtin_bit_cast(dkv_bf16x4, b), c, 0, 0,
                                                     0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(dkv_f16x4, a),
                                                 __builtin_bit_cast(dkv_f16x4, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  dkv_f16x2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return dkv_f32_to_bf16_bits(lo) | (dkv_f32_to_bf16_bits(hi) << 16);
}
template <int DT>
__device__ __forceinline__ float elt_to_f32(uint32_t bits16) {
  if constexpr (DT == DKV_BF16)
    return dkv_bf16_bits_to_f32(bits16);
  else
    return dkv_f16_bits_to_f32(bits16);
}

__device__ __forceinline__ dkv_f32x4 mfma_f16(const dkv_u32x4& a, const dkv_u32x4& b,
                                              dkv_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dkv_f16x8, a),
                                                __builtin_bit_cast(dkv_f16x8, b), c, 0, 0, 0);
}

// x ~= hi + lo with hi = fp16(x) and lo = fp16(x - hi), for two values packed per dword.
__device__ __forceinline__ void split_f16x2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
  const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
  hi = __builtin_bit_cast(uint32_t, dkv_f16x2{h0, h1});
  lo = __builtin_bit_cast(uint32_t, dkv_f16x2{l0, l1});
}

// Element-wise gather of the first nv (1..8) 16-bit values at element offset e; the rest zero.
__device__ __forceinline__ dkv_u32x4 gather8_b16(__amdgpu_buffer_rsrc_t r, int e, int nv) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (t < nv) {
      const uint32_t v = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (e + t) * 2, 0, 0);
      w[t >> 1] |= v << (16 * (t & 1));
    }
  }
  return dkv_u32x4{w[0], w[1], w[2], w[3]};
}

// Zero the elements at index >= nv (0 <= nv < 8) of an 8 x 16-bit vector.
__device__ __forceinline__ dkv_u32x4 mask_prefix8(dkv_u32x4 v, int nv) {
  const int nlo = min(nv, 4), nhi = max(nv - 4, 0);
  const unsigned long long mlo = nlo >= 4 ? ~0ull : ((1ull << (16 * nlo)) - 1ull);
  const unsigned long long mhi = nhi >= 4 ? ~0ull : ((1ull << (16 * nhi)) - 1ull);
  v.x &= (uint32_t)mlo;
  v.y &= (uint32_t)(mlo >> 32);
  v.z &= (uint32_t)mhi;
  v.w &= (uint32_t)(mhi >> 32);
  return v;
}

// Wave-uniform maximum of a per-lane int, returned in a scalar register.
__device__ __forceinline__ int wave_max_uniform(int v) {
  return __builtin_amdgcn_readfirstlane(dkv_wave_max_i(v));
}

// ---------------------------------------------------------------------------------------
// RoPE table prologue: cos/sin of tile-base positions, in-tile deltas and the per-step
// rotation, evaluated in double from the fp32 angle the reference forms
// (angle = float(pos) * inv_freq, reference fused.py:65-66,97 / two_stage.py:36-44).
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rope_table_kernel(float* __restrict__ rope, int n_tb,
                                                         float log_theta) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int total = (n_tb + TILE + 1) * 64;
  if (idx >= total) return;
  const int r = idx / 64, i = idx % 64;
  const float inv = dkv_inv_freq(i, DH, log_theta);
  float ang;
  if (r < n_tb)
    ang = (float)(r * TILE) * inv;
  else if (r < n_tb + TILE)
    ang = (float)(r - n_tb) * inv;
  else
    ang = (float)(TILE * WAVES) * inv;
  double s, c;
  sincos((double)ang, &s, &c);
  rope[2 * idx] = (float)c;
  rope[2 * idx + 1] = (float)s;
}

template <int DT, int ROUTE>
__global__ __launch_bounds__(256, 2) void splitk_kernel(SplitParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sBK[DH * BK_LD];

  // XCD-aware mapping: consecutive workgroup ids land on different XCDs (id % 8), so give
  // every split of one unit the same id % 8 to keep that unit's basis in one L2.
  const int nunits = p.B * p.Hkv;
  int unit, split;
  {
    const int id = blockIdx.x;
    if ((nunits & 7) == 0) {
      const int xcd = id & 7, k = id >> 3;
      unit = xcd + 8 * (k / p.n_splits);
      split = k % p.n_splits;
    } else {
      unit = id / p.n_splits;
      split = id % p.n_splits;
    }
  }
  const int b = unit / p.Hkv, kvh = unit % p.Hkv;
  const int row = b * p.G + kvh / (p.Hkv / p.G);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int R = p.R;

  // ---- stage BK^T ([dim][rank], ranks >= R zero) into LDS --------------------------------
  {
    const uint16_t* kb = p.k_basis + (long long)kvh * p.k_unit;
    for (int idx = tid; idx < 128 * 16; idx += 256) {
      const int j = idx >> 4, d8 = (idx & 15) * 8;
      dkv_u32x4 v = {0u, 0u, 0u, 0u};
      if (j < R) v = *(const dkv_u32x4*)(kb + (long long)j * p.k_sr + d8);
      const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        sBK[(d8 + 2 * t) * BK_LD + j] = (uint16_t)(e[t] & 0xffffu);
        sBK[(d8 + 2 * t + 1) * BK_LD + j] = (uint16_t)(e[t] >> 16);
      }
    }
  }

  // ---- scaled query as the B operand of the QK MFMA: lane (head slot n, k-group g) holds
  //      (q_i, q_{i+64}) for i = 16*qi + 4*g + w, w = 0..3 --------------------------------
  dkv_u32x4 bq[4], bql[4];  // fp16 hi and lo parts of the scaled query
  {
    const int hs = n;
    const bool real = hs < p.hpg;
    const long long qo = (long long)b * p.q_sb + (long long)(kvh * p.hpg + (real ? hs : 0)) * p.q_sh;
#pragma unroll
    for (int qi = 0; qi < 4; ++qi) {
      uint32_t w4[4], l4[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int i = 16 * qi + 4 * g + w;
        const float a = real ? elt_to_f32<DT>(p.q[qo + i]) * p.q_scale : 0.f;
        const float c = real ? elt_to_f32<DT>(p.q[qo + i + 64]) * p.q_scale : 0.f;
        split_f16x2(a, c, w4[w], l4[w]);
      }
      bq[qi] = dkv_u32x4{w4[0], w4[1], w4[2], w4[3]};
      bql[qi] = dkv_u32x4{l4[0], l4[1], l4[2], l4[3]};
    }
  }

  const int tiles_per_split = p.split_len / TILE;
  const int tile0 = split * tiles_per_split + wave;
  const int s_end = min(p.S, (split + 1) * p.split_len);

  // ---- RoPE state for this lane's token slot n and its 16 frequencies ---------------------
  float rc[16], rs[16], dc[16], ds[16];
  {
    const int tb = min(tile0, p.n_tb - 1);
    const float* base = p.rope + (long long)tb * 128;
    const float* delt = p.rope + (long long)(p.n_tb + n) * 128;
    const float* step = p.rope + (long long)(p.n_tb + TILE) * 128;
#pragma unroll
    for (int qi = 0; qi < 4; ++qi)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int i = 16 * qi + 4 * g + w, f = qi * 4 + w;
        const float bc = base[2 * i], bs = base[2 * i + 1];
        const float ec = delt[2 * i], es = delt[2 * i + 1];
        rc[f] = bc * ec - bs * es;
        rs[f] = bs * ec + bc * es;
        dc[f] = step[2 * i];
        ds[f] = step[2 * i + 1];
      }
  }

  __syncthreads();  // sBK ready

  const __amdgpu_buffer_rsrc_t rk_src =
      dkv_make_rsrc(p.k_flat + (long long)row * p.k_ld, (uint32_t)(p.k_ld * 2));
  const __amdgpu_buffer_rsrc_t rv_src =
      dkv_make_rsrc(p.v_flat + (long long)row * p.v_ld, (uint32_t)(p.v_ld * 2));
  const int* lk = p.lens_k + (long long)row * p.tk_sb;
  const int* ok_ = p.offs_k + (long long)row * p.tk_sb;
  const int* lv = p.lens_v + (long long)row * p.tv_sb;
  const int* ov_ = p.offs_v + (long long)row * p.tv_sb;

  dkv_f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // per head slot n (log2 units), identical across g
  float l_run = 0.f;        // partial over this lane's 4 tokens per tile

  for (int T = tile0; T * TILE < s_end; T += WAVES) {
    const int t = T * TILE + n;
    const bool valid = t < s_end;
    const int rk = valid ? lk[(long long)t * p.tk_ss] : 0;
    const int ok = valid ? ok_[(long long)t * p.tk_ss] : 0;
    const int rv = valid ? lv[(long long)t * p.tv_ss] : 0;
    const int ov = valid ? ov_[(long long)t * p.tv_ss] : 0;
    const int rkc = max(0, min(rk, R));
    const int rvc = max(0, min(rv, R));

    // ---- 1. K reconstruction ----------------------------------------------------------------
    dkv_f32x4 ck[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ck[i] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
    const int nck = (wave_max_uniform(rkc) + 31) >> 5;
    for (int c = 0; c < nck; ++c) {
      const int j0 = 32 * c + 8 * g;
      const int nv = rkc - j0;
      const int boff = nv > 0 ? (ok + j0) * 2 : 0x7ffffff0;
      dkv_u32x4 xv;
      if (nv > 0 && (long long)(ok + j0 + 8) > p.k_ld) {
        // the 16-byte window would cross the end of the row's buffer, where an out-of-range
        // vector access reads as all zeros: gather element by element instead
        xv = gather8_b16(rk_src, ok + j0, nv);
      } else {
        xv = __builtin_amdgcn_raw_buffer_load_b128(rk_src, boff, 0, 0);
        if (nv < 8) xv = mask_prefix8(xv, max(nv, 0));
      }
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) {
        const dkv_u32x4 a = *(const dkv_u32x4*)&sBK[(16 * blk + n) * BK_LD + 32 * c + 8 * g];
        ck[blk] = mfma_k<DT>(a, xv, ck[blk]);
      }
    }

    // ---- 2. RoPE on (i, i+64) pairs, packed to fp16 as the QK A operand -----------------------
    dkv_u32x4 aq[4], aql[4];
#pragma unroll
    for (int qi = 0; qi < 4; ++qi) {
      uint32_t w4[4], l4[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int f = qi * 4 + w;
        const float k0 = ck[qi][w], k1 = ck[qi + 4][w];
        const float r0 = k0 * rc[f] - k1 * rs[f];
        const float r1 = k1 * rc[f] + k0 * rs[f];
        split_f16x2(r0, r1, w4[w], l4[w]);
      }
      aq[qi] = dkv_u32x4{w4[0], w4[1], w4[2], w4[3]};
      aql[qi] = dkv_u32x4{l4[0], l4[1], l4[2], l4[3]};
    }
    // advance the rotation by WAVES*TILE positions
#pragma unroll
    for (int f = 0; f < 16; ++f) {
      const float c2 = rc[f] * dc[f] - rs[f] * ds[f];
      const float s2 = rs[f] * dc[f] + rc[f] * ds[f];
      rc[f] = c2;
      rs[f] = s2;
    }

    // ---- 3. scores: lane (head slot n, tokens 4g+u) -----------------------------------------
    // scores = K'.Q with hi/lo fp16 parts on both sides (~22-bit products, fp32 accumulate)
    dkv_f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int qi = 0; qi < 4; ++qi) {
      sc = mfma_f16(aql[qi], bq[qi], sc);
      sc = mfma_f16(aq[qi], bql[qi], sc);
      sc = mfma_f16(aq[qi], bq[qi], sc);
    }
    const unsigned long long has_bits = __ballot(valid && rk > 0);
    const unsigned long long in_bits = __ballot(valid);
    float z[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tok = 4 * g + u;
      const bool has = (has_bits >> tok) & 1ull;
      const bool inr = (in_bits >> tok) & 1ull;
      float v;
      if constexpr (ROUTE == DKV_ROUTE_FUSED) {
        v = has ? sc[u] : -INFINITY;  // q already carries sm_scale * log2(e)
      } else {
        v = dkv_round_to<DT>(has ? sc[u] : p.masked_score) * LOG2E;
      }
      z[u] = inr ? v : -INFINITY;
    }

    // ---- 4. online softmax (per head slot) --------------------------------------------------
    float tmax = fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3]));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const bool grow = tmax > m_run + RESCALE_THRESH;
    if (__ballot(grow)) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
      float au[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) au[u] = __shfl(alpha, 4 * g + u, 64);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[i][u] *= au[u];
    }
    float pu[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      pu[u] = (z[u] == -INFINITY) ? 0.f : exp2f(z[u] - m_run);
      l_run += pu[u];
    }

    // ---- 5. P . X^V in coefficient space ----------------------------------------------------
    int rvu[4], ovu[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      rvu[u] = __shfl(rvc, 4 * g + u, 64);
      ovu[u] = __shfl(ov, 4 * g + u, 64);
    }
    const int nbv = (wave_max_uniform(rvc) + 15) >> 4;
    dkv_u32x2 pa_hi, pa_lo;
    if constexpr (DT == DKV_F16) {
      pa_hi = dkv_u32x2{pack_f16x2(pu[0], pu[1]), pack_f16x2(pu[2], pu[3])};
      pa_lo = pa_hi;
    } else {
      const uint32_t h0 = dkv_f32_to_bf16_bits(pu[0]), h1 = dkv_f32_to_bf16_bits(pu[1]);
      const uint32_t h2 = dkv_f32_to_bf16_bits(pu[2]), h3 = dkv_f32_to_bf16_bits(pu[3]);
      pa_hi = dkv_u32x2{h0 | (h1 << 16), h2 | (h3 << 16)};
      pa_lo = dkv_u32x2{pack_bf16x2(pu[0] - dkv_bf16_bits_to_f32(h0), pu[1] - dkv_bf16_bits_to_f32(h1)),
                        pack_bf16x2(pu[2] - dkv_bf16_bits_to_f32(h2), pu[3] - dkv_bf16_bits_to_f32(h3))};
    }
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      if (blk < nbv) {  // wave-uniform
        const int j = 16 * blk + n;
        uint32_t e[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int boff = j < rvu[u] ? (ovu[u] + j) * 2 : 0x7ffffff0;
          e[u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rv_src, boff, 0, 0);
        }
        const dkv_u32x2 xb = {e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
        // acc rows = head slots 4g+u, column = rank j
        acc[blk] = mfma_pv<DT>(pa_hi, xb, acc[blk]);
        if constexpr (DT == DKV_BF16) acc[blk] = mfma_pv<DT>(pa_lo, xb, acc[blk]);
      }
    }
  }

  // ---- combine the 4 waves through LDS and write the partial record ----------------------
  float l_tot = l_run;
  l_tot += __shfl_xor(l_tot, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  __syncthreads();  // all waves done with sBK
  float* sw = reinterpret_cast<float*>(sBK);  // [WAVES][16 m | 16 l | 16 x 128 acc]
  constexpr int WREC = 32 + 16 * DH;
  float* my = sw + wave * WREC;
  if (g == 0) {
    my[n] = m_run;
    my[16 + n] = l_tot;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u) my[32 + (4 * g + u) * DH + 16 * i + n] = acc[i][u];
  __syncthreads();
  float* out = p.partials + ((long long)unit * p.n_splits + split) * p.hpg * PREC;
  for (int idx = tid; idx < p.hpg * (DH + 2); idx += 256) {
    const int hs = idx / (DH + 2), e = idx % (DH + 2);
    float mw[WAVES], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      mw[w] = sw[w * WREC + hs];
      M = fmaxf(M, mw[w]);
    }
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float wt = (M == -INFINITY) ? 0.f : exp2f(mw[w] - M);
      const float x = e == 1 ? sw[w * WREC + 16 + hs] : (e >= 2 ? sw[w * WREC + 32 + hs * DH + (e - 2)] : 0.f);
      v += wt * x;
    }
    out[hs * PREC + e] = e == 0 ? M : v;
  }
}

// One block per unit: LSE-merge the splits of each head slot, normalise, project through the
// V basis of the unit's KV head, store in the query dtype.
template <int DT, int ROUTE, int ODT>
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ partials,
                                                    const uint16_t* __restrict__ v_basis,
                                                    long long v_unit, long long v_sr,
                                                    void* __restrict__ out, long long out_sb,
                                                    long long out_sh, int Hkv, int hpg,
                                                    int n_splits, int R) {
  __shared__ float s_a[16][DH];
  __shared__ float s_w[16][64];
  const int unit = blockIdx.x;
  const int b = unit / Hkv, kvh = unit % Hkv;
  const int tid = threadIdx.x;
  const float* pr = partials + (long long)unit * n_splits * hpg * PREC;
  // per head slot: max over splits, then weighted sums
  for (int hs = tid >> 4; hs < hpg; hs += 16) {
    // 16 threads per head slot cooperate over splits
    const int lane16 = tid & 15;
    float M = -INFINITY;
    for (int s = lane16; s < n_splits; s += 16) M = fmaxf(M, pr[((long long)s * hpg + hs) * PREC]);
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) M = fmaxf(M, __shfl_xor(M, m, 16));
    float L = 0.f;
    for (int s = lane16; s < n_splits; s += 16) {
      const float* rec = pr + ((long long)s * hpg + hs) * PREC;
      const float w = (M == -INFINITY) ? 0.f : exp2f(rec[0] - M);
      if (s < 64) s_w[hs][s] = w;
      L += w * rec[1];
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) L += __shfl_xor(L, m, 16);
    if (lane16 == 0) s_w[hs][63] = L;  // slot 63 reused for L when n_splits <= 63
  }
  __syncthreads();
  // weighted accumulator sums; n_splits <= 63 guaranteed by the host
  for (int idx = tid; idx < hpg * DH; idx += 256) {
    const int hs = idx / DH, j = idx % DH;
    float a = 0.f;
    if (j < R) {
      for (int s = 0; s < n_splits; ++s) a += s_w[hs][s] * pr[((long long)s * hpg + hs) * PREC + 2 + j];
    }
    const float L = s_w[hs][63];
    const float den = ROUTE == DKV_ROUTE_TWO_STAGE ? fmaxf(L, 1e-6f) : L;
    s_a[hs][j] = a / den;
  }
  __syncthreads();
  const uint16_t* vb = v_basis + (long long)kvh * v_unit;
  const int d = tid & 127, hh = tid >> 7;
  for (int hs = hh; hs < hpg; hs += 2) {
    float o = 0.f;
    for (int j = 0; j < R; ++j) o = fmaf(s_a[hs][j], elt_to_f32<DT>(vb[(long long)j * v_sr + d]), o);
    const long long oi = (long long)b * out_sb + (long long)(kvh * hpg + hs) * out_sh + d;
    dkv_store_f32<ODT>(out, oi, o);
  }
}

// ---------------------------------------------------------------------------------------
// Self test of the operand layouts and unaligned gathers assumed above.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void selftest_kernel(int* __restrict__ mismatches) {
  __shared__ uint16_t buf[512];
  const int l = threadIdx.x;
  const int n = l & 15, g = l >> 4;
  int bad = 0;
  // A[m][k] = (m + 2k) % 7 - 3, B[k][n] = (3k + n) % 5 - 2 (small integers: exact in 16-bit fp)
  auto Aval = [](int m, int k) { return (float)(((m + 2 * k) % 7) - 3); };
  auto Bval = [](int k, int nn) { return (float)(((3 * k + nn) % 5) - 2); };
  // 16x16x32 bf16 and f16: lane holds A[n][8g+v], B[8g+v][n]; C lane holds C[4g+u][n]
  {
    uint32_t a4b[4], b4b[4], a4h[4], b4h[4];
    for (int w = 0; w < 4; ++w) {
      const float a0 = Aval(n, 8 * g + 2 * w), a1 = Aval(n, 8 * g + 2 * w + 1);
      const float b0 = Bval(8 * g + 2 * w, n), b1 = Bval(8 * g + 2 * w + 1, n);
      a4b[w] = pack_bf16x2(a0, a1);
      b4b[w] = pack_bf16x2(b0, b1);
      a4h[w] = pack_f16x2(a0, a1);
      b4h[w] = pack_f16x2(b0, b1);
    }
    dkv_f32x4 c0 = {0.f, 0.f, 0.f, 0.f};
    dkv_f32x4 cb = mfma_k<DKV_BF16>(dkv_u32x4{a4b[0], a4b[1], a4b[2], a4b[3]},
                                    dkv_u32x4{b4b[0], b4b[1], b4b[2], b4b[3]}, c0);
    dkv_f32x4 ch = mfma_k<DKV_F16>(dkv_u32x4{a4h[0], a4h[1], a4h[2], a4h[3]},
                                   dkv_u32x4{b4h[0], b4h[1], b4h[2], b4h[3]}, c0);
    for (int u = 0; u < 4; ++u) {
      float ref = 0.f;
      for (int k = 0; k < 32; ++k) ref += Aval(4 * g + u, k) * Bval(k, n);
      bad += (cb[u] != ref) + (ch[u] != ref);
    }
  }
  // 16x16x16: lane holds A[n][4g+v], B[4g+v][n]
  {
    const uint32_t a0b = pack_bf16x2(Aval(n, 4 * g), Aval(n, 4 * g + 1));
    const uint32_t a1b = pack_bf16x2(Aval(n, 4 * g + 2), Aval(n, 4 * g + 3));
    const uint32_t b0b = pack_bf16x2(Bval(4 * g, n), Bval(4 * g + 1, n));
    const uint32_t b1b = pack_bf16x2(Bval(4 * g + 2, n), Bval(4 * g + 3, n));
    const uint32_t a0h = pack_f16x2(Aval(n, 4 * g), Aval(n, 4 * g + 1));
    const uint32_t a1h = pack_f16x2(Aval(n, 4 * g + 2), Aval(n, 4 * g + 3));
    const uint32_t b0h = pack_f16x2(Bval(4 * g, n), Bval(4 * g + 1, n));
    const uint32_t b1h = pack_f16x2(Bval(4 * g + 2, n), Bval(4 * g + 3, n));
    dkv_f32x4 c0 = {0.f, 0.f, 0.f, 0.f};
    dkv_f32x4 cb = mfma_pv<DKV_BF16>(dkv_u32x2{a0b, a1b}, dkv_u32x2{b0b, b1b}, c0);
    dkv_f32x4 ch = mfma_pv<DKV_F16>(dkv_u32x2{a0h, a1h}, dkv_u32x2{b0h, b1h}, c0);
    for (int u = 0; u < 4; ++u) {
      float ref = 0.f;
      for (int k = 0; k < 16; ++k) ref += Aval(4 * g + u, k) * Bval(k, n);
      bad += (cb[u] != ref) + (ch[u] != ref);
    }
  }
  // unaligned 16-byte and 2-byte buffer gathers, with out-of-range offsets reading zero
  {
    for (int i = l; i < 512; i += 64) buf[i] = (uint16_t)(i * 7 + 1);
    __syncthreads();
    // global copy for buffer loads lives right after the mismatch counter
    uint16_t* gbuf = reinterpret_cast<uint16_t*>(mismatches + 64);
    for (int i = l; i < 512; i += 64) gbuf[i] = buf[i];
    __threadfence();
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rs = dkv_make_rsrc(gbuf, 512 * 2);
    const int e0 = 3 + 5 * l;  // odd and even element offsets
    dkv_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, e0 * 2, 0, 0);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    for (int t = 0; t < 8; ++t) {
      const uint16_t got = (uint16_t)(w[t >> 1] >> (16 * (t & 1)));
      const int idx = e0 + t;
      const uint16_t want = idx < 512 ? buf[idx] : 0;
      bad += got != want;
    }
    const uint16_t h = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (e0 + 1) * 2, 0, 0);
    bad += h != (e0 + 1 < 512 ? buf[e0 + 1] : 0);
    const uint16_t z = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, 0x7ffffff0, 0, 0);
    bad += z != 0;
    dkv_u32x4 zz = __builtin_amdgcn_raw_buffer_load_b128(rs, 0x7ffffff0, 0, 0);
    bad += (zz.x | zz.y | zz.z | zz.w) != 0;
  }
  atomicAdd(mismatches, bad);
}

}  // namespace

static int splitk_tiles_bases(int S) { return (S + TILE - 1) / TILE; }

extern "C" int dkv_splitk_choose_split(int B, int Hkv, int S) {
  if (B <= 0 || Hkv <= 0 || S <= 0) return 64;
  const long long units = (long long)B * Hkv;
  const long long target_groups = 2048;  // 256 CUs x 8
  long long sl = ((long long)S * units + target_groups - 1) / target_groups;
  sl = ((sl + 63) / 64) * 64;
  if (sl < 64) sl = 64;
  // at most 63 splits per unit (merge kernel staging)
  const long long min_sl = (((long long)S + 62) / 63 + 63) / 64 * 64;
  if (sl < min_sl) sl = min_sl;
  return (int)sl;
}

extern "C" long long dkv_splitk_workspace_floats(int B, int Hq, int Hkv, int S, int R,
                                                 int split_len) {
  (void)R;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0) return 0;
  if (split_len <= 0) split_len = dkv_splitk_choose_split(B, Hkv, S);
  const long long n_splits = (S + split_len - 1) / split_len;
  const long long hpg = Hq / Hkv;
  const long long rope = (long long)(splitk_tiles_bases(S) + TILE + 1) * 128;
  const long long parts = (long long)B * Hkv * n_splits * hpg * PREC;
  return ((rope + 63) / 64) * 64 + parts;
}

namespace {

struct SplitLaunch {
  SplitParams p;
  int route, dtype, out_dtype, n_tb;
  long long units;
  const void* v_basis;
  long long v_unit, v_sr;
  void* out;
  long long out_sb, out_sh;
  float log_theta;
};

int splitk_prepare(SplitLaunch& L, int route, int dtype, const void* q, long long q_sb,
                   long long q_sh, const void* k_basis, long long k_unit_stride,
                   long long k_basis_sr, const void* v_basis, long long v_unit_stride,
                   long long v_basis_sr, const void* k_flat, long long k_ld, const void* v_flat,
                   long long v_ld, const int* lens_k, const int* offs_k, long long tk_sb,
                   long long tk_ss, const int* lens_v, const int* offs_v, long long tv_sb,
                   long long tv_ss, float* partials, long long partials_floats, void* out,
                   long long out_sb, long long out_sh, int out_dtype, int B, int Hq, int Hkv,
                   int G, int S, int R, int Dh, float log_theta, int split_len) {
  if (route != DKV_ROUTE_FUSED && route != DKV_ROUTE_TWO_STAGE) return DKV_E_ARG;
  if (out_dtype != dtype && out_dtype != DKV_F32) return DKV_E_ARG;
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || G <= 0 || S < 0 || R <= 0) return DKV_E_ARG;
  if (Hq % Hkv != 0 || Hkv % G != 0) return DKV_E_ARG;
  if (Dh != DH || R > DH || Hq / Hkv > 16) return DKV_E_UNSUPPORTED;
  if (S == 0) return DKV_E_UNSUPPORTED;  // empty cache: the generic path defines the result
  if (!q || !k_basis || !v_basis || !k_flat || !v_flat || !lens_k || !offs_k || !lens_v ||
      !offs_v || !partials || !out)
    return DKV_E_ARG;
  // 16-byte aligned basis rows for the vector LDS staging
  if (((uintptr_t)k_basis & 15) || (k_basis_sr & 7) || (k_unit_stride & 7))
    return DKV_E_UNSUPPORTED;
  if (k_ld * 2 > 0x7fffffffLL || v_ld * 2 > 0x7fffffffLL) return DKV_E_UNSUPPORTED;
  if (split_len <= 0) split_len = dkv_splitk_choose_split(B, Hkv, S);
  if (split_len % 64 != 0) return DKV_E_ARG;
  const int n_splits = (S + split_len - 1) / split_len;
  if (n_splits > 63) return DKV_E_ARG;
  const long long need = dkv_splitk_workspace_floats(B, Hq, Hkv, S, R, split_len);
  if (partials_floats < need) return DKV_E_WORKSPACE;
  L.units = (long long)B * Hkv;
  if (L.units * n_splits > 0x7fffffffLL) return DKV_E_UNSUPPORTED;
  L.n_tb = splitk_tiles_bases(S);
  const long long rope_floats = ((long long)(L.n_tb + TILE + 1) * 128 + 63) / 64 * 64;
  SplitParams& p = L.p;
  p.q = (const uint16_t*)q;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.k_basis = (const uint16_t*)k_basis;
  p.k_unit = k_unit_stride;
  p.k_sr = k_basis_sr;
  p.k_flat = (const uint16_t*)k_flat;
  p.v_flat = (const uint16_t*)v_flat;
  p.k_ld = k_ld;
  p.v_ld = v_ld;
  p.lens_k = lens_k;
  p.offs_k = offs_k;
  p.tk_sb = tk_sb;
  p.tk_ss = tk_ss;
  p.lens_v = lens_v;
  p.offs_v = offs_v;
  p.tv_sb = tv_sb;
  p.tv_ss = tv_ss;
  p.rope = partials;
  p.partials = partials + rope_floats;
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.G = G;
  p.S = S;
  p.R = R;
  p.hpg = Hq / Hkv;
  p.n_splits = n_splits;
  p.split_len = split_len;
  p.n_tb = L.n_tb;
  const float sm_scale = 1.0f / sqrtf((float)Dh);
  p.q_scale = route == DKV_ROUTE_FUSED ? sm_scale * LOG2E : sm_scale;
  p.masked_score = -1.0e4f * sm_scale;
  L.route = route;
  L.dtype = dtype;
  L.out_dtype = out_dtype;
  L.v_basis = v_basis;
  L.v_unit = v_unit_stride;
  L.v_sr = v_basis_sr;
  L.out = out;
  L.out_sb = out_sb;
  L.out_sh = out_sh;
  L.log_theta = log_theta;
  return DKV_OK;
}

int launch_rope(const SplitLaunch& L, hipStream_t st) {
  const int total = (L.n_tb + TILE + 1) * 64;
  hipLaunchKernelGGL(rope_table_kernel, dim3((total + 255) / 256), dim3(256), 0, st,
                     const_cast<float*>(L.p.rope), L.n_tb, L.log_theta);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

int launch_split(const SplitLaunch& L, hipStream_t st) {
  const dim3 grid((unsigned)(L.units * L.p.n_splits)), block(256);
  if (L.dtype == DKV_BF16) {
    if (L.route == DKV_ROUTE_FUSED)
      hipLaunchKernelGGL((splitk_kernel<DKV_BF16, DKV_ROUTE_FUSED>), grid, block, 0, st, L.p);
    else
      hipLaunchKernelGGL((splitk_kernel<DKV_BF16, DKV_ROUTE_TWO_STAGE>), grid, block, 0, st, L.p);
  } else {
    if (L.route == DKV_ROUTE_FUSED)
      hipLaunchKernelGGL((splitk_kernel<DKV_F16, DKV_ROUTE_FUSED>), grid, block, 0, st, L.p);
    else
      hipLaunchKernelGGL((splitk_kernel<DKV_F16, DKV_ROUTE_TWO_STAGE>), grid, block, 0, st, L.p);
  }
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

template <int DT, int RT>
void launch_merge_t(const SplitLaunch& L, hipStream_t st) {
  const dim3 mgrid((unsigned)L.units), block(256);
  if (L.out_dtype == DKV_F32)
    hipLaunchKernelGGL((merge_kernel<DT, RT, DKV_F32>), mgrid, block, 0, st, L.p.partials,
                       (const uint16_t*)L.v_basis, L.v_unit, L.v_sr, L.out, L.out_sb, L.out_sh,
                       L.p.Hkv, L.p.hpg, L.p.n_splits, L.p.R);
  else
    hipLaunchKernelGGL((merge_kernel<DT, RT, DT>), mgrid, block, 0, st, L.p.partials,
                       (const uint16_t*)L.v_basis, L.v_unit, L.v_sr, L.out, L.out_sb, L.out_sh,
                       L.p.Hkv, L.p.hpg, L.p.n_splits, L.p.R);
}

int launch_merge(const SplitLaunch& L, hipStream_t st) {
  if (L.dtype == DKV_BF16) {
    if (L.route == DKV_ROUTE_FUSED) launch_merge_t<DKV_BF16, DKV_ROUTE_FUSED>(L, st);
    else launch_merge_t<DKV_BF16, DKV_ROUTE_TWO_STAGE>(L, st);
  } else {
    if (L.route == DKV_ROUTE_FUSED) launch_merge_t<DKV_F16, DKV_ROUTE_FUSED>(L, st);
    else launch_merge_t<DKV_F16, DKV_ROUTE_TWO_STAGE>(L, st);
  }
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

}  // namespace

#define DKV_SPLITK_ARGS                                                                         \
  void *stream, int route, int dtype, const void *q, long long q_sb, long long q_sh,            \
      const void *k_basis, long long k_unit_stride, long long k_basis_sr, const void *v_basis,  \
      long long v_unit_stride, long long v_basis_sr, const void *k_flat, long long k_ld,        \
      const void *v_flat, long long v_ld, const int *lens_k, const int *offs_k, long long tk_sb, \
      long long tk_ss, const int *lens_v, const int *offs_v, long long tv_sb, long long tv_ss,  \
      float *partials, long long partials_floats, void *out, long long out_sb, long long out_sh, \
      int out_dtype, int B, int Hq, int Hkv, int G, int S, int R, int Dh, float log_theta,       \
      int split_len
#define DKV_SPLITK_FWD                                                                          \
  route, dtype, q, q_sb, q_sh, k_basis, k_unit_stride, k_basis_sr, v_basis, v_unit_stride,      \
      v_basis_sr, k_flat, k_ld, v_flat, v_ld, lens_k, offs_k, tk_sb, tk_ss, lens_v, offs_v,     \
      tv_sb, tv_ss, partials, partials_floats, out, out_sb, out_sh, out_dtype, B, Hq, Hkv, G, S,  \
      R, Dh, log_theta, split_len

extern "C" int dkv_decode_splitk(DKV_SPLITK_ARGS) {
  if (B == 0) return DKV_OK;
  SplitLaunch L;
  int rc = splitk_prepare(L, DKV_SPLITK_FWD);
  if (rc != DKV_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = launch_rope(L, st)) != DKV_OK) return rc;
  if ((rc = launch_split(L, st)) != DKV_OK) return rc;
  return launch_merge(L, st);
}

extern "C" int dkv_decode_splitk_phase(int phase, DKV_SPLITK_ARGS) {
  if (B == 0) return DKV_OK;
  SplitLaunch L;
  int rc = splitk_prepare(L, DKV_SPLITK_FWD);
  if (rc != DKV_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  switch (phase) {
    case 0: return launch_rope(L, st);
    case 1: return launch_split(L, st);
    case 2: return launch_merge(L, st);
    default: return DKV_E_ARG;
  }
}

extern "C" int dkv_selftest_layouts(void* stream, int* mismatches) {
  if (!mismatches) return DKV_E_ARG;
  // mismatches must point at >= 64 ints + 1 KiB of scratch (see selftest_kernel)
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, mismatches);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
