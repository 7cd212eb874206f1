// Split-K compressed decode attention for gfx950 (MFMA), the fast path behind both router
// routes (reference src/dynakv/kernels/fused.py:28-170, two_stage.py:48-324, router.py:20-59).
//
// Work unit: (batch b, KV head k) with hpg query heads sharing K/V basis k; its packed
// coefficients are cache row b*G + k/(Hkv/G). A workgroup (4 waves) owns one unit and one
// contiguous token range ("split", <= 512 tokens); waves take 16-token tiles round-robin.
//
// Workgroup prologue: the K basis (transposed, [dim][rank]) and the split's length/offset
// tables go to LDS, together with each tile's largest retained count, so a tile's gathers need
// no dependent global round trip. Each wave then runs a two-stage software pipeline: the
// current tile's gathered K and V coefficients are zero-masked past each token's count and
// stored to the wave's LDS tiles, then the next tile's gathers (16-byte buffer loads, one lane =
// one token x 8 ranks, out-of-range reads return zero) are issued and stay in flight while the
// current tile computes from LDS:
//   1. K^T[128 x 16] = BK^T . X^T on v_mfma_f32_16x16x32_{bf16,f16}, two 16-dim blocks at a
//      time ((i, i+64) rotate-half pairs), rank chunks of 32 up to the tile's largest count;
//   2. RoPE by cache row index on the accumulators (cos/sin advanced by angle addition from a
//      precomputed table), K' split into fp16 hi/lo parts;
//   3. scores on 16x16x32 f16 MFMA (K'hi.q + K'lo.q; a bf16 or fp16 query is exact in fp16,
//      the softmax scale is applied to the fp32 result);
//   4. online softmax in the log2 domain, lazily rescaled (only when the running max grows by
//      more than 2^11.5);
//   5. P.X^V in coefficient space on 16x16x16 MFMA; X^V goes through a per-wave LDS tile so
//      the operand (4 tokens x 1 rank per lane) is read transposed.
// Epilogue: the 4 waves combine through LDS into one (m, l, acc[128]) record per head.
// merge_kernel (same stream, one workgroup per unit and head) LSE-merges the split records and
// projects once through the V basis; stream order makes the records visible to it without
// device-scope fences (an agent-scope acquire would invalidate the XCD's L2).
#include "dkv_common.h"

namespace {

constexpr int DH = 128;
constexpr int TILE = 16;
constexpr int WAVES = 4;
constexpr int BK_LD = 136;    // LDS row pitch (elements) of the transposed K basis
constexpr int VT_LD = 136;    // LDS row pitch (elements) of a wave's V tile
constexpr int PREC = DH + 2;  // floats per partial record: m, l, acc[128]
constexpr int MAX_SPLIT = 512;
constexpr int MAX_TILES = MAX_SPLIT / TILE;
constexpr int ROPE_FIXED_ROWS = TILE + 1;  // rows 0..15: in-tile deltas; row 16: per-step
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_THRESH = 11.5f;  // log2 units
constexpr int OOB = 0x7ffffff0;          // buffer offset that reads as zero

struct SplitParams {
  const uint16_t* q;
  long long q_sb, q_sh;
  const uint16_t* k_basis;
  long long k_unit, k_sr;
  const uint16_t* v_basis;
  long long v_unit, v_sr;
  const uint16_t* k_flat;
  const uint16_t* v_flat;
  int k_ld, v_ld;
  uint32_t k_end, v_end;  // elements covered by the buffer resources: rows * ld
  const int* lens_k;
  const int* offs_k;
  long long tk_sb, tk_ss;
  const int* lens_v;
  const int* offs_v;
  long long tv_sb, tv_ss;
  const float* rope;   // rows of 64 (cos, sin): 16 in-tile deltas, 1 step, then tile bases
  float* partials;     // [unit][split][hpg][PREC]
  void* out;
  long long out_sb, out_sh;
  int B, Hq, Hkv, G, S, R, hpg, n_splits, split_len;
  float score_scale;   // applied to q.k' after the MFMA (fused: sm_scale*log2e, else sm_scale)
  float masked_score;  // two-stage route: -1e4 * (1/sqrt(Dh)) in fp32
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

// Element-wise gather of the first nv (1..8) 16-bit values at element offset e, the rest zero:
// eight unconditional 2-byte loads, those past nv aimed at the out-of-range offset.
__device__ __forceinline__ dkv_u32x4 gather8_b16(__amdgpu_buffer_rsrc_t r, int e, int nv) {
  uint32_t v[8];
#pragma unroll
  for (int t = 0; t < 8; ++t)
    v[t] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, t < nv ? (e + t) * 2 : 0x7ffffff0, 0, 0);
  return dkv_u32x4{v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16),
                   v[6] | (v[7] << 16)};
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

// Zero-fill masks for the first k (0..8) 16-bit elements of an 8-element vector.
__device__ __forceinline__ uint32_t prefix_mask_word(int k, int d) {
  return k >= 2 * d + 2 ? 0xffffffffu : (k == 2 * d + 1 ? 0x0000ffffu : 0u);
}

// 16-byte gather of ranks [32c + 8g, +8) of one token at element offset o (from the start of
// the buffer resource) with clamped count r; lanes with nothing to load read the out-of-range
// offset (zero, no memory traffic). A window that would cross the end of the resource (only
// the last token of the buffer's last row can) falls back to element loads, because an
// out-of-range vector access reads as zero in full.
__device__ __forceinline__ dkv_u32x4 gather_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t end, int o,
                                                  int r, int c, int g) {
  const int j0 = 32 * c + 8 * g;
  const int nv = r - j0;
  if (nv > 0 && (uint32_t)(o + j0 + 8) > end) return gather8_b16(rs, o + j0, min(nv, 8));
  return __builtin_amdgcn_raw_buffer_load_b128(rs, nv > 0 ? (o + j0) * 2 : OOB, 0, 0);
}

struct TileMeta {
  int rk;   // this lane's token: raw K length (only its sign matters: has a key)
  int rkc;  // clamped K length
  int rvc;  // clamped V length
  int nck;  // wave-uniform: 32-rank K chunks
  int nvc;  // wave-uniform: 32-rank V chunks
  int nbv;  // wave-uniform: 16-rank V blocks
  bool valid;
};

template <int DT, int ROUTE>
__global__ __launch_bounds__(256, 2) void splitk_kernel(SplitParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sBK[DH * BK_LD];
  __shared__ __attribute__((aligned(16))) int sTab[4][MAX_SPLIT];
  __shared__ int sTmax[2][MAX_TILES];
  __shared__ __attribute__((aligned(16))) uint16_t sKT[WAVES][TILE * VT_LD];
  __shared__ __attribute__((aligned(16))) uint16_t sVT[WAVES][TILE * VT_LD];
  __shared__ __attribute__((aligned(16))) uint32_t sMask[9][4];
  __shared__ __attribute__((aligned(16))) float sStep[2][64];

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
  const int s_begin = split * p.split_len;
  const int s_end = min(p.S, s_begin + p.split_len);
  const int ns = s_end - s_begin;

  // ---- prologue: K basis, tables, masks, per-step rotation --------------------------------
  {
    // transpose to [dim][rank]: consecutive lanes take consecutive ranks, so each 2-byte LDS
    // store of a wave covers 128 contiguous bytes (no bank conflicts)
    const uint16_t* kb = p.k_basis + (long long)kvh * p.k_unit;
    const int j = tid & 127;
    dkv_u32x4 v[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int d8 = ((tid >> 7) + 2 * it) * 8;
      v[it] = dkv_u32x4{0u, 0u, 0u, 0u};
      if (j < R) v[it] = *(const dkv_u32x4*)(kb + (long long)j * p.k_sr + d8);
    }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int d8 = ((tid >> 7) + 2 * it) * 8;
      const uint32_t e[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        sBK[(d8 + 2 * t) * BK_LD + j] = (uint16_t)(e[t] & 0xffffu);
        sBK[(d8 + 2 * t + 1) * BK_LD + j] = (uint16_t)(e[t] >> 16);
      }
    }
    const int* lk = p.lens_k + (long long)row * p.tk_sb;
    const int* okp = p.offs_k + (long long)row * p.tk_sb;
    const int* lv = p.lens_v + (long long)row * p.tv_sb;
    const int* ovp = p.offs_v + (long long)row * p.tv_sb;
    for (int i = tid; i < ns; i += 256) {
      const long long t = s_begin + i;
      sTab[0][i] = lk[t * p.tk_ss];
      sTab[1][i] = okp[t * p.tk_ss];
      sTab[2][i] = lv[t * p.tv_ss];
      sTab[3][i] = ovp[t * p.tv_ss];
    }
    if (tid < 36) sMask[tid >> 2][tid & 3] = prefix_mask_word(tid >> 2, tid & 3);
    if (tid < 64) {
      sStep[0][tid] = p.rope[TILE * 128 + 2 * tid];
      sStep[1][tid] = p.rope[TILE * 128 + 2 * tid + 1];
    }
  }
  __syncthreads();
  {  // largest clamped K and V count of each tile of the split (4 threads per tile)
    const int tile = tid >> 2, qq = tid & 3;
    int mk = 0, mv = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = tile * TILE + qq * 4 + e;
      if (tile < MAX_TILES && i < ns) {
        mk = max(mk, min(max(sTab[0][i], 0), R));
        mv = max(mv, min(max(sTab[2][i], 0), R));
      }
    }
    mk = max(mk, __shfl_xor(mk, 1, 64));
    mk = max(mk, __shfl_xor(mk, 2, 64));
    mv = max(mv, __shfl_xor(mv, 1, 64));
    mv = max(mv, __shfl_xor(mv, 2, 64));
    if (qq == 0 && tile < MAX_TILES) {
      sTmax[0][tile] = mk;
      sTmax[1][tile] = mv;
    }
  }

  // ---- query as the fp16 B operand of the QK MFMA: lane (head slot n, k-group g) holds
  //      (q_i, q_{i+64}) for i = 16*pp + 4*g + w; bf16 and fp16 values are exact in fp16 ------
  dkv_u32x4 bq[4];
  {
    const bool real = n < p.hpg;
    const long long qo = (long long)b * p.q_sb + (long long)(kvh * p.hpg + min(n, p.hpg - 1)) * p.q_sh;
    uint32_t qa[16], qb[16];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int i = 16 * pp + 4 * g + w;
        qa[pp * 4 + w] = p.q[qo + i];
        qb[pp * 4 + w] = p.q[qo + i + 64];
      }
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      uint32_t w4[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float a = real ? elt_to_f32<DT>(qa[pp * 4 + w]) : 0.f;
        const float c = real ? elt_to_f32<DT>(qb[pp * 4 + w]) : 0.f;
        w4[w] = pack_f16x2(a, c);
      }
      bq[pp] = dkv_u32x4{w4[0], w4[1], w4[2], w4[3]};
    }
  }

  const int tile_first = s_begin / TILE;  // splits are multiples of 64 tokens
  const int tile0 = tile_first + wave;
  const int n_tb = (p.S + TILE - 1) / TILE;

  // ---- RoPE state of this lane's token slot for its 16 frequencies -----------------------
  float rc[16], rs[16];
  {
    const int tb = min(tile0, n_tb - 1);
    const float* base = p.rope + (long long)(ROPE_FIXED_ROWS + tb) * 128;
    const float* delt = p.rope + (long long)n * 128;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int i = 16 * pp + 4 * g + w, f = pp * 4 + w;
        const float bc = base[2 * i], bs = base[2 * i + 1];
        const float ec = delt[2 * i], es = delt[2 * i + 1];
        rc[f] = bc * ec - bs * es;
        rs[f] = bs * ec + bc * es;
      }
  }
  __syncthreads();  // sTmax ready

  // one resource per buffer, ranges [flat, flat + rows * ld); row offsets go in the voffset
  const __amdgpu_buffer_rsrc_t rk_src = dkv_make_rsrc(p.k_flat, p.k_end * 2u);
  const __amdgpu_buffer_rsrc_t rv_src = dkv_make_rsrc(p.v_flat, p.v_end * 2u);
  const int k_row0 = row * p.k_ld, v_row0 = row * p.v_ld;
  uint16_t* kt = sKT[wave];
  uint16_t* vt = sVT[wave];

  // per-tile metadata from the LDS tables
  auto meta_of = [&](int T) {
    TileMeta d;
    const int tl = T * TILE + n - s_begin;
    d.valid = T * TILE + n < s_end;
    d.rk = d.valid ? sTab[0][tl] : 0;
    const int rv = d.valid ? sTab[2][tl] : 0;
    d.rkc = min(max(d.rk, 0), R);
    d.rvc = min(max(rv, 0), R);
    const int tt = T - tile_first;
    const int mk = __builtin_amdgcn_readfirstlane(sTmax[0][tt]);
    const int mv = __builtin_amdgcn_readfirstlane(sTmax[1][tt]);
    d.nck = (mk + 31) >> 5;
    d.nvc = (mv + 31) >> 5;
    d.nbv = (mv + 15) >> 4;
    return d;
  };
  dkv_u32x4 kx[4], vx[4];  // in-flight gathers of the next tile
  auto issue = [&](const TileMeta& d, int T) {
    const int tl = T * TILE + n - s_begin;
    const int ok = k_row0 + (d.valid ? sTab[1][tl] : 0);
    const int ov = v_row0 + (d.valid ? sTab[3][tl] : 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      kx[c] = dkv_u32x4{0u, 0u, 0u, 0u};
      if (c < d.nck) kx[c] = gather_chunk(rk_src, p.k_end, ok, d.rkc, c, g);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      vx[c] = dkv_u32x4{0u, 0u, 0u, 0u};
      if (c < d.nvc) vx[c] = gather_chunk(rv_src, p.v_end, ov, d.rvc, c, g);
    }
  };

  dkv_f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // per head slot n (log2 units), identical across g
  float l_run = 0.f;        // partial over this lane's 4 tokens per tile

  TileMeta cur;
  if (tile0 * TILE < s_end) {
    cur = meta_of(tile0);
    issue(cur, tile0);
  }
  for (int T = tile0; T * TILE < s_end; T += WAVES) {
    // chunk counts are wave-uniform: keep them in scalar registers
    cur.nck = __builtin_amdgcn_readfirstlane(cur.nck);
    cur.nvc = __builtin_amdgcn_readfirstlane(cur.nvc);
    cur.nbv = __builtin_amdgcn_readfirstlane(cur.nbv);
    // ---- store the current tile (masked) to the wave's LDS tiles, then issue the next ------
    // all four chunks are stored (chunks past the tile's count hold zeros), so the compute
    // below is straight-line code
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int nvk = min(max(cur.rkc - 32 * c - 8 * g, 0), 8);
      const dkv_u32x4 mk = *(const dkv_u32x4*)sMask[nvk];
      *(dkv_u32x4*)&kt[n * VT_LD + 32 * c + 8 * g] =
          dkv_u32x4{kx[c].x & mk.x, kx[c].y & mk.y, kx[c].z & mk.z, kx[c].w & mk.w};
      const int nvv = min(max(cur.rvc - 32 * c - 8 * g, 0), 8);
      const dkv_u32x4 mv = *(const dkv_u32x4*)sMask[nvv];
      *(dkv_u32x4*)&vt[n * VT_LD + 32 * c + 8 * g] =
          dkv_u32x4{vx[c].x & mv.x, vx[c].y & mv.y, vx[c].z & mv.z, vx[c].w & mv.w};
    }
    const bool more = (T + WAVES) * TILE < s_end;
    TileMeta nxt = cur;
    if (more) {
      nxt = meta_of(T + WAVES);
      issue(nxt, T + WAVES);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- 1-3: K reconstruction, RoPE, hi/lo split, scores ---------------------------------
    dkv_f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      dkv_f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const dkv_u32x4 xk = *(const dkv_u32x4*)&kt[n * VT_LD + 32 * c + 8 * g];
        const dkv_u32x4 a0 = *(const dkv_u32x4*)&sBK[(16 * pp + n) * BK_LD + 32 * c + 8 * g];
        const dkv_u32x4 a1 = *(const dkv_u32x4*)&sBK[(16 * (pp + 4) + n) * BK_LD + 32 * c + 8 * g];
        c0 = mfma_k<DT>(a0, xk, c0);
        c1 = mfma_k<DT>(a1, xk, c1);
      }
      uint32_t h4[4], l4[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int f = pp * 4 + w;
        const float r0 = c0[w] * rc[f] - c1[w] * rs[f];
        const float r1 = c1[w] * rc[f] + c0[w] * rs[f];
        split_f16x2(r0, r1, h4[w], l4[w]);
      }
      sc = mfma_f16(dkv_u32x4{l4[0], l4[1], l4[2], l4[3]}, bq[pp], sc);
      sc = mfma_f16(dkv_u32x4{h4[0], h4[1], h4[2], h4[3]}, bq[pp], sc);
    }
    // advance the rotation by WAVES*TILE positions
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const dkv_f32x4 dc = *(const dkv_f32x4*)&sStep[0][16 * pp + 4 * g];
      const dkv_f32x4 ds = *(const dkv_f32x4*)&sStep[1][16 * pp + 4 * g];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int f = pp * 4 + w;
        const float c2 = rc[f] * dc[w] - rs[f] * ds[w];
        const float s2 = rs[f] * dc[w] + rc[f] * ds[w];
        rc[f] = c2;
        rs[f] = s2;
      }
    }

    // scores of lane (head slot n, tokens 4g+u) -> log2 domain with the route's masking
    const unsigned long long has_bits = __ballot(cur.valid && cur.rk > 0);
    const unsigned long long in_bits = __ballot(cur.valid);
    float z[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tok = 4 * g + u;
      const bool has = (has_bits >> tok) & 1ull;
      const bool inr = (in_bits >> tok) & 1ull;
      float v;
      if constexpr (ROUTE == DKV_ROUTE_FUSED) {
        v = has ? sc[u] * p.score_scale : -INFINITY;  // score_scale = sm_scale * log2(e)
      } else {
        v = dkv_round_to<DT>(has ? sc[u] * p.score_scale : p.masked_score) * LOG2E;
      }
      z[u] = inr ? v : -INFINITY;
    }

    // ---- 4. online softmax (per head slot) --------------------------------------------------
    float tmax = fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3]));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    if (__ballot(tmax > m_run + RESCALE_THRESH)) {
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

    // ---- 5. P.X^V from the wave's LDS V tile (4 tokens x 1 rank per lane) ---------------------
    dkv_u32x2 pa_hi, pa_lo;
    if constexpr (DT == DKV_F16) {
      pa_hi = dkv_u32x2{pack_f16x2(pu[0], pu[1]), pack_f16x2(pu[2], pu[3])};
      pa_lo = pa_hi;
    } else {
      const __bf16 h0 = (__bf16)pu[0], h1 = (__bf16)pu[1], h2 = (__bf16)pu[2], h3 = (__bf16)pu[3];
      const __bf16 e0 = (__bf16)(pu[0] - (float)h0), e1 = (__bf16)(pu[1] - (float)h1);
      const __bf16 e2 = (__bf16)(pu[2] - (float)h2), e3 = (__bf16)(pu[3] - (float)h3);
      pa_hi = dkv_u32x2{(uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16),
                        (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16)};
      pa_lo = dkv_u32x2{(uint32_t)__builtin_bit_cast(uint16_t, e0) | ((uint32_t)__builtin_bit_cast(uint16_t, e1) << 16),
                        (uint32_t)__builtin_bit_cast(uint16_t, e2) | ((uint32_t)__builtin_bit_cast(uint16_t, e3) << 16)};
    }
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const uint16_t* src = vt + (4 * g) * VT_LD + 16 * blk + n;
      const uint32_t e0 = src[0], e1 = src[VT_LD], e2 = src[2 * VT_LD], e3 = src[3 * VT_LD];
      const dkv_u32x2 xb = {e0 | (e1 << 16), e2 | (e3 << 16)};
      acc[blk] = mfma_pv<DT>(pa_hi, xb, acc[blk]);
      if constexpr (DT == DKV_BF16) acc[blk] = mfma_pv<DT>(pa_lo, xb, acc[blk]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    cur = nxt;
  }

  // ---- combine the 4 waves through LDS and write the partial record ----------------------
  float l_tot = l_run;
  l_tot += __shfl_xor(l_tot, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  __syncthreads();  // all waves done with sBK and their tiles
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
  float* prec = p.partials + ((long long)unit * p.n_splits + split) * p.hpg * PREC;
  for (int idx = tid; idx < p.hpg * PREC; idx += 256) {
    const int hs = idx / PREC, e = idx % PREC;
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
    prec[hs * PREC + e] = e == 0 ? M : v;
  }

}

// One workgroup per (unit, head slot): LSE-merge the split records of that head, normalise with
// the route's denominator, project once through the unit's V basis, store in the output dtype.
template <int DT, int ROUTE, int ODT>
__global__ __launch_bounds__(256) void merge_kernel(SplitParams p) {
  __shared__ float sW[1024];  // split weights (n_splits <= 1024 handled in chunks)
  __shared__ float sA[DH];
  __shared__ float sO[2][DH];
  __shared__ float sRed[2][4];
  const int unit = blockIdx.x / p.hpg, hs = blockIdx.x % p.hpg;
  const int b = unit / p.Hkv, kvh = unit % p.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int R = p.R;
  const long long stride = (long long)p.hpg * PREC;  // between splits of one head
  const float* pr = p.partials + (long long)unit * p.n_splits * stride + (long long)hs * PREC;
  // M = max over splits
  float M = -INFINITY;
  for (int s = tid; s < p.n_splits; s += 256) M = fmaxf(M, pr[s * stride]);
  M = dkv_wave_max(M);
  if (lane == 0) sRed[0][wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(sRed[0][0], sRed[0][1]), fmaxf(sRed[0][2], sRed[0][3]));
  // weights and L
  float L = 0.f;
  for (int s = tid; s < p.n_splits; s += 256) {
    const float w = (M == -INFINITY) ? 0.f : exp2f(pr[s * stride] - M);
    if (s < 1024) sW[s] = w;
    L += w * pr[s * stride + 1];
  }
  L = dkv_wave_sum(L);
  if (lane == 0) sRed[1][wave] = L;
  __syncthreads();
  L = sRed[1][0] + sRed[1][1] + sRed[1][2] + sRed[1][3];
  const float den = ROUTE == DKV_ROUTE_TWO_STAGE ? fmaxf(L, 1e-6f) : L;
  // A[j] = sum_s w_s acc_s[j] / den; two halves of the splits per rank, summed through LDS
  {
    const int j = tid & 127, half = tid >> 7;
    float a = 0.f;
    if (j < R) {
      for (int s = half; s < p.n_splits; s += 2) {
        const float w = s < 1024 ? sW[s] : ((M == -INFINITY) ? 0.f : exp2f(pr[s * stride] - M));
        a += w * pr[s * stride + 2 + j];
      }
    }
    sO[half][j] = a;
    __syncthreads();
    if (half == 0) sA[j] = (sO[0][j] + sO[1][j]) / den;
    __syncthreads();
  }
  // out[d] = sum_j A[j] * V[j][d]: two halves of the ranks, summed through LDS
  {
    const int d = tid & 127, half = tid >> 7;
    const uint16_t* vb = p.v_basis + (long long)kvh * p.v_unit;
    float o = 0.f;
#pragma unroll 8
    for (int j = half; j < R; j += 2) o = fmaf(sA[j], elt_to_f32<DT>(vb[(long long)j * p.v_sr + d]), o);
    __syncthreads();
    sO[half][d] = o;
    __syncthreads();
    if (half == 0) {
      const long long oi = (long long)b * p.out_sb + (long long)(kvh * p.hpg + hs) * p.out_sh + d;
      dkv_store_f32<ODT>(p.out, oi, sO[0][d] + sO[1][d]);
    }
  }
}

// RoPE table rows (64 x (cos, sin) each): 0..15 in-tile deltas (angle = delta * inv_freq),
// 16 the per-step rotation (64 positions), 17 + T the base of tile T (angle = 16T * inv_freq).
// Angles are formed in fp32 as the reference does (angle = float(pos) * inv_freq, reference
// fused.py:65-66,97 / two_stage.py:36-44); cos/sin are evaluated in double and rounded.
__global__ __launch_bounds__(256) void rope_table_kernel(float* __restrict__ rope, int row_from,
                                                         int row_to, float log_theta) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int r = row_from + idx / 64, i = idx % 64;
  if (r >= row_to) return;
  const float inv = dkv_inv_freq(i, DH, log_theta);
  float ang;
  if (r < TILE)
    ang = (float)r * inv;
  else if (r == TILE)
    ang = (float)(TILE * WAVES) * inv;
  else
    ang = (float)((r - ROPE_FIXED_ROWS) * TILE) * inv;
  double s, c;
  sincos((double)ang, &s, &c);
  rope[(long long)r * 128 + 2 * i] = (float)c;
  rope[(long long)r * 128 + 2 * i + 1] = (float)s;
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

extern "C" int dkv_splitk_choose_split(int B, int Hkv, int S) {
  if (B <= 0 || Hkv <= 0 || S <= 0) return 64;
  const long long units = (long long)B * Hkv;
  const long long target_groups = 2048;  // 256 CUs x 8
  long long sl = ((long long)S * units + target_groups - 1) / target_groups;
  sl = ((sl + 63) / 64) * 64;
  if (sl < 64) sl = 64;
  if (sl > MAX_SPLIT) sl = MAX_SPLIT;
  return (int)sl;
}

extern "C" long long dkv_splitk_workspace_floats(int B, int Hq, int Hkv, int S, int R,
                                                 int split_len) {
  (void)R;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0) return 0;
  if (split_len <= 0) split_len = dkv_splitk_choose_split(B, Hkv, S);
  const long long n_splits = (S + split_len - 1) / split_len;
  const long long units = (long long)B * Hkv;
  return units * n_splits * (Hq / Hkv) * PREC;
}

extern "C" long long dkv_rope_table_floats(int n_tiles) {
  if (n_tiles < 0) return 0;
  return (long long)(ROPE_FIXED_ROWS + n_tiles) * 128;
}

extern "C" int dkv_rope_table(void* stream, float* rope, int from_tile, int to_tile,
                              float log_theta) {
  if (!rope || from_tile < 0 || to_tile < from_tile) return DKV_E_ARG;
  const int row_from = from_tile == 0 ? 0 : ROPE_FIXED_ROWS + from_tile;
  const int row_to = ROPE_FIXED_ROWS + to_tile;
  const long long total = (long long)(row_to - row_from) * 64;
  if (total == 0) return DKV_OK;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, rope, row_from, row_to, log_theta);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

template <int DT, int RT>
static void launch_splitk_t(const SplitParams& p, int out_dtype, dim3 grid, dim3 mgrid,
                            hipStream_t st) {
  hipLaunchKernelGGL((splitk_kernel<DT, RT>), grid, dim3(256), 0, st, p);
  if (out_dtype == DKV_F32)
    hipLaunchKernelGGL((merge_kernel<DT, RT, DKV_F32>), mgrid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((merge_kernel<DT, RT, DT>), mgrid, dim3(256), 0, st, p);
}

extern "C" int dkv_decode_splitk(void* stream, int route, int dtype, const void* q, long long q_sb,
                                 long long q_sh, const void* k_basis, long long k_unit_stride,
                                 long long k_basis_sr, const void* v_basis,
                                 long long v_unit_stride, long long v_basis_sr,
                                 const void* k_flat, long long k_ld, const void* v_flat,
                                 long long v_ld, const int* lens_k, const int* offs_k,
                                 long long tk_sb, long long tk_ss, const int* lens_v,
                                 const int* offs_v, long long tv_sb, long long tv_ss,
                                 const float* rope, int rope_tiles, float* workspace,
                                 long long workspace_floats, void* out, long long out_sb,
                                 long long out_sh, int out_dtype, int B, int Hq, int Hkv, int G,
                                 int S, int R, int Dh, int split_len) {
  if (route != DKV_ROUTE_FUSED && route != DKV_ROUTE_TWO_STAGE) return DKV_E_ARG;
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (out_dtype != dtype && out_dtype != DKV_F32) return DKV_E_ARG;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || G <= 0 || S < 0 || R <= 0) return DKV_E_ARG;
  if (Hq % Hkv != 0 || Hkv % G != 0) return DKV_E_ARG;
  if (Dh != DH || R > DH || Hq / Hkv > 16) return DKV_E_UNSUPPORTED;
  if (B == 0) return DKV_OK;
  if (S == 0) return DKV_E_UNSUPPORTED;  // empty cache: the vector path defines the result
  if (!q || !k_basis || !v_basis || !k_flat || !v_flat || !lens_k || !offs_k || !lens_v ||
      !offs_v || !rope || !workspace || !out)
    return DKV_E_ARG;
  // 16-byte aligned K basis rows for the vector LDS staging
  if (((uintptr_t)k_basis & 15) || (k_basis_sr & 7) || (k_unit_stride & 7))
    return DKV_E_UNSUPPORTED;
  if (k_ld <= 0 || v_ld <= 0) return DKV_E_ARG;
  // buffer offsets are 32-bit byte offsets from the first row
  const long long rows = (long long)B * G;
  if (rows * k_ld >= (1LL << 30) || rows * v_ld >= (1LL << 30)) return DKV_E_UNSUPPORTED;
  if (rope_tiles < (S + TILE - 1) / TILE) return DKV_E_ARG;
  if (split_len <= 0) split_len = dkv_splitk_choose_split(B, Hkv, S);
  if (split_len % 64 != 0 || split_len > MAX_SPLIT) return DKV_E_ARG;
  const long long n_splits = ((long long)S + split_len - 1) / split_len;
  const long long units = (long long)B * Hkv;
  if (units * n_splits > 0x7fffffffLL) return DKV_E_UNSUPPORTED;
  if (workspace_floats < dkv_splitk_workspace_floats(B, Hq, Hkv, S, R, split_len))
    return DKV_E_WORKSPACE;
  SplitParams p;
  p.q = (const uint16_t*)q;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.k_basis = (const uint16_t*)k_basis;
  p.k_unit = k_unit_stride;
  p.k_sr = k_basis_sr;
  p.v_basis = (const uint16_t*)v_basis;
  p.v_unit = v_unit_stride;
  p.v_sr = v_basis_sr;
  p.k_flat = (const uint16_t*)k_flat;
  p.v_flat = (const uint16_t*)v_flat;
  p.k_ld = (int)k_ld;
  p.v_ld = (int)v_ld;
  p.k_end = (uint32_t)(rows * k_ld);
  p.v_end = (uint32_t)(rows * v_ld);
  p.lens_k = lens_k;
  p.offs_k = offs_k;
  p.tk_sb = tk_sb;
  p.tk_ss = tk_ss;
  p.lens_v = lens_v;
  p.offs_v = offs_v;
  p.tv_sb = tv_sb;
  p.tv_ss = tv_ss;
  p.rope = rope;
  p.partials = workspace;
  p.out = out;
  p.out_sb = out_sb;
  p.out_sh = out_sh;
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.G = G;
  p.S = S;
  p.R = R;
  p.hpg = Hq / Hkv;
  p.n_splits = (int)n_splits;
  p.split_len = split_len;
  const float sm_scale = 1.0f / sqrtf((float)Dh);
  p.score_scale = route == DKV_ROUTE_FUSED ? sm_scale * LOG2E : sm_scale;
  p.masked_score = -1.0e4f * sm_scale;
  const dim3 grid((unsigned)(units * n_splits)), mgrid((unsigned)(units * (Hq / Hkv)));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DKV_BF16) {
    if (route == DKV_ROUTE_FUSED)
      launch_splitk_t<DKV_BF16, DKV_ROUTE_FUSED>(p, out_dtype, grid, mgrid, st);
    else
      launch_splitk_t<DKV_BF16, DKV_ROUTE_TWO_STAGE>(p, out_dtype, grid, mgrid, st);
  } else {
    if (route == DKV_ROUTE_FUSED)
      launch_splitk_t<DKV_F16, DKV_ROUTE_FUSED>(p, out_dtype, grid, mgrid, st);
    else
      launch_splitk_t<DKV_F16, DKV_ROUTE_TWO_STAGE>(p, out_dtype, grid, mgrid, st);
  }
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_selftest_layouts(void* stream, int* mismatches) {
  if (!mismatches) return DKV_E_ARG;
  // mismatches must point at >= 64 ints + 1 KiB of scratch (see selftest_kernel)
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, mismatches);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
