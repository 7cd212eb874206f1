// Split-K compressed decode attention for gfx950 (MFMA), the fast path behind both router
// routes (reference src/dynakv/kernels/fused.py:28-170, two_stage.py:48-324, router.py:20-59).
//
// Work unit: (batch b, KV head k) with hpg query heads sharing K/V basis k; its packed
// coefficients are cache row b*G + k/(Hkv/G). A workgroup (8 waves, one per CU) owns one unit
// and one contiguous token range ("split", a multiple of 64 tokens); waves take 16-token tiles
// round-robin, or, in splits of at least 16 tiles, pairs of consecutive tiles that share the
// per-tile query operand (the second tile's token slots rotated by R(16 + n)).
//
// Prologue: the K basis goes to registers (MFMA A operands; NREG_PP < 4 keeps part of it in
// LDS instead, [dim][rank], read per tile), the mask table and the table of every lane's fixed
// token-slot rotation R(n) to LDS; each lane keeps the query pairs of its frequency. Each wave then runs a software pipeline
// over its tiles: the length/offset tables of tile j+2 and the coefficient windows of tile j+1
// (direct-to-LDS buffer loads, one lane = one token x 8 ranks, empty pieces read from an
// out-of-range offset as zeros) are in flight while tile j computes:
//   1. the partial piece of each token is masked in place; the K windows go to registers;
//   2. the query rotated back by the tile's base position, R(-16T) q (RoPE by angle addition:
//      q . R(16T+n) k = (R(-16T) q) . (R(n) k)), split into bf16 hi/lo and staged through LDS
//      into the B operand of the score MFMA;
//   3. K^T[128 x 16] = BK^T . X^T on v_mfma_f32_16x16x32_{bf16,f16}, two 16-dim blocks at a
//      time ((i, i+64) rotate-half pairs), R(n) per lane in fp32, K' split into bf16 hi + lo,
//      scores on 16x16x32 bf16 MFMA (K'hi and K'lo products; hi and lo query columns added by
//      one DPP step);
//   4. online softmax in the log2 domain, lazily rescaled (only when the running max grows by
//      more than 2^11.5);
//   5. P.X^V in coefficient space on MFMA, the X^V operand read transposed from the windows.
// Epilogue: the 8 waves combine through LDS into one (m, l, acc[128]) record per head; the
// last split of a unit to arrive merges the unit's records by LSE and projects once through
// the V basis (merge_kernel does this instead when a call has more units than counters). A
// unit with a single split (caches up to 256 tokens) merges its waves in LDS and projects
// directly, with no record.
#include "dkv_common.h"

#include <mutex>
#include <type_traits>

namespace {

constexpr int DH = 128;
constexpr int TILE = 16;
constexpr int WAVES = 8;        // per workgroup: two per SIMD
constexpr int NTHREADS = WAVES * 64;
constexpr int BK_LD = 136;    // LDS row pitch (elements) of the transposed K basis
// K^T is formed as 4 pairs pp of 16-dim blocks (pp, pp + 4); the basis rows of the first
// NREG_PP pairs stay in registers, the others are read from LDS per tile
constexpr int NREG_PP = 4;
constexpr int SBH_ROWS = 32 * (4 - NREG_PP);
constexpr int VT_LD = 136;    // LDS row pitch (elements) of a wave's V tile
constexpr int PREC = DH + 2;  // floats per partial record: m, l, acc[128]
constexpr int NSLOT = 2;        // gather slots per wave: the current tile + one in flight
constexpr int TSLOT = 4;        // table slots per wave (tables run a tile ahead of gathers)
constexpr int GSLOT_BYTES = 8192;  // 4 K chunks + 4 V chunks of 64 lanes x 16 bytes
constexpr int QROW_BYTES = 256;    // one row of the per-tile query operand (64 dwords)
constexpr int MERGE_COUNTERS = 16384;  // leading workspace ints: per-unit arrival counters
constexpr int VB_CHUNKS = DH * DH / 8 / NTHREADS;  // 16-byte V-basis pieces per thread
constexpr int MASK_BIAS = 24;  // mask-table row of dk = 0 (dk: a lane's elements, -24 .. 128)
constexpr int MASK_ROWS = MASK_BIAS + DH + 1;
constexpr int ROPE_FIXED_ROWS = TILE + 1;  // rows 0..15: in-tile deltas; row 16: per-step
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_THRESH = 11.5f;  // log2 units
constexpr int OOB = 0x7ffffff0;          // buffer offset that reads as zero
// elements a flat-buffer resource covers at most (its byte size stays below OOB), and the
// largest row stride the kernel accepts (a row's last 16-byte window stays inside that range)
constexpr int FLAT_ELEM_CAP = DKV_FLAT_RSRC_CAP;
constexpr int FLAT_LD_MAX = FLAT_ELEM_CAP - 8;
constexpr int DPP_ROW_SHL8 = 0x108;      // DPP row_shl:8: lane i of a 16-lane row reads lane i+8

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
  int rows;               // cache rows of the flat buffers (B * G)
  const int* lens_k;
  const int* offs_k;
  long long tk_sb, tk_ss;
  const int* lens_v;
  const int* offs_v;
  long long tv_sb, tv_ss;
  const float* rope;   // rows of 64 (cos, sin): 16 in-tile deltas, 1 step, then tile bases
  float* partials;     // [unit][split][hpg][PREC]
  int* counters;       // [unit] arrival counts of the fused merge (zero between calls)
  int fused_merge;     // 1: the last split of a unit merges; 0: merge_kernel follows
  int out_f32;         // output dtype: 1 fp32, 0 the cache dtype
  void* out;
  long long out_sb, out_sh;
  int B, Hq, Hkv, G, S, R, hpg, n_splits, split_len;
  float score_scale;   // applied to q.k' after the MFMA (fused: sm_scale*log2e, else sm_scale)
  float masked_score;  // two-stage route: -1e4 * (1/sqrt(Dh)) in fp32
  float minus_one;     // -1.0f (see split_f16x2)
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

// x ~= hi + lo with hi = fp16(x) and lo = fp16(x - hi), for two values packed per dword
// (x - hi is exact in fp32, so lo is that difference rounded once to fp16). minus_one is -1.0f
// passed at run time: as a literal the compiler folds fma(h, -1, x) into a subtraction and
// converts in several steps, while fma(h, m, x) maps to one mixed-precision fma per half.
__device__ __forceinline__ void split_f16x2(float x0, float x1, float minus_one, uint32_t& hi,
                                            uint32_t& lo) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  const dkv_f16x2 hv = __builtin_convertvector(f32x2{x0, x1}, dkv_f16x2);  // one packed convert
  const _Float16 l0 = (_Float16)__builtin_fmaf((float)hv[0], minus_one, x0);
  const _Float16 l1 = (_Float16)__builtin_fmaf((float)hv[1], minus_one, x1);
  hi = __builtin_bit_cast(uint32_t, hv);
  lo = __builtin_bit_cast(uint32_t, dkv_f16x2{l0, l1});
}

__device__ __forceinline__ dkv_f32x4 mfma_bf16(const dkv_u32x4& a, const dkv_u32x4& b,
                                               dkv_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dkv_bf16x8, a),
                                                 __builtin_bit_cast(dkv_bf16x8, b), c, 0, 0, 0);
}

// x ~= hi + lo in bf16 for two values packed per dword: hi = RNE(x), lo = RNE(x - hi). x - hi is
// exact in fp32 (a bf16 value as fp32 is its bits in the upper half of a dword), so the pair
// carries 16 significant bits over fp32's exponent range (no overflow where fp32 has none).
__device__ __forceinline__ void split_bf16x2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, dkv_bf16x2));
  const float l0 = x0 - __uint_as_float(h << 16);
  const float l1 = x1 - __uint_as_float(h & 0xffff0000u);
  hi = h;
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{l0, l1}, dkv_bf16x2));
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

// Loads that write LDS directly (M0 = wave-uniform LDS base; lane i's bytes land at
// M0 + size*i). They are issued as inline assembly so that the compiler neither reorders LDS
// accesses around them nor guards later LDS reads with a full drain of the load queue: the
// kernel waits for them itself (wait_vm) at the points where the data is consumed. No other
// code of the kernel uses M0.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base,
                                           uint32_t byte_off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(lds_base), "v"(byte_off), "s"(rsrc)
               : "memory", "m0");
}
// Chunk C of a lane's 8-rank pieces: the 16 bytes at byte offset off + 64*C, through the
// instruction offset. The hardware adds the instruction offset to the LDS address too, so M0
// is the chunk's LDS base minus 64*C. An out-of-range offset loads nothing and writes zeros.
template <int C>
__device__ __forceinline__ void lds_load16_chunk(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_chunk,
                                                 uint32_t off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen offset:%3 lds"
               ::"s"(lds_chunk - 64u * C), "v"(off), "s"(rsrc), "i"(64 * C)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_load4(const void* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               ::"s"(lds_base), "v"(gptr)
               : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// Float maxima without the NaN-quieting the compiler adds around fmaxf (the scores are never NaN
// for finite inputs; -inf is an ordinary operand here).
__device__ __forceinline__ float max2_f32(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// max(x, x of lane l ^ 32) and max(x, x of lane l ^ 16): a permlane swap of a value with
// itself leaves each lane its own value in one result and its partner's in the other.
__device__ __forceinline__ float lane_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return max2_f32(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float lane_max16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return max2_f32(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// An opaque definition of x: a value loaded before a loop and settled after the load is, to the
// compiler's wait insertion, produced here rather than by the load, so no wait for that load
// is placed inside the loop.
template <typename T>
__device__ __forceinline__ void settle(T& x) {
  asm volatile("" : "+v"(x));
}

// Wait until at most N vector-memory loads of this wave are outstanding (loads complete in
// issue order); the "memory" clobber keeps LDS accesses from moving across the wait.
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Split records are exchanged between the workgroups of a unit with relaxed agent-scope atomic
// accesses: such loads and stores are coherent across the XCDs' L2 caches by themselves, so
// publishing a record needs only the wait for its stores before the arrival is counted, and
// the last arrival reads the records without an L2 write-back or invalidation (the fences an
// acquire/release pair at agent scope would add for ordinary accesses).
__device__ __forceinline__ float rec_load(const float* a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void rec_store(float* a, float v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LSE-merge the split records of one unit, normalise with the route's denominator, project
// once through the unit's V basis and store the hpg output rows (all threads of the block).
// scratch: LDS for the basis ([128][DH] bf16/fp16, zero past rank R) and 16 * DH floats.
// The LSE merge of one unit's split records into sA[16][DH] (merged, normalised coefficients;
// head slots past hpg zero), MB splits per batch of loads.
template <int MB, int ROUTE>
__device__ __forceinline__ void merge_records(const SplitParams& p, const float* base,
                                              long long stride, float* sA) {
  for (int idx = threadIdx.x; idx < 16 * DH; idx += NTHREADS) {
    const int hs = idx / DH, r = idx % DH;
    float a = 0.f;
    if (hs < p.hpg) {
      float M = -INFINITY, L = 0.f, A = 0.f;
      for (int sp0 = 0; sp0 < p.n_splits; sp0 += MB) {
        float mb[MB], lb[MB], xb[MB];
#pragma unroll
        for (int u = 0; u < MB; ++u) {
          const int sp = min(sp0 + u, p.n_splits - 1);
          const float* rec = base + sp * stride + hs * PREC;
          mb[u] = rec_load(rec);
          lb[u] = rec_load(rec + 1);
          xb[u] = r < p.R ? rec_load(rec + 2 + r) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < MB; ++u) {
          if (sp0 + u >= p.n_splits) break;
          const float m = mb[u];
          const float Mn = fmaxf(M, m);
          const float so = M == -INFINITY ? 0.f : exp2f(M - Mn);
          const float sn = m == -INFINITY ? 0.f : exp2f(m - Mn);
          L = L * so + lb[u] * sn;
          A = A * so + xb[u] * sn;
          M = Mn;
        }
      }
      const float den = ROUTE == DKV_ROUTE_TWO_STAGE ? fmaxf(L, 1e-6f) : L;
      a = A / den;
    }
    sA[idx] = a;
  }
}

// The same merge with the weights formed once per (head, split) for up to MERGE_WSPLITS
// splits: w = 2^(m - M) / den from the head's maximum M and denominator, then each (head,
// rank) thread only loads its coefficient of every split and sums the weighted values (a third
// of the loads and none of the exponentials of merge_records per thread).
constexpr int MERGE_WSPLITS = 64;
template <int MB, int ROUTE>
__device__ __forceinline__ void merge_records_w(const SplitParams& p, const float* base,
                                                long long stride, float* sA, float* sM,
                                                float* sL, float* sW) {
  const int tid = threadIdx.x, ns = p.n_splits;
  // this thread's (head, rank) pairs: idx = tid + k * NTHREADS. For the first (head slots
  // 0..3) the coefficients of the first MB splits are loaded here, in flight with the (m, l)
  // loads below; the others are loaded once the weights are known.
  constexpr int NIDX = 16 * DH / NTHREADS;
  float x0[MB];
  {
    const int hsc = min(tid / DH, p.hpg - 1), rc = min(tid % DH, p.R - 1);
#pragma unroll
    for (int u = 0; u < MB; ++u) x0[u] = rec_load(base + min(u, ns - 1) * stride + hsc * PREC + 2 + rc);
  }
  for (int t = tid; t < p.hpg * ns; t += NTHREADS) {
    const int hs = t / ns, sp = t % ns;
    const float* rec = base + sp * stride + hs * PREC;
    sM[hs * MERGE_WSPLITS + sp] = rec_load(rec);
    sL[hs * MERGE_WSPLITS + sp] = rec_load(rec + 1);
  }
  __syncthreads();
  for (int t = tid; t < p.hpg * ns; t += NTHREADS) {
    const int hs = t / ns, sp = t % ns;
    const float* mh = sM + hs * MERGE_WSPLITS;
    const float* lh = sL + hs * MERGE_WSPLITS;
    float M = -INFINITY;
    for (int u = 0; u < ns; ++u) M = fmaxf(M, mh[u]);
    float L = 0.f;
    for (int u = 0; u < ns; ++u) L += mh[u] == -INFINITY ? 0.f : lh[u] * exp2f(mh[u] - M);
    const float den = ROUTE == DKV_ROUTE_TWO_STAGE ? fmaxf(L, 1e-6f) : L;
    sW[hs * MERGE_WSPLITS + sp] = mh[sp] == -INFINITY ? 0.f : exp2f(mh[sp] - M) / den;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NIDX; ++k) {
    const int idx = tid + k * NTHREADS, hs = idx / DH, r = idx % DH;
    float a = 0.f;
    if (hs < p.hpg && r < p.R) {
      int sp0 = 0;
      if (k == 0) {
#pragma unroll
        for (int u = 0; u < MB; ++u)
          if (u < ns) a += sW[hs * MERGE_WSPLITS + u] * x0[u];
        sp0 = MB;
      }
      for (; sp0 < ns; sp0 += MB) {
        float xb[MB];
#pragma unroll
        for (int u = 0; u < MB; ++u) xb[u] = rec_load(base + min(sp0 + u, ns - 1) * stride + hs * PREC + 2 + r);
#pragma unroll
        for (int u = 0; u < MB; ++u)
          if (sp0 + u < ns) a += sW[hs * MERGE_WSPLITS + sp0 + u] * xb[u];
      }
    }
    sA[idx] = a;
  }
}

// This thread's share of the unit's V basis (16-byte piece ch: rank ch / 16, dims
// 8 * (ch % 16)); unconditional loads (pieces of ranks past R read rank R-1's and are zeroed
// when staged), so that none waits for another.
__device__ __forceinline__ void load_vbasis(const SplitParams& p, int kvh, dkv_u32x4 (&vbr)[VB_CHUNKS]) {
  const uint16_t* vb = p.v_basis + (long long)kvh * p.v_unit;
#pragma unroll
  for (int k = 0; k < VB_CHUNKS; ++k) {
    const int ch = min((int)threadIdx.x + k * NTHREADS, p.R * (DH / 8) - 1);
    vbr[k] = *(const dkv_u32x4*)(vb + (long long)(ch >> 4) * p.v_sr + 8 * (ch & 15));
  }
}

template <int DT, int ODT>
__device__ __forceinline__ void project_store(const SplitParams& p, int unit, uint8_t* scratch,
                                              const dkv_u32x4 (&vbr)[VB_CHUNKS]);

template <int DT, int ROUTE, int ODT>
__device__ __forceinline__ void merge_unit_t(const SplitParams& p, int unit, uint8_t* scratch) {
  const int kvh = unit % p.Hkv;
  const long long stride = (long long)p.hpg * PREC;  // between splits of one head
  const float* base = p.partials + (long long)unit * p.n_splits * stride;
  float* sA = reinterpret_cast<float*>(scratch + DH * DH * 2);    // [16][DH] merged, normalised
  // the V basis in flight while the records are read and merged
  dkv_u32x4 vbr[VB_CHUNKS];
  load_vbasis(p, kvh, vbr);
  // merged coefficient of (head slot hs, rank r); slots past hpg are zero. A batch of MB
  // splits' record loads is issued before any is used, so a call pays one load latency per
  // MB splits (MB the smallest of 8, 16, 32 that covers the splits). Up to 8 splits merge
  // in one pass of running maxima; from 9 on the weights are formed once per (head, split)
  // (measured on MI355X: ~1 us less at 32 splits, ~0.5 us more at 2).
  float* sM = sA + 16 * DH;
  float* sL = sM + 16 * MERGE_WSPLITS;
  float* sW = sL + 16 * MERGE_WSPLITS;
  if (p.n_splits <= 8)
    merge_records<8, ROUTE>(p, base, stride, sA);
  else if (p.n_splits <= 16)
    merge_records_w<16, ROUTE>(p, base, stride, sA, sM, sL, sW);
  else if (p.n_splits <= MERGE_WSPLITS)
    merge_records_w<32, ROUTE>(p, base, stride, sA, sM, sL, sW);
  else
    merge_records<32, ROUTE>(p, base, stride, sA);
  project_store<DT, ODT>(p, unit, scratch, vbr);
}

// out = the merged, normalised coefficients sA (scratch + DH * DH * 2, [16][DH], written by
// every thread before the call) through the V basis (vbr, staged here at scratch), stored in
// the output dtype (all threads of the block).
template <int DT, int ODT>
__device__ __forceinline__ void project_store(const SplitParams& p, int unit, uint8_t* scratch,
                                              const dkv_u32x4 (&vbr)[VB_CHUNKS]) {
  const int b = unit / p.Hkv, kvh = unit % p.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  uint16_t* sVB = reinterpret_cast<uint16_t*>(scratch);          // [128][DH], rank-major
  const float* sA = reinterpret_cast<const float*>(scratch + DH * DH * 2);
#pragma unroll
  for (int k = 0; k < VB_CHUNKS; ++k)
    *(dkv_u32x4*)(sVB + (tid + k * NTHREADS) * 8) =
        tid + k * NTHREADS < p.R * (DH / 8) ? vbr[k] : dkv_u32x4{0u, 0u, 0u, 0u};
  __syncthreads();
  // out[hs][d] = sum_r a[hs][r] VB[r][d] on 16x16x32 MFMA: wave w takes dims 16w..16w+15.
  // A: the merged coefficients of head slot n, ranks 32c + 8g..+7, as hi + lo parts in the
  // basis dtype (two products); B: the basis read transposed -- within a 16-lane group, lane i
  // gets element i%4 of the 8 bytes read by lane 4j + i/4 as its element j, so lane L reading
  // VB[k0 + L/4][d0 + 4*(L%4) ..] hands lane i the four ranks k0..k0+3 of dim d0 + i.
  const int d0 = 16 * wave;
  dkv_f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int k0 = 32 * c + 8 * g;
    const float* ar = sA + n * DH + k0;
    const dkv_f32x4 x0 = *(const dkv_f32x4*)ar, x1 = *(const dkv_f32x4*)(ar + 4);
    const float xs[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (DT == DKV_BF16) {
        typedef __attribute__((ext_vector_type(2))) float f32x2;
        const dkv_bf16x2 h = __builtin_convertvector(f32x2{xs[2 * e], xs[2 * e + 1]}, dkv_bf16x2);
        const dkv_bf16x2 l = __builtin_convertvector(
            f32x2{xs[2 * e] - (float)h[0], xs[2 * e + 1] - (float)h[1]}, dkv_bf16x2);
        hi[e] = __builtin_bit_cast(uint32_t, h);
        lo[e] = __builtin_bit_cast(uint32_t, l);
      } else {
        split_f16x2(xs[2 * e], xs[2 * e + 1], p.minus_one, hi[e], lo[e]);
      }
    }
    const uint16_t* src = sVB + (k0 + (n >> 2)) * DH + d0 + 4 * (n & 3);
    typedef __attribute__((address_space(3))) dkv_i16x4 lds_i16x4;
    const dkv_u32x2 b0 = __builtin_bit_cast(
        dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                       (lds_i16x4*)(__attribute__((address_space(3))) uint16_t*)src));
    const dkv_u32x2 b1 = __builtin_bit_cast(
        dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                       (lds_i16x4*)(__attribute__((address_space(3))) uint16_t*)(src + 4 * DH)));
    const dkv_u32x4 bop = dkv_u32x4{b0.x, b0.y, b1.x, b1.y};
    o = mfma_k<DT>(dkv_u32x4{lo[0], lo[1], lo[2], lo[3]}, bop, o);
    o = mfma_k<DT>(dkv_u32x4{hi[0], hi[1], hi[2], hi[3]}, bop, o);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int hs = 4 * g + u;
    if (hs < p.hpg) {
      const long long oi =
          (long long)b * p.out_sb + (long long)(kvh * p.hpg + hs) * p.out_sh + d0 + n;
      dkv_store_f32<ODT>(p.out, oi, o[u]);
    }
  }
}
template <int DT, int ROUTE>
__device__ __forceinline__ void merge_unit(const SplitParams& p, int unit, uint8_t* scratch) {
  if (p.out_f32)
    merge_unit_t<DT, ROUTE, DKV_F32>(p, unit, scratch);
  else
    merge_unit_t<DT, ROUTE, DT>(p, unit, scratch);
}

// HMAX: the most query heads per unit the instance handles (4, 8 or 16); each lane keeps HMAX
// query registers, so the common 4-head groups carry no registers for absent heads. Past 8
// heads (WIDE) the query operand carries the heads' hi parts in its 16 columns and a second
// product takes the lo parts; with up to 8 heads the hi parts sit in columns 0..7 and the lo
// parts in columns 8..15 of one product.
template <int DT, int ROUTE, int HMAX, bool PAIR>
__global__ __launch_bounds__(NTHREADS, 1) void splitk_kernel(SplitParams p) {
  constexpr bool WIDE = HMAX > 8;
  // LDS: per-wave rings (NSLOT gather slots: K then V, 4 chunks x 64 lanes x 16 bytes each;
  // TSLOT table slots: lens_k, offs_k, lens_v, offs_v x 16 tokens), the part of the K basis not
  // held in registers ([dim][rank] rows; none with NREG_PP = 4), the R(n) table and the mask
  // table. The full basis
  // staging copy, the per-tile query operand and the epilogue scratch alias the rings.
  __shared__ __attribute__((aligned(16))) uint32_t sMask[MASK_ROWS][4];
  __shared__ __attribute__((aligned(16))) int sTabRing[WAVES][TSLOT][4][TILE];
  __shared__ __attribute__((aligned(16))) uint16_t sBH[(SBH_ROWS > 0 ? SBH_ROWS : 1) * BK_LD];
  // R(n) of every lane's token slot, in lane order: entry [2*pp + k][lane] holds (cos, sin) of
  // the lane's frequencies 16*pp + 4*g + 2k and + 1 (one conflict-free 16-byte read per lane)
  __shared__ __attribute__((aligned(16))) dkv_f32x4 sRn[8][64];
  // R(16 + n): the token slots of the second tile of a wave's pair (same layout as sRn)
  __shared__ __attribute__((aligned(16))) dkv_f32x4 sRn2[8][64];
  // the unit's query pairs per lane (qh, below) and the rotation step of the per-tile query
  // rotation, read per tile instead of held in registers (the same for every wave)
  __shared__ __attribute__((aligned(16))) dkv_u32x4 sQh[(HMAX + 3) / 4][64];
  __shared__ __attribute__((aligned(16))) float sStep[64][4];
  // 256-byte aligned: the query operand's row swizzle XORs bits 4..7 of ring addresses
  __shared__ __attribute__((aligned(256))) uint8_t sRing[WAVES * NSLOT * GSLOT_BYTES];
  static_assert(DH * BK_LD * 2 <= WAVES * NSLOT * GSLOT_BYTES, "basis staging fits the rings");
  static_assert(16 * QROW_BYTES <= GSLOT_BYTES / 2, "query operand fits a slot's K half");
  constexpr int QH = HMAX;  // head registers per lane
  uint16_t* sBK = reinterpret_cast<uint16_t*>(sRing);

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
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int R = p.R;
  const int s_begin = split * p.split_len;
  const int s_end = min(p.S, s_begin + p.split_len);
  const int ns = s_end - s_begin;

  const int tile_first = s_begin / TILE;  // splits are whole tiles (multiples of 64 tokens)
  // PAIR: a wave takes pairs of consecutive tiles (2*wave, 2*wave + 1, then 16 tiles on), which
  // share one query operand (the second tile's token slots use R(16 + n)); otherwise waves
  // take single tiles round-robin. The host pairs splits of at least 2 * WAVES tiles, where
  // both schemes give every wave the same number of tiles.
  const int n_tiles = (ns + TILE - 1) / TILE;
  constexpr bool paired = PAIR;
  const int tile0 = tile_first + (paired ? 2 * wave : wave);
  auto tix = [&](int j) {
    return paired ? tile0 + (j & 1) + 2 * WAVES * (j >> 1) : tile0 + WAVES * j;
  };
  const int n_tb = (p.S + TILE - 1) / TILE;
  const int n_iter = paired ? 2 * (n_tiles / (2 * WAVES)) +
                                   max(0, min(2, n_tiles % (2 * WAVES) - 2 * wave))
                             : max(0, (n_tiles - wave + WAVES - 1) / WAVES);
  // table loads: lane (table l/16, token l%16) -> one 4-byte load per lane and tile
  const int* tab_base;
  int tab_ss;
  {
    const int tsel = lane >> 4;
    const int* bases[4] = {p.lens_k + (long long)row * p.tk_sb, p.offs_k + (long long)row * p.tk_sb,
                           p.lens_v + (long long)row * p.tv_sb, p.offs_v + (long long)row * p.tv_sb};
    tab_base = tsel == 0 ? bases[0] : tsel == 1 ? bases[1] : tsel == 2 ? bases[2] : bases[3];
    tab_ss = tsel < 2 ? (int)p.tk_ss : (int)p.tv_ss;
  }
  auto load_tab = [&](int j) {  // one load per lane into table slot j % TSLOT
    const uint32_t t = (uint32_t)min(tix(j) * TILE + n, s_end - 1);
    lds_load4(tab_base + __umul24(t, (uint32_t)tab_ss), lds_addr(&sTabRing[wave][j % TSLOT][0][0]));
  };
  // the first two tiles' tables (the table ring does not alias the staging copy) are in
  // flight during the prologue
  load_tab(0);
  load_tab(1);
  // rotation R(16*T) of the wave's current tile T for frequency i = lane, times the score
  // scale (the fused route's scores come out in log2 units, the two-stage route's in natural
  // units), advanced by angle addition (WAVES*TILE positions per tile); bc/bs start at the
  // table's exact value for the wave's first tile. Loaded here, with the tables, so that their
  // round trip overlaps the prologue's instead of following its barriers.
  float bc, bs;
  {
    const int t = min(tile0, n_tb - 1);
    const float* rrow = p.rope + (long long)(ROPE_FIXED_ROWS + t) * 128 + 2 * lane;
    bc = rrow[0] * p.score_scale;
    bs = rrow[1] * p.score_scale;
  }

  // ---- prologue: K basis, mask table, rotation step ---------------------------------------
  {
    // transpose to [dim][rank]: consecutive lanes take consecutive ranks, so each 2-byte LDS
    // store of a wave covers 128 contiguous bytes (no bank conflicts). The dims of the block
    // pairs past NREG_PP go to their permanent place in sBH (low blocks, then high blocks),
    // the others to the staging copy.
    const uint16_t* kb = p.k_basis + (long long)kvh * p.k_unit;
    const int j = tid & 127, dq = tid >> 7;  // 4 groups of 8-dim slices
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int d8 = (dq + 4 * it) * 8;
      dkv_u32x4 v = dkv_u32x4{0u, 0u, 0u, 0u};
      if (j < R) v = *(const dkv_u32x4*)(kb + (long long)j * p.k_sr + d8);
      const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int d = d8 + t;
        const uint16_t x = (uint16_t)((e[t >> 1] >> (16 * (t & 1))) & 0xffffu);
        const int pp = (d & 63) >> 4;
        if (pp >= NREG_PP)
          sBH[(((d >> 6) * (4 - NREG_PP) + pp - NREG_PP) * 16 + (d & 15)) * BK_LD + j] = x;
        else
          sBK[d * BK_LD + j] = x;
      }
    }
    // row MASK_BIAS + dk: keep-mask of the lane's last piece when its token has dk elements from
    // the lane's first piece on (that piece is chunk clamp((dk - 1) / 32, 0, 3))
    for (int r = tid; r < MASK_ROWS * 4; r += NTHREADS) {
      const int dk = (r >> 2) - MASK_BIAS;
      const int ck = min(max((dk - 1) >> 5, 0), 3);
      sMask[r >> 2][r & 3] = prefix_mask_word(min(max(dk - 32 * ck, 0), 8), r & 3);
    }
  }

  // RoPE is split by angle addition: the key of position 16*T + n is rotated by R(n) here,
  // on its own lane (token slot n, fixed for the whole kernel), and R(16*T) goes to the query
  // of tile T instead: q . R(16T + n) k = (R(-16T) q) . (R(n) k).
  // qh[h]: (q_i, q_{i+64}) of head h for frequency i = lane, as the cache's 16-bit values.
  uint32_t qh[QH];
  {
    const long long qo = (long long)b * p.q_sb + (long long)kvh * p.hpg * p.q_sh + lane;
    // unconditional loads (slots past the heads read head 0), so that they are all in flight
    // at once rather than one round trip per head
#pragma unroll
    for (int h = 0; h < QH; ++h) {
      const long long o = qo + (h < p.hpg ? h : 0) * p.q_sh;
      const uint32_t v = (uint32_t)p.q[o] | ((uint32_t)p.q[o + 64] << 16);
      qh[h] = h < p.hpg ? v : 0u;
    }
    if (wave == 0) {
#pragma unroll
      for (int k = 0; k < (QH + 3) / 4; ++k)
        sQh[k][lane] = dkv_u32x4{qh[4 * k], 4 * k + 1 < QH ? qh[4 * k + 1] : 0u,
                                 4 * k + 2 < QH ? qh[4 * k + 2] : 0u,
                                 4 * k + 3 < QH ? qh[4 * k + 3] : 0u};
      // the rotation by WAVES * TILE positions (single tiles) and by twice that (pairs),
      // R(128) doubled
      const float c = p.rope[TILE * 128 + 2 * lane], sn = p.rope[TILE * 128 + 2 * lane + 1];
      sStep[lane][0] = c;
      sStep[lane][1] = sn;
      sStep[lane][2] = c * c - sn * sn;
      sStep[lane][3] = 2.f * c * sn;
    }
  }
  // R(n) table in LDS (see sRn): thread t fills entry t (8 x 64 entries, 512 threads)
  {
    const int k = tid >> 6, ln = tid & 63;
    const int nn = ln & 15, gg = ln >> 4, i0 = 16 * (k >> 1) + 4 * gg + 2 * (k & 1);
    const float* delt = p.rope + (long long)nn * 128 + 2 * i0;
    sRn[k][ln] = dkv_f32x4{delt[0], delt[1], delt[2], delt[3]};
    // R(16) = R(15) R(1) by angle addition, then R(16 + n) = R(16) R(n)
    if constexpr (PAIR) {
    const float* r15 = p.rope + 15 * 128 + 2 * i0;
    const float* r1 = p.rope + 1 * 128 + 2 * i0;
    float o[4];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float c16 = r15[2 * e] * r1[2 * e] - r15[2 * e + 1] * r1[2 * e + 1];
      const float s16 = r15[2 * e + 1] * r1[2 * e] + r15[2 * e] * r1[2 * e + 1];
      o[2 * e] = c16 * delt[2 * e] - s16 * delt[2 * e + 1];
      o[2 * e + 1] = s16 * delt[2 * e] + c16 * delt[2 * e + 1];
    }
    sRn2[k][ln] = dkv_f32x4{o[0], o[1], o[2], o[3]};
    }
  }
  // The per-tile query operand lives in the K half of the tile's gather slot once the K
  // coefficients are in registers: row r (one per operand column), chunk c (16 bytes: dwords
  // 4c..4c+3, i.e. frequencies 4c..4c+3) stored at chunk position c ^ r, so that the 16 rows
  // read by one k-group land in 16 different bank groups. Column n reads row qrow: its head's
  // hi (n < 8) or lo (n >= 8) row, or, for columns past the heads, a real row (finite values
  // in columns that are never used).
  uint8_t* ring = sRing + wave * NSLOT * GSLOT_BYTES;
  uint32_t q_rd[4];  // LDS address of chunk 4*pp + g of row qrow in slot 0
  uint32_t q_wr;     // ring base | 4*lane: this lane's dword in row r of slot 0 is q_wr ^ (16*r)
  {
    const int hn = WIDE ? n : (n & 7);
    const int head = hn < p.hpg ? hn : hn % p.hpg;
    const int qrow = WIDE ? head : (n & 8) + head;
    const uint32_t rb = lds_addr(ring);
#pragma unroll
    for (int pp = 0; pp < 4; ++pp)
      q_rd[pp] = rb + (uint32_t)(qrow * QROW_BYTES) + 16u * (uint32_t)((4 * pp + g) ^ qrow);
    q_wr = rb | (4u * (uint32_t)lane);
  }

  __syncthreads();  // staging copy, sBH, sMask ready

  // recon A operands of the block pairs pp < NREG_PP (blocks pp and pp + 4; block blk = dims
  // 16*blk + n, rank chunk c = ranks 32c + 8g .. +8), read into the registers the MFMAs take
  // as their A operand; the other pairs are read from sBH per tile.
  dkv_u32x4 bA[2 * NREG_PP][4];  // [k][c], k -> block (k&1 ? 4 : 0) + (k >> 1)
  {
    const uint32_t a0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)(
        sBK + n * BK_LD + 8 * g);
    // one statement per block: its four reads and the wait for them, so that the outputs
    // hold their data when the statement ends (the compiler may copy or spill an asm output
    // right after the statement)
#pragma unroll
    for (int k = 0; k < 2 * NREG_PP; ++k) {
      const int blk = (k & 1 ? 4 : 0) + (k >> 1);
      asm volatile(
          "ds_read_b128 %0, %4 offset:%5\n\t"
          "ds_read_b128 %1, %4 offset:%6\n\t"
          "ds_read_b128 %2, %4 offset:%7\n\t"
          "ds_read_b128 %3, %4 offset:%8\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(bA[k][0]), "=&v"(bA[k][1]), "=&v"(bA[k][2]), "=&v"(bA[k][3])
          : "v"(a0), "i"((16 * blk * BK_LD) * 2), "i"((16 * blk * BK_LD + 32) * 2),
            "i"((16 * blk * BK_LD + 64) * 2), "i"((16 * blk * BK_LD + 96) * 2)
          : "memory");
    }
  }
  __syncthreads();  // every wave holds its operands: the rings may now be overwritten

  // one resource per buffer, ranges [flat, flat + rows * ld); row offsets go in the voffset
  // one resource per buffer, based at this workgroup's row (a workgroup reads one row only),
  // covering the rest of the buffer up to FLAT_ELEM_CAP elements; token offsets go in the
  // voffset. Row strides are at most FLAT_LD_MAX, so a row's last window stays in range unless
  // the row is the buffer's last.
  const uint32_t k_end = (uint32_t)dkv_flat_tail_elems(p.rows, row, p.k_ld, FLAT_ELEM_CAP);
  const uint32_t v_end = (uint32_t)dkv_flat_tail_elems(p.rows, row, p.v_ld, FLAT_ELEM_CAP);
  const __amdgpu_buffer_rsrc_t rk_src = dkv_make_rsrc(p.k_flat + (long long)row * p.k_ld, k_end * 2u);
  const __amdgpu_buffer_rsrc_t rv_src = dkv_make_rsrc(p.v_flat + (long long)row * p.v_ld, v_end * 2u);
  constexpr int k_row0 = 0, v_row0 = 0;
  // only the buffers' last row can hold a token whose 16-byte window crosses the end
  const bool last_row = row == p.B * p.G - 1;
  // token metadata of this lane's token in tile j (table slot must have arrived). A slot past
  // the split's end holds the entries of the split's last token (the table loads clamp): its
  // gathers read real data and its score is excluded in the softmax.
  struct Tok {
    int ko, rkc, rvc, vo;
  };
  auto tok_of = [&](int j) {
    Tok d;
    const int(*tb)[TILE] = sTabRing[wave][j % TSLOT];
    d.rkc = min(max(tb[0][n], 0), R);
    d.rvc = min(max(tb[2][n], 0), R);
    d.ko = k_row0 + tb[1][n];
    d.vo = v_row0 + tb[3][n];
    return d;
  };
  // gathers of tile j into gather slot j % NSLOT: lane l's 16 bytes of chunk c land at
  // slot + c*1024 + 16*l (K) and slot + 4096 + c*1024 + 16*l (V). A lane whose token has no
  // element in its 8-rank piece of chunk c reads the out-of-range offset instead: no memory
  // traffic, and zeros land in its LDS bytes.
  auto issue = [&](int j) {
    const Tok d = tok_of(j);
    const uint32_t slot = lds_addr(ring + (j % NSLOT) * GSLOT_BYTES);
    const int dk = d.rkc - 8 * g, dv = d.rvc - 8 * g;  // elements from the lane's first piece
    const uint32_t kb = (uint32_t)(d.ko + 8 * g) * 2u, vb = (uint32_t)(d.vo + 8 * g) * 2u;
    lds_load16_chunk<0>(rk_src, slot, dk > 0 ? kb : OOB);
    lds_load16_chunk<1>(rk_src, slot + 1024, dk > 32 ? kb : OOB);
    lds_load16_chunk<2>(rk_src, slot + 2048, dk > 64 ? kb : OOB);
    lds_load16_chunk<3>(rk_src, slot + 3072, dk > 96 ? kb : OOB);
    lds_load16_chunk<0>(rv_src, slot + 4096, dv > 0 ? vb : OOB);
    lds_load16_chunk<1>(rv_src, slot + 5120, dv > 32 ? vb : OOB);
    lds_load16_chunk<2>(rv_src, slot + 6144, dv > 64 ? vb : OOB);
    lds_load16_chunk<3>(rv_src, slot + 7168, dv > 96 ? vb : OOB);
  };
  // A 16-byte window that crosses the end of a resource reads as zero in full; only the last
  // tokens of the last row can need one. Such a tile is gathered again with element loads
  // once its slot has landed.
  auto regather_if_needed = [&](const Tok& d, uint8_t* slot) {
    const bool risky = (d.rkc > 0 && (uint32_t)(d.ko + d.rkc + 7) > k_end) ||
                       (d.rvc > 0 && (uint32_t)(d.vo + d.rvc + 7) > v_end);
    if (__builtin_expect(__ballot(risky) != 0ull, 0)) {
      // one chunk at a time: this cold path must not raise the loop's register pressure
#pragma unroll 1
      for (int c = 0; c < 8; ++c) {
        const bool isv = c >= 4;
        *(dkv_u32x4*)(slot + c * 1024 + 16 * lane) =
            gather_chunk(isv ? rv_src : rk_src, isv ? v_end : k_end, isv ? d.vo : d.ko,
                         isv ? d.rvc : d.rkc, c & 3, g);
      }
    }
  };

  dkv_f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
  // running max per head slot n (log2 units), identical across g. It starts at a finite floor
  // far below any score, so that excluded tokens (-inf) give exp2(-inf) = 0 without a select
  // and a record without any included token carries l = 0 and acc = 0 under that floor.
  float m_run = -1.0e30f;
  float l_run = 0.f;        // partial over this lane's 4 tokens per tile

  // ---- pipeline: one tile per iteration; the gathers of tile j+1 and the table of tile j+2
  //      are in flight while tile j computes (two waves per SIMD hide each other's latency).
  //      Loads are issued for every iteration, also past the wave's last tile (indices clamp
  //      to the split's last token), so at the top of iteration j nothing but G(j) and T(j+1)
  //      can be in flight and a full wait costs nothing extra. -------------------------------
  // loop-invariant loaded values: settled here, so the loop carries no wait for their loads
  // (such a wait would also drain the gathers in flight)
  settle(bc);
  settle(bs);

  // T0 and T1 (a full wait: compiler-generated memory operations of the prologue, such as
  // register spill stores, may lie between them and here and need not complete in order)
  wait_vm<0>();
  issue(0);

  dkv_u32x4 bq[4], bq_lo[4];  // the query operand of the wave's current pair of tiles
  // one tile; par = j % NSLOT (par 0: the first tile of a pair, which forms the query operand)
  auto tile = [&](int j, const int par) {
    wait_vm<0>();  // G(j), T(j+1)
    const Tok cur = tok_of(j);
    uint8_t* slot = ring + par * GSLOT_BYTES;
    if (last_row) regather_if_needed(cur, slot);
    load_tab(j + 2);
    issue(j + 1);
    // issue priority by phase (measured on MI355X, ~3% at config 3 over one level): the tile's
    // front (masks, K windows, query rotation) 2, the reconstruction products 0, scores,
    // softmax and P.V 1
    __builtin_amdgcn_s_setprio(2);
    // ---- masks: elements past a token's count belong to the next tokens. Pieces wholly past
    //      the count were loaded as zeros, so only the partial piece of each token needs one:
    //      the lane masks its own partial K and V piece in place, then reads the K windows ----
    {
      const int dk = cur.rkc - 8 * g, dv = cur.rvc - 8 * g;
      const int ck = min(max((dk - 1) >> 5, 0), 3);  // chunk of the lane's last K element
      const int cv = min(max((dv - 1) >> 5, 0), 3);
      dkv_u32x4* kp = (dkv_u32x4*)(slot + ck * 1024 + 16 * lane);
      dkv_u32x4* vp = (dkv_u32x4*)(slot + 4096 + cv * 1024 + 16 * lane);
      const dkv_u32x4 mk = *(const dkv_u32x4*)&sMask[dk + MASK_BIAS][0];
      const dkv_u32x4 mv = *(const dkv_u32x4*)&sMask[dv + MASK_BIAS][0];
      const dkv_u32x4 kr = *kp, vr = *vp;
      *kp = dkv_u32x4{kr.x & mk.x, kr.y & mk.y, kr.z & mk.z, kr.w & mk.w};
      *vp = dkv_u32x4{vr.x & mv.x, vr.y & mv.y, vr.z & mv.z, vr.w & mv.w};
    }
    dkv_u32x4 xk[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) xk[c] = *(const dkv_u32x4*)(slot + c * 1024 + 16 * lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- query of this tile: R(-16T) q times the score scale, as bf16 hi + lo, written to the
    //      K half of the slot (its coefficients are in xk; LDS accesses of a wave run in order)
    //      and read back as the B operand of the score MFMAs (lane: column n, k-group g) ----
    if (par == 0 || !paired) {
      const float cb = bc, sb = bs;
      // formed per tile (not hoisted as one register per row)
      uint32_t wr = q_wr + (uint32_t)(par * GSLOT_BYTES);
      settle(wr);
      uint32_t qv[4 * ((QH + 3) / 4)];
#pragma unroll
      for (int k = 0; k < (QH + 3) / 4; ++k) {
        const dkv_u32x4 v = sQh[k][lane];
        qv[4 * k] = v.x;
        qv[4 * k + 1] = v.y;
        qv[4 * k + 2] = v.z;
        qv[4 * k + 3] = v.w;
      }
      auto rotate = [&](int h, uint32_t& hi, uint32_t& lo) {
        const float x = elt_to_f32<DT>(qv[h] & 0xffffu), y = elt_to_f32<DT>(qv[h] >> 16);
        split_bf16x2(cb * x + sb * y, cb * y - sb * x, hi, lo);
      };
      // the next tile's base rotation
      const float stc = sStep[lane][paired ? 2 : 0], sts = sStep[lane][paired ? 3 : 1];
      bc = cb * stc - sb * sts;
      bs = sb * stc + cb * sts;
      auto put = [&](uint32_t v, int r) {
        *(__attribute__((address_space(3))) uint32_t*)(uintptr_t)(
            (wr ^ (16u * r)) + (uint32_t)(r * QROW_BYTES)) = v;
      };
      auto get = [&](dkv_u32x4 (&dst)[4]) {
#pragma unroll
        for (int pp = 0; pp < 4; ++pp)
          dst[pp] = *(const __attribute__((address_space(3))) dkv_u32x4*)(uintptr_t)(
              q_rd[pp] + (uint32_t)(par * GSLOT_BYTES));
      };
      if constexpr (!WIDE) {
#pragma unroll
        for (int h = 0; h < QH; ++h)
          if (h < p.hpg) {
            uint32_t hi, lo;
            rotate(h, hi, lo);
            put(hi, h);
            put(lo, 8 + h);
          }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        get(bq);
      } else {
        uint32_t lo16[QH];
#pragma unroll
        for (int h = 0; h < QH; ++h)
          if (h < p.hpg) {
            uint32_t hi;
            rotate(h, hi, lo16[h]);
            put(hi, h);
          }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        get(bq);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // hi rows read before the lo rows
#pragma unroll
        for (int h = 0; h < QH; ++h)
          if (h < p.hpg) put(lo16[h], h);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        get(bq_lo);
      }
    }

    // ---- 1-3: K reconstruction, R(n) on the lane's token, K' as bf16 hi + lo, scores -------
    dkv_f32x4 sc = {0.f, 0.f, 0.f, 0.f};
    // blocks pp and pp+4 of K^T for the tile; pp < NREG_PP from the registers, the others
    // from the streamed rows in sBH
    auto recon = [&](int pp, dkv_f32x4& c0, dkv_f32x4& c1) {
      c0 = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
      c1 = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
      if (pp < NREG_PP) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          c0 = mfma_k<DT>(bA[2 * pp][c], xk[c], c0);
          c1 = mfma_k<DT>(bA[2 * pp + 1][c], xk[c], c1);
        }
      } else {
        const uint16_t* r0 = sBH + ((pp - NREG_PP) * 16 + n) * BK_LD + 8 * g;
        const uint16_t* r1 = r0 + (4 - NREG_PP) * 16 * BK_LD;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          c0 = mfma_k<DT>(*(const dkv_u32x4*)(r0 + 32 * c), xk[c], c0);
          c1 = mfma_k<DT>(*(const dkv_u32x4*)(r1 + 32 * c), xk[c], c1);
        }
      }
    };
    // R(n), or R(16 + n) for the second tile of a pair
    const dkv_f32x4(*rtab)[64] = (par == 1 && paired) ? sRn2 : sRn;
    // software-pipelined by one block pair: the products of pp+1 are issued before the
    // rotation of pp, so the MFMA pipe and the VALU work of one wave overlap
    __builtin_amdgcn_s_setprio(0);
    dkv_f32x4 C0[2], C1[2];
    recon(0, C0[0], C1[0]);
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      if (pp + 1 < 4) recon(pp + 1, C0[(pp + 1) & 1], C1[(pp + 1) & 1]);
      const dkv_f32x4 c0 = C0[pp & 1], c1 = C1[pp & 1];
      // K' rotated in fp32 and split into bf16 hi + lo parts: the score products are
      // (K'hi + K'lo) . (q hi + q lo) to ~16 bits per factor, with fp32's range
      uint32_t kh[4], kl[4];
      const dkv_f32x4 r01 = rtab[2 * pp][lane], r23 = rtab[2 * pp + 1][lane];
      const float rc[4] = {r01.x, r01.z, r23.x, r23.z}, rs[4] = {r01.y, r01.w, r23.y, r23.w};
#pragma unroll
      for (int w = 0; w < 4; ++w)
        split_bf16x2(c0[w] * rc[w] - c1[w] * rs[w], c1[w] * rc[w] + c0[w] * rs[w], kh[w], kl[w]);
      const dkv_u32x4 ka = dkv_u32x4{kh[0], kh[1], kh[2], kh[3]};
      const dkv_u32x4 kal = dkv_u32x4{kl[0], kl[1], kl[2], kl[3]};
      sc = mfma_bf16(ka, bq[pp], sc);
      sc = mfma_bf16(kal, bq[pp], sc);
      if constexpr (WIDE) sc = mfma_bf16(ka, bq_lo[pp], sc);
    }
    if constexpr (!WIDE) {
      // column n += column n + 8 (the lo part of head n) within each row of 16 lanes
#pragma unroll
      for (int u = 0; u < 4; ++u)
        sc[u] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sc[u]),
                                                            DPP_ROW_SHL8, 0xf, 0xf, false));
    }

    __builtin_amdgcn_s_setprio(1);
    // scores of lane (head slot n, tokens 4g+u) with the route's masking: the fused route in
    // log2 units, the two-stage route as the rounded scores (natural units; the factor log2(e)
    // is applied to their maximum and inside the exponent's fma)
    float z[4];
    {
      const dkv_i32x4 lk4 = *(const dkv_i32x4*)&sTabRing[wave][j % TSLOT][0][4 * g];
      const int lk[4] = {lk4.x, lk4.y, lk4.z, lk4.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool has = lk[u] > 0;
        if constexpr (ROUTE == DKV_ROUTE_FUSED)
          z[u] = has ? sc[u] : -INFINITY;
        else
          z[u] = dkv_round_to<DT>(has ? sc[u] : p.masked_score);
      }
      const int nvalid = s_end - tix(j) * TILE;  // tokens of the tile in range
      if (__builtin_expect(nvalid < TILE, 0)) {  // wave-uniform: the split's last tile
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (4 * g + u >= nvalid) z[u] = -INFINITY;
      }
    }

    // ---- 4. online softmax (per head slot; its 16 tokens sit in lanes n, n+16, n+32, n+48) --
    float tmax = max3_f32(max3_f32(z[0], z[1], z[2]), z[3], z[3]);
    tmax = lane_max32(tmax);
    tmax = lane_max16(tmax);
    if constexpr (ROUTE != DKV_ROUTE_FUSED) tmax *= LOG2E;
    if (__ballot(tmax > m_run + RESCALE_THRESH)) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // m_run is finite
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
      // exp2 of a value <= RESCALE_THRESH (-inf for excluded tokens gives 0); results below
      // fp32's normal range may flush to zero
      if constexpr (ROUTE == DKV_ROUTE_FUSED)
        pu[u] = __builtin_amdgcn_exp2f(z[u] - m_run);
      else
        pu[u] = __builtin_amdgcn_exp2f(__builtin_fmaf(z[u], LOG2E, -m_run));
      l_run += pu[u];
    }

    // ---- 5. P.X^V in coefficient space ----------------------------------------------------------
    dkv_u32x2 pa_hi, pa_lo;
    if constexpr (DT == DKV_F16) {
      pa_hi = dkv_u32x2{pack_f16x2(pu[0], pu[1]), pack_f16x2(pu[2], pu[3])};
      pa_lo = pa_hi;
    } else {
      // P = hi + lo in bf16 (hi = bf16(p), lo = bf16(p - hi); p - hi is exact in fp32)
      typedef __attribute__((ext_vector_type(2))) float f32x2;
      const dkv_bf16x2 h01 = __builtin_convertvector(f32x2{pu[0], pu[1]}, dkv_bf16x2);
      const dkv_bf16x2 h23 = __builtin_convertvector(f32x2{pu[2], pu[3]}, dkv_bf16x2);
      const dkv_bf16x2 l01 = __builtin_convertvector(
          f32x2{pu[0] - (float)h01[0], pu[1] - (float)h01[1]}, dkv_bf16x2);
      const dkv_bf16x2 l23 = __builtin_convertvector(
          f32x2{pu[2] - (float)h23[0], pu[3] - (float)h23[1]}, dkv_bf16x2);
      pa_hi = dkv_u32x2{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
      pa_lo = dkv_u32x2{__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
    }
    // B operand (tokens 4g..4g+3 x rank 16*blk + n) by transposed reads: within each 16-lane
    // group, lane i receives element i%4 of the 8 bytes read by lane 4*u + i/4 of that group,
    // so lane (g, u = n/4, q = n%4) reads ranks 16*blk + 4q .. +3 of token 4g + u. Rank r of
    // token t sits in chunk r/32 at lane slot 16*((r%32)/8) + t, element r%8.
    {
      const int u = n >> 2, q = n & 3;
      const uint8_t* vbase = slot + 4096 + 16 * (16 * (q >> 1) + 4 * g + u) + 8 * (q & 1);
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) {
        const uint8_t* src = vbase + (blk >> 1) * 1024 + (blk & 1) * 512;
        const dkv_u32x2 xb = __builtin_bit_cast(
            dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                           (__attribute__((address_space(3))) dkv_i16x4*)(
                               (__attribute__((address_space(3))) uint8_t*)src)));
        if constexpr (DT == DKV_BF16)
          // hi and lo parts in one 16x16x32 product: k = 8*g + e pairs part e/4 of token
          // 4*g + e%4 (A: this lane's hi then lo values) with that token's coefficients (B: the
          // same four values twice)
          acc[blk] = mfma_k<DT>(
              dkv_u32x4{pa_hi.x, pa_hi.y, pa_lo.x, pa_lo.y},
              __builtin_bit_cast(dkv_u32x4, dkv_u64x2{__builtin_bit_cast(uint64_t, xb),
                                                      __builtin_bit_cast(uint64_t, xb)}),
              acc[blk]);
        else
          acc[blk] = mfma_pv<DT>(pa_hi, xb, acc[blk]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

  // two tiles per loop iteration, so that the gather slot of each is a constant; the
  // scheduling barrier keeps the two tiles from being interleaved, which would double the
  // live registers
  static_assert(NSLOT == 2, "tile j uses gather slot j % 2");
  for (int j = 0; j < n_iter; j += 2) {
    tile(j, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < n_iter) tile(j + 1, 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vm<0>();  // nothing may land in the ring once it is reused below

  // ---- combine the waves through LDS and write the partial record -----------------------
  float l_tot = l_run;
  l_tot += __shfl_xor(l_tot, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  __syncthreads();  // all waves done with their rings
  float* sw = reinterpret_cast<float*>(sRing);  // [WAVES][16 m | 16 l | 16 x 128 acc]
  constexpr int WREC = 32 + 16 * DH;
  static_assert(WAVES * WREC * 4 <= WAVES * NSLOT * GSLOT_BYTES, "epilogue scratch fits");
  static_assert(DH * DH * 2 + 16 * DH * 4 + 3 * 16 * MERGE_WSPLITS * 4 <= WAVES * NSLOT * GSLOT_BYTES,
                "merge scratch fits");
  static_assert(WAVES * 16 == DH, "the merge projection gives each wave 16 output dims");
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
  if (p.n_splits == 1 && p.fused_merge) {
    // the unit's only split merges its waves' partials here: the same weights and sums as
    // its record and the record merge (a single record's weight is 1), without writing the
    // record, counting the arrival and reading the record back
    dkv_u32x4 vbr[VB_CHUNKS];
    load_vbasis(p, kvh, vbr);
    constexpr int NA = 16 * DH / NTHREADS;
    float av[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      const int idx = tid + k * NTHREADS, hs = idx / DH, r = idx % DH;
      float a = 0.f;
      if (hs < p.hpg && r < R) {
        float mw[WAVES], M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
          mw[w] = sw[w * WREC + hs];
          M = fmaxf(M, mw[w]);
        }
        float L = 0.f, X = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
          const float wt = (M == -INFINITY) ? 0.f : exp2f(mw[w] - M);
          L += wt * sw[w * WREC + 16 + hs];
          X += wt * sw[w * WREC + 32 + hs * DH + r];
        }
        const float den = ROUTE == DKV_ROUTE_TWO_STAGE ? fmaxf(L, 1e-6f) : L;
        a = X / den;
      }
      av[k] = a;
    }
    __syncthreads();  // every read of the waves' partials is done: the scratch is reused
    float* sA = reinterpret_cast<float*>(sRing + DH * DH * 2);
#pragma unroll
    for (int k = 0; k < NA; ++k) sA[tid + k * NTHREADS] = av[k];
    if (p.out_f32)
      project_store<DT, DKV_F32>(p, unit, sRing, vbr);
    else
      project_store<DT, DT>(p, unit, sRing, vbr);
    return;
  }
  float* prec = p.partials + ((long long)unit * p.n_splits + split) * p.hpg * PREC;
  for (int idx = tid; idx < p.hpg * PREC; idx += NTHREADS) {
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
    rec_store(prec + hs * PREC + e, e == 0 ? M : v);
  }
  if (!p.fused_merge) return;

  // ---- fused merge: the last split of the unit to finish combines the unit's records -------
  // The records are written with device-coherent stores (rec_store); each wave waits until its
  // stores have completed, then one thread counts the arrival. The last arrival reads the
  // records with device-coherent loads (rec_load) issued after it has seen the count (the
  // splits of a unit may run on different XCDs), and only it loads the V basis.
  __shared__ int sLast;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(p.counters + unit, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    sLast = old == p.n_splits - 1;
  }
  __syncthreads();
  if (!sLast) return;
  merge_unit<DT, ROUTE>(p, unit, sRing);
  if (tid == 0) p.counters[unit] = 0;  // ready for the next call (calls are stream-ordered)
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
  // rounds of 256 workgroups against a workgroup's fixed cost of ~1500 token-equivalents
  // (prologue, record exchange and merge), at least one 16-token tile per wave (a 64-token
  // split leaves half of a workgroup's waves idle: measured on MI355X at batch 1 and 2K tokens,
  // 19.0 against 20.6 us per call). With 8 KV heads at power-of-two batches up to 32 this is one
  // full round (config 3: 128 units -> 2 splits of 4160 tokens). Measured on MI355X (bf16, 8 KV
  // heads, 8K tokens, us per call, the chosen count first): 80 units 56.4 with three splits
  // against 74.3 with two; 96 units 74.5 with two against 98.2 with three (the previous
  // ceil(256 / units) splits); 160 units 103.0 with three against 120.5 with one and 139.9 with
  // two; 288 units 214.5 with two against 251.6 with one; 384 units 233.8 with two against
  // 269.9 with one; 384 and 512 units at 2K tokens best with one.
  const long long units = (long long)B * Hkv;
  long long sl = dkv_rounds_split(units, S, 1500, (long long)WAVES * TILE);
  // up to two tiles per wave, one split per unit: its workgroup merges its waves in LDS, with
  // no record exchange (measured on MI355X: 15.3 against 16.5 us per call at 192 tokens, about
  // even at 256, the exchange ahead from 384)
  if (S <= 2 * WAVES * TILE) sl = ((long long)S + 63) / 64 * 64;
  if (sl < 64) sl = 64;
  if (sl > (1LL << 30)) sl = 1LL << 30;
  return (int)sl;
}

extern "C" long long dkv_splitk_workspace_floats(int B, int Hq, int Hkv, int S, int R,
                                                 int split_len) {
  (void)R;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0) return 0;
  if (split_len <= 0) split_len = dkv_splitk_choose_split(B, Hkv, S);
  const long long n_splits = (S + split_len - 1) / split_len;
  const long long units = (long long)B * Hkv;
  return MERGE_COUNTERS + units * n_splits * (Hq / Hkv) * PREC;
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

// launch timing hooks (dkv_profile_begin / dkv_profile_end)
struct ProfileState {
  bool on = false;
  int cap = 0, n = 0;
  hipEvent_t* ev = nullptr;  // 3 per recorded call
  bool* merged = nullptr;    // per recorded call: a separate merge kernel ran (events 1..2)
};
static ProfileState g_prof;

template <int DT, int RT>
static void launch_splitk_t(const SplitParams& p, int out_dtype, dim3 grid, dim3 mgrid,
                            hipStream_t st) {
  const int slot = (g_prof.on && g_prof.n < g_prof.cap) ? g_prof.n++ : -1;
  hipEvent_t* ev = slot >= 0 ? g_prof.ev + 3 * slot : nullptr;
  if (ev) (void)hipEventRecord(ev[0], st);
  // tile pairs for splits of at least 2 * WAVES tiles (up to 8 heads per unit: with 16 the
  // pair's query operand of hi and lo rows would add spills)
  const bool pair = p.split_len >= 2 * WAVES * TILE;
  if (p.hpg > 8)
    hipLaunchKernelGGL((splitk_kernel<DT, RT, 16, false>), grid, dim3(NTHREADS), 0, st, p);
  else if (p.hpg > 4 && pair)
    hipLaunchKernelGGL((splitk_kernel<DT, RT, 8, true>), grid, dim3(NTHREADS), 0, st, p);
  else if (p.hpg > 4)
    hipLaunchKernelGGL((splitk_kernel<DT, RT, 8, false>), grid, dim3(NTHREADS), 0, st, p);
  else if (pair)
    hipLaunchKernelGGL((splitk_kernel<DT, RT, 4, true>), grid, dim3(NTHREADS), 0, st, p);
  else
    hipLaunchKernelGGL((splitk_kernel<DT, RT, 4, false>), grid, dim3(NTHREADS), 0, st, p);
  if (ev) (void)hipEventRecord(ev[1], st);
  if (!p.fused_merge) {
    if (out_dtype == DKV_F32)
      hipLaunchKernelGGL((merge_kernel<DT, RT, DKV_F32>), mgrid, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((merge_kernel<DT, RT, DT>), mgrid, dim3(256), 0, st, p);
    if (ev) (void)hipEventRecord(ev[2], st);
  }
  if (slot >= 0) g_prof.merged[slot] = !p.fused_merge;
}

static void profile_release() {
  for (int i = 0; i < 3 * g_prof.cap; ++i) (void)hipEventDestroy(g_prof.ev[i]);
  delete[] g_prof.ev;
  delete[] g_prof.merged;
  g_prof = ProfileState{};
}

extern "C" int dkv_profile_begin(int max_calls) {
  if (max_calls <= 0 || max_calls > (1 << 20)) return DKV_E_ARG;
  if (g_prof.ev) profile_release();
  g_prof.ev = new hipEvent_t[3 * (size_t)max_calls];
  g_prof.merged = new bool[(size_t)max_calls]();
  for (int i = 0; i < 3 * max_calls; ++i) {
    const hipError_t e = hipEventCreate(&g_prof.ev[i]);
    if (e != hipSuccess) {
      g_prof.cap = i;
      profile_release();
      return -(1000 + (int)e);
    }
  }
  g_prof.cap = max_calls;
  g_prof.n = 0;
  g_prof.on = true;
  return DKV_OK;
}

extern "C" int dkv_profile_end(double* split_ms, double* merge_ms, int* calls) {
  if (!split_ms || !merge_ms || !calls) return DKV_E_ARG;
  *split_ms = *merge_ms = 0.0;
  *calls = 0;
  if (!g_prof.ev) return DKV_E_ARG;
  int rc = DKV_OK;
  for (int i = 0; i < g_prof.n && rc == DKV_OK; ++i) {
    hipEvent_t* e = g_prof.ev + 3 * i;
    float a = 0.f, m = 0.f;
    hipError_t err = hipEventSynchronize(g_prof.merged[i] ? e[2] : e[1]);
    if (err == hipSuccess) err = hipEventElapsedTime(&a, e[0], e[1]);
    if (err == hipSuccess && g_prof.merged[i]) err = hipEventElapsedTime(&m, e[1], e[2]);
    if (err != hipSuccess) rc = -(1000 + (int)err);
    *split_ms += a;
    *merge_ms += m;
  }
  *calls = g_prof.n;
  profile_release();
  return rc;
}

// Argument checks shared by both entry points; 0 when the call is valid, or a status.
// On success *n_floats receives the workspace size the call needs (0 when nothing is launched).
static int splitk_check(int route, int dtype, const void* q, const void* k_basis,
                        long long k_unit_stride, long long k_basis_sr, const void* v_basis,
                        long long v_unit_stride, long long v_basis_sr, const void* k_flat,
                        long long k_ld, const void* v_flat, long long v_ld, const int* lens_k,
                        const int* offs_k, long long tk_ss, const int* lens_v,
                        const int* offs_v, long long tv_ss, const float* rope, int rope_tiles,
                        const void* out, int out_dtype, int B, int Hq, int Hkv, int G, int S,
                        int R, int Dh, int* split_len, long long* n_floats) {
  *n_floats = 0;
  if (route != DKV_ROUTE_FUSED && route != DKV_ROUTE_TWO_STAGE) return DKV_E_ARG;
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (out_dtype != dtype && out_dtype != DKV_F32) return DKV_E_ARG;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || G <= 0 || S < 0 || R <= 0) return DKV_E_ARG;
  if (Hq % Hkv != 0 || Hkv % G != 0) return DKV_E_ARG;
  if (Dh != DH || R > DH || Hq / Hkv > 16) return DKV_E_UNSUPPORTED;
  if (B == 0) return DKV_OK;
  if (S == 0) return DKV_E_UNSUPPORTED;  // empty cache: the vector path defines the result
  if (!q || !k_basis || !v_basis || !k_flat || !v_flat || !lens_k || !offs_k || !lens_v ||
      !offs_v || !rope || !out)
    return DKV_E_ARG;
  // 16-byte aligned K basis rows for the vector LDS staging
  if (((uintptr_t)k_basis & 15) || (k_basis_sr & 7) || (k_unit_stride & 7))
    return DKV_E_UNSUPPORTED;
  // 16-byte aligned V basis rows for the vector loads of the fused merge
  if (((uintptr_t)v_basis & 15) || (v_basis_sr & 7) || (v_unit_stride & 7))
    return DKV_E_UNSUPPORTED;
  if (k_ld <= 0 || v_ld <= 0) return DKV_E_ARG;
  // buffer offsets are 32-bit byte offsets from the start of a row
  const long long rows = (long long)B * G;
  if (k_ld > FLAT_LD_MAX || v_ld > FLAT_LD_MAX || rows > 0x7fffffffLL) return DKV_E_UNSUPPORTED;
  if (rope_tiles < (S + TILE - 1) / TILE) return DKV_E_ARG;
  if (*split_len <= 0) *split_len = dkv_splitk_choose_split(B, Hkv, S);
  if (*split_len % 64 != 0) return DKV_E_ARG;
  // token indices times table strides stay 32-bit inside the kernel, both factors 24-bit
  if ((long long)S * tk_ss >= (1LL << 31) || (long long)S * tv_ss >= (1LL << 31) || tk_ss < 0 ||
      tv_ss < 0 || S >= (1 << 24) || tk_ss >= (1 << 24) || tv_ss >= (1 << 24))
    return DKV_E_UNSUPPORTED;
  const long long n_splits = ((long long)S + *split_len - 1) / *split_len;
  const long long units = (long long)B * Hkv;
  if (units * n_splits > 0x7fffffffLL) return DKV_E_UNSUPPORTED;
  *n_floats = dkv_splitk_workspace_floats(B, Hq, Hkv, S, R, *split_len);
  return DKV_OK;
}

// Launch the split kernel (and the merge kernel when one is needed) of a call that passed
// splitk_check, with `workspace` holding at least the floats splitk_check asked for.
static int splitk_launch(void* stream, int route, int dtype, const void* q, long long q_sb,
                         long long q_sh, const void* k_basis, long long k_unit_stride,
                         long long k_basis_sr, const void* v_basis, long long v_unit_stride,
                         long long v_basis_sr, const void* k_flat, long long k_ld,
                         const void* v_flat, long long v_ld, const int* lens_k,
                         const int* offs_k, long long tk_sb, long long tk_ss,
                         const int* lens_v, const int* offs_v, long long tv_sb, long long tv_ss,
                         const float* rope, float* workspace, void* out, long long out_sb,
                         long long out_sh, int out_dtype, int B, int Hq, int Hkv, int G, int S,
                         int R, int Dh, int split_len) {
  const long long rows = (long long)B * G;
  const long long n_splits = ((long long)S + split_len - 1) / split_len;
  const long long units = (long long)B * Hkv;
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
  p.rows = (int)rows;
  p.lens_k = lens_k;
  p.offs_k = offs_k;
  p.tk_sb = tk_sb;
  p.tk_ss = tk_ss;
  p.lens_v = lens_v;
  p.offs_v = offs_v;
  p.tv_sb = tv_sb;
  p.tv_ss = tv_ss;
  p.rope = rope;
  // workspace: MERGE_COUNTERS ints (zero between calls), then the split records
  p.counters = reinterpret_cast<int*>(workspace);
  p.partials = workspace + MERGE_COUNTERS;
  p.fused_merge = units <= MERGE_COUNTERS ? 1 : 0;
  p.out_f32 = out_dtype == DKV_F32 ? 1 : 0;
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
  p.minus_one = -1.0f;
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
  long long need = 0;
  const int rc = splitk_check(route, dtype, q, k_basis, k_unit_stride, k_basis_sr, v_basis,
                              v_unit_stride, v_basis_sr, k_flat, k_ld, v_flat, v_ld, lens_k,
                              offs_k, tk_ss, lens_v, offs_v, tv_ss, rope, rope_tiles, out,
                              out_dtype, B, Hq, Hkv, G, S, R, Dh, &split_len, &need);
  if (rc != DKV_OK || need == 0) return rc;
  if (!workspace) return DKV_E_ARG;
  if (workspace_floats < need) return DKV_E_WORKSPACE;
  return splitk_launch(stream, route, dtype, q, q_sb, q_sh, k_basis, k_unit_stride, k_basis_sr,
                       v_basis, v_unit_stride, v_basis_sr, k_flat, k_ld, v_flat, v_ld, lens_k,
                       offs_k, tk_sb, tk_ss, lens_v, offs_v, tv_sb, tv_ss, rope, workspace, out,
                       out_sb, out_sh, out_dtype, B, Hq, Hkv, G, S, R, Dh, split_len);
}

// ---------------------------------------------------------------------------------------
// The entry point that allocates nothing: the split workspace lives in a fixed device array.
// ---------------------------------------------------------------------------------------
// One copy per GPU (each device that loads the code object gets its own, at its own address),
// held until the process ends. Host code never passes `scratch` itself to a kernel: on the host
// the name only stands in for the symbol; the device address comes from hipGetSymbolAddress.
__device__ __align__(256) float scratch[DKV_NOALLOC_SCRATCH_FLOATS];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[MAX_DEVICES] = {};

__global__ __launch_bounds__(256) void zero_ints_kernel(int* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Device address of this GPU's scratch array (the device of `stream`, or the current device for
// the null stream). The first call on a device looks the address up with that device current
// and zeroes the arrival counters with a fill kernel on `stream`; later calls reuse the address.
int noalloc_scratch(hipStream_t stream, float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(DKV_E_HIP_BASE + (int)e);
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return -(DKV_E_HIP_BASE + (int)e);
    if (sdev != dev) return DKV_E_ARG;  // the stream must belong to the current device
  }
  if (dev < 0 || dev >= MAX_DEVICES) return DKV_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return -(DKV_E_HIP_BASE + (int)e);
    if (!ptr) return -(DKV_E_HIP_BASE + (int)hipErrorInvalidSymbol);
    hipLaunchKernelGGL(zero_ints_kernel, dim3((MERGE_COUNTERS + 255) / 256), dim3(256), 0,
                       stream, reinterpret_cast<int*>(ptr), MERGE_COUNTERS);
    DKV_HIP_CHECK_LAUNCH();
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return DKV_OK;
}
}  // namespace

extern "C" int dkv_decode_splitk_noalloc(
    void* stream, int route, int dtype, const void* q, long long q_sb, long long q_sh,
    const void* k_basis, long long k_unit_stride, long long k_basis_sr, const void* v_basis,
    long long v_unit_stride, long long v_basis_sr, const void* k_flat, long long k_ld,
    const void* v_flat, long long v_ld, const int* lens_k, const int* offs_k, long long tk_sb,
    long long tk_ss, const int* lens_v, const int* offs_v, long long tv_sb, long long tv_ss,
    const float* rope, int rope_tiles, void* out, long long out_sb, long long out_sh,
    int out_dtype, int B, int Hq, int Hkv, int G, int S, int R, int Dh, int split_len) {
  long long need = 0;
  int rc = splitk_check(route, dtype, q, k_basis, k_unit_stride, k_basis_sr, v_basis,
                        v_unit_stride, v_basis_sr, k_flat, k_ld, v_flat, v_ld, lens_k, offs_k,
                        tk_ss, lens_v, offs_v, tv_ss, rope, rope_tiles, out, out_dtype, B, Hq,
                        Hkv, G, S, R, Dh, &split_len, &need);
  if (rc != DKV_OK || need == 0) return rc;
  if (need > DKV_NOALLOC_SCRATCH_FLOATS) return DKV_E_SCRATCH;
  float* ws = nullptr;
  rc = noalloc_scratch((hipStream_t)stream, &ws);
  if (rc != DKV_OK) return rc;
  return splitk_launch(stream, route, dtype, q, q_sb, q_sh, k_basis, k_unit_stride, k_basis_sr,
                       v_basis, v_unit_stride, v_basis_sr, k_flat, k_ld, v_flat, v_ld, lens_k,
                       offs_k, tk_sb, tk_ss, lens_v, offs_v, tv_sb, tv_ss, rope, ws, out, out_sb,
                       out_sh, out_dtype, B, Hq, Hkv, G, S, R, Dh, split_len);
}

extern "C" int dkv_selftest_layouts(void* stream, int* mismatches) {
  if (!mismatches) return DKV_E_ARG;
  // mismatches must point at >= 64 ints + 1 KiB of scratch (see selftest_kernel)
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, mismatches);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
