// Dense GQA decode attention for gfx950: the uncompressed-cache baseline of the end-to-end
// comparison. The reference's baseline is the unmodified Llama model with transformers' KV cache
// (scripts/benchmark_throughput.py:17-77 runs the compressed and the original model side by
// side); its decode attention reads every cached token's rotated key and value at full head
// width. This kernel does that on the device: no reconstruction, no RoPE (the cache holds
// rotated keys, the query arrives rotated).
//
// Cache layout: row b * Hkv + g of `ld` elements per buffer; token t of a row at elements
// t * 128 .. t * 128 + 127 (K and V in separate buffers, same layout). Work unit = (batch b,
// KV head g) with its hpg query heads; a workgroup (8 waves) owns one unit and one contiguous
// token range (a split, a multiple of 64 tokens); waves take 16-token tiles round-robin.
// Per tile: the K and V tiles (4 KB each, contiguous in memory) land in LDS by direct-to-LDS
// loads, 16-byte pieces XOR-swizzled by token; scores S^T = K Q^T on 16x16x32 MFMA (the query
// heads in the operand's columns, exact 16-bit products, fp32 accumulation); online softmax in
// the log2 domain; P.V on MFMA with P as hi + lo parts (bf16) or fp16, V read transposed from
// LDS. Each split writes (m, l, acc[128]) per head; the last split of a unit to arrive merges
// the records by LSE and stores the output (fused-route semantics: fp32 scores, den = l).
#include "dkv_common.h"
#include "dkv_mfma_ops.h"

namespace {

constexpr int DH = 128;
constexpr int TILE = 16;
constexpr int DW = 8;                   // waves per workgroup (two per SIMD)
constexpr int DT_THREADS = DW * 64;
constexpr int DSLOT = 2;                // tile slots per wave: the current tile + one in flight
constexpr int TILE_BYTES = TILE * DH * 2;  // 4 KB of K or of V
constexpr int SLOT_BYTES = 2 * TILE_BYTES;
constexpr int DPREC = DH + 2;           // floats per record: m, l, acc[128]
constexpr int D_COUNTERS = 16384;       // leading workspace ints: per-unit arrival counters
constexpr float LOG2E_F = 1.4426950408889634f;
constexpr float D_RESCALE = 11.5f;      // log2 units

struct DenseParams {
  const uint16_t* q;
  long long q_sb, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  long long ld;
  float* partials;  // [unit][split][hpg][DPREC]
  int* counters;    // [unit] (zero between calls)
  int fused_merge;
  int out_f32;
  void* out;
  long long out_sb, out_sh;
  int B, Hq, Hkv, S, hpg, n_splits, split_len;
  float scale_log2;  // softmax scale * log2(e)
};

// 16 bytes at byte offset `off` of a buffer resource into LDS at M0 + 16 * lane (inline assembly
// so that the compiler neither reorders LDS accesses around it nor drains the load queue before
// later LDS reads; the kernel waits for these loads itself).
__device__ __forceinline__ void d_lds_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base,
                                             uint32_t off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(lds_base), "v"(off), "s"(rsrc)
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void d_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ float d_rec_load(const float* a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void d_rec_store(float* a, float v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT>
__device__ __forceinline__ dkv_f32x4 d_mfma_pv16(const dkv_u32x2& a, const dkv_u32x2& b,
                                                 dkv_f32x4 c) {
  if constexpr (DT == DKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(dkv_bf16x4, a),
                                                     __builtin_bit_cast(dkv_bf16x4, b), c, 0, 0,
                                                     0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(dkv_f16x4, a),
                                                 __builtin_bit_cast(dkv_f16x4, b), c, 0, 0, 0);
}

template <int DT>
__global__ __launch_bounds__(DT_THREADS, 1) void dense_decode_kernel(DenseParams p) {
  // per wave: DSLOT slots of [K tile | V tile]; piece (token t, 16-byte piece c) of a tile at
  // byte 256 t + 16 (c ^ t)
  __shared__ __attribute__((aligned(256))) uint8_t sRing[DW * DSLOT * SLOT_BYTES];
  __shared__ int sLast;

  const int nunits = p.B * p.Hkv;
  int unit, split;
  {
    // all splits of a unit on one XCD (id % 8), as the compressed split kernel maps them
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
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int s_begin = split * p.split_len;
  const int s_end = min(p.S, s_begin + p.split_len);
  const int tile_first = s_begin / TILE;
  const int n_tiles = (s_end - s_begin + TILE - 1) / TILE;
  const int n_iter = max(0, (n_tiles - wave + DW - 1) / DW);
  auto tix = [&](int j) { return tile_first + wave + DW * j; };

  // the unit's rows; tokens at or past S read as zero (the resource ends at token S)
  const uint32_t row_bytes = (uint32_t)p.S * DH * 2u;
  const __amdgpu_buffer_rsrc_t rk = dkv_make_rsrc(p.k + (long long)unit * p.ld, row_bytes);
  const __amdgpu_buffer_rsrc_t rv = dkv_make_rsrc(p.v + (long long)unit * p.ld, row_bytes);
  uint8_t* ring = sRing + wave * DSLOT * SLOT_BYTES;
  // this lane's piece of each of the four 1 KB direct-to-LDS loads of a tile: token
  // t = 4 * i + lane / 16 and LDS piece lane % 16, which holds memory piece (lane % 16) ^ t
  uint32_t piece_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * i + (lane >> 4);
    piece_off[i] = (uint32_t)(t * 256 + 16 * ((lane & 15) ^ t));
  }
  auto issue = [&](int j) {
    const uint32_t slot = dkv_lds_addr(ring + (j % DSLOT) * SLOT_BYTES);
    const uint32_t base = (uint32_t)tix(j) * (TILE * DH * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) d_lds_load16(rk, slot + 1024 * i, base + piece_off[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) d_lds_load16(rv, slot + TILE_BYTES + 1024 * i, base + piece_off[i]);
  };
  issue(0);

  // query operand: column n = head n (heads past hpg zero), rows k = dims 32c + 8g .. +8
  dkv_u32x4 bq[4];
  {
    const bool has = n < p.hpg;
    const uint16_t* qr = p.q + (long long)b * p.q_sb + (long long)(kvh * p.hpg + (has ? n : 0)) * p.q_sh;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const dkv_u32x4 v = *(const dkv_u32x4*)(qr + 32 * c + 8 * g);
      bq[c] = has ? v : dkv_u32x4{0u, 0u, 0u, 0u};
    }
    // settled here (the compiler's wait for these loads falls before the loop, together with
    // tile 0's, instead of inside it, where its count would also drain the tile in flight)
#pragma unroll
    for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(bq[c]));
  }

  dkv_f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -1.0e30f;  // log2 units; a finite floor (see the compressed split kernel)
  float l_run = 0.f;

  for (int j = 0; j < n_iter; ++j) {
    d_wait_vm<0>();  // tile j
    issue(j + 1);    // the next tile (past the split: zeros or real rows, never used)
    const uint8_t* slot = ring + (j % DSLOT) * SLOT_BYTES;
    // K operand: token n, dims 32c + 8g .. +8 = piece 4c + g
    dkv_u32x4 xk[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      xk[c] = *(const dkv_u32x4*)(slot + n * 256 + 16 * ((4 * c + g) ^ n));
    dkv_f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) sc = dkv_mfma32<DT>(xk[c], bq[c], sc);
    // lane (head n, tokens 4g + u): scores in log2 units, tokens past the split excluded
    const int nvalid = s_end - tix(j) * TILE;
    float z[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) z[u] = 4 * g + u < nvalid ? sc[u] * p.scale_log2 : -INFINITY;
    float tmax = dkv_max3(dkv_max3(z[0], z[1], z[2]), z[3], z[3]);
    tmax = dkv_lane_max32(tmax);
    tmax = dkv_lane_max16(tmax);
    if (__ballot(tmax > m_run + D_RESCALE)) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
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
      pu[u] = __builtin_amdgcn_exp2f(z[u] - m_run);
      l_run += pu[u];
    }
    // P.V: A = P (row = head n, k = tokens), B = V (k = tokens 4g .. 4g + 3, column = dim
    // 16 blk + n) read transposed: lane (n, g) reads 8 bytes of token 4g + n / 4 at dims
    // 16 blk + 4 (n % 4) and receives the four tokens of dim 16 blk + n
    const uint8_t* vt = slot + TILE_BYTES;
    const int vtok = 4 * g + (n >> 2);
    if constexpr (DT == DKV_BF16) {
      typedef __attribute__((ext_vector_type(2))) float f32x2;
      const dkv_bf16x2 h01 = __builtin_convertvector(f32x2{pu[0], pu[1]}, dkv_bf16x2);
      const dkv_bf16x2 h23 = __builtin_convertvector(f32x2{pu[2], pu[3]}, dkv_bf16x2);
      const dkv_bf16x2 l01 = __builtin_convertvector(
          f32x2{pu[0] - (float)h01[0], pu[1] - (float)h01[1]}, dkv_bf16x2);
      const dkv_bf16x2 l23 = __builtin_convertvector(
          f32x2{pu[2] - (float)h23[0], pu[3] - (float)h23[1]}, dkv_bf16x2);
      const dkv_u32x4 pa = dkv_u32x4{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23),
                                     __builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) {
        const int dd = 16 * blk + 4 * (n & 3);  // first dim of this lane's 8 bytes
        const uint8_t* src = vt + vtok * 256 + 16 * (((dd >> 3)) ^ vtok) + 2 * (dd & 7);
        const dkv_u32x2 xb = __builtin_bit_cast(
            dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                           (__attribute__((address_space(3))) dkv_i16x4*)(
                               (__attribute__((address_space(3))) uint8_t*)src)));
        // k = 8g + e: part e / 4 (hi, lo) of token 4g + e % 4 against that token's value twice
        acc[blk] = dkv_mfma32<DT>(
            pa, __builtin_bit_cast(dkv_u32x4, dkv_u64x2{__builtin_bit_cast(uint64_t, xb),
                                                        __builtin_bit_cast(uint64_t, xb)}),
            acc[blk]);
      }
    } else {
      const dkv_u32x2 pa = dkv_u32x2{dkv_pack_f16x2(pu[0], pu[1]), dkv_pack_f16x2(pu[2], pu[3])};
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) {
        const int dd = 16 * blk + 4 * (n & 3);
        const uint8_t* src = vt + vtok * 256 + 16 * (((dd >> 3)) ^ vtok) + 2 * (dd & 7);
        const dkv_u32x2 xb = __builtin_bit_cast(
            dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                           (__attribute__((address_space(3))) dkv_i16x4*)(
                               (__attribute__((address_space(3))) uint8_t*)src)));
        acc[blk] = d_mfma_pv16<DT>(pa, xb, acc[blk]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  d_wait_vm<0>();  // nothing lands in the ring once it is reused below

  // ---- combine the waves through LDS into this split's record ----
  float l_tot = l_run;
  l_tot += __shfl_xor(l_tot, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  __syncthreads();
  float* sw = reinterpret_cast<float*>(sRing);  // [DW][16 m | 16 l | 16 x 128 acc]
  constexpr int WREC = 32 + 16 * DH;
  static_assert(DW * WREC * 4 <= DW * DSLOT * SLOT_BYTES, "epilogue scratch fits the ring");
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
  float* prec = p.partials + ((long long)unit * p.n_splits + split) * p.hpg * DPREC;
  for (int idx = tid; idx < p.hpg * DPREC; idx += DT_THREADS) {
    const int hs = idx / DPREC, e = idx % DPREC;
    float mw[DW], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < DW; ++w) {
      mw[w] = sw[w * WREC + hs];
      M = fmaxf(M, mw[w]);
    }
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < DW; ++w) {
      const float wt = (M == -INFINITY) ? 0.f : exp2f(mw[w] - M);
      const float x = e == 1 ? sw[w * WREC + 16 + hs] : (e >= 2 ? sw[w * WREC + 32 + hs * DH + (e - 2)] : 0.f);
      v += wt * x;
    }
    d_rec_store(prec + hs * DPREC + e, e == 0 ? M : v);
  }
  if (!p.fused_merge) return;

  // ---- the unit's last split to arrive merges the records (see the compressed kernel) ----
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(p.counters + unit, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    sLast = old == p.n_splits - 1;
  }
  __syncthreads();
  if (!sLast) return;
  const long long stride = (long long)p.hpg * DPREC;
  const float* base = p.partials + (long long)unit * p.n_splits * stride;
  for (int idx = tid; idx < p.hpg * DH; idx += DT_THREADS) {
    const int hs = idx / DH, d = idx % DH;
    float M = -INFINITY, L = 0.f, A = 0.f;
    for (int sp0 = 0; sp0 < p.n_splits; sp0 += 8) {
      float mb[8], lb[8], xb[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sp = min(sp0 + u, p.n_splits - 1);
        const float* rec = base + sp * stride + hs * DPREC;
        mb[u] = d_rec_load(rec);
        lb[u] = d_rec_load(rec + 1);
        xb[u] = d_rec_load(rec + 2 + d);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
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
    const float o = A / L;
    const long long oi = (long long)b * p.out_sb + (long long)(kvh * p.hpg + hs) * p.out_sh + d;
    if (p.out_f32)
      dkv_store_f32<DKV_F32>(p.out, oi, o);
    else
      dkv_store_f32<DT>(p.out, oi, o);
  }
  if (tid == 0) p.counters[unit] = 0;
}

// One workgroup per (unit, head): the LSE merge when a call has more units than counters.
template <int DT>
__global__ __launch_bounds__(128) void dense_merge_kernel(DenseParams p) {
  const int unit = blockIdx.x / p.hpg, hs = blockIdx.x % p.hpg;
  const int b = unit / p.Hkv, kvh = unit % p.Hkv;
  const int d = threadIdx.x;
  const long long stride = (long long)p.hpg * DPREC;
  const float* base = p.partials + (long long)unit * p.n_splits * stride + (long long)hs * DPREC;
  float M = -INFINITY, L = 0.f, A = 0.f;
  for (int sp = 0; sp < p.n_splits; ++sp) {
    const float* rec = base + sp * stride;
    const float m = rec[0];
    const float Mn = fmaxf(M, m);
    const float so = M == -INFINITY ? 0.f : exp2f(M - Mn);
    const float sn = m == -INFINITY ? 0.f : exp2f(m - Mn);
    L = L * so + rec[1] * sn;
    A = A * so + rec[2 + d] * sn;
    M = Mn;
  }
  const long long oi = (long long)b * p.out_sb + (long long)(kvh * p.hpg + hs) * p.out_sh + d;
  if (p.out_f32)
    dkv_store_f32<DKV_F32>(p.out, oi, A / L);
  else
    dkv_store_f32<DT>(p.out, oi, A / L);
}

// One decode step's cache write for the dense baseline, from the fused q/k/v projection row of
// each batch element (Hq query heads, then Hkv key heads, then Hkv value heads, 128 each): the
// query heads rotated in place at position q_pos, the key heads rotated at position k_pos into
// k_cache row b * Hkv + g at token k_pos, the value heads copied into v_cache likewise. One thread
// per rotate-half pair (i, i + 64) of a head, the rotation of dkv_rope_pair (fp32 angle and
// rotation, rounded once to the dtype).
template <int DT>
__global__ __launch_bounds__(256) void dense_append_kernel(uint16_t* __restrict__ y,
                                                           long long y_ld,
                                                           uint16_t* __restrict__ kc,
                                                           uint16_t* __restrict__ vc,
                                                           long long kv_ld, int q_pos, int k_pos,
                                                           int B, int Hq, int Hkv,
                                                           float log_theta) {
  const int heads = Hq + 2 * Hkv;
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)B * heads * 64) return;
  const int i = (int)(idx & 63);
  const long long bh = idx >> 6;
  const int b = (int)(bh / heads), h = (int)(bh % heads);
  uint16_t* src = y + (long long)b * y_ld + (long long)h * DH;
  if (h < Hq) {
    dkv_rope_pair<DT>(src, i, q_pos, log_theta);
    return;
  }
  const bool is_k = h < Hq + Hkv;
  const int g = is_k ? h - Hq : h - Hq - Hkv;
  uint16_t* dst = (is_k ? kc : vc) + ((long long)b * Hkv + g) * kv_ld + (long long)k_pos * DH;
  if (is_k) {
    const float inv = dkv_inv_freq(i, DH, log_theta);
    const float ang = (float)k_pos * inv;
    const float c = cosf(ang), sn = sinf(ang);
    const float a = dkv_load_f32<DT>(src, i), bb = dkv_load_f32<DT>(src, i + 64);
    dkv_store_f32<DT>(dst, i, a * c - bb * sn);
    dkv_store_f32<DT>(dst, i + 64, bb * c + a * sn);
  } else {
    dst[i] = src[i];
    dst[i + 64] = src[i + 64];
  }
}

}  // namespace

extern "C" int dkv_dense_append(void* stream, int dtype, void* y, long long y_ld, void* k_cache,
                                void* v_cache, long long kv_ld, int q_pos, int k_pos, int B,
                                int Hq, int Hkv, float log_theta) {
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || q_pos < 0 || k_pos < 0) return DKV_E_ARG;
  if (B == 0) return DKV_OK;
  if (!y || !k_cache || !v_cache) return DKV_E_ARG;
  if (y_ld < (long long)(Hq + 2 * Hkv) * DH || kv_ld < (long long)(k_pos + 1) * DH)
    return DKV_E_ARG;
  const long long total = (long long)B * (Hq + 2 * Hkv) * 64;
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DKV_BF16)
    hipLaunchKernelGGL(dense_append_kernel<DKV_BF16>, grid, dim3(256), 0, st, (uint16_t*)y, y_ld,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, kv_ld, q_pos, k_pos, B, Hq, Hkv,
                       log_theta);
  else
    hipLaunchKernelGGL(dense_append_kernel<DKV_F16>, grid, dim3(256), 0, st, (uint16_t*)y, y_ld,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, kv_ld, q_pos, k_pos, B, Hq, Hkv,
                       log_theta);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_dense_choose_split(int B, int Hkv, int S) {
  if (B <= 0 || Hkv <= 0 || S <= 0) return 128;
  // rounds of 256 workgroups (one per CU) against a workgroup's fixed cost of ~3000
  // token-equivalents, at least one tile per wave (128 tokens) unless the cache is shorter.
  // Measured on MI355X (bf16, 8 KV heads, 8K tokens, us per call, the chosen count first): 48
  // units 32.8 with five splits against 41.3 with six (the previous ceil(256 / units)); 96
  // units 71.4 with two against 90.8 with three; 160 units 115.5 with one against 118.9 with
  // three and 138.3 with two; 192 units 141.7 with one against 151.3 with two.
  const long long units = (long long)B * Hkv;
  long long sl = dkv_rounds_split(units, S, 3000, (long long)DW * TILE);
  if (sl > (1LL << 30)) sl = 1LL << 30;
  return (int)sl;
}

extern "C" long long dkv_dense_workspace_floats(int B, int Hq, int Hkv, int S, int split_len) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0) return 0;
  if (split_len <= 0) split_len = dkv_dense_choose_split(B, Hkv, S);
  const long long n_splits = (S + split_len - 1) / split_len;
  return D_COUNTERS + (long long)B * Hkv * n_splits * (Hq / Hkv) * DPREC;
}

extern "C" int dkv_decode_dense(void* stream, int dtype, const void* q, long long q_sb,
                                long long q_sh, const void* k, const void* v, long long kv_ld,
                                int S, float* workspace, long long workspace_floats, void* out,
                                long long out_sb, long long out_sh, int out_dtype, int B, int Hq,
                                int Hkv, int Dh, int split_len) {
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (out_dtype != dtype && out_dtype != DKV_F32) return DKV_E_ARG;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || S < 0 || Hq % Hkv != 0) return DKV_E_ARG;
  if (Dh != DH || Hq / Hkv > 16) return DKV_E_UNSUPPORTED;
  if (B == 0) return DKV_OK;
  if (S == 0) return DKV_E_UNSUPPORTED;  // nothing to attend
  if (!q || !k || !v || !out || !workspace) return DKV_E_ARG;
  // 16-byte aligned query rows and cache rows; every byte offset into a row fits 32 bits
  if (((uintptr_t)q & 15) || (q_sb & 7) || (q_sh & 7) || ((uintptr_t)k & 15) ||
      ((uintptr_t)v & 15) || (kv_ld & 7))
    return DKV_E_UNSUPPORTED;
  if (kv_ld < (long long)S * DH) return DKV_E_ARG;
  if ((long long)S * DH * 2 + TILE * DH * 2 * (DSLOT + DW) >= 0x7fffffffLL) return DKV_E_UNSUPPORTED;
  if (split_len <= 0) split_len = dkv_dense_choose_split(B, Hkv, S);
  if (split_len % 64 != 0) return DKV_E_ARG;
  const long long n_splits = ((long long)S + split_len - 1) / split_len;
  const long long units = (long long)B * Hkv;
  if (units * n_splits > 0x7fffffffLL) return DKV_E_UNSUPPORTED;
  if (workspace_floats < dkv_dense_workspace_floats(B, Hq, Hkv, S, split_len)) return DKV_E_WORKSPACE;
  DenseParams p;
  p.q = (const uint16_t*)q;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.ld = kv_ld;
  p.counters = reinterpret_cast<int*>(workspace);
  p.partials = workspace + D_COUNTERS;
  p.fused_merge = units <= D_COUNTERS ? 1 : 0;
  p.out_f32 = out_dtype == DKV_F32 ? 1 : 0;
  p.out = out;
  p.out_sb = out_sb;
  p.out_sh = out_sh;
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.S = S;
  p.hpg = Hq / Hkv;
  p.n_splits = (int)n_splits;
  p.split_len = split_len;
  p.scale_log2 = (1.0f / sqrtf((float)Dh)) * LOG2E_F;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)(units * n_splits));
  if (dtype == DKV_BF16)
    hipLaunchKernelGGL(dense_decode_kernel<DKV_BF16>, grid, dim3(DT_THREADS), 0, st, p);
  else
    hipLaunchKernelGGL(dense_decode_kernel<DKV_F16>, grid, dim3(DT_THREADS), 0, st, p);
  DKV_HIP_CHECK_LAUNCH();
  if (!p.fused_merge) {
    const dim3 mgrid((unsigned)(units * p.hpg));
    if (dtype == DKV_BF16)
      hipLaunchKernelGGL(dense_merge_kernel<DKV_BF16>, mgrid, dim3(DH), 0, st, p);
    else
      hipLaunchKernelGGL(dense_merge_kernel<DKV_F16>, mgrid, dim3(DH), 0, st, p);
    DKV_HIP_CHECK_LAUNCH();
  }
  return DKV_OK;
}
