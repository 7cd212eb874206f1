// Prefill attention over the reconstructed cache.
//
// Reference behaviour: the prefill branch of CustomAttention.forward
// (src/dynakv/kernels/compressed_attention.py:359-386) packs the prompt's coefficients into the
// cache (update_sp), re-expands the whole cache (get_origin_states, compressed_cache.py:70-81),
// projects it through k_up / v_up (:160-165), applies RoPE at positions 0..S-1 to K
// (calc_cos_sin, :193-200, then apply_rotary_pos_emb_) and runs causal attention of the
// prompt's (RoPE'd) queries over it (eager / SDPA, :373-383).
//
// Here: dkv_rope_dense rotates dense K in place (rotate-half RoPE, fp32 angles
// float(pos) * inv_freq as the decode kernels form them, result rounded to the cache dtype);
// dkv_prefill_attention is a causal GQA flash-attention forward on MFMA:
//   one workgroup = 128 queries of one query head (4 waves x 2 blocks of 16 queries, so every
//   K and V operand read from LDS serves two products), the work items handed out longest
//   first and evenly over the 8 XCDs, a KV head's query heads on one XCD (the grid's own
//   order gave XCD k only the query blocks k, k+8, ...: 0.40 ms against 0.25 at B=4,
//   S=2048); key tiles of 64
//   are staged in LDS (double-buffered, direct-to-LDS loads, 16-byte chunks XOR-swizzled by
//   key so that both the row reads of K and the transposed reads of V avoid bank conflicts);
//   S^T = K Q^T on 16x16x32 MFMA (each lane then holds one query's scores for 16 keys), online
//   softmax in fp32 with lane maxima by permlane swaps (the running maximum raised only when a
//   tile's exceeds it by more than 2^8, so most tiles skip the rescale), P kept as a bf16/fp16
//   hi + lo pair and
//   P.V on 16x16x32 MFMA with both parts in the k dimension (V read transposed from LDS).
#include "dkv_common.h"

namespace {

constexpr int FA_DH = 128;
constexpr int FA_QB = 2;      // 16-query blocks per wave
constexpr int FA_QW = 16 * FA_QB;  // queries per wave
constexpr int FA_BQ = 4 * FA_QW;   // queries per workgroup (4 waves)
constexpr float FA_RESCALE = 8.f;  // log2 units a tile's maximum may exceed the running one
constexpr int FA_BK = 64;     // keys per tile
constexpr int FA_TILE_BYTES = FA_BK * FA_DH * 2;  // 16 KB

struct PrefillParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  void* out;
  long long q_sb, q_sh, q_ss;
  long long k_sb, k_sh, k_ss;
  long long v_sb, v_sh, v_ss;
  long long o_sb, o_sh, o_ss;
  int B, Hq, Hkv, Sq, Sk, q_offset, causal;
  float scale_log2;  // softmax scale * log2(e)
  uint32_t k_bytes, v_bytes;
  const int* kstart;  // per batch row: keys before it are masked (left padding); may be null
};

template <int DT>
__device__ __forceinline__ dkv_f32x4 mfma32(const dkv_u32x4& a, const dkv_u32x4& b, dkv_f32x4 c) {
  if constexpr (DT == DKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dkv_bf16x8, a),
                                                   __builtin_bit_cast(dkv_bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dkv_f16x8, a),
                                                  __builtin_bit_cast(dkv_f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ void fa_lds_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base,
                                              uint32_t byte_off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(lds_base), "v"(byte_off), "s"(rsrc)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t fa_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

__device__ __forceinline__ float fa_max(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// max over the four lanes n, n+16, n+32, n+48
__device__ __forceinline__ float fa_max4(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fa_max(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fa_max(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <int DT>
__device__ __forceinline__ void split_hi_lo(const float (&p)[4], dkv_u32x2& hi, dkv_u32x2& lo) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  if constexpr (DT == DKV_BF16) {
    const dkv_bf16x2 h01 = __builtin_convertvector(f32x2{p[0], p[1]}, dkv_bf16x2);
    const dkv_bf16x2 h23 = __builtin_convertvector(f32x2{p[2], p[3]}, dkv_bf16x2);
    const dkv_bf16x2 l01 =
        __builtin_convertvector(f32x2{p[0] - (float)h01[0], p[1] - (float)h01[1]}, dkv_bf16x2);
    const dkv_bf16x2 l23 =
        __builtin_convertvector(f32x2{p[2] - (float)h23[0], p[3] - (float)h23[1]}, dkv_bf16x2);
    hi = dkv_u32x2{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
    lo = dkv_u32x2{__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
  } else {
    const dkv_f16x2 h01 = __builtin_convertvector(f32x2{p[0], p[1]}, dkv_f16x2);
    const dkv_f16x2 h23 = __builtin_convertvector(f32x2{p[2], p[3]}, dkv_f16x2);
    const dkv_f16x2 l01 =
        __builtin_convertvector(f32x2{p[0] - (float)h01[0], p[1] - (float)h01[1]}, dkv_f16x2);
    const dkv_f16x2 l23 =
        __builtin_convertvector(f32x2{p[2] - (float)h23[0], p[3] - (float)h23[1]}, dkv_f16x2);
    hi = dkv_u32x2{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
    lo = dkv_u32x2{__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
  }
}

// grid: (ceil(Sq / 128), Hq, B); 256 threads (the workgroup's item is remapped from its
// linear id, see below). ODT: output dtype (DT or fp32).
template <int DT, int ODT>
__global__ __launch_bounds__(256, 2) void fa_prefill_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t sK[2][FA_TILE_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t sV[2][FA_TILE_BYTES];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  // Work item of this workgroup. Workgroups go to the 8 XCDs round-robin by linear id L (XCD
  // L % 8, in order of L on each), so items are handed out by L in longest-first order of
  // causal work: units (query block, b, KV head) from the last query block down, unit
  // c + 8j to XCD c, each unit's query heads consecutive on it (they read the same K and V
  // tiles, from that XCD's L2). Every XCD then gets the same mix of query blocks, each
  // longest first. (The grid's own order gave XCD k the query blocks k, k+8, ... only: 2.4x
  // the work on XCD 7 as on XCD 0 at 16 blocks.) When the units do not divide among the
  // XCDs the items go out by L in the same longest-first order, query heads spread.
  int b, h, qblk;
  {
    const int nx = gridDim.x, ny = gridDim.y, nz = gridDim.z;
    const int L = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    const int grp = p.Hq / p.Hkv;       // query heads per KV head
    const int units = nx * nz * p.Hkv;  // (query block, b, KV head)
    if (units % 8 == 0) {
      const int xcd = L & 7, rank = L >> 3;
      const int u = xcd + 8 * (rank / grp);
      const int per = nz * p.Hkv;  // units per query block
      qblk = nx - 1 - u / per;
      b = (u % per) / p.Hkv;
      h = ((u % per) % p.Hkv) * grp + rank % grp;
    } else {
      const int per = ny * nz;  // items per query block
      qblk = nx - 1 - L / per;
      h = (L % per) % ny;
      b = (L % per) / ny;
    }
  }
  const int kvh = h / (p.Hq / p.Hkv);
  const int q0 = qblk * FA_BQ;
  const int wq0 = q0 + FA_QW * wave;  // the wave's first query
  // this lane's query in block qb (B operand column, output row)
  auto qrow = [&](int qb) { return wq0 + 16 * qb + n; };

  // Q^T operands: lane (query n of block qb, k-group g) holds dims 32s + 8g .. +8
  dkv_u32x4 qop[FA_QB][4];
#pragma unroll
  for (int qb = 0; qb < FA_QB; ++qb) {
    const uint16_t* qp = p.q + (long long)b * p.q_sb + (long long)h * p.q_sh +
                         (long long)min(qrow(qb), p.Sq - 1) * p.q_ss + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[qb][s] = *(const dkv_u32x4*)(qp + 32 * s);
  }

  // keys this workgroup needs: causal limit of its last query; the wave's own limit
  const int q_last_pos = p.q_offset + min(q0 + FA_BQ, p.Sq) - 1;
  const int k_end = p.causal ? min(p.Sk, q_last_pos + 1) : p.Sk;
  const int n_tiles = (k_end + FA_BK - 1) / FA_BK;
  // keys before ks are masked (a left-padded row's padding); tiles wholly before it are skipped
  const int ks = p.kstart ? min(max(p.kstart[b], 0), p.Sk) : 0;
  const int t0 = ks / FA_BK;
  const int wave_k_end =
      p.causal ? min(k_end, p.q_offset + min(wq0 + FA_QW, p.Sq)) : k_end;  // <= k_end

  const __amdgpu_buffer_rsrc_t rk = dkv_make_rsrc(p.k, p.k_bytes);
  const __amdgpu_buffer_rsrc_t rv = dkv_make_rsrc(p.v, p.v_bytes);
  const long long kbase = (long long)b * p.k_sb + (long long)kvh * p.k_sh;
  const long long vbase = (long long)b * p.v_sb + (long long)kvh * p.v_sh;
  // tile loads: wave w, instruction c stores keys 16w + 4c + l/16, LDS chunk position l%16,
  // which holds the key's 16-byte dims chunk (l%16) ^ (key % 16)
  auto issue = [&](int t) {
    const int buf = t & 1;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kk = 16 * wave + 4 * c + (lane >> 4);
      const int key = t * FA_BK + kk;
      const int chunk = (lane & 15) ^ (kk & 15);
      const bool ok = key < k_end;
      const uint32_t ko = ok ? (uint32_t)((kbase + (long long)key * p.k_ss + 8 * chunk) * 2) : 0x7ffffff0u;
      const uint32_t vo = ok ? (uint32_t)((vbase + (long long)key * p.v_ss + 8 * chunk) * 2) : 0x7ffffff0u;
      fa_lds_load16(rk, fa_lds_addr(&sK[buf][(16 * wave + 4 * c) * 256]), ko);
      fa_lds_load16(rv, fa_lds_addr(&sV[buf][(16 * wave + 4 * c) * 256]), vo);
    }
  };

  dkv_f32x4 acc[FA_QB][8];
#pragma unroll
  for (int qb = 0; qb < FA_QB; ++qb)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[qb][i] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
  // running maxima (log2 units) and sums per query block; a maximum is only raised when the
  // tile's exceeds it by more than FA_RESCALE, so P may reach 2^FA_RESCALE
  float m_run[FA_QB], l_run[FA_QB];
#pragma unroll
  for (int qb = 0; qb < FA_QB; ++qb) {
    m_run[qb] = -1.0e30f;
    l_run[qb] = 0.f;
  }

  if (t0 < n_tiles) issue(t0);
  for (int t = t0; t < n_tiles; ++t) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // tile t is in LDS for every wave; tile t-1's buffer is free
    if (t + 1 < n_tiles) issue(t + 1);
    const int key0 = t * FA_BK;
    if (key0 >= wave_k_end) continue;  // every key of the tile is past the wave's queries
    const uint8_t* kt = sK[t & 1];
    const uint8_t* vt = sV[t & 1];

    // S^T = K Q^T: A = K rows (lane: key 16kb + n, dims 32s + 8g .. +8), B = Q^T of block qb;
    // lane (query n, g) then holds keys 16kb + 4g + u
    float z[FA_QB][4][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      dkv_f32x4 sacc[FA_QB];
#pragma unroll
      for (int qb = 0; qb < FA_QB; ++qb) sacc[qb] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
      const uint8_t* row = kt + (16 * kb + n) * 256;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const dkv_u32x4 a = *(const dkv_u32x4*)(row + 16 * ((4 * s + g) ^ n));
#pragma unroll
        for (int qb = 0; qb < FA_QB; ++qb) sacc[qb] = mfma32<DT>(a, qop[qb][s], sacc[qb]);
      }
#pragma unroll
      for (int qb = 0; qb < FA_QB; ++qb)
#pragma unroll
        for (int u = 0; u < 4; ++u) z[qb][kb][u] = sacc[qb][u];  // unscaled (see below)
    }
    if (key0 + FA_BK > k_end || key0 < ks || (p.causal && key0 + FA_BK - 1 > p.q_offset + wq0)) {
#pragma unroll
      for (int qb = 0; qb < FA_QB; ++qb) {
        const int my_pos = p.q_offset + qrow(qb);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int key = key0 + 16 * kb + 4 * g + u;
            if (key >= k_end || key < ks || (p.causal && key > my_pos)) z[qb][kb][u] = -INFINITY;
          }
      }
    }
    float tmax[FA_QB];
#pragma unroll
    for (int qb = 0; qb < FA_QB; ++qb) {
      float m = z[qb][0][0];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int u = 0; u < 4; ++u) m = fa_max(m, z[qb][kb][u]);
      // the scale is applied to the tile's maximum and inside the exponent's fma (one VALU
      // per score less than scaling every score: 2-3% of the launch); it is positive (the
      // entry point checks), so the maximum commutes with it
      tmax[qb] = fa_max4(m) * p.scale_log2;
    }
    if (__ballot(tmax[0] > m_run[0] + FA_RESCALE || tmax[FA_QB - 1] > m_run[FA_QB - 1] + FA_RESCALE)) {
#pragma unroll
      for (int qb = 0; qb < FA_QB; ++qb) {
        const float m_new = fa_max(m_run[qb], tmax[qb]);
        const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
        m_run[qb] = m_new;
        l_run[qb] *= alpha;
        // acc rows are dims, columns queries: lane (query n, g) holds dims 16db + 4g + u of
        // query n, so its rescale factor is its own alpha
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int u = 0; u < 4; ++u) acc[qb][i][u] *= alpha;
      }
    }

    // P.V: for each key block kb, one 16x16x32 product per 16 dims and query block with
    // k = 8g + e pairing part e/4 of key 16kb + 4g + e%4 (B: this lane's P hi then lo) with that
    // key's V values (A: the four keys' values of dim 16db + n, twice)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      dkv_u32x4 bop[FA_QB];
#pragma unroll
      for (int qb = 0; qb < FA_QB; ++qb) {
        float pu[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          pu[u] = __builtin_amdgcn_exp2f(__builtin_fmaf(z[qb][kb][u], p.scale_log2, -m_run[qb]));
          l_run[qb] += pu[u];
        }
        dkv_u32x2 ph, pl;
        split_hi_lo<DT>(pu, ph, pl);
        bop[qb] = dkv_u32x4{ph.x, ph.y, pl.x, pl.y};
      }
      // transposed read: lane L = 4j + q of each 16-lane group reads key 16kb + 4g + j,
      // dims 16db + 4q .. +3 (8 bytes); lane i then holds dim 16db + i of keys 4g .. 4g+3
      const int key = 16 * kb + 4 * g + (n >> 2);
      const uint8_t* vrow = vt + key * 256;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const int dchunk = 2 * db + ((n & 3) >> 1);
        const uint8_t* src = vrow + 16 * (dchunk ^ (key & 15)) + 8 * (n & 1);
        const dkv_u32x2 xv = __builtin_bit_cast(
            dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                           (__attribute__((address_space(3))) dkv_i16x4*)(
                               (__attribute__((address_space(3))) uint8_t*)src)));
        const dkv_u32x4 aop = __builtin_bit_cast(
            dkv_u32x4, dkv_u64x2{__builtin_bit_cast(uint64_t, xv), __builtin_bit_cast(uint64_t, xv)});
#pragma unroll
        for (int qb = 0; qb < FA_QB; ++qb) acc[qb][db] = mfma32<DT>(aop, bop[qb], acc[qb][db]);
      }
    }
  }

#pragma unroll
  for (int qb = 0; qb < FA_QB; ++qb) {
    // l over each tile's 64 keys sits in the lane's 16 keys x 4 lanes of the query
    float l = l_run[qb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int qr = qrow(qb);
    if (qr < p.Sq) {
      // a query with no key to attend (a padding position before the row's first key) gets 0
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const long long ob = (long long)b * p.o_sb + (long long)h * p.o_sh + (long long)qr * p.o_ss;
#pragma unroll
      for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int u = 0; u < 4; ++u)
          dkv_store_f32<ODT>(p.out, ob + 16 * db + 4 * g + u, acc[qb][db][u] * inv);
    }
  }
}

// In-place rotate-half RoPE on dense rows x[r][s][d] (d < 128): position pos0 + s, angle
// float(pos) * inv_freq_i in fp32, the rotation in fp32, the result rounded to the dtype.
template <int DT>
__global__ __launch_bounds__(256) void rope_dense_kernel(uint16_t* __restrict__ x, long long r_ld,
                                                         long long s_ld, int rows, int S, int pos0,
                                                         float log_theta) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long total = (long long)rows * S * 64;
  if (idx >= total) return;
  const int i = (int)(idx % 64);
  const long long rs = idx / 64;
  const int s = (int)(rs % S);
  const long long r = rs / S;
  dkv_rope_pair<DT>(x + r * r_ld + (long long)s * s_ld, i, pos0 + s, log_theta);
}

// In-place rotate-half RoPE of x (B, H, S, 128) with given cos / sin tables (B, S, 128) in the
// dtype, rounded as the reference's apply_rotary_pos_emb_ computes (x * cos) + (rotate_half(x)
// * sin) in the dtype (compressed_attention.py:18-22): each product rounded, then their sum.
template <int DT>
__global__ __launch_bounds__(256) void rope_apply_kernel(uint16_t* __restrict__ x, long long x_sb,
                                                         long long x_sh, long long x_ss,
                                                         const uint16_t* __restrict__ cs,
                                                         const uint16_t* __restrict__ sn,
                                                         long long c_sb, long long c_ss, int B,
                                                         int H, int S) {
  // no contraction: for fp16 the compiler narrows the products and the sum to half arithmetic
  // and would fuse them into one fma, skipping the product's rounding
#pragma clang fp contract(off)
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long total = (long long)B * H * S * 64;
  if (idx >= total) return;
  const int i = (int)(idx % 64);
  long long r = idx / 64;
  const int s = (int)(r % S);
  r /= S;
  const int h = (int)(r % H);
  const int b = (int)(r / H);
  uint16_t* xr = x + (long long)b * x_sb + (long long)h * x_sh + (long long)s * x_ss;
  const long long co = (long long)b * c_sb + (long long)s * c_ss;
  const float x1 = dkv_load_f32<DT>(xr, i), x2 = dkv_load_f32<DT>(xr, i + 64);
  const float c1 = dkv_load_f32<DT>(cs, co + i), c2 = dkv_load_f32<DT>(cs, co + i + 64);
  const float s1 = dkv_load_f32<DT>(sn, co + i), s2 = dkv_load_f32<DT>(sn, co + i + 64);
  const float o1 = dkv_round_to<DT>(x1 * c1) + dkv_round_to<DT>(-x2 * s1);
  const float o2 = dkv_round_to<DT>(x2 * c2) + dkv_round_to<DT>(x1 * s2);
  dkv_store_f32<DT>(xr, i, o1);
  dkv_store_f32<DT>(xr, i + 64, o2);
}

}  // namespace

extern "C" int dkv_rope_dense(void* stream, int dtype, void* x, long long row_ld, long long tok_ld,
                              int rows, int S, int pos0, float log_theta) {
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (rows < 0 || S < 0) return DKV_E_ARG;
  if (rows == 0 || S == 0) return DKV_OK;
  if (!x) return DKV_E_ARG;
  const long long total = (long long)rows * S * 64;
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DKV_BF16)
    hipLaunchKernelGGL(rope_dense_kernel<DKV_BF16>, grid, dim3(256), 0, st, (uint16_t*)x, row_ld,
                       tok_ld, rows, S, pos0, log_theta);
  else
    hipLaunchKernelGGL(rope_dense_kernel<DKV_F16>, grid, dim3(256), 0, st, (uint16_t*)x, row_ld,
                       tok_ld, rows, S, pos0, log_theta);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_rope_apply(void* stream, int dtype, void* x, long long x_sb, long long x_sh,
                              long long x_ss, const void* cos, const void* sin, long long cs_sb,
                              long long cs_ss, int B, int H, int S) {
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (B < 0 || H < 0 || S < 0 || cs_sb < 0 || cs_ss < 0) return DKV_E_ARG;
  const long long total = (long long)B * H * S * 64;
  if (total == 0) return DKV_OK;
  if (!x || !cos || !sin) return DKV_E_ARG;
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DKV_BF16)
    hipLaunchKernelGGL(rope_apply_kernel<DKV_BF16>, grid, dim3(256), 0, st, (uint16_t*)x, x_sb,
                       x_sh, x_ss, (const uint16_t*)cos, (const uint16_t*)sin, cs_sb, cs_ss, B, H,
                       S);
  else
    hipLaunchKernelGGL(rope_apply_kernel<DKV_F16>, grid, dim3(256), 0, st, (uint16_t*)x, x_sb,
                       x_sh, x_ss, (const uint16_t*)cos, (const uint16_t*)sin, cs_sb, cs_ss, B, H,
                       S);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_prefill_attention(void* stream, int dtype, const void* q, long long q_sb,
                                     long long q_sh, long long q_ss, const void* k, long long k_sb,
                                     long long k_sh, long long k_ss, long long k_elems,
                                     const void* v, long long v_sb, long long v_sh, long long v_ss,
                                     long long v_elems, void* out, int out_dtype, long long o_sb,
                                     long long o_sh, long long o_ss, int B, int Hq, int Hkv,
                                     int Sq, int Sk, int Dh, int causal, float scale,
                                     const int* kstart) {
  // the kernel takes each tile's maximum before scaling: a positive, finite scale only
  if (!(scale > 0.f) || !(scale < INFINITY)) return DKV_E_UNSUPPORTED;
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (out_dtype != dtype && out_dtype != DKV_F32) return DKV_E_ARG;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Sq < 0 || Sk < 0) return DKV_E_ARG;
  if (Dh != FA_DH || Hq % Hkv != 0) return DKV_E_UNSUPPORTED;
  if (B == 0 || Sq == 0) return DKV_OK;
  if (!q || !k || !v || !out) return DKV_E_ARG;
  if (causal && Sk < Sq) return DKV_E_ARG;  // queries are the last Sq positions of the keys
  // 16-byte operand loads: unit dim stride, row strides in whole 16-byte units
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 || q_ss % 8 || k_ss % 8 || v_ss % 8 ||
      k_sh % 8 || v_sh % 8 || k_sb % 8 || v_sb % 8 || q_sh % 8 || q_sb % 8)
    return DKV_E_UNSUPPORTED;
  if (k_elems * 2 >= (1LL << 31) || v_elems * 2 >= (1LL << 31)) return DKV_E_UNSUPPORTED;
  PrefillParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.out = out;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_ss = q_ss;
  p.k_sb = k_sb; p.k_sh = k_sh; p.k_ss = k_ss;
  p.v_sb = v_sb; p.v_sh = v_sh; p.v_ss = v_ss;
  p.o_sb = o_sb; p.o_sh = o_sh; p.o_ss = o_ss;
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.Sq = Sq; p.Sk = Sk;
  p.q_offset = causal ? Sk - Sq : 0;
  p.causal = causal ? 1 : 0;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.k_bytes = (uint32_t)(k_elems * 2);
  p.v_bytes = (uint32_t)(v_elems * 2);
  p.kstart = kstart;
  const dim3 grid((unsigned)((Sq + FA_BQ - 1) / FA_BQ), (unsigned)Hq, (unsigned)B);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DKV_BF16) {
    if (out_dtype == DKV_F32)
      hipLaunchKernelGGL((fa_prefill_kernel<DKV_BF16, DKV_F32>), grid, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((fa_prefill_kernel<DKV_BF16, DKV_BF16>), grid, dim3(256), 0, st, p);
  } else {
    if (out_dtype == DKV_F32)
      hipLaunchKernelGGL((fa_prefill_kernel<DKV_F16, DKV_F32>), grid, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((fa_prefill_kernel<DKV_F16, DKV_F16>), grid, dim3(256), 0, st, p);
  }
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
