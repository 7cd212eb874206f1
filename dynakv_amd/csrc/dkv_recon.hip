// Dense K and V of a prompt from its masked coefficient rows, for the compressed prefill
// attention (reference compressed_attention.py:359-386 reconstructs the prompt's keys and
// values through the up-projection bases, get_origin_states in compressed_cache.py:36-56 returns
// the coefficients zero past each token's count, and the keys are rotated before the causal
// attention, :375-378). One launch reconstructs both: K[t] = R(t) (B_K^T c_K[t]) and
// V[t] = B_V^T c_V[t] per cache row (b, g), the products on 16x16x32 MFMA with fp32
// accumulation; the keys rounded to the dtype, rotated in fp32 and rounded again, as the
// reference rounds the projection and then the rotation. The rotation of position p = 16T + n
// is R(16T) R(n) composed in fp32 from the rows of the RoPE table (dkv_rope_table: cos and sin
// of the fp32 angles n * inv_freq and 16T * inv_freq), not a sine and cosine per element.
//
// Workgroup = (64 tokens, cache row, K | V), four waves of 16 tokens. The row's basis ([rank]
// [dim], ranks past R zero) is staged in LDS and read transposed (ds_read_b64_tr_b16) as the A
// operand (dims x ranks); each lane loads its token's 8 coefficients of a 32-rank chunk as the B
// operand; the result out^T[dim][token] leaves every lane four consecutive dims of one token
// for each 16-dim block, and the rotate-half pairs (d, d + 64) in the same lane.
#include "dkv_common.h"
#include "dkv_mfma_ops.h"

namespace {

constexpr int DH = 128;
constexpr int RW = 4;  // waves per workgroup (16 tokens each)
constexpr int RT_FIXED = 17;  // RoPE table rows before the tile rows R(16T)

template <int DT>
__global__ __launch_bounds__(RW * 64) void recon_kv_kernel(
    const uint16_t* __restrict__ ck, const uint16_t* __restrict__ cv, long long c_sr,
    long long c_st, const uint16_t* __restrict__ kb, const uint16_t* __restrict__ vb,
    long long b_sg, long long b_sr, uint16_t* __restrict__ ko, uint16_t* __restrict__ vo,
    long long o_sr, long long o_st, int G, int S, int R, int pos0, const float* __restrict__ rope) {
  __shared__ __attribute__((aligned(16))) uint16_t sB[DH * DH];  // [rank][dim]
  const bool is_k = blockIdx.z == 0;
  const int row = blockIdx.y, grp = row % G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const uint16_t* c = is_k ? ck : cv;
  const uint16_t* bg = (is_k ? kb : vb) + (long long)grp * b_sg;
  uint16_t* o = is_k ? ko : vo;

  // this lane's token and its coefficient pieces (ranks 32 cc + 8g .. +8; R is a multiple of 8)
  const int t = (blockIdx.x * RW + wave) * 16 + n;
  const uint16_t* cr = c + (long long)row * c_sr + (long long)min(t, S - 1) * c_st;
  dkv_u32x4 xc[4];
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    const int r0 = 32 * cc + 8 * g;
    xc[cc] = (t < S && r0 < R) ? *(const dkv_u32x4*)(cr + r0) : dkv_u32x4{0u, 0u, 0u, 0u};
  }
  // the basis, 16-byte pieces (rank r, dims d8 .. d8 + 7), ranks past R as zeros
  for (int pc = tid; pc < DH * DH / 8; pc += RW * 64) {
    const int r = pc >> 4, d8 = (pc & 15) * 8;
    *(dkv_u32x4*)(sB + r * DH + d8) =
        r < R ? *(const dkv_u32x4*)(bg + (long long)r * b_sr + d8) : dkv_u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  dkv_f32x4 acc[8];
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) acc[blk] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
  typedef __attribute__((address_space(3))) dkv_i16x4 lds_i16x4;
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    if (32 * cc >= R) break;  // uniform: chunks wholly past the rank are zero
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      // lane (n, g) receives ranks 32 cc + 8g .. +3 and +4 .. +7 of dim 16 blk + n
      const uint16_t* src = sB + (32 * cc + 8 * g + (n >> 2)) * DH + 16 * blk + 4 * (n & 3);
      const dkv_u32x2 b0 = __builtin_bit_cast(
          dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                         (lds_i16x4*)(__attribute__((address_space(3))) uint16_t*)src));
      const dkv_u32x2 b1 = __builtin_bit_cast(
          dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                         (lds_i16x4*)(__attribute__((address_space(3))) uint16_t*)(src + 4 * DH)));
      acc[blk] = dkv_mfma32<DT>(dkv_u32x4{b0.x, b0.y, b1.x, b1.y}, xc[cc], acc[blk]);
    }
  }
  if (t >= S) return;
  // lane (n, g): dims 16 blk + 4g + u of token t in acc[blk][u]
  if (is_k) {
    const int pos = pos0 + t;
    // (cos, sin) of frequencies 16 blk + 4g .. +3: 32 contiguous bytes of a table row
    const float* rn = rope + (pos & 15) * 128 + 8 * g;
    const float* rt = rope + (RT_FIXED + (pos >> 4)) * 128 + 8 * g;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const dkv_f32x4 n0 = *(const dkv_f32x4*)(rn + 32 * blk), n1 = *(const dkv_f32x4*)(rn + 32 * blk + 4);
      const dkv_f32x4 t0 = *(const dkv_f32x4*)(rt + 32 * blk), t1 = *(const dkv_f32x4*)(rt + 32 * blk + 4);
      const float nc[4] = {n0.x, n0.z, n1.x, n1.z}, ns[4] = {n0.y, n0.w, n1.y, n1.w};
      const float tc[4] = {t0.x, t0.z, t1.x, t1.z}, ts[4] = {t0.y, t0.w, t1.y, t1.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float cs = tc[u] * nc[u] - ts[u] * ns[u], sn = ts[u] * nc[u] + tc[u] * ns[u];
        // the projection rounded to the dtype first, then rotated: the reference's two steps
        // (the up-projection's product in the dtype, then apply_rotary_pos_emb_)
        const float a = dkv_round_to<DT>(acc[blk][u]), bb = dkv_round_to<DT>(acc[blk + 4][u]);
        acc[blk][u] = a * cs - bb * sn;
        acc[blk + 4][u] = bb * cs + a * sn;
      }
    }
  }
  uint16_t* orow = o + (long long)row * o_sr + (long long)t * o_st;
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
    uint32_t w[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float lo = acc[blk][2 * e], hi = acc[blk][2 * e + 1];
      if constexpr (DT == DKV_BF16)
        w[e] = dkv_f32_to_bf16_bits(lo) | (dkv_f32_to_bf16_bits(hi) << 16);
      else
        w[e] = dkv_f32_to_f16_bits(lo) | (dkv_f32_to_f16_bits(hi) << 16);
    }
    *(dkv_u32x2*)(orow + 16 * blk + 4 * g) = dkv_u32x2{w[0], w[1]};
  }
}

}  // namespace

extern "C" int dkv_recon_kv(void* stream, int dtype, const void* ck, const void* cv,
                            long long c_sr, long long c_st, const void* k_basis,
                            const void* v_basis, long long b_sg, long long b_sr, void* k_out,
                            void* v_out, long long o_sr, long long o_st, int rows, int G, int S,
                            int R, int pos0, const float* rope, int rope_tiles) {
  if (dtype != DKV_F16 && dtype != DKV_BF16) return DKV_E_UNSUPPORTED;
  if (rows < 0 || G <= 0 || S < 0 || R <= 0 || pos0 < 0) return DKV_E_ARG;
  if (rows == 0 || S == 0) return DKV_OK;
  if (!ck || !cv || !k_basis || !v_basis || !k_out || !v_out || !rope) return DKV_E_ARG;
  if ((long long)rope_tiles * 16 < (long long)pos0 + S) return DKV_E_ARG;
  if ((uintptr_t)rope & 15) return DKV_E_UNSUPPORTED;
  if (R > DH || R % 8 != 0 || rows % G != 0) return DKV_E_UNSUPPORTED;
  // 16-byte coefficient pieces and basis rows, 8-byte output pieces
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!a16(ck) || !a16(cv) || !a16(k_basis) || !a16(v_basis) || (c_sr & 7) || (c_st & 7) ||
      (b_sg & 7) || (b_sr & 7) || ((uintptr_t)k_out & 7) || ((uintptr_t)v_out & 7) ||
      (o_sr & 3) || (o_st & 3))
    return DKV_E_UNSUPPORTED;
  if (S > 65535 * 64 || rows > 65535) return DKV_E_UNSUPPORTED;
  const dim3 grid((unsigned)((S + 63) / 64), (unsigned)rows, 2);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DKV_BF16)
    hipLaunchKernelGGL(recon_kv_kernel<DKV_BF16>, grid, dim3(RW * 64), 0, st,
                       (const uint16_t*)ck, (const uint16_t*)cv, c_sr, c_st,
                       (const uint16_t*)k_basis, (const uint16_t*)v_basis, b_sg, b_sr,
                       (uint16_t*)k_out, (uint16_t*)v_out, o_sr, o_st, G, S, R, pos0, rope);
  else
    hipLaunchKernelGGL(recon_kv_kernel<DKV_F16>, grid, dim3(RW * 64), 0, st,
                       (const uint16_t*)ck, (const uint16_t*)cv, c_sr, c_st,
                       (const uint16_t*)k_basis, (const uint16_t*)v_basis, b_sg, b_sr,
                       (uint16_t*)k_out, (uint16_t*)v_out, o_sr, o_st, G, S, R, pos0, rope);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
