// Decode attention for the reference's joint layout on MFMA: one packed coefficient row per batch
// element with ranks up to 1024 shared by every KV head, one (R, 128) basis per KV head (or per
// query head, as the reference's repeated k_up).
//
// Reference behaviour: abx_sparse / _abx_sparse_fwd (src/dynakv/kernels/two_stage.py:48-189) and
// avx / _avx_proj_fwd (:207-324), the router's long route for this layout; the fused route
// (fused.py:28-170) is the same scores with -inf masking and the V pass without the 1e-6 clamp.
// The entry points take what dkv_scores / dkv_av take for these shapes (the K basis transposed
// in 32-rank chunks, [chunk][dim][rank], a RoPE table, a workspace for the V pass) and compute
// the same results to fp32 accuracy:
//
// joint_sort_kernel -- workgroup = (window of up to 2048 positions, batch row b): the window's
//   tokens ordered by their count of 32-rank chunks (a counting sort) into a workspace.
// joint_scores_sorted_kernel -- workgroup = (512 sorted tokens of a window, basis head h, batch
//   row b), or with the heads in pairs (256 tokens, heads 2h and 2h+1, b) so that each
//   coefficient load serves both heads' products; the longest ranges are dispatched first. The
//   workgroup's tokens form blocks of 16; wave w takes blocks w and NBLK-1-w (one short, one
//   long). K^T = B_h^T . X^T accumulates on 16x16x32 MFMA over the rank chunks of
//   32, each block only up to its own longest token's chunk. Each basis chunk ([128 dims][32
//   ranks], 8 KB contiguous in HBM) is loaded once per workgroup into LDS (four buffers per
//   head, one barrier per two chunks) and every A operand read from it serves the wave's active
//   blocks; the coefficients go straight into B operand registers (lane = one token x 8 ranks,
//   elements past the token's count zeroed), two chunks ahead, each serving every head of the
//   workgroup. Then per block: the lane's token rotated by R(p) = R(16T) R(n) (p = 16T + n, its
//   position; composed from LDS tables) in fp32, K' split into bf16 hi + lo, scores on MFMA
//   against the unrotated query (hi and lo parts in separate operand columns, formed once per
//   head), the route's masking and rounding, stored at the token's position.
// joint_av_kernel -- workgroup = (token split, 16 or 32 query heads, batch row b); wave w takes
//   ranks [128w, 128w + 128). Per 16-token tile: each set of 16 heads' scores through an online
//   softmax in the log2 domain (every wave computes the same values), P as bf16 hi + lo (fp16
//   for fp16 caches), the wave's V coefficients of the tile staged in LDS and read transposed
//   (ds_read_b64_tr_b16) once as the B operand of every set's P.X^V. Each split writes (m, l,
//   acc[R]) per head.
// joint_merge_kernel -- workgroup = (rank block of 128, V basis and up to 8 of its query heads,
//   batch row b): LSE weights of the split records with the route's denominator, the block's
//   merged coefficients, their projection through the block's basis rows (each basis value
//   loaded once for the group's heads); joint_project_sum_kernel adds the blocks' partial
//   projections and rounds the output.
#include <type_traits>

#include "dkv_common.h"
#include "dkv_mfma_ops.h"

namespace {

constexpr int JDH = 128;
constexpr int JWAVES = 8;
constexpr int JTHREADS = JWAVES * 64;
constexpr int JCB = 4;                   // 16-token column blocks per wave (scores)
constexpr int JTOK = JWAVES * JCB * 16;  // tokens per scores workgroup
constexpr int JCH = 32;                  // ranks per basis chunk
constexpr int JRMAX = 1024;
constexpr int JPREC = 4 + JRMAX;         // split record: m (log2 units), l, 2 unused, acc[R]
constexpr int JRB = 128;                 // ranks per merge workgroup
constexpr int JROPE_FIXED = 17;          // rows of the RoPE table before the per-tile rows
constexpr int JFLAT_CAP = DKV_FLAT_RSRC_CAP;  // elements one buffer resource covers
constexpr int JMAX_SPLITS = 1024;  // token splits of the V pass
constexpr float JLOG2E = 1.4426950408889634f;
constexpr float JRESCALE = 11.5f;        // log2 units: rescale when the running max grows more
// the scores kernel's tokens are ordered by chunk count within windows of at most JSWIN
// positions (a multiple of every scores workgroup's token count); the R(16T) rows of a window's
// tiles fit in LDS
constexpr int JSWIN = 2048;
constexpr int JSORT_THREADS = 1024;

// piece swizzle of the basis chunk buffers (a function of d mod 16): the 16-byte slot of ranks
// 8k..8k+7 of row d is k ^ ((d >> 1) & 3). Measured on MI355X for ds_read_b128 with lane
// (n, g) reading slot g of row 16*blk + n: 270-290 bytes per clock and CU, as fast as
// consecutive addresses (168-177 for (d ^ (d >> 2)) & 3 or no swizzle)
__device__ __forceinline__ int jswz(int d) { return (d >> 1) & 3; }

__device__ __forceinline__ dkv_f32x4 mfma_bf16x32(const dkv_u32x4& a, const dkv_u32x4& b,
                                                  dkv_f32x4 c) {
  return dkv_mfma32<DKV_BF16>(a, b, c);
}

struct JScoresParams {
  const uint16_t* q;
  long long q_sb, q_sh;
  const uint16_t* bt;  // K basis [n_basis][Dh][R-stride]
  long long bt_sh, bt_sc;  // basis [h][chunk][dim][32 ranks]: head and chunk strides
  const uint16_t* flat;
  long long flat_ld;
  const int* lens;
  long long lens_sb, lens_ss;
  const int* offs;
  long long offs_sb, offs_ss;
  const float* rope;
  int rope_tiles;
  void* out;
  long long out_sb, out_sh, out_ss;
  int B, S, R, hpg;
  float scale;
  // per (batch row, window): 3 x win ints, the window's (length, offset, position) triplets in
  // ascending chunk-count order, pad entries (0, 0, -1) first up to a multiple of the
  // workgroup's tokens (joint_sort_kernel)
  const int* sorted;
  int win, nwin, n_basis;
};

// Window length for S positions: JSWIN, or S rounded up to 512 when shorter.
__host__ __device__ inline int joint_window(int S) {
  return S >= JSWIN ? JSWIN : ((S + 511) / 512) * 512;
}

// joint_sort_kernel -- workgroup = (window of win positions, batch row): the window's tokens in
// ascending order of their count of 32-rank chunks (a counting sort: per-wave bucket counts by
// ballots, bucket starts, scatter; within a bucket by (pass, wave, lane), an order no score
// depends on), preceded by pad entries up to a multiple of tok, as (length, offset, position)
// triplets.
struct JSortParams {
  const int* lens;
  long long lens_sb, lens_ss;
  const int* offs;
  long long offs_sb, offs_ss;
  int* sorted;
  int S, R, win, nwin, tok;
};

__global__ __launch_bounds__(JSORT_THREADS) void joint_sort_kernel(JSortParams p) {
  constexpr int NK = JRMAX / JCH + 1;             // chunk-count buckets 0..32
  constexpr int NW = JSORT_THREADS / 64;          // waves
  constexpr int IT = JSWIN / JSORT_THREADS;       // tokens per thread
  static_assert(NK <= 64, "one lane per bucket");
  // per bucket and (pass it, wave w): the wave's token count in the bucket, then its first slot
  __shared__ int sW[NK][IT * NW];
  __shared__ int sTot[NK];
  const int w = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6;
  const int base = w * p.win;
  const int nt = min(p.win, p.S - base);
  const int npad = (nt + p.tok - 1) / p.tok * p.tok - nt;
  const int* lr = p.lens + (long long)b * p.lens_sb;
  const int* orow = p.offs + (long long)b * p.offs_sb;
  int* out = p.sorted + ((long long)b * p.nwin + w) * 3 * p.win;
  for (int e = tid; e < IT * NW * NK; e += JSORT_THREADS) (&sW[0][0])[e] = 0;
  // token i = it * JSORT_THREADS + tid of the window: its length, offset, bucket and its rank
  // among the wave's lanes of the same bucket (lanes in order)
  int len[IT], off[IT], bk[IT], rk[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int i = it * JSORT_THREADS + tid;
    len[it] = 0;
    off[it] = 0;
    bk[it] = -1;
    if (i < nt) {
      len[it] = min(max(lr[(long long)(base + i) * p.lens_ss], 0), p.R);
      off[it] = orow[(long long)(base + i) * p.offs_ss];
      bk[it] = (len[it] + JCH - 1) / JCH;
    }
  }
  __syncthreads();  // sW cleared
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int k = bk[it];
    uint64_t pending = __ballot(k >= 0);
    rk[it] = 0;
    while (pending) {  // one step per distinct bucket of the wave
      const int kk = __shfl(k, __ffsll((unsigned long long)pending) - 1, 64);
      const uint64_t same = __ballot(k == kk);
      if (k == kk)
        rk[it] = __builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32),
                                           __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
      if (lane == 0) sW[kk][it * NW + wave] = __popcll(same);
      pending &= ~same;
    }
  }
  __syncthreads();
  // bucket k (wave k % NW, lane j = (pass, wave)): the exclusive scan of its counts over j and
  // its total; then the buckets' starts (pad entries first) by a scan over the first wave
  static_assert(IT * NW <= 64, "one lane per (pass, wave)");
  for (int k = wave; k < NK; k += NW) {
    const int c = lane < IT * NW ? sW[k][lane] : 0;
    int incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    if (lane < IT * NW) sW[k][lane] = incl - c;
    if (lane == 63) sTot[k] = incl;
  }
  __syncthreads();
  if (wave == 0) {
    const int tot = lane < NK ? sTot[lane] : 0;
    int incl = tot;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    if (lane < NK) sTot[lane] = npad + incl - tot;  // the bucket's first slot
  }
  for (int i = tid; i < npad; i += JSORT_THREADS) {
    out[i] = 0;
    out[p.win + i] = 0;
    out[2 * p.win + i] = -1;
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (bk[it] >= 0) {
      const int slot = sTot[bk[it]] + sW[bk[it]][it * NW + wave] + rk[it];
      out[slot] = len[it];
      out[p.win + slot] = off[it];
      out[2 * p.win + slot] = base + it * JSORT_THREADS + tid;
    }
  }
}

// joint_scores_sorted_kernel: the scores with the rank chunks bounded per 16-token block instead of
// per workgroup. joint_sort_kernel orders each window of JSWIN positions by the tokens' count of
// 32-rank chunks, and a workgroup takes TOK consecutive sorted tokens of one window, so each
// block of 16 of them needs the chunks up to its own last token's count (a block's products and
// coefficient loads stop there) and the workgroup's basis chunks only up to its last token's:
// in the reference's joint layout a few full-rank tokens sit in almost every 256-token range of
// positions, which made a workgroup of consecutive positions stage all 32 basis chunks (~12.9 on
// average with sorted windows of 2048 at the config-3 shape, 11.8 -> 11.0 products per block).
// Wave w takes sorted blocks w and NBLK-1-w (with one basis head: also 16+w and 31-w), one short
// and one long, so the waves' products per chunk stay balanced. A token's position is arbitrary
// within the window, so the key takes the whole rotation R(p) = R(16T) R(n) (p = 16T + n),
// composed per lane from the R(n) table and the window's R(16T) rows in LDS; the query operand
// is then the same for every token and formed once per head. Scores are stored at the tokens'
// positions.
template <int DT, int MODE, int ODT, int NHB>
__global__ __launch_bounds__(JTHREADS, 1) void joint_scores_sorted_kernel(JScoresParams p) {
  constexpr int CB = JCB / NHB;            // 16-token blocks per wave
  constexpr int TOK = JWAVES * CB * 16;    // tokens per workgroup
  static_assert(JSWIN % TOK == 0 && 512 % TOK == 0, "windows hold whole workgroups");
  __shared__ __attribute__((aligned(16))) dkv_u32x4 sB[4][NHB][JDH * JCH / 8];
  // R(n): [2*pp + k][16*g + n] holds (cos, sin) of frequencies 16pp + 4g + 2k and + 1 at delta n
  __shared__ __attribute__((aligned(16))) dkv_f32x4 sRn[8][64];
  // R(16T) of the window's tiles: [T - T0][(2*pp + k) * 4 + g], the same frequencies; rows of 33
  // entries (one of padding), so that lanes reading different tiles' entry (k, g) fall in
  // different banks (with 32-entry rows every tile's entry sits in the same four banks)
  constexpr int RT_ROW = 33;
  __shared__ __attribute__((aligned(16))) dkv_f32x4 sRT[JSWIN / 16][RT_ROW];
  // the query operand of each head: row r = head r's hi part (r < 8) or head r-8's lo part,
  // dword i = frequency i, 16-byte chunk c stored at chunk position c ^ r
  __shared__ __attribute__((aligned(16))) uint32_t sQ[NHB][16 * 64];
  __shared__ int sLen[TOK], sOff[TOK], sPos[TOK];  // in sorted order; sPos -1: a pad entry

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  // workgroup id -> (range of TOK sorted slots, unit = (batch row, window), head group): the
  // ranges from the windows' longest tokens down are the slowest index, so the heaviest
  // workgroups of the whole launch are dispatched first; the head groups of one (range, unit)
  // are consecutive on one XCD (ids are dispatched to the 8 XCDs round-robin), so their shared
  // coefficient loads meet in that XCD's L2
  const int nhg = p.n_basis / NHB, nunits = p.B * p.nwin;
  int rix, unit, hg;
  {
    const int id = blockIdx.x;
    if ((nunits & 7) == 0) {
      const int xcd = id & 7, k = id >> 3;
      hg = k % nhg;
      const int k2 = k / nhg;
      unit = (k2 % (nunits >> 3)) * 8 + xcd;
      rix = k2 / (nunits >> 3);
    } else {
      hg = id % nhg;
      unit = (id / nhg) % nunits;
      rix = id / nhg / nunits;
    }
  }
  const int b = unit / p.nwin, win = unit % p.nwin;
  const int rng = p.win / TOK - 1 - rix;
  const int wbase = win * p.win;  // the window's first position
  const int wlen = min(p.win, p.S - wbase);
  const int s0 = rng * TOK;
  if (s0 >= (wlen + TOK - 1) / TOK * TOK) return;  // past the window's slots (uniform)
  const int h0 = hg * NHB;

  // ---- this thread's token (tid < TOK), the query and table loads, all issued first ----------
  int tlen0 = 0, toff0 = 0, tpos0 = -1;
  if (tid < TOK) {
    const int* srt = p.sorted + ((long long)b * p.nwin + win) * 3 * p.win + s0 + tid;
    tlen0 = srt[0];
    toff0 = srt[p.win];
    tpos0 = srt[2 * p.win];
  }
  tlen0 = min(max(tlen0, 0), p.R);
  // query: (q_i, q_{i+64}) of head slot hh for frequency i = lane; wave hb of the first NHB
  // forms head h0 + hb's operand
  uint32_t qh[8];
  if (wave < NHB) {
    const long long qo = (long long)b * p.q_sb + (long long)(h0 + wave) * p.hpg * p.q_sh + lane;
#pragma unroll
    for (int hh = 0; hh < 8; ++hh) {
      const long long o = qo + (hh < p.hpg ? hh : 0) * p.q_sh;
      qh[hh] = (uint32_t)p.q[o] | ((uint32_t)p.q[o + 64] << 16);
    }
  }
  {
    const int k = tid >> 6;
    const int i0 = 16 * (k >> 1) + 4 * g + 2 * (k & 1);
    const float* delt = p.rope + n * 128 + 2 * i0;
    sRn[k][lane] = dkv_f32x4{delt[0], delt[1], delt[2], delt[3]};
  }
  {
    const int T0 = wbase / 16, ntl = (wlen + 15) / 16;
    for (int e = tid; e < ntl * 32; e += JTHREADS) {
      const int tl = e >> 5, k = (e >> 2) & 7, gg = e & 3;
      const int i0 = 16 * (k >> 1) + 4 * gg + 2 * (k & 1);
      const int T = min(T0 + tl, p.rope_tiles - 1);
      // 16-byte aligned (2 * i0 is a multiple of 4; the host checks the table's alignment)
      sRT[tl][4 * k + gg] = *(const dkv_f32x4*)(p.rope + (long long)(JROPE_FIXED + T) * 128 + 2 * i0);
    }
  }
  // the tokens arrive sorted by chunk count (joint_sort_kernel): a token's products and
  // rotation do not depend on its place in the block, and chunks past its count add zeros
  if (tid < TOK) {
    sLen[tid] = tlen0;
    sOff[tid] = toff0;
    sPos[tid] = tpos0;
  }
  if (wave < NHB) {
    // the query operand of head h0 + wave: R(0) (no rotation) times the score scale, bf16 hi + lo
    uint32_t* qw = sQ[wave];
#pragma unroll
    for (int hh = 0; hh < 8; ++hh)
      if (hh < p.hpg) {
        const float x = dkv_elt_to_f32<DT>(qh[hh] & 0xffffu) * p.scale;
        const float y = dkv_elt_to_f32<DT>(qh[hh] >> 16) * p.scale;
        uint32_t hi, lo;
        dkv_split_bf16x2(x, y, hi, lo);
        qw[hh * 64 + 4 * ((lane >> 2) ^ hh) + (lane & 3)] = hi;
        qw[(8 + hh) * 64 + 4 * ((lane >> 2) ^ (8 + hh)) + (lane & 3)] = lo;
      }
  }
  __syncthreads();

  // this wave's blocks: 8*cb + (w or 7-w), short and long alternately
  int tlen[CB], toff[CB], nchk[CB];
  uint32_t pmask[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int blk = 8 * cb + ((cb & 1) ? 7 - wave : wave);
    tlen[cb] = sLen[16 * blk + n];
    toff[cb] = sOff[16 * blk + n];
    nchk[cb] = __builtin_amdgcn_readfirstlane((sLen[16 * blk + 15] + JCH - 1) / JCH);
    const int e = tlen[cb] - 8 * g;  // 1..7 past a multiple of 32: partial in chunk e / 32
    uint32_t bit = (e > 0 && (e & 31) != 0 && (e & 31) < 8) ? (1u << (e >> 5)) : 0u;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) bit |= (uint32_t)__shfl_xor((int)bit, m, 64);
    pmask[cb] = __builtin_amdgcn_readfirstlane(bit);
  }
  int wmax = 0;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) wmax = max(wmax, nchk[cb]);
  const int nch = (sLen[TOK - 1] + JCH - 1) / JCH;  // the workgroup's longest token

  const uint32_t end = (uint32_t)dkv_flat_tail_elems(p.B, b, p.flat_ld, JFLAT_CAP);
  const __amdgpu_buffer_rsrc_t rs = dkv_make_rsrc(p.flat + (long long)b * p.flat_ld, end * 2u);
  const int bd = tid >> 2, bk = (tid & 3) ^ jswz(bd);
  const uint16_t* bsrc = p.bt + (long long)h0 * p.bt_sh + (long long)bd * JCH + 8 * bk;

  dkv_f32x4 acc[NHB][8][CB];
#pragma unroll
  for (int hh = 0; hh < NHB; ++hh)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) acc[hh][i][cb] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};

  // The rank loop: chunk c's basis sits in sB[c & 3], written at step c-2 (or before the loop),
  // and a barrier follows every odd step, so buffer (c+2) & 3 (last read at step c-2) may take
  // chunk c+2's basis, loaded two steps ago, and the registers it came from the basis of c+4.
  // The coefficients of chunk c+2 are loaded, after chunk c's products are issued, into the
  // registers chunk c used. Each block's products and coefficient loads stop at its own chunk
  // count (wave-uniform branches); loads past the last chunk clamp the basis index.
  auto rank_loop = [&](auto safe_tag) {
    constexpr bool SAFE = decltype(safe_tag)::value;
    auto load_x = [&](int c, dkv_u32x4(&x)[CB]) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        if (c < nchk[cb]) {
          const int j0 = JCH * c + 8 * g;
          if constexpr (SAFE)
            x[cb] = dkv_load8_safe(rs, end, toff[cb] + j0, tlen[cb] - j0);
          else
            x[cb] = dkv_load8_raw(rs, toff[cb] + j0, tlen[cb] - j0);
        }
      }
    };
    dkv_u32x4 xa[CB], xb[CB];
    dkv_u32x4 ba[NHB], bb[NHB];
#pragma unroll
    for (int hh = 0; hh < NHB; ++hh) ba[hh] = bb[hh] = dkv_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) xa[cb] = xb[cb] = dkv_u32x4{0u, 0u, 0u, 0u};
    auto load_b = [&](int c, int hh) {
      return *(const dkv_u32x4*)(bsrc + hh * p.bt_sh + p.bt_sc * min(c, nch - 1));
    };
    if (nch > 0) {
#pragma unroll
      for (int hh = 0; hh < NHB; ++hh) {
        sB[0][hh][tid] = load_b(0, hh);
        sB[1][hh][tid] = load_b(1, hh);
        ba[hh] = load_b(2, hh);
        bb[hh] = load_b(3, hh);
      }
      load_x(0, xa);
      load_x(1, xb);
    }
    __syncthreads();
    auto step = [&](int c, dkv_u32x4(&x)[CB], dkv_u32x4(&bn)[NHB], bool sync) {
#pragma unroll
      for (int hh = 0; hh < NHB; ++hh) {
        sB[(c + 2) & 3][hh][tid] = bn[hh];
        bn[hh] = load_b(c + 4, hh);
      }
      if (c < wmax) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          if (c < nchk[cb] && ((pmask[cb] >> c) & 1u))
            x[cb] = dkv_mask8(x[cb], tlen[cb] - (JCH * c + 8 * g));
        dkv_u32x4 a[NHB][8];
#pragma unroll
        for (int hh = 0; hh < NHB; ++hh)
#pragma unroll
          for (int blk = 0; blk < 8; ++blk)
            a[hh][blk] = sB[c & 3][hh][4 * (16 * blk + n) + (g ^ jswz(n))];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          if (c < nchk[cb]) {
#pragma unroll
            for (int hh = 0; hh < NHB; ++hh)
#pragma unroll
              for (int blk = 0; blk < 8; ++blk)
                acc[hh][blk][cb] = dkv_mfma32<DT>(a[hh][blk], x[cb], acc[hh][blk][cb]);
          }
        load_x(c + 2, x);
      }
      if (sync) __syncthreads();
    };
    int c = 0;
    for (; c + 1 < nch; c += 2) {
      step(c, xa, ba, false);
      step(c + 1, xb, bb, true);
    }
    if (c < nch) step(c, xa, ba, false);
  };
  if (b == p.B - 1)
    rank_loop(std::integral_constant<bool, true>{});
  else
    rank_loop(std::integral_constant<bool, false>{});

  // ---- per block: R(p) of the lane's token, K' hi + lo, scores, masking, stores --------------
  const int hn = n & 7;
  const int qrow = (n & 8) + (hn < p.hpg ? hn : hn % p.hpg);
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int blk = 8 * cb + ((cb & 1) ? 7 - wave : wave);
    const int pos_n = sPos[16 * blk + n];
    // R(p) = R(16T) R(n) for the lane's token: (cos, sin) of its 16 frequencies
    float rc[16], rsn[16];
    {
      const int pl = pos_n < 0 ? 0 : pos_n - wbase;
      const int tl = pl >> 4, nn = pl & 15;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const dkv_f32x4 d = sRn[k][16 * g + nn];
        const dkv_f32x4 t = sRT[tl][4 * k + g];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float ct = t[2 * e], st = t[2 * e + 1], cn = d[2 * e], sn = d[2 * e + 1];
          // frequency 16pp + 4g + 2k' + e with k = 2pp + k': element w = 2k' + e of pair pp
          rc[4 * (k >> 1) + 2 * (k & 1) + e] = ct * cn - st * sn;
          rsn[4 * (k >> 1) + 2 * (k & 1) + e] = st * cn + ct * sn;
        }
      }
    }
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb) {
      const int h = h0 + hb;
      const uint32_t* qw = sQ[hb];
      dkv_f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const dkv_u32x4 bq = *(const dkv_u32x4*)&qw[qrow * 64 + 4 * ((4 * pp + g) ^ qrow)];
        const dkv_f32x4 c0 = acc[hb][pp][cb], c1 = acc[hb][pp + 4][cb];
        uint32_t kh[4], kl[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float cw = rc[4 * pp + w], sw = rsn[4 * pp + w];
          dkv_split_bf16x2(c0[w] * cw - c1[w] * sw, c1[w] * cw + c0[w] * sw, kh[w], kl[w]);
        }
        sc = mfma_bf16x32(dkv_u32x4{kh[0], kh[1], kh[2], kh[3]}, bq, sc);
        sc = mfma_bf16x32(dkv_u32x4{kl[0], kl[1], kl[2], kl[3]}, bq, sc);
      }
      // column n += column n + 8 (the lo part of head n) within each row of 16 lanes
#pragma unroll
      for (int u = 0; u < 4; ++u)
        sc[u] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sc[u]),
                                                            DKV_DPP_ROW_SHL8, 0xf, 0xf, false));
      if (n < p.hpg) {
        const long long ob = (long long)b * p.out_sb + (long long)(h * p.hpg + n) * p.out_sh;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 16 * blk + 4 * g + u;
          const int t = sPos[r];
          if (t >= 0) {
            float z;
            if constexpr (MODE == 0)
              z = sLen[r] > 0 ? sc[u] : -1.0e4f * p.scale;
            else
              z = sLen[r] > 0 ? sc[u] : -INFINITY;
            dkv_store_f32<ODT>(p.out, ob + (long long)t * p.out_ss, z);
          }
        }
      }
    }
  }
}

struct JAvParams {
  const void* scores;
  long long sc_sb, sc_sh, sc_ss;
  const uint16_t* flat;
  long long flat_ld;
  const int* lens;
  long long lens_sb, lens_ss;
  const int* offs;
  long long offs_sb, offs_ss;
  float* rec;  // [B][Hq][n_splits][JPREC]
  uint32_t sc_bytes;  // extent of the scores from their base (vector score loads)
  int B, Hq, S, R, n_splits, split_len;
};

// VEC: the scores are token-contiguous with rows aligned to 4 elements, and a lane loads its 4
// tokens' scores of a tile in one 8- or 16-byte access (else one access per score)
// NHS sets of 16 query heads per workgroup (1 or 2): with 2, each V window is staged and read
// once for both sets' products
template <int DT, int SDT, bool VEC, int NHS>
__global__ __launch_bounds__(JTHREADS, 1) void joint_av_kernel(JAvParams p) {
  // per wave: its rank slice of the current tile's V coefficients, the split kernel's V-window
  // layout: rank r of token t in chunk r/32 at lane slot 16*((r%32)/8) + t, element r%8
  __shared__ __attribute__((aligned(16))) dkv_u32x4 sV[JWAVES][4 * 64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int split = blockIdx.x, hset = blockIdx.y, b = blockIdx.z;
  const int s_begin = split * p.split_len;
  const int s_end = min(p.S, s_begin + p.split_len);
  const int ntiles = s_end > s_begin ? (s_end - s_begin + 15) / 16 : 0;
  const int r0 = 128 * wave;
  int hq[NHS];     // head slot n of each set: this lane's softmax values
  bool hq_ok[NHS];
  long long sbase[NHS];
#pragma unroll
  for (int s = 0; s < NHS; ++s) {
    hq[s] = 16 * (NHS * hset + s) + n;
    hq_ok[s] = hq[s] < p.Hq;
    sbase[s] = (long long)b * p.sc_sb + (long long)(hq_ok[s] ? hq[s] : 0) * p.sc_sh;
  }

  const uint32_t end = (uint32_t)dkv_flat_tail_elems(p.B, b, p.flat_ld, JFLAT_CAP);
  const __amdgpu_buffer_rsrc_t rs = dkv_make_rsrc(p.flat + (long long)b * p.flat_ld, end * 2u);

  // Tile j's inputs for this lane: the metadata (count, offset) of token n, its V pieces (ranks
  // r0 + 32c + 8g .. +8) and the scores of head slot n for tokens 4g .. 4g+3. Every lane issues
  // every load (indices past the split clamp to its last token) and keeps the raw value; counts
  // are clamped, pieces masked and excluded scores replaced where the values are used, two tiles
  // later, so no load is waited for where it is issued.
  auto load_meta = [&](int j, int& l, int& o) {
    const int tc = min(s_begin + 16 * j + n, s_end - 1);
    l = p.lens[(long long)b * p.lens_sb + (long long)tc * p.lens_ss];
    o = p.offs[(long long)b * p.offs_sb + (long long)tc * p.offs_ss];
  };
  auto count = [&](int j, int l) { return s_begin + 16 * j + n < s_end ? min(max(l, 0), p.R) : 0; };
  const __amdgpu_buffer_rsrc_t rz = dkv_make_rsrc(p.scores, p.sc_bytes);
  auto load_z1 = [&](int j, int hs, uint32_t(&z)[4]) {
    if constexpr (VEC) {
      // tokens past the split read their neighbours (zeros past the scores' last element, where
      // the buffer range ends): replaced at use
      const uint32_t e = (uint32_t)(sbase[hs] + s_begin + 16 * j + 4 * g);
      if constexpr (SDT == DKV_F32) {
        const dkv_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rz, e * 4u, 0, 0);
        z[0] = v.x;
        z[1] = v.y;
        z[2] = v.z;
        z[3] = v.w;
      } else {
        // kept packed (two scores per register) until used
        const dkv_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rz, e * 2u, 0, 0);
        z[0] = v.x;
        z[1] = v.y;
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const long long i =
            sbase[hs] + (long long)min(s_begin + 16 * j + 4 * g + u, s_end - 1) * p.sc_ss;
        if constexpr (SDT == DKV_F32)
          z[u] = ((const uint32_t*)p.scores)[i];
        else
          z[u] = ((const uint16_t*)p.scores)[i];
      }
    }
  };
  auto load_z = [&](int j, uint32_t(&z)[NHS][4]) {
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) load_z1(j, hs, z[hs]);
  };
  auto score = [&](int j, int hs, int u, const uint32_t(&zr)[4]) {
    uint32_t raw;
    if constexpr (VEC && SDT != DKV_F32)
      raw = (zr[u >> 1] >> (16 * (u & 1))) & 0xffffu;
    else
      raw = zr[u];
    float v;
    if constexpr (SDT == DKV_F32)
      v = __uint_as_float(raw);
    else
      v = dkv_elt_to_f32<SDT>(raw);
    return (hq_ok[hs] && s_begin + 16 * j + 4 * g + u < s_end) ? v * JLOG2E : -INFINITY;
  };

  dkv_f32x4 acc[NHS][8];
  float m_run[NHS], l_run[NHS];
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[hs][i] = dkv_f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[hs] = -1.0e30f;  // finite floor: excluded tokens give exp2(-inf) = 0
    l_run[hs] = 0.f;
  }
  dkv_u32x4* slot = sV[wave];

  auto tile_loop = [&](auto safe_tag) {
    constexpr bool SAFE = decltype(safe_tag)::value;
    auto load_v = [&](int len, int off, dkv_u32x4(&x)[4]) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int j0 = r0 + 32 * c + 8 * g;
        if constexpr (SAFE)
          x[c] = dkv_load8_safe(rs, end, off + j0, len - j0);
        else
          x[c] = dkv_load8_raw(rs, off + j0, len - j0);
      }
    };
    // Set A holds even tiles, set B odd ones: the V pieces x and raw scores z of its current
    // tile, that tile's count, and the raw metadata (ml, mo) of the tile two ahead. A tile's
    // loads go into the registers its set just used, so no loaded value is ever copied.
    dkv_u32x4 xA[4], xB[4];
    uint32_t zA[NHS][4], zB[NHS][4];
    int cA, cB, mlA, moA, mlB, moB;
    {
      int l0, o0, l1, o1;
      load_meta(0, l0, o0);
      load_meta(1, l1, o1);
      load_meta(2, mlA, moA);
      load_meta(3, mlB, moB);
      cA = count(0, l0);
      cB = count(1, l1);
      load_v(cA, o0, xA);
      load_z(0, zA);
      load_v(cB, o1, xB);
      load_z(1, zB);
    }
    auto step = [&](int j, dkv_u32x4(&x)[4], uint32_t(&zr)[NHS][4], int& cnt, int& ml, int& mo) {
      // a tile none of whose tokens reaches this wave's ranks has only zero pieces here: its
      // products would add exact zeros, so the wave skips them (the online softmax still runs)
      const bool live = __ballot(cnt > r0) != 0ull;
      if (live) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          slot[c * 64 + lane] = dkv_mask8(x[c], cnt - (r0 + 32 * c + 8 * g));
      }
      float z[NHS][4];
#pragma unroll
      for (int hs = 0; hs < NHS; ++hs)
#pragma unroll
        for (int u = 0; u < 4; ++u) z[hs][u] = score(j, hs, u, zr[hs]);
      cnt = count(j + 2, ml);
      load_v(cnt, mo, x);
      load_z(j + 2, zr);
      load_meta(j + 4, ml, mo);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // the wave's V operands of the tile: B of P.X^V by transposed reads
      dkv_u32x2 xv[8];
      if (live) {
        const int u = n >> 2, q = n & 3;
        const uint8_t* vbase =
            (const uint8_t*)slot + 16 * (16 * (q >> 1) + 4 * g + u) + 8 * (q & 1);
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) {
          const uint8_t* src = vbase + (blk >> 1) * 1024 + (blk & 1) * 512;
          xv[blk] = __builtin_bit_cast(
              dkv_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                             (__attribute__((address_space(3))) dkv_i16x4*)(
                                 (__attribute__((address_space(3))) uint8_t*)src)));
        }
      }
      // per set: online softmax of head slot n (its 16 tokens sit in lanes n, n+16, n+32,
      // n+48), P as the A operand, the set's products; one set at a time
#pragma unroll
      for (int hs = 0; hs < NHS; ++hs) {
        float tmax = dkv_max3(dkv_max3(z[hs][0], z[hs][1], z[hs][2]), z[hs][3], z[hs][3]);
        tmax = dkv_lane_max32(tmax);
        tmax = dkv_lane_max16(tmax);
        if (__ballot(tmax > m_run[hs] + JRESCALE)) {
          const float m_new = fmaxf(m_run[hs], tmax);
          const float alpha = __builtin_amdgcn_exp2f(m_run[hs] - m_new);
          l_run[hs] *= alpha;
          m_run[hs] = m_new;
          float au[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) au[u] = __shfl(alpha, 4 * g + u, 64);
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[hs][i][u] *= au[u];
        }
        float pu[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          pu[u] = __builtin_amdgcn_exp2f(z[hs][u] - m_run[hs]);
          l_run[hs] += pu[u];
        }
        if (!live) continue;
        // P.X^V in coefficient space (A: P of head slot n, tokens 4g..4g+3; B: the V reads)
        dkv_u32x4 pa;
        if constexpr (DT == DKV_F16) {
          pa = dkv_u32x4{dkv_pack_f16x2(pu[0], pu[1]), dkv_pack_f16x2(pu[2], pu[3]), 0u, 0u};
        } else {
          uint32_t h01, l01, h23, l23;
          dkv_split_bf16x2(pu[0], pu[1], h01, l01);
          dkv_split_bf16x2(pu[2], pu[3], h23, l23);
          pa = dkv_u32x4{h01, h23, l01, l23};
        }
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) {
          if constexpr (DT == DKV_BF16)
            acc[hs][blk] = dkv_mfma32<DT>(
                pa,
                __builtin_bit_cast(dkv_u32x4, dkv_u64x2{__builtin_bit_cast(uint64_t, xv[blk]),
                                                        __builtin_bit_cast(uint64_t, xv[blk])}),
                acc[hs][blk]);
          else
            acc[hs][blk] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                __builtin_bit_cast(dkv_f16x4, dkv_u32x2{pa.x, pa.y}),
                __builtin_bit_cast(dkv_f16x4, xv[blk]), acc[hs][blk], 0, 0, 0);
        }
        if (NHS > 1) __builtin_amdgcn_sched_barrier(0);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // whole pairs in the loop (every path back to its head has issued both tiles' loads)
    int j = 0;
    for (; j + 1 < ntiles; j += 2) {
      step(j, xA, zA, cA, mlA, moA);
      if (NHS > 1) __builtin_amdgcn_sched_barrier(0);
      step(j + 1, xB, zB, cB, mlB, moB);
      if (NHS > 1) __builtin_amdgcn_sched_barrier(0);
    }
    if (j < ntiles) step(j, xA, zA, cA, mlA, moA);
  };
  if (ntiles > 0) {
    if (b == p.B - 1)
      tile_loop(std::integral_constant<bool, true>{});
    else
      tile_loop(std::integral_constant<bool, false>{});
  }

  // the split's record per head: m and l (identical in every wave: wave 0 writes them), the
  // wave's rank slice of acc (head slot 4g+u, rank r0 + 16*blk + n)
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs) {
    float l_tot = l_run[hs];
    l_tot += __shfl_xor(l_tot, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
    if (wave == 0 && g == 0 && hq_ok[hs]) {
      float* rec = p.rec + (((long long)b * p.Hq + hq[hs]) * p.n_splits + split) * JPREC;
      rec[0] = m_run[hs];
      rec[1] = l_tot;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int head = 16 * (NHS * hset + hs) + 4 * g + u;
      if (head < p.Hq) {
        float* rec = p.rec + (((long long)b * p.Hq + head) * p.n_splits + split) * JPREC + 4;
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) {
          const int r = r0 + 16 * blk + n;
          if (r < p.R) rec[r] = acc[hs][blk][u];
        }
      }
    }
  }
}

struct JMergeParams {
  const float* rec;
  float* part;  // [B][Hq][R/128 rank blocks][Dh] partial projections
  const uint16_t* vb;  // V basis [n_basis][R][Dh] with strides (vb_sh, vb_sr)
  long long vb_sh, vb_sr;
  void* out;
  long long out_sb, out_sh;
  int Hq, R, n_splits, hpg, n_rb;
};

// workgroup = (rank block of 128, V basis hv and up to NH of its query heads, batch row b): the
// split weights, the block's merged coefficients, their projection through the block's basis rows.
// Every load that does not depend on another is issued up front, in the order the values are
// needed (split maxima and sums, the first 16 splits' coefficients, the basis rows), so the
// workgroup waits about one memory latency. NH (4 or 8, the instance for the heads per basis)
// fixes the product loops' trip counts; heads past the group's own count carry zeros.
template <int DT, int MODE, int NH>
__global__ __launch_bounds__(256) void joint_merge_kernel(JMergeParams p) {
  extern __shared__ float sWt[];  // [NH][n_splits]: split weights 2^(m_s - M) / den per head
  __shared__ __attribute__((aligned(16))) float sA[NH][JRB];
  __shared__ float sOut[4][NH][JDH];
  const int rb = blockIdx.x;
  const int chunks = (p.hpg + NH - 1) / NH;
  const int hv = blockIdx.y / chunks, j0 = (blockIdx.y % chunks) * NH;
  const int b = blockIdx.z;
  const int nh = min(NH, p.hpg - j0);
  const int nr = min(JRB, p.R - JRB * rb);  // ranks of this block
  const int ns = p.n_splits;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long long head0 = (long long)b * p.Hq + hv * p.hpg + j0;

  // (1) m, l of split `lane` for heads wave and wave + 4 (up to 64 splits in registers)
  float mv[2], lv[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int j = wave + 4 * i;
    const float* base =
        p.rec + (head0 + min(j, nh - 1)) * ns * JPREC + (long long)min(lane, ns - 1) * JPREC;
    mv[i] = base[0];
    lv[i] = base[1];
  }
  // (2) coefficients of the first 16 splits: thread = (head jc, ranks 4q .. 4q+3 of the block)
  const int jc = tid >> 5, q = tid & 31;
  const float* cbase =
      p.rec + (head0 + min(jc, nh - 1)) * ns * JPREC + 4 + JRB * rb + 4 * min(q, (nr - 1) / 4);
  dkv_f32x4 x[16];
  auto load_coef = [&](int s0) {
#pragma unroll
    for (int u = 0; u < 16; ++u)
      x[u] = *(const dkv_f32x4*)(cbase + (long long)min(s0 + u, ns - 1) * JPREC);
  };
  if (jc < NH) load_coef(0);
  // (3) basis rows: thread = (dims 2dp, 2dp+1, ranks 32rq .. 32rq+31 of the block)
  const int dp = tid & 63, rq = tid >> 6;
  uint32_t vbv[32];
  {
    const uint16_t* vb = p.vb + (long long)hv * p.vb_sh +
                         (long long)(JRB * rb + 32 * rq) * p.vb_sr + 2 * dp;
    const int kmax = nr - 1 - 32 * rq;  // rows past the block's end read its last row
    if (kmax >= 31) {
#pragma unroll
      for (int k = 0; k < 32; ++k) vbv[k] = *(const uint32_t*)(vb + (long long)k * p.vb_sr);
    } else {
#pragma unroll
      for (int k = 0; k < 32; ++k)
        vbv[k] = *(const uint32_t*)(vb + (long long)max(min(k, kmax), -32 * rq) * p.vb_sr);
    }
  }

  // weights: one wave per head
  auto weights = [&](int j, float m_in, float l_in) {
    const float* base = p.rec + (head0 + j) * ns * JPREC;
    float M, L;
    if (ns <= 64) {
      const float m = lane < ns ? m_in : -INFINITY;
      M = dkv_wave_max(m);
      L = dkv_wave_sum(lane < ns ? __builtin_amdgcn_exp2f(m - M) * l_in : 0.f);
    } else {
      M = -INFINITY;
      for (int s = lane; s < ns; s += 64) M = fmaxf(M, base[(long long)s * JPREC]);
      M = dkv_wave_max(M);
      L = 0.f;
      for (int s = lane; s < ns; s += 64)
        L += __builtin_amdgcn_exp2f(base[(long long)s * JPREC] - M) * base[(long long)s * JPREC + 1];
      L = dkv_wave_sum(L);
    }
    const float den = MODE == 0 ? fmaxf(L, 1e-6f) : L;
    if (ns <= 64) {
      if (lane < ns) sWt[j * ns + lane] = __builtin_amdgcn_exp2f(m_in - M) / den;
    } else {
      for (int s = lane; s < ns; s += 64)
        sWt[j * ns + s] = __builtin_amdgcn_exp2f(base[(long long)s * JPREC] - M) / den;
    }
  };
  if (wave < nh) weights(wave, mv[0], lv[0]);
  if (wave + 4 < nh) weights(wave + 4, mv[1], lv[1]);
  __syncthreads();

  // merged, normalised coefficients of the block (rows of heads past nh: zeros)
  if (jc < NH) {
    dkv_f32x4 a = {0.f, 0.f, 0.f, 0.f};
    if (jc < nh) {
      for (int s0 = 0;;) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const float w = s0 + u < ns ? sWt[jc * ns + s0 + u] : 0.f;
          a += w * x[u];
        }
        s0 += 16;
        if (s0 >= ns) break;
        load_coef(s0);
      }
      // ranks past the block's end (never written by the V pass) hold zeros
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = 4 * q + e < nr ? a[e] : 0.f;
    }
    *(dkv_f32x4*)&sA[jc][4 * q] = a;
  }
  __syncthreads();

  // partial[j][d] = sum over the block's ranks of a[j][r] VB[r][d], per quarter of the block
  float o0[NH], o1[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j) o0[j] = o1[j] = 0.f;
#pragma unroll
  for (int k4 = 0; k4 < 8; ++k4) {
    dkv_f32x4 av[NH];
#pragma unroll
    for (int j = 0; j < NH; ++j) av[j] = *(const dkv_f32x4*)&sA[j][32 * rq + 4 * k4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = vbv[4 * k4 + e];
      const float v0 = dkv_elt_to_f32<DT>(w & 0xffffu), v1 = dkv_elt_to_f32<DT>(w >> 16);
#pragma unroll
      for (int j = 0; j < NH; ++j) {  // a = 0 past the block's end and for absent heads
        o0[j] = fmaf(av[j][e], v0, o0[j]);
        o1[j] = fmaf(av[j][e], v1, o1[j]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    sOut[rq][j][2 * dp] = o0[j];
    sOut[rq][j][2 * dp + 1] = o1[j];
  }
  __syncthreads();
  for (int i = tid; i < nh * JDH; i += 256) {
    const int j = i / JDH, d = i % JDH;
    p.part[((head0 + j) * p.n_rb + rb) * JDH + d] =
        (sOut[0][j][d] + sOut[1][j][d]) + (sOut[2][j][d] + sOut[3][j][d]);
  }
}

// workgroup = (query head, batch row b), thread = output dim: the sum of the rank blocks' partial
// projections, the output rounding
template <int ODT>
__global__ __launch_bounds__(JDH) void joint_project_sum_kernel(JMergeParams p) {
  const int hq = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const float* part = p.part + (((long long)b * p.Hq + hq) * p.n_rb) * JDH + d;
  float o = 0.f;
  for (int k = 0; k < p.n_rb; ++k) o += part[(long long)k * JDH];
  dkv_store_f32<ODT>(p.out, (long long)b * p.out_sb + (long long)hq * p.out_sh + d, o);
}

// sets of 16 query heads per V-pass workgroup: two when the sets pair up
int joint_av_hsets(int Hq) { return ((Hq + 15) / 16) % 2 == 0 ? 2 : 1; }

int joint_av_split_len(int B, int Hq, int S) {
  // One 8-wave workgroup per CU (200 VGPRs with two head sets, 132 with one): rounds of 256
  // workgroups, each (token split, head-set workgroup, batch row), at a fixed cost of about 150
  // tokens per workgroup (measured on MI355X at B = 16, S = 8192: V pass + merge 72 us with 16
  // splits of 512 tokens, 88 with 32 of 256).
  const long long units = (long long)B * ((Hq + 15) / 16 / joint_av_hsets(Hq));
  const long long sl = dkv_rounds_split(units, S, 150, 16, 16, JMAX_SPLITS);
  return (int)(sl < 16 ? 16 : sl);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace

extern "C" long long dkv_joint_scores_workspace_ints(int B, int S) {
  if (B <= 0 || S <= 0) return 0;
  const long long win = joint_window(S);
  return (long long)B * ((S + win - 1) / win) * 3 * win;
}

extern "C" int dkv_joint_scores(void* stream, int mode, int dtype, int out_dtype, const void* q,
                                long long q_sb, long long q_sh, const void* basis_t,
                                long long bt_sh, long long bt_sc, int n_basis, const void* flat,
                                long long flat_ld, const int* lens, long long lens_sb,
                                long long lens_ss, const int* offs, long long offs_sb,
                                long long offs_ss, const float* rope, int rope_tiles,
                                int* workspace, long long workspace_ints, void* out,
                                long long out_sb, long long out_sh, long long out_ss, int B,
                                int Hq, int S, int R, int Dh) {
  if (mode != 0 && mode != 1) return DKV_E_ARG;
  if (dtype != DKV_BF16 && dtype != DKV_F16) return DKV_E_UNSUPPORTED;
  if (out_dtype != DKV_F32 && out_dtype != DKV_F16 && out_dtype != DKV_BF16) return DKV_E_ARG;
  if (mode == 1 && out_dtype != DKV_F32) return DKV_E_ARG;
  if (B < 0 || Hq < 0 || S < 0 || R <= 0 || n_basis <= 0) return DKV_E_ARG;
  if (Dh != JDH || R % JCH != 0 || R > JRMAX) return DKV_E_UNSUPPORTED;
  if (Hq % n_basis != 0 || Hq / n_basis > 8) return DKV_E_UNSUPPORTED;
  if (B == 0 || Hq == 0 || S == 0) return DKV_OK;
  if (!q || !basis_t || !flat || !lens || !offs || !rope || !out) return DKV_E_ARG;
  if (!aligned16(basis_t) || bt_sc < JDH * JCH || bt_sc % 8 != 0 || bt_sh % 8 != 0)
    return DKV_E_UNSUPPORTED;
  if (flat_ld <= 0 || flat_ld > JFLAT_CAP - 8) return DKV_E_UNSUPPORTED;
  if (rope_tiles < (S + 15) / 16) return DKV_E_ARG;
  if (B > 65535 || n_basis > 65535) return DKV_E_UNSUPPORTED;
  if (!aligned16(rope)) return DKV_E_UNSUPPORTED;
  if (!workspace || ((uintptr_t)workspace & 3) ||
      workspace_ints < dkv_joint_scores_workspace_ints(B, S))
    return DKV_E_ARG;
  JScoresParams p;
  p.q = (const uint16_t*)q;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.bt = (const uint16_t*)basis_t;
  p.bt_sh = bt_sh;
  p.bt_sc = bt_sc;
  p.flat = (const uint16_t*)flat;
  p.flat_ld = flat_ld;
  p.lens = lens;
  p.lens_sb = lens_sb;
  p.lens_ss = lens_ss;
  p.offs = offs;
  p.offs_sb = offs_sb;
  p.offs_ss = offs_ss;
  p.rope = rope;
  p.rope_tiles = rope_tiles;
  p.out = out;
  p.out_sb = out_sb;
  p.out_sh = out_sh;
  p.out_ss = out_ss;
  p.B = B;
  p.S = S;
  p.R = R;
  p.hpg = Hq / n_basis;
  p.scale = 1.0f / sqrtf((float)Dh);
  p.sorted = workspace;
  p.win = joint_window(S);
  p.nwin = (S + p.win - 1) / p.win;
  // two basis heads per workgroup when the heads pair up (each coefficient load then serves
  // both heads' products)
  const int nhb = n_basis % 2 == 0 ? 2 : 1;
  const int tok = JTOK / nhb;
  p.n_basis = n_basis;
  const long long n_wg = (long long)p.nwin * (p.win / tok) * (n_basis / nhb) * B;
  if (n_wg > 0x7fffffffLL) return DKV_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  {
    JSortParams sp;
    sp.lens = lens;
    sp.lens_sb = lens_sb;
    sp.lens_ss = lens_ss;
    sp.offs = offs;
    sp.offs_sb = offs_sb;
    sp.offs_ss = offs_ss;
    sp.sorted = workspace;
    sp.S = S;
    sp.R = R;
    sp.win = p.win;
    sp.nwin = p.nwin;
    sp.tok = tok;
    hipLaunchKernelGGL(joint_sort_kernel, dim3((unsigned)p.nwin, (unsigned)B), dim3(JSORT_THREADS),
                       0, st, sp);
  }
  const dim3 grid((unsigned)n_wg);
#define DKV_JS_LAUNCH(DT_, MODE_, ODT_)                                                        \
  do {                                                                                         \
    if (nhb == 2)                                                                              \
      hipLaunchKernelGGL((joint_scores_sorted_kernel<DT_, MODE_, ODT_, 2>), grid,              \
                         dim3(JTHREADS), 0, st, p);                                            \
    else                                                                                       \
      hipLaunchKernelGGL((joint_scores_sorted_kernel<DT_, MODE_, ODT_, 1>), grid,              \
                         dim3(JTHREADS), 0, st, p);                                            \
  } while (0)
  if (mode == 1) {
    if (dtype == DKV_BF16) DKV_JS_LAUNCH(DKV_BF16, 1, DKV_F32);
    else DKV_JS_LAUNCH(DKV_F16, 1, DKV_F32);
  } else if (dtype == DKV_BF16) {
    if (out_dtype == DKV_BF16) DKV_JS_LAUNCH(DKV_BF16, 0, DKV_BF16);
    else if (out_dtype == DKV_F16) DKV_JS_LAUNCH(DKV_BF16, 0, DKV_F16);
    else DKV_JS_LAUNCH(DKV_BF16, 0, DKV_F32);
  } else {
    if (out_dtype == DKV_BF16) DKV_JS_LAUNCH(DKV_F16, 0, DKV_BF16);
    else if (out_dtype == DKV_F16) DKV_JS_LAUNCH(DKV_F16, 0, DKV_F16);
    else DKV_JS_LAUNCH(DKV_F16, 0, DKV_F32);
  }
#undef DKV_JS_LAUNCH
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" long long dkv_joint_av_workspace_floats(int B, int Hq, int S, int R) {
  if (B <= 0 || Hq <= 0 || S <= 0 || R <= 0 || R > JRMAX) return 0;
  const int sl = joint_av_split_len(B, Hq, S);
  const long long ns = (S + sl - 1) / sl;
  const long long n_rb = (R + JRB - 1) / JRB;
  return (long long)B * Hq * (ns * JPREC + n_rb * JDH);
}

extern "C" int dkv_joint_av(void* stream, int mode, int scores_dtype, int dtype, int out_dtype,
                            const void* scores, long long sc_sb, long long sc_sh, long long sc_ss,
                            const void* basis, long long basis_sh, long long basis_sr, int n_basis,
                            const void* flat, long long flat_ld, const int* lens, long long lens_sb,
                            long long lens_ss, const int* offs, long long offs_sb,
                            long long offs_ss, float* workspace, long long workspace_floats,
                            void* out, long long out_sb, long long out_sh, int B, int Hq, int S,
                            int R, int Dh) {
  if (mode != 0 && mode != 1) return DKV_E_ARG;
  if (dtype != DKV_BF16 && dtype != DKV_F16) return DKV_E_UNSUPPORTED;
  if (scores_dtype != DKV_F32 && scores_dtype != DKV_F16 && scores_dtype != DKV_BF16)
    return DKV_E_ARG;
  if (out_dtype != DKV_F32 && out_dtype != DKV_F16 && out_dtype != DKV_BF16) return DKV_E_ARG;
  if (B < 0 || Hq < 0 || S < 0 || R <= 0 || n_basis <= 0) return DKV_E_ARG;
  if (Dh != JDH || R > JRMAX) return DKV_E_UNSUPPORTED;
  if (Hq % n_basis != 0) return DKV_E_ARG;
  if (B == 0 || Hq == 0) return DKV_OK;
  if (S == 0) return DKV_E_UNSUPPORTED;  // the reference's empty-cache result: generic path
  if (!scores || !basis || !flat || !lens || !offs || !out || !workspace) return DKV_E_ARG;
  if (flat_ld <= 0 || flat_ld > JFLAT_CAP - 8) return DKV_E_UNSUPPORTED;
  if (B > 65535 || Hq > 65535) return DKV_E_UNSUPPORTED;
  const int sl = joint_av_split_len(B, Hq, S);
  const int ns = (S + sl - 1) / sl;
  const int n_rb = (R + JRB - 1) / JRB;
  const long long rec_floats = (long long)B * Hq * ns * JPREC;
  if (workspace_floats < rec_floats + (long long)B * Hq * n_rb * JDH) return DKV_E_WORKSPACE;
  if (!aligned16(workspace)) return DKV_E_ARG;
  // the merge reads the V basis two dims (4 bytes) at a time
  if (((uintptr_t)basis & 3u) || (basis_sr & 1) || (basis_sh & 1)) return DKV_E_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;

  JAvParams a;
  a.scores = scores;
  a.sc_sb = sc_sb;
  a.sc_sh = sc_sh;
  a.sc_ss = sc_ss;
  a.flat = (const uint16_t*)flat;
  a.flat_ld = flat_ld;
  a.lens = lens;
  a.lens_sb = lens_sb;
  a.lens_ss = lens_ss;
  a.offs = offs;
  a.offs_sb = offs_sb;
  a.offs_ss = offs_ss;
  a.rec = workspace;
  a.B = B;
  a.Hq = Hq;
  a.S = S;
  a.R = R;
  a.n_splits = ns;
  a.split_len = sl;
  const int nhs = joint_av_hsets(Hq);
  const dim3 agrid((unsigned)ns, (unsigned)((Hq + 15) / 16 / nhs), (unsigned)B);
  // vector score loads: token-contiguous rows whose starts are 4-element aligned and a token
  // count that is a multiple of 4, so each lane's group of 4 scores lies wholly inside or
  // wholly past the scores' last element; the buffer range ends exactly at that element (the
  // prefetch of tiles past the last row's end returns zeros and touches no memory), within
  // what a 32-bit byte offset covers
  const int sc_elt = scores_dtype == DKV_F32 ? 4 : 2;
  const long long sc_shape[3] = {B, Hq, S}, sc_stride[3] = {sc_sb, sc_sh, sc_ss};
  const long long sc_extent = dkv_view_extent(3, sc_shape, sc_stride) * sc_elt;
  const bool vec = sc_ss == 1 && S % 4 == 0 && sc_sb % 4 == 0 && sc_sh % 4 == 0 && sc_sb >= 0 &&
                   sc_sh >= 0 && ((uintptr_t)scores % (4 * sc_elt)) == 0 &&
                   sc_extent < (1LL << 31);
  a.sc_bytes = vec ? (uint32_t)sc_extent : 0u;
#define DKV_JA_LAUNCH(DT_, SDT_)                                                              \
  do {                                                                                        \
    if (vec && nhs == 2)                                                                      \
      hipLaunchKernelGGL((joint_av_kernel<DT_, SDT_, true, 2>), agrid, dim3(JTHREADS), 0, st, a); \
    else if (vec)                                                                             \
      hipLaunchKernelGGL((joint_av_kernel<DT_, SDT_, true, 1>), agrid, dim3(JTHREADS), 0, st, a); \
    else if (nhs == 2)                                                                        \
      hipLaunchKernelGGL((joint_av_kernel<DT_, SDT_, false, 2>), agrid, dim3(JTHREADS), 0, st, a); \
    else                                                                                      \
      hipLaunchKernelGGL((joint_av_kernel<DT_, SDT_, false, 1>), agrid, dim3(JTHREADS), 0, st, a); \
  } while (0)
  if (dtype == DKV_BF16) {
    if (scores_dtype == DKV_F32) DKV_JA_LAUNCH(DKV_BF16, DKV_F32);
    else if (scores_dtype == DKV_BF16) DKV_JA_LAUNCH(DKV_BF16, DKV_BF16);
    else DKV_JA_LAUNCH(DKV_BF16, DKV_F16);
  } else {
    if (scores_dtype == DKV_F32) DKV_JA_LAUNCH(DKV_F16, DKV_F32);
    else if (scores_dtype == DKV_BF16) DKV_JA_LAUNCH(DKV_F16, DKV_BF16);
    else DKV_JA_LAUNCH(DKV_F16, DKV_F16);
  }
#undef DKV_JA_LAUNCH
  DKV_HIP_CHECK_LAUNCH();

  JMergeParams m;
  m.rec = workspace;
  m.part = workspace + rec_floats;
  m.vb = (const uint16_t*)basis;
  m.vb_sh = basis_sh;
  m.vb_sr = basis_sr;
  m.out = out;
  m.out_sb = out_sb;
  m.out_sh = out_sh;
  m.Hq = Hq;
  m.R = R;
  m.n_splits = ns;
  const int hpg = Hq / n_basis;
  m.hpg = hpg;
  m.n_rb = n_rb;
  const int nhm = hpg <= 4 ? 4 : 8;  // query heads merged and projected together
  const dim3 mgrid((unsigned)n_rb, (unsigned)(n_basis * ((hpg + nhm - 1) / nhm)), (unsigned)B);
  const size_t wt_bytes = sizeof(float) * nhm * (size_t)ns;
  if (dtype == DKV_BF16) {
    if (mode == 0)
      {
        if (nhm == 4)
          hipLaunchKernelGGL((joint_merge_kernel<DKV_BF16, 0, 4>), mgrid, dim3(256), wt_bytes, st, m);
        else
          hipLaunchKernelGGL((joint_merge_kernel<DKV_BF16, 0, 8>), mgrid, dim3(256), wt_bytes, st, m);
      }
    else
      {
        if (nhm == 4)
          hipLaunchKernelGGL((joint_merge_kernel<DKV_BF16, 1, 4>), mgrid, dim3(256), wt_bytes, st, m);
        else
          hipLaunchKernelGGL((joint_merge_kernel<DKV_BF16, 1, 8>), mgrid, dim3(256), wt_bytes, st, m);
      }
  } else {
    if (mode == 0)
      {
        if (nhm == 4)
          hipLaunchKernelGGL((joint_merge_kernel<DKV_F16, 0, 4>), mgrid, dim3(256), wt_bytes, st, m);
        else
          hipLaunchKernelGGL((joint_merge_kernel<DKV_F16, 0, 8>), mgrid, dim3(256), wt_bytes, st, m);
      }
    else
      {
        if (nhm == 4)
          hipLaunchKernelGGL((joint_merge_kernel<DKV_F16, 1, 4>), mgrid, dim3(256), wt_bytes, st, m);
        else
          hipLaunchKernelGGL((joint_merge_kernel<DKV_F16, 1, 8>), mgrid, dim3(256), wt_bytes, st, m);
      }
  }
  DKV_HIP_CHECK_LAUNCH();
  const dim3 pgrid((unsigned)Hq, (unsigned)B);
  if (out_dtype == DKV_BF16)
    hipLaunchKernelGGL((joint_project_sum_kernel<DKV_BF16>), pgrid, dim3(JDH), 0, st, m);
  else if (out_dtype == DKV_F16)
    hipLaunchKernelGGL((joint_project_sum_kernel<DKV_F16>), pgrid, dim3(JDH), 0, st, m);
  else
    hipLaunchKernelGGL((joint_project_sum_kernel<DKV_F32>), pgrid, dim3(JDH), 0, st, m);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
