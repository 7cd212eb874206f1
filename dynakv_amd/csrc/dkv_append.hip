// Packed-cache writers: decode append (one token per row), K+V decode append in one
// launch, sync-free prefill packing, and dense re-expansion.
//
// Reference behaviour: src/dynakv/kernels/compressed_cache.py:7-34 (decode kernel),
// :182-209 (prefill branch), :36-56 (simple_decompress).
#include "dkv_common.h"

namespace {

// One wave per row. Lane 0 claims the row's range by bumping ptr (one writer per row, so no
// atomic is needed), then the wave copies the first min(len, max_dim) elements.
template <typename T>
__device__ __forceinline__ void append_row(const T* __restrict__ states, long long states_ld,
                                           const int* __restrict__ new_len, long long new_len_ld,
                                           T* __restrict__ flat, long long flat_ld,
                                           int* __restrict__ lens, int* __restrict__ offs,
                                           long long tab_sb, long long tab_ss,
                                           int* __restrict__ ptr, int seq_pos, int row,
                                           int max_dim) {
  const int lane = threadIdx.x & 63;
  const int len = new_len[(long long)row * new_len_ld];
  const int off = ptr[row];
  if (lane == 0) {
    ptr[row] = off + len;
    lens[(long long)row * tab_sb + (long long)seq_pos * tab_ss] = len;
    offs[(long long)row * tab_sb + (long long)seq_pos * tab_ss] = off;
  }
  const int n = min(len, max_dim);
  const T* src = states + (long long)row * states_ld;
  T* dst = flat + (long long)row * flat_ld + off;
  for (int j = lane; j < n; j += 64) dst[j] = src[j];
}

template <typename T>
__global__ __launch_bounds__(256) void append_decode_kernel(
    const T* __restrict__ states, long long states_ld, const int* __restrict__ new_len,
    long long new_len_ld, T* __restrict__ flat, long long flat_ld, int* __restrict__ lens,
    int* __restrict__ offs, long long tab_sb, long long tab_ss, int* __restrict__ ptr,
    int seq_pos, int rows, int max_dim) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  append_row<T>(states, states_ld, new_len, new_len_ld, flat, flat_ld, lens, offs, tab_sb,
                tab_ss, ptr, seq_pos, row, max_dim);
}

struct AppendSlot {
  const void* states;
  long long states_ld;
  const int* new_len;
  long long new_len_ld;
  void* flat;
  long long flat_ld;
  int* lens;
  int* offs;
  long long tab_sb, tab_ss;
  int* ptr;
};

// blockIdx.y selects the K (0) or V (1) slot.
template <typename T>
__global__ __launch_bounds__(256) void append_decode_kv_kernel(AppendSlot k, AppendSlot v,
                                                               int seq_pos, int rows,
                                                               int max_dim) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const AppendSlot s = blockIdx.y == 0 ? k : v;
  append_row<T>((const T*)s.states, s.states_ld, s.new_len, s.new_len_ld, (T*)s.flat,
                s.flat_ld, s.lens, s.offs, s.tab_sb, s.tab_ss, s.ptr, seq_pos, row, max_dim);
}

// Prefill append, workgroup (row, chunk): AP_CHUNK tokens of one row. The row's offsets before
// the chunk come from a reduction over the earlier tokens' counts (every workgroup reads the
// row's old pointer, so the pointer itself is advanced by append_prefill_ptr_kernel, launched
// after); wave 0 scans the chunk, then each wave copies its tokens four at a time (all loads
// of a group issued before its stores). Offsets follow the unclipped counts, the coefficients
// are stored at the clipped ones (min(len, max_dim)), as in the one-token append.
constexpr int AP_CHUNK = 64;
// one slot (K or V cache of a layer) of a prefill append
struct PrefillSlot {
  const void* states;
  long long states_sb, states_ss;
  const int* new_len;
  long long len_sb, len_ss;
  void* flat;
  long long flat_ld;
  int* lens;
  int* offs;
  long long tab_sb, tab_ss;
  int* ptr;
};

template <typename T>
__global__ __launch_bounds__(256) void append_prefill_kernel(PrefillSlot s0, PrefillSlot s1,
                                                             int seq_pos, int n_new, int max_dim) {
  // slot blockIdx.z: K, or V in a two-slot launch
  const PrefillSlot& sl = blockIdx.z ? s1 : s0;
  const T* __restrict__ states = (const T*)sl.states;
  const long long states_sb = sl.states_sb, states_ss = sl.states_ss;
  const int* __restrict__ new_len = sl.new_len;
  const long long len_sb = sl.len_sb, len_ss = sl.len_ss;
  T* __restrict__ flat = (T*)sl.flat;
  const long long flat_ld = sl.flat_ld;
  int* __restrict__ lens = sl.lens;
  int* __restrict__ offs = sl.offs;
  const long long tab_sb = sl.tab_sb, tab_ss = sl.tab_ss;
  const int* __restrict__ ptr = sl.ptr;
  __shared__ long long s_red[2][4];
  __shared__ long long s_dst[AP_CHUNK];
  __shared__ int s_clen[AP_CHUNK];
  const int row = blockIdx.x, c0 = blockIdx.y * AP_CHUNK;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long long start = ptr[row];
  const int* lrow = new_len + (long long)row * len_sb;
  // counts of the tokens before the chunk
  long long pu = 0, pc = 0;
  for (int t = tid; t < c0; t += 256) {
    const int len = lrow[(long long)t * len_ss];
    pu += len;
    pc += max(0, min(len, max_dim));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    pu += __shfl_xor(pu, o, 64);
    pc += __shfl_xor(pc, o, 64);
  }
  if (lane == 0) {
    s_red[0][wave] = pu;
    s_red[1][wave] = pc;
  }
  __syncthreads();
  if (wave == 0) {
    const long long bu = s_red[0][0] + s_red[0][1] + s_red[0][2] + s_red[0][3];
    const long long bc = s_red[1][0] + s_red[1][1] + s_red[1][2] + s_red[1][3];
    const int t = c0 + lane;
    const int len = t < n_new ? lrow[(long long)t * len_ss] : 0;
    const int clen = max(0, min(len, max_dim));
    long long iu = len, ic = clen;  // inclusive scans over the chunk
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const long long ou = __shfl_up(iu, d, 64), oc = __shfl_up(ic, d, 64);
      if (lane >= d) {
        iu += ou;
        ic += oc;
      }
    }
    if (t < n_new) {
      const long long ti = (long long)row * tab_sb + (long long)(seq_pos + t) * tab_ss;
      lens[ti] = len;
      offs[ti] = (int)(start + bu + iu - len);
    }
    s_dst[lane] = start + bc + ic - clen;
    s_clen[lane] = clen;
  }
  __syncthreads();
  T* frow = flat + (long long)row * flat_ld;
  const T* srow = states + (long long)row * states_sb;
  const int nt = min(AP_CHUNK, n_new - c0);
  for (int t0 = 4 * wave; t0 < nt; t0 += 16) {
    // tokens t0 .. t0+3 of the chunk: lane j copies element j (and j + 64) of each
    T v[4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tt = t0 + u;
      const int c = tt < nt ? s_clen[tt] : 0;
      const T* src = srow + (long long)(c0 + tt) * states_ss;
#pragma unroll
      for (int h = 0; h < 2; ++h) v[u][h] = lane + 64 * h < c ? src[lane + 64 * h] : T(0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tt = t0 + u;
      const int c = tt < nt ? s_clen[tt] : 0;
      T* dst = frow + s_dst[tt < nt ? tt : 0];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (lane + 64 * h < c) dst[lane + 64 * h] = v[u][h];
    }
    // counts above 128 (max_dim past the per-head rank): the rest element by element
    for (int u = 0; u < 4; ++u) {
      const int tt = t0 + u;
      if (tt >= nt) break;
      const int c = s_clen[tt];
      const T* src = srow + (long long)(c0 + tt) * states_ss;
      T* dst = frow + s_dst[tt];
      for (int j = 128 + lane; j < c; j += 64) dst[j] = src[j];
    }
  }
}

// ptr[row] += sum over the appended tokens of min(len, max_dim)
__global__ __launch_bounds__(256) void append_prefill_ptr_kernel(PrefillSlot s0, PrefillSlot s1,
                                                                int n_new, int max_dim) {
  const PrefillSlot& sl = blockIdx.y ? s1 : s0;
  const int* __restrict__ new_len = sl.new_len;
  const long long len_sb = sl.len_sb, len_ss = sl.len_ss;
  int* __restrict__ ptr = sl.ptr;
  __shared__ long long s_red[4];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  long long pc = 0;
  for (int t = tid; t < n_new; t += 256)
    pc += max(0, min(new_len[(long long)row * len_sb + (long long)t * len_ss], max_dim));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) pc += __shfl_xor(pc, o, 64);
  if (lane == 0) s_red[wave] = pc;
  __syncthreads();
  if (tid == 0) ptr[row] = (int)(ptr[row] + s_red[0] + s_red[1] + s_red[2] + s_red[3]);
}

// out[b, t, j] = flat[b, offs[b,t] + j] for j < min(lens, max_dim), else 0.
template <typename T>
__global__ __launch_bounds__(256) void decompress_kernel(const T* __restrict__ flat,
                                                         long long flat_ld,
                                                         const int* __restrict__ lens,
                                                         const int* __restrict__ offs,
                                                         long long tab_sb, long long tab_ss,
                                                         T* __restrict__ out, int seq,
                                                         int max_dim) {
  const int row = blockIdx.y;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= seq) return;
  const int lane = threadIdx.x & 63;
  const long long ti = (long long)row * tab_sb + (long long)t * tab_ss;
  const int n = max(0, min(lens[ti], max_dim));
  const T* src = flat + (long long)row * flat_ld + offs[ti];
  T* dst = out + ((long long)row * seq + t) * max_dim;
  for (int j = lane; j < max_dim; j += 64) dst[j] = j < n ? src[j] : (T)0;
}

}  // namespace

extern "C" int dkv_version(void) { return DKV_VERSION; }

extern "C" long long dkv_flat_range_elems(long long rows, long long row, long long ld) {
  return dkv_flat_tail_elems(rows, row, ld, DKV_FLAT_RSRC_CAP);
}

extern "C" long long dkv_view_extent_elems(int nd, const long long* shape,
                                           const long long* stride) {
  if (nd < 0 || (nd > 0 && (!shape || !stride))) return -1;
  return dkv_view_extent(nd, shape, stride);
}

extern "C" const char* dkv_status_string(int status) {
  switch (status) {
    case DKV_OK: return "ok";
    case DKV_E_ARG: return "invalid argument";
    case DKV_E_UNSUPPORTED: return "unsupported configuration";
    case DKV_E_WORKSPACE: return "workspace too small";
    case DKV_E_SCRATCH: return "call needs more than the fixed no-allocation scratch";
    default: break;
  }
  if (status <= -DKV_E_HIP_BASE) return hipGetErrorString((hipError_t)(-status - DKV_E_HIP_BASE));
  return "unknown status";
}

extern "C" int dkv_append_decode(void* stream, int dtype, const void* states, long long states_ld,
                                 const int* new_len, long long new_len_ld, void* flat,
                                 long long flat_ld, int* lens, int* offs, long long tab_sb,
                                 long long tab_ss, int* ptr, int seq_pos, int rows, int max_dim) {
  if (rows < 0 || max_dim < 0 || seq_pos < 0) return DKV_E_ARG;
  if (rows == 0) return DKV_OK;
  if (!states || !new_len || !flat || !lens || !offs || !ptr) return DKV_E_ARG;
  const int es = dkv_elt_size(dtype);
  if (es == 0) return DKV_E_ARG;
  dim3 grid((rows + 3) / 4), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (es == 4)
    hipLaunchKernelGGL(append_decode_kernel<uint32_t>, grid, block, 0, s, (const uint32_t*)states,
                       states_ld, new_len, new_len_ld, (uint32_t*)flat, flat_ld, lens, offs,
                       tab_sb, tab_ss, ptr, seq_pos, rows, max_dim);
  else
    hipLaunchKernelGGL(append_decode_kernel<uint16_t>, grid, block, 0, s, (const uint16_t*)states,
                       states_ld, new_len, new_len_ld, (uint16_t*)flat, flat_ld, lens, offs,
                       tab_sb, tab_ss, ptr, seq_pos, rows, max_dim);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_append_decode_kv(
    void* stream, int dtype, int rows, int max_dim, int seq_pos, const void* states_k,
    long long states_k_ld, const int* new_len_k, long long new_len_k_ld, void* flat_k,
    long long flat_k_ld, int* lens_k, int* offs_k, long long tab_k_sb, long long tab_k_ss,
    int* ptr_k, const void* states_v, long long states_v_ld, const int* new_len_v,
    long long new_len_v_ld, void* flat_v, long long flat_v_ld, int* lens_v, int* offs_v,
    long long tab_v_sb, long long tab_v_ss, int* ptr_v) {
  if (rows < 0 || max_dim < 0 || seq_pos < 0) return DKV_E_ARG;
  if (rows == 0) return DKV_OK;
  if (!states_k || !new_len_k || !flat_k || !lens_k || !offs_k || !ptr_k) return DKV_E_ARG;
  if (!states_v || !new_len_v || !flat_v || !lens_v || !offs_v || !ptr_v) return DKV_E_ARG;
  const int es = dkv_elt_size(dtype);
  if (es == 0) return DKV_E_ARG;
  AppendSlot k{states_k, states_k_ld, new_len_k, new_len_k_ld, flat_k, flat_k_ld,
               lens_k,   offs_k,      tab_k_sb,  tab_k_ss,     ptr_k};
  AppendSlot v{states_v, states_v_ld, new_len_v, new_len_v_ld, flat_v, flat_v_ld,
               lens_v,   offs_v,      tab_v_sb,  tab_v_ss,     ptr_v};
  dim3 grid((rows + 3) / 4, 2), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (es == 4)
    hipLaunchKernelGGL(append_decode_kv_kernel<uint32_t>, grid, block, 0, s, k, v, seq_pos, rows,
                       max_dim);
  else
    hipLaunchKernelGGL(append_decode_kv_kernel<uint16_t>, grid, block, 0, s, k, v, seq_pos, rows,
                       max_dim);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

static int append_prefill_launch(void* stream, int dtype, const PrefillSlot& k,
                                 const PrefillSlot& v, int nslots, int seq_pos, int rows,
                                 int n_new, int max_dim) {
  const int es = dkv_elt_size(dtype);
  if (es == 0) return DKV_E_ARG;
  if ((n_new + AP_CHUNK - 1) / AP_CHUNK > 65535) return DKV_E_UNSUPPORTED;
  const dim3 grid((unsigned)rows, (unsigned)((n_new + AP_CHUNK - 1) / AP_CHUNK), (unsigned)nslots),
      block(256);
  hipStream_t s = (hipStream_t)stream;
  if (es == 4)
    hipLaunchKernelGGL(append_prefill_kernel<uint32_t>, grid, block, 0, s, k, v, seq_pos, n_new,
                       max_dim);
  else
    hipLaunchKernelGGL(append_prefill_kernel<uint16_t>, grid, block, 0, s, k, v, seq_pos, n_new,
                       max_dim);
  DKV_HIP_CHECK_LAUNCH();
  hipLaunchKernelGGL(append_prefill_ptr_kernel, dim3((unsigned)rows, (unsigned)nslots), block, 0,
                     s, k, v, n_new, max_dim);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}

extern "C" int dkv_append_prefill(void* stream, int dtype, const void* states,
                                  long long states_sb, long long states_ss, const int* new_len,
                                  long long len_sb, long long len_ss, void* flat,
                                  long long flat_ld, int* lens, int* offs, long long tab_sb,
                                  long long tab_ss, int* ptr, int seq_pos, int rows, int n_new,
                                  int max_dim) {
  if (rows < 0 || n_new < 0 || max_dim < 0 || seq_pos < 0) return DKV_E_ARG;
  if (rows == 0 || n_new == 0) return DKV_OK;
  if (!states || !new_len || !flat || !lens || !offs || !ptr) return DKV_E_ARG;
  const PrefillSlot k{states, states_sb, states_ss, new_len, len_sb, len_ss,
                      flat,   flat_ld,   lens,      offs,    tab_sb, tab_ss, ptr};
  return append_prefill_launch(stream, dtype, k, k, 1, seq_pos, rows, n_new, max_dim);
}

extern "C" int dkv_append_prefill_kv(
    void* stream, int dtype, int seq_pos, int rows, int n_new, int max_dim, const void* states_k,
    long long states_k_sb, long long states_k_ss, const int* new_len_k, long long len_k_sb,
    long long len_k_ss, void* flat_k, long long flat_k_ld, int* lens_k, int* offs_k,
    long long tab_k_sb, long long tab_k_ss, int* ptr_k, const void* states_v,
    long long states_v_sb, long long states_v_ss, const int* new_len_v, long long len_v_sb,
    long long len_v_ss, void* flat_v, long long flat_v_ld, int* lens_v, int* offs_v,
    long long tab_v_sb, long long tab_v_ss, int* ptr_v) {
  if (rows < 0 || n_new < 0 || max_dim < 0 || seq_pos < 0) return DKV_E_ARG;
  if (rows == 0 || n_new == 0) return DKV_OK;
  if (!states_k || !new_len_k || !flat_k || !lens_k || !offs_k || !ptr_k || !states_v ||
      !new_len_v || !flat_v || !lens_v || !offs_v || !ptr_v)
    return DKV_E_ARG;
  const PrefillSlot k{states_k, states_k_sb, states_k_ss, new_len_k, len_k_sb, len_k_ss,
                      flat_k,   flat_k_ld,   lens_k,      offs_k,    tab_k_sb, tab_k_ss, ptr_k};
  const PrefillSlot v{states_v, states_v_sb, states_v_ss, new_len_v, len_v_sb, len_v_ss,
                      flat_v,   flat_v_ld,   lens_v,      offs_v,    tab_v_sb, tab_v_ss, ptr_v};
  return append_prefill_launch(stream, dtype, k, v, 2, seq_pos, rows, n_new, max_dim);
}

extern "C" int dkv_decompress(void* stream, int dtype, const void* flat, long long flat_ld,
                              const int* lens, const int* offs, long long tab_sb,
                              long long tab_ss, void* out, int rows, int seq, int max_dim) {
  if (rows < 0 || seq < 0 || max_dim < 0) return DKV_E_ARG;
  if (rows == 0 || seq == 0 || max_dim == 0) return DKV_OK;
  if (!flat || !lens || !offs || !out) return DKV_E_ARG;
  const int es = dkv_elt_size(dtype);
  if (es == 0) return DKV_E_ARG;
  if (rows > 65535) return DKV_E_UNSUPPORTED;
  dim3 grid((seq + 3) / 4, rows), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (es == 4)
    hipLaunchKernelGGL(decompress_kernel<uint32_t>, grid, block, 0, s, (const uint32_t*)flat,
                       flat_ld, lens, offs, tab_sb, tab_ss, (uint32_t*)out, seq, max_dim);
  else
    hipLaunchKernelGGL(decompress_kernel<uint16_t>, grid, block, 0, s, (const uint16_t*)flat,
                       flat_ld, lens, offs, tab_sb, tab_ss, (uint16_t*)out, seq, max_dim);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
}
