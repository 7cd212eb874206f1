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

// Block-wide inclusive scan of one long long per thread (256 threads).
__device__ __forceinline__ long long block_scan_incl(long long v, long long* s_tmp) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    long long o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  if (lane == 63) s_tmp[wave] = v;
  __syncthreads();
  long long add = 0;
  for (int w = 0; w < wave; ++w) add += s_tmp[w];
  __syncthreads();
  return v + add;
}

// One 256-thread block per row; tokens processed in chunks of 256.
template <typename T>
__global__ __launch_bounds__(256) void append_prefill_kernel(
    const T* __restrict__ states, long long states_sb, long long states_ss,
    const int* __restrict__ new_len, long long len_sb, long long len_ss, T* __restrict__ flat,
    long long flat_ld, int* __restrict__ lens, int* __restrict__ offs, long long tab_sb,
    long long tab_ss, int* __restrict__ ptr, int seq_pos, int n_new, int max_dim) {
  __shared__ long long s_tmp[4];
  __shared__ long long s_dst[256];
  __shared__ int s_clen[256];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const long long start = ptr[row];
  long long carry_u = 0, carry_c = 0;
  T* frow = flat + (long long)row * flat_ld;
  const T* srow = states + (long long)row * states_sb;
  for (int base = 0; base < n_new; base += 256) {
    const int t = base + tid;
    const int len = t < n_new ? new_len[(long long)row * len_sb + (long long)t * len_ss] : 0;
    const int clen = max(0, min(len, max_dim));
    const long long inc_u = block_scan_incl((long long)len, s_tmp);
    const long long inc_c = block_scan_incl((long long)clen, s_tmp);
    if (t < n_new) {
      const long long ti = (long long)row * tab_sb + (long long)(seq_pos + t) * tab_ss;
      lens[ti] = len;
      offs[ti] = (int)(start + carry_u + inc_u - len);
    }
    s_dst[tid] = start + carry_c + inc_c - clen;
    s_clen[tid] = clen;
    // chunk totals, identical in every thread after the broadcast
    if (tid == 255) {
      s_tmp[0] = inc_u;
      s_tmp[1] = inc_c;
    }
    __syncthreads();
    carry_u += s_tmp[0];
    carry_c += s_tmp[1];
    for (int tt = wave; tt < 256 && base + tt < n_new; tt += 4) {
      const T* src = srow + (long long)(base + tt) * states_ss;
      T* dst = frow + s_dst[tt];
      const int c = s_clen[tt];
      for (int j = lane; j < c; j += 64) dst[j] = src[j];
    }
    __syncthreads();
  }
  if (tid == 0) ptr[row] = (int)(start + carry_c);
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

extern "C" const char* dkv_status_string(int status) {
  switch (status) {
    case DKV_OK: return "ok";
    case DKV_E_ARG: return "invalid argument";
    case DKV_E_UNSUPPORTED: return "unsupported configuration";
    case DKV_E_WORKSPACE: return "workspace too small";
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

extern "C" int dkv_append_prefill(void* stream, int dtype, const void* states,
                                  long long states_sb, long long states_ss, const int* new_len,
                                  long long len_sb, long long len_ss, void* flat,
                                  long long flat_ld, int* lens, int* offs, long long tab_sb,
                                  long long tab_ss, int* ptr, int seq_pos, int rows, int n_new,
                                  int max_dim) {
  if (rows < 0 || n_new < 0 || max_dim < 0 || seq_pos < 0) return DKV_E_ARG;
  if (rows == 0 || n_new == 0) return DKV_OK;
  if (!states || !new_len || !flat || !lens || !offs || !ptr) return DKV_E_ARG;
  const int es = dkv_elt_size(dtype);
  if (es == 0) return DKV_E_ARG;
  dim3 grid(rows), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (es == 4)
    hipLaunchKernelGGL(append_prefill_kernel<uint32_t>, grid, block, 0, s, (const uint32_t*)states,
                       states_sb, states_ss, new_len, len_sb, len_ss, (uint32_t*)flat, flat_ld,
                       lens, offs, tab_sb, tab_ss, ptr, seq_pos, n_new, max_dim);
  else
    hipLaunchKernelGGL(append_prefill_kernel<uint16_t>, grid, block, 0, s, (const uint16_t*)states,
                       states_sb, states_ss, new_len, len_sb, len_ss, (uint16_t*)flat, flat_ld,
                       lens, offs, tab_sb, tab_ss, ptr, seq_pos, n_new, max_dim);
  DKV_HIP_CHECK_LAUNCH();
  return DKV_OK;
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
