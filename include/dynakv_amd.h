/*
 * dynakv_amd.h — C ABI of the MI355X (gfx950) compressed-KV-cache decode path.
 *
 * Every entry point:
 *   - takes plain device pointers, element strides and sizes (no framework types);
 *   - is stream-ordered and asynchronous on `stream` (a hipStream_t passed as void*;
 *     NULL means the default stream) and never synchronises the device;
 *   - never allocates or frees device memory: outputs and workspaces belong to the caller;
 *   - returns DKV_OK (0) or a negative status (DKV_E_*), or -(DKV_E_HIP_BASE + hipError_t)
 *     when a HIP launch fails.
 *
 * Cache layout (one "slot" = one layer's K or V cache, mirroring the reference's
 * per-layer list [flat, lens, offs, flat_ptr, seq_ptr, ub]):
 *   flat  (rows, cap_flat)   coefficient payload, dtype = cache dtype; token t of row b
 *                            occupies flat[b, offs[b,t] : offs[b,t] + lens[b,t]]
 *   lens  (rows, cap_seq)    int32 retained-dimension count per token
 *   offs  (rows, cap_seq)    int32 start of each token's packed row (exclusive prefix sum)
 *   ptr   (rows,)            int32 next free element per row
 * A row is one batch element (reference "joint" layout) or one (batch, KV-group) pair
 * (per-head layout: row = b * G + g).
 */
#ifndef DYNAKV_AMD_H
#define DYNAKV_AMD_H

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define DKV_F32 0
#define DKV_F16 1
#define DKV_BF16 2

/* status codes */
#define DKV_OK 0
#define DKV_E_ARG (-1)       /* invalid argument (shape, stride, dtype, null pointer) */
#define DKV_E_UNSUPPORTED (-2) /* valid arguments outside what the kernel implements */
#define DKV_E_WORKSPACE (-3) /* caller workspace too small */
#define DKV_E_SCRATCH (-4)   /* call needs more than the fixed scratch of dkv_decode_splitk_noalloc */
#define DKV_E_HIP_BASE 1000  /* -(1000 + hipError_t) for HIP runtime failures */

/* decode-attention semantics ("route") */
#define DKV_ROUTE_FUSED 0     /* reference fused.py: -inf for len_K==0, no score rounding, acc/l */
#define DKV_ROUTE_TWO_STAGE 1 /* reference two_stage.py: -1e4*scale for len_K==0, scores rounded
                                 to the query dtype, acc/max(l,1e-6) */

/* Library version (major*10000 + minor*100 + patch). */
int dkv_version(void);

/* Human-readable message for a status code (static storage). */
const char* dkv_status_string(int status);

/*
 * Buffer-resource ranges (no reference counterpart: they state the memory contract of the
 * kernels that read through raw buffer resources, and let host-side tests check it).
 *
 * Packed flat buffers (rows, ld) passed to dkv_decode_splitk, dkv_decode_layer,
 * dkv_joint_scores and dkv_joint_av: rows * ld elements must be addressable from the base
 * pointer (a whole (rows, capacity) buffer, or a column slice of one whose storage runs to the
 * end of its last row). A workgroup reading row `row` covers the elements from that row to the
 * buffer's end, at most 0x3ffffff0: dkv_flat_range_elems returns that count.
 * dkv_view_extent_elems: one past the last element of a view of nd dimensions with non-negative
 * strides (0 when empty; -1 for a bad argument), the range of a strided operand such as
 * dkv_joint_av's scores.
 */
long long dkv_flat_range_elems(long long rows, long long row, long long ld);
long long dkv_view_extent_elems(int nd, const long long* shape, const long long* stride);

/*
 * Decode append: one new token per row.
 * Replaces update_cache_decode_kernel and its launch
 * (reference src/dynakv/kernels/compressed_cache.py:7-34, launch :170-181).
 * For each row b:  off = ptr[b]; ptr[b] += new_len[b];
 *                  lens[b, seq_pos] = new_len[b]; offs[b, seq_pos] = off;
 *                  flat[b, off + j] = states[b, j]  for j < min(new_len[b], max_dim).
 * states: (rows, max_dim) with row stride states_ld (elements); new_len: int32 with stride
 * new_len_ld; lens/offs tables share strides (tab_sb, tab_ss); flat row stride flat_ld.
 * The caller guarantees capacity (host-side growth policy), exactly as the reference does.
 */
int dkv_append_decode(void* stream, int dtype,
                      const void* states, long long states_ld,
                      const int* new_len, long long new_len_ld,
                      void* flat, long long flat_ld,
                      int* lens, int* offs, long long tab_sb, long long tab_ss,
                      int* ptr, int seq_pos, int rows, int max_dim);

/*
 * Decode append for K and V of one layer in one launch (the reference issues two
 * update_cache_decode_kernel launches per layer, compressed_cache.py:222-223).
 * Same per-slot semantics as dkv_append_decode; *_k arguments describe the K slot and
 * *_v arguments the V slot. Both slots have the same dtype, rows, max_dim and seq_pos.
 */
int dkv_append_decode_kv(void* stream, int dtype, int rows, int max_dim, int seq_pos,
                         const void* states_k, long long states_k_ld,
                         const int* new_len_k, long long new_len_k_ld,
                         void* flat_k, long long flat_k_ld,
                         int* lens_k, int* offs_k, long long tab_k_sb, long long tab_k_ss,
                         int* ptr_k,
                         const void* states_v, long long states_v_ld,
                         const int* new_len_v, long long new_len_v_ld,
                         void* flat_v, long long flat_v_ld,
                         int* lens_v, int* offs_v, long long tab_v_sb, long long tab_v_ss,
                         int* ptr_v);

/*
 * Prefill append of n_new tokens per row, without host synchronisation.
 * Replaces the per-row Python loop of the prefill branch
 * (reference src/dynakv/kernels/compressed_cache.py:182-209).
 * For each row b, with start = ptr[b]:
 *   offs[b, seq_pos + t] = start + sum_{t' < t} new_len[b, t']          (unclamped lengths)
 *   lens[b, seq_pos + t] = new_len[b, t]
 *   the first min(new_len[b,t], max_dim) elements of states[b, t, :] are written back to
 *   back starting at start (clamped prefix sums), and ptr[b] += sum_t min(new_len[b,t], max_dim).
 * states: (rows, n_new, max_dim) with strides (states_sb, states_ss), unit inner stride;
 * new_len: int32 (rows, n_new) with strides (len_sb, len_ss).
 */
int dkv_append_prefill(void* stream, int dtype,
                       const void* states, long long states_sb, long long states_ss,
                       const int* new_len, long long len_sb, long long len_ss,
                       void* flat, long long flat_ld,
                       int* lens, int* offs, long long tab_sb, long long tab_ss,
                       int* ptr, int seq_pos, int rows, int n_new, int max_dim);

/*
 * dkv_append_prefill for a layer's K and V slots in one launch (plus one pointer launch): the
 * prefill appends of update_sp (reference src/dynakv/kernels/compressed_cache.py:219-227 with
 * :182-209 per slot), both slots at the same seq_pos with the same rows and n_new. Each slot's
 * arguments mean what dkv_append_prefill's do; the results equal two dkv_append_prefill calls.
 */
int dkv_append_prefill_kv(void* stream, int dtype, int seq_pos, int rows, int n_new, int max_dim,
                          const void* states_k, long long states_k_sb, long long states_k_ss,
                          const int* new_len_k, long long len_k_sb, long long len_k_ss,
                          void* flat_k, long long flat_k_ld, int* lens_k, int* offs_k,
                          long long tab_k_sb, long long tab_k_ss, int* ptr_k,
                          const void* states_v, long long states_v_sb, long long states_v_ss,
                          const int* new_len_v, long long len_v_sb, long long len_v_ss,
                          void* flat_v, long long flat_v_ld, int* lens_v, int* offs_v,
                          long long tab_v_sb, long long tab_v_ss, int* ptr_v);

/*
 * Dense re-expansion of a packed slot: out[b, t, j] = flat[b, offs[b,t] + j] for
 * j < min(lens[b,t], max_dim), else 0. out is (rows, seq, max_dim) contiguous, cache dtype.
 * Replaces simple_decompress (reference src/dynakv/kernels/compressed_cache.py:36-56),
 * which lays tokens back to back from element 0 of each row, i.e. uses the prefix sum of the
 * lengths rather than offs; both agree whenever offs is the exclusive prefix sum from 0.
 */
int dkv_decompress(void* stream, int dtype,
                   const void* flat, long long flat_ld,
                   const int* lens, const int* offs, long long tab_sb, long long tab_ss,
                   void* out, int rows, int seq, int max_dim);

/*
 * Reference-semantics QK scores (abx_sparse / _abx_sparse_fwd, reference two_stage.py:48-189).
 *   z[b,h,s] = round_out( ((len>0) ? q_h . RoPE_s(x_s @ basis[h / hpg]) : -1e4) / sqrt(Dh) )
 * with x_s = flat[b, offs[b,s] : offs[b,s] + min(len, R)], rotate-half RoPE at position s,
 * inv_freq_i = exp(-(2i/Dh) ln theta) in fp32, hpg = Hq / n_basis.
 * mode 0: abx semantics (out dtype = out_dtype, -1e4 masking before the scale).
 * mode 1: fused semantics (out must be fp32, -inf masking, no rounding).
 * q: (B, Hq, Dh) strides (q_sb, q_sh), unit dim stride, dtype = q_dtype.
 * basis: (n_basis, R, Dh) strides (basis_sh, basis_sr), unit dim stride, dtype = cache dtype.
 * out: (B, Hq, S) strides (out_sb, out_sh, out_ss).
 * Dh must be even and <= 128.
 */
int dkv_scores(void* stream, int mode, int q_dtype, int cache_dtype, int out_dtype,
               const void* q, long long q_sb, long long q_sh,
               const void* basis, long long basis_sh, long long basis_sr, int n_basis,
               const void* flat, long long flat_ld,
               const int* lens, long long lens_sb, long long lens_ss,
               const int* offs, long long offs_sb, long long offs_ss,
               void* out, long long out_sb, long long out_sh, long long out_ss,
               int B, int Hq, int S, int R, int Dh, float log_theta);

/*
 * Reference-semantics softmax-weighted V (avx / _avx_proj_fwd, reference two_stage.py:207-324):
 *   out[b,h] = ((sum_s e^{z_s - m} x^V_s) @ basis[h / hpg]) / D,
 *   D = max(sum_s e^{z_s - m}, 1e-6) in mode 0 (avx), D = sum_s e^{z_s - m} in mode 1 (fused).
 * scores: (B, Hq, S) strides (sc_sb, sc_sh, sc_ss) of dtype scores_dtype.
 * out: (B, Hq, Dh) strides (out_sb, out_sh), unit dim stride, dtype out_dtype.
 * R <= 1024, Dh <= 128.
 */
int dkv_av(void* stream, int mode, int scores_dtype, int cache_dtype, int out_dtype,
           const void* scores, long long sc_sb, long long sc_sh, long long sc_ss,
           const void* basis, long long basis_sh, long long basis_sr, int n_basis,
           const void* flat, long long flat_ld,
           const int* lens, long long lens_sb, long long lens_ss,
           const int* offs, long long offs_sb, long long offs_ss,
           void* out, long long out_sb, long long out_sh,
           int B, int Hq, int S, int R, int Dh);

/*
 * dkv_scores on MFMA for the reference's joint layout and any 16-bit cache with ranks up to 1024
 * (abx_sparse / _abx_sparse_fwd, reference two_stage.py:48-189; with mode 1 the scores of the
 * fused route, fused.py:28-140). Same semantics and outputs as dkv_scores (mode, masking,
 * rounding to out_dtype), with the K basis given transposed in 32-rank chunks: basis_t
 * (n_basis, R/32, Dh, 32), element B_h[32c + k][d] at h*bt_sh + c*bt_sc + d*32 + k (each
 * chunk's 8 KB contiguous), 16-byte aligned, bt_sc >= Dh*32, bt_sh and bt_sc multiples of 8.
 * RoPE: the rope table of dkv_rope_table with rope_tiles >= ceil(S/16), 16-byte aligned.
 * workspace: dkv_joint_scores_workspace_ints(B, S) int32s, 4-byte aligned (the tokens of each
 * window of up to 2048 positions ordered by their count of 32-rank chunks, written by the call's
 * first launch and read by its second; contents need not be initialised).
 * q: (B, Hq, Dh) strides (q_sb, q_sh), unit dim stride; dtype (q and cache) DKV_BF16 or DKV_F16.
 * DKV_E_UNSUPPORTED unless Dh == 128, R % 32 == 0, R <= 1024, Hq / n_basis <= 8,
 * flat_ld <= 0x3fffffe8 (the caller then uses dkv_scores).
 */
int dkv_joint_scores(void* stream, int mode, int dtype, int out_dtype,
                     const void* q, long long q_sb, long long q_sh,
                     const void* basis_t, long long bt_sh, long long bt_sc, int n_basis,
                     const void* flat, long long flat_ld,
                     const int* lens, long long lens_sb, long long lens_ss,
                     const int* offs, long long offs_sb, long long offs_ss,
                     const float* rope, int rope_tiles,
                     int* workspace, long long workspace_ints,
                     void* out, long long out_sb, long long out_sh, long long out_ss,
                     int B, int Hq, int S, int R, int Dh);

/* int32 workspace dkv_joint_scores needs for B rows of S tokens (0 when B or S is 0). */
long long dkv_joint_scores_workspace_ints(int B, int S);

/* fp32 workspace dkv_joint_av needs for these sizes (split records and per rank block partial
 * projections); 0 for sizes dkv_joint_av does not take. */
long long dkv_joint_av_workspace_floats(int B, int Hq, int S, int R);

/*
 * dkv_av on MFMA (avx / _avx_proj_fwd, reference two_stage.py:207-324; mode 1: the fused route's V
 * pass): the same inputs and outputs as dkv_av plus a caller workspace of
 * dkv_joint_av_workspace_floats(B, Hq, S, R) floats, 16-byte aligned. Token splits write (m, l,
 * acc[R]) records; a second launch merges them by LSE per block of 128 ranks and projects each
 * block through its rows of the V basis, a third adds the blocks. dtype (cache) DKV_BF16 or
 * DKV_F16, Dh == 128, R <= 1024, the basis 4-byte aligned with even strides; S == 0 returns
 * DKV_E_UNSUPPORTED (dkv_av covers it).
 */
int dkv_joint_av(void* stream, int mode, int scores_dtype, int dtype, int out_dtype,
                 const void* scores, long long sc_sb, long long sc_sh, long long sc_ss,
                 const void* basis, long long basis_sh, long long basis_sr, int n_basis,
                 const void* flat, long long flat_ld,
                 const int* lens, long long lens_sb, long long lens_ss,
                 const int* offs, long long offs_sb, long long offs_ss,
                 float* workspace, long long workspace_floats,
                 void* out, long long out_sb, long long out_sh,
                 int B, int Hq, int S, int R, int Dh);

/*
 * RoPE cos/sin table for the split-K kernel, (17 + n_tiles) rows of 64 (cos, sin) fp32 pairs:
 * rows 0..15 the in-tile offsets (angle = d * inv_freq), row 16 the rotation by 128 positions (8 waves x 16),
 * row 17 + T the base of 16-token tile T (angle = 16T * inv_freq); inv_freq_i =
 * exp(-(2i/128) ln theta) and every angle formed in fp32 as the reference does (fused.py:65-66,
 * 97; two_stage.py:36-44). dkv_rope_table fills the fixed rows when from_tile == 0 and the tile
 * rows [from_tile, to_tile), so a caller can extend a table as the cache grows.
 */
long long dkv_rope_table_floats(int n_tiles);
int dkv_rope_table(void* stream, float* rope, int from_tile, int to_tile, float log_theta);

/*
 * Split-K compressed decode attention on MFMA (the fast path for both router routes,
 * reference fused.py:28-170 and two_stage.py:48-324 as called from router.py:20-59).
 * One work unit = (batch b, KV head k) with hpg = Hq / Hkv query heads sharing the K/V basis
 * of KV head k; its coefficients live in cache row b * G + k / (Hkv / G).
 *   q: (B, Hq, Dh) strides (q_sb, q_sh), already RoPE'd by the caller.
 *   k_basis / v_basis: base pointers with basis of KV head k at  base + k * unit_stride,
 *                      rank stride basis_sr, unit dim stride (R x Dh).
 *   lens/offs tables for K and V with their own (sb, ss) strides.
 *   rope: table from dkv_rope_table with rope_tiles >= ceil(S / 16) tile rows (it carries theta).
 *   workspace: fp32 buffer of dkv_splitk_workspace_floats(...) floats: 16384 leading ints of
 *              per-unit arrival counters, then the split records. The counters must be zero
 *              before the first call (a zero-filled buffer) and every call leaves them zero;
 *              calls that share a workspace must be ordered (same stream). With at most 16384
 *              units the last split of each unit to finish merges the unit's records itself
 *              (one launch); beyond that a merge kernel follows on the same stream.
 *   out: (B, Hq, Dh) strides (out_sb, out_sh), dtype out_dtype = the cache dtype (what the
 *        reference returns) or DKV_F32 (the merged result before rounding).
 * Requirements: q and cache dtype f16 or bf16 (same), Dh == 128, R <= 128, hpg <= 16,
 * Hkv % G == 0, flat row strides k_ld, v_ld <= 0x3fffffe8 elements (each workgroup addresses
 * the buffer from its own row, so the number of rows is not limited), S and the table token
 * strides < 2^24 with S * table token stride < 2^31. split_len is a multiple of 64
 * (0 = dkv_splitk_choose_split: about one workgroup per CU, at least 128 tokens per split when
 * the cache is that long). Splits of 256 tokens or more run their waves on pairs of tiles.
 */
long long dkv_splitk_workspace_floats(int B, int Hq, int Hkv, int S, int R, int split_len);
int dkv_splitk_choose_split(int B, int Hkv, int S);
int dkv_decode_splitk(void* stream, int route, int dtype,
                      const void* q, long long q_sb, long long q_sh,
                      const void* k_basis, long long k_unit_stride, long long k_basis_sr,
                      const void* v_basis, long long v_unit_stride, long long v_basis_sr,
                      const void* k_flat, long long k_ld, const void* v_flat, long long v_ld,
                      const int* lens_k, const int* offs_k, long long tk_sb, long long tk_ss,
                      const int* lens_v, const int* offs_v, long long tv_sb, long long tv_ss,
                      const float* rope, int rope_tiles,
                      float* workspace, long long workspace_floats,
                      void* out, long long out_sb, long long out_sh, int out_dtype,
                      int B, int Hq, int Hkv, int G, int S, int R, int Dh, int split_len);

/*
 * Dense GQA decode attention over an uncompressed cache: the baseline of the end-to-end
 * comparison (the reference's uncompressed model, scripts/benchmark_throughput.py:17-77, reads
 * every cached token's rotated key and value at full width; it has no kernel of its own for it).
 *   q: (B, Hq, Dh) strides (q_sb, q_sh), rotated by the caller.
 *   k / v: rows b * Hkv + g of kv_ld elements; token t of a row at elements t * Dh .. + Dh - 1,
 *          keys already rotated.
 *   workspace: dkv_dense_workspace_floats(...) floats, the same contract as dkv_decode_splitk's
 *              (16384 leading arrival counters, zero before the first call and after each).
 *   out: (B, Hq, Dh) strides (out_sb, out_sh), out_dtype = the cache dtype or DKV_F32.
 * Semantics: softmax(q . k / sqrt(Dh)) v over tokens 0..S-1 with fp32 scores and accumulation.
 * Requirements: dtype f16 or bf16, Dh == 128, hpg <= 16, 16-byte aligned q rows and cache
 * rows (kv_ld % 8 == 0, kv_ld >= S * Dh), S * Dh * 2 < 2^31, split_len a multiple of 64
 * (0 = dkv_dense_choose_split).
 */
long long dkv_dense_workspace_floats(int B, int Hq, int Hkv, int S, int split_len);
/*
 * A decode step's cache write for the dense baseline (the uncompressed model's KV-cache update
 * and its q/k rotation, transformers' Llama attention, run as one launch): y holds B rows (stride
 * y_ld) of the fused q/k/v projection, Hq query heads then Hkv key heads then Hkv value heads of
 * 128; the query heads are rotated in place at q_pos, the key heads rotated at k_pos into
 * k_cache[(b * Hkv + g) * kv_ld + k_pos * 128 ..], the value heads copied into v_cache likewise.
 * RoPE as dkv_rope_dense (angle float(pos) * inv_freq in fp32, rotation in fp32).
 */
int dkv_dense_append(void* stream, int dtype, void* y, long long y_ld, void* k_cache,
                     void* v_cache, long long kv_ld, int q_pos, int k_pos, int B, int Hq,
                     int Hkv, float log_theta);
int dkv_dense_choose_split(int B, int Hkv, int S);
int dkv_decode_dense(void* stream, int dtype, const void* q, long long q_sb, long long q_sh,
                     const void* k, const void* v, long long kv_ld, int S,
                     float* workspace, long long workspace_floats,
                     void* out, long long out_sb, long long out_sh, int out_dtype,
                     int B, int Hq, int Hkv, int Dh, int split_len);

/*
 * dkv_decode_splitk without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has no
 * counterpart in the reference. Same arguments, semantics and results as dkv_decode_splitk; the
 * split records and arrival counters live in a fixed device array of DKV_NOALLOC_SCRATCH_FLOATS
 * floats (4 MiB) per GPU, held until the process ends. The call allocates nothing: a call whose
 * dkv_splitk_workspace_floats(...) exceeds that size returns DKV_E_SCRATCH. The first call on a
 * device looks the array up and zeroes its counters with a fill kernel on `stream`; every call
 * leaves the counters zero. All calls on one GPU share the array: calls that overlap in time
 * (different streams without ordering, or different host threads) race and give wrong results.
 * `stream` must belong to the current device (DKV_E_ARG otherwise).
 */
#define DKV_NOALLOC_SCRATCH_FLOATS (1 << 20)
int dkv_decode_splitk_noalloc(void* stream, int route, int dtype,
                              const void* q, long long q_sb, long long q_sh,
                              const void* k_basis, long long k_unit_stride, long long k_basis_sr,
                              const void* v_basis, long long v_unit_stride, long long v_basis_sr,
                              const void* k_flat, long long k_ld, const void* v_flat, long long v_ld,
                              const int* lens_k, const int* offs_k, long long tk_sb, long long tk_ss,
                              const int* lens_v, const int* offs_v, long long tv_sb, long long tv_ss,
                              const float* rope, int rope_tiles,
                              void* out, long long out_sb, long long out_sh, int out_dtype,
                              int B, int Hq, int Hkv, int G, int S, int R, int Dh, int split_len);

/*
 * Launch timing hooks (measurement only, no reference counterpart). Between
 * dkv_profile_begin(max_calls) and dkv_profile_end, each dkv_decode_splitk call (the first
 * max_calls of them) records HIP events on its stream before and after its split launch and,
 * when a separate merge kernel runs, after the merge. dkv_profile_end waits for the recorded
 * events, returns the summed split and merge milliseconds (merge 0 when the split kernel
 * merged itself) and the number of calls recorded, and destroys the events. Not thread-safe.
 */
int dkv_profile_begin(int max_calls);
int dkv_profile_end(double* split_ms, double* merge_ms, int* calls);

/*
 * Launch-layout self test (diagnostic, no reference counterpart): runs the MFMA operand
 * layouts and unaligned buffer gathers the split-K kernel relies on against a scalar
 * computation of the same products, on the device. `mismatches` points at a zeroed device
 * buffer of at least 1280 bytes; the number of mismatching elements is added to its first
 * int (the rest is scratch). Used by the GPU test suite before parity tests.
 */
int dkv_selftest_layouts(void* stream, int* mismatches);

/*
 * Cutoff head for K and V (reference KVProcessor.kv_process_fused,
 * src/dynakv/kernels/compressed_attention.py:84-119, replayed per decode step at :321-327).
 * Per row m (M = B*S tokens) and group g (G groups of D dims; G = 1 is the reference's joint
 * head): logits = round(b_g + x_g @ W_g), p = round(softmax(logits)), c_m = round(prefix sums
 * of p accumulated in fp32), all rounded to the compute dtype; len = min(#{m : c_m >= thr},
 * low_rank) with thr = threshold rounded to the compute dtype (the reference's
 * flip(cumsum) >= 0.1 prefix mask, mask[low_rank:] = 0); out = x * (j < len).
 *   x*, out*: (M, G*D) rows with row strides x_ld / out_ld (x_ld a multiple of 8 elements,
 *             x and wt 16-byte aligned); len*: (M, G) int32, row stride len_ld.
 *   wt*: (G, D, D) transposed weights, wt[g][n][k] = W_g[k][n]; b*: (G, D).
 *   low_rank < 0 means D. dtype: DKV_F16 or DKV_BF16; D a power of two in 64 .. 1024.
 *   workspace: >= dkv_cutoff_workspace_bytes(M, G, D) bytes (the rounded logits).
 */
long long dkv_cutoff_workspace_bytes(int M, int G, int D);
int dkv_cutoff_kv(void* stream, int dtype, const void* xk, const void* xv, long long x_ld,
                  const void* wt_k, const void* wt_v, const void* b_k, const void* b_v,
                  float threshold, int low_rank, void* out_k, void* out_v, long long out_ld,
                  int* len_k, int* len_v, long long len_ld, void* workspace,
                  long long workspace_bytes, int M, int G, int D);

/*
 * Prefill attention over the reconstructed cache (reference prefill branch,
 * src/dynakv/kernels/compressed_attention.py:359-386: get_origin_states, the k_up / v_up
 * projection, RoPE of K at positions 0..S-1 via calc_cos_sin :193-200, causal attention).
 *
 * dkv_rope_dense: in-place rotate-half RoPE of dense rows x[r][s][0..127] (row stride row_ld,
 * token stride tok_ld, unit dim stride) at positions pos0 + s; angle float(pos) * inv_freq_i
 * in fp32 (inv_freq_i = exp(-(2i/128) ln theta)), rotation in fp32, result rounded to dtype.
 * Replaces the reference's apply_rotary_pos_emb_ on the projected K (:375-378).
 *
 * dkv_prefill_attention: out[b,h,i] = softmax_j(scale * q[b,h,i] . k[b,h/(Hq/Hkv),j]) v[...]
 * over keys j <= (Sk - Sq) + i when causal (queries are the last Sq positions), else all Sk.
 * q (B,Hq,Sq,128), k/v (B,Hkv,Sk,128), out (B,Hq,Sq,128): strides in elements per batch, head
 * and token, unit dim stride, 16-byte aligned rows; k_elems / v_elems: elements addressable
 * from k / v (bounds of the buffer loads). fp32 softmax, probabilities as a hi + lo pair in
 * the compute dtype for the P.V product. dtype: DKV_F16 or DKV_BF16; out_dtype: dtype or
 * DKV_F32 (the normalised result before rounding). scale: positive and finite (else
 * DKV_E_UNSUPPORTED; the reference passes 1/sqrt(128)). kstart: NULL, or B int32 on the
 * device; keys j < kstart[b] are masked for every query of row b (a left-padded prompt: the
 * reference passes create_causal_mask(attention_mask, ...) to this call, custom_llama.py:161-168);
 * a query left with no key (a padding position) gets 0. Replaces the eager / SDPA attention
 * call of the prefill branch (:373-383).
 *
 * dkv_rope_apply: in-place rotate-half RoPE of x (B, H, S, 128) (strides x_sb / x_sh / x_ss,
 * unit dim stride) with given cos / sin tables (B, S, 128) in the dtype (batch stride cs_sb,
 * 0 to share one table, token stride cs_ss, unit dim stride): x <- (x * cos) +
 * (rotate_half(x) * sin), each product and the sum rounded to the dtype as the reference's
 * apply_rotary_pos_emb_ computes it (compressed_attention.py:18-22). Rotates q by the
 * position embeddings of the HF decoder (LlamaRotaryEmbedding, rope_scaling included,
 * :314,:360) and the prefill K by calc_cos_sin's (:193-200, :375-378).
 */
int dkv_rope_dense(void* stream, int dtype, void* x, long long row_ld, long long tok_ld,
                   int rows, int S, int pos0, float log_theta);
int dkv_prefill_attention(void* stream, int dtype, const void* q, long long q_sb, long long q_sh,
                          long long q_ss, const void* k, long long k_sb, long long k_sh,
                          long long k_ss, long long k_elems, const void* v, long long v_sb,
                          long long v_sh, long long v_ss, long long v_elems, void* out,
                          int out_dtype, long long o_sb, long long o_sh, long long o_ss, int B,
                          int Hq, int Hkv, int Sq, int Sk, int Dh, int causal, float scale,
                          const int* kstart);
/*
 * Dense K and V of a prompt from masked coefficient rows, for the compressed prefill attention
 * (compressed_attention.py:359-386 with get_origin_states, compressed_cache.py:36-56): per cache
 * row r = b * G + g, K[t] = RoPE_{pos0 + t}(B_K[g]^T ck[r, t]) and V[t] = B_V[g]^T cv[r, t] in one
 * launch (fp32 accumulation and one rounding to the dtype; the keys then rotated in fp32 by
 * R(16T) R(n) for position 16T + n, composed from the rows of the RoPE table rope (dkv_rope_table,
 * rope_tiles >= ceil((pos0 + S) / 16), 16-byte aligned), and rounded again, the reference's
 * two steps).
 * ck / cv: (rows, S, R) element strides (c_sr, c_st, 1), zero past each token's count; bases
 * (G, R, 128) strides (b_sg, b_sr, 1); outputs (rows, S, 128) strides (o_sr, o_st, 1). R <= 128
 * and a multiple of 8; 16-byte aligned coefficient and basis rows, 8-byte aligned output rows.
 */
int dkv_recon_kv(void* stream, int dtype, const void* ck, const void* cv, long long c_sr,
                 long long c_st, const void* k_basis, const void* v_basis, long long b_sg,
                 long long b_sr, void* k_out, void* v_out, long long o_sr, long long o_st,
                 int rows, int G, int S, int R, int pos0, const float* rope, int rope_tiles);
int dkv_rope_apply(void* stream, int dtype, void* x, long long x_sb, long long x_sh,
                   long long x_ss, const void* cos, const void* sin, long long cs_sb,
                   long long cs_ss, int B, int H, int S);

/*
 * One decode step of one attention layer (per-head layout, rows b*G + g) in one call: the
 * reference's decode branch, src/dynakv/kernels/compressed_attention.py:312-357 -- cutoff head
 * (:321-327, dkv_cutoff_kv), K+V append at position seq (:330-334, dkv_append_decode_kv), RoPE
 * of q at position pos (:314, dkv_rope_dense), decode attention over seq + 1 tokens routed at
 * switch_tokens (:335-348 and router.py:20-59, dkv_decode_splitk). The caller fills a
 * DkvDecodeLayer once per layer (and again after the cache grows or the RoPE table is
 * extended) and calls dkv_decode_layer per step with the step's q (B, Hq, Dh) (batch stride
 * q_sb, rotated in place at position pos; pos == -1: q arrives rotated by the caller, as the
 * reference rotates it with the decoder's position embeddings), the layer's K/V coefficients
 * (B, G*R) (row stride coef_ld) and the
 * output (B, Hq, Dh) contiguous in the cache dtype. The caller guarantees room for one more token:
 * seq + 1 <= the tables' capacity, every row's used length + R <= the flat capacity, and
 * rope_tiles * 16 >= seq + 1. Three launches: the cutoff logits; the counts, the appends of
 * the first len coefficients and the q rotation; the attention. coef_k / coef_v (B, G*R) and
 * len_k / len_v (B*G) int32 are scratch the current implementation does not touch.
 */
typedef struct DkvDecodeLayer {
  int dtype, B, G, Hq, R, Dh, low_rank, switch_tokens;
  float threshold, log_theta;
  const void *wt_k, *wt_v, *b_k, *b_v;         /* cutoff head, (G, R, R) transposed / (G, R) */
  void* cut_ws;
  long long cut_ws_bytes;
  void *coef_k, *coef_v;
  int *len_k, *len_v;
  void* flat_k;
  long long flat_k_ld;
  int *lens_k, *offs_k;
  long long tab_k_sb, tab_k_ss;
  int* ptr_k;
  void* flat_v;
  long long flat_v_ld;
  int *lens_v, *offs_v;
  long long tab_v_sb, tab_v_ss;
  int* ptr_v;
  const void* k_basis;
  long long k_unit, k_sr;
  const void* v_basis;
  long long v_unit, v_sr;
  const float* rope;
  int rope_tiles;
  float* split_ws;
  long long split_ws_floats;
  /* row strides in elements of q (per batch row; its heads are contiguous 128-element rows)
   * and of k_coef / v_coef; 0 means contiguous (Hq * Dh, G * R) */
  long long q_sb, coef_ld;
} DkvDecodeLayer;
int dkv_decode_layer(void* stream, const DkvDecodeLayer* layer, void* q, const void* k_coef,
                     const void* v_coef, void* out, int seq, int pos);

/*
 * Element-wise stages of the end-to-end decoder around the attention (the HF Llama decoder
 * layer the reference runs, custom_llama.py:93-323 on transformers' LlamaDecoderLayer and
 * LlamaRMSNorm / LlamaMLP), one kernel each instead of torch's chains of element-wise kernels.
 *
 * dkv_add_rmsnorm: for each of rows rows (H <= 8192, H % 8 == 0): if delta is non-NULL,
 * x = round(x + delta) in place (the residual add); then out = round(round(x * rsqrt(mean(x^2)
 * + eps)) * w) (LlamaRMSNorm: fp32 statistics, the normalised value rounded to dtype, times the
 * weight in dtype). Row strides x_ld / delta_ld / out_ld in elements; 16-byte aligned rows.
 *
 * dkv_silu_mul: out[r][j] = round(round(silu(g)) * u), g = gu[r][j], u = gu[r][F + j] (the
 * gate and up projections of one concatenated GEMM), silu(g) = g / (1 + e^-g) in fp32 (LlamaMLP
 * act_fn(gate_proj(x)) * up_proj(x)). F % 8 == 0, 16-byte aligned rows.
 *
 * dkv_silu_mul_pairs: the same with g = gu[r][2j], u = gu[r][2j + 1] (one GEMM by a gate/up
 * weight whose rows interleave gate j and up j); bit-identical to dkv_silu_mul of the
 * de-interleaved halves.
 */
int dkv_add_rmsnorm(void* stream, int dtype, void* x, long long x_ld, const void* delta,
                    long long delta_ld, const void* w, void* out, long long out_ld, int rows,
                    int H, float eps);
int dkv_silu_mul(void* stream, int dtype, const void* gu, long long gu_ld, void* out,
                 long long out_ld, int rows, int F);
int dkv_silu_mul_pairs(void* stream, int dtype, const void* gu, long long gu_ld, void* out,
                       long long out_ld, int rows, int F);

/*
 * dkv_gemv: y[m][n] = sum_k x[m][k] W[n][k] for m < M <= 8 (the decode-time linear layers of
 * the decoder, torch's F.linear(x, W) with W (N, K) row-major): fp32 accumulation, y rounded
 * once to dtype. K % 8 == 0, 16-byte aligned x and W rows; row strides x_ld, w_ld, y_ld in
 * elements. DKV_E_UNSUPPORTED for other shapes (the caller uses a library GEMM then).
 */
int dkv_gemv(void* stream, int dtype, const void* x, long long x_ld, const void* W,
             long long w_ld, void* y, long long y_ld, int M, int N, int K);

/*
 * dkv_gemv_rmsnorm: dkv_gemv of the normalised rows, h = rmsnorm(x + delta) * norm_w with the
 * roundings and summation order of dkv_add_rmsnorm (h is bit-identical to its output), y = h
 * W^T. With delta non-NULL the updated residual x + delta (rounded) is stored to r_out (a
 * buffer other than x and delta: every workgroup reads x while one writes r_out). M * K * 2
 * <= 64 KiB, K % 8 == 0; DKV_E_UNSUPPORTED otherwise (the caller runs dkv_add_rmsnorm and a
 * GEMM then).
 */
int dkv_gemv_rmsnorm(void* stream, int dtype, const void* x, long long x_ld, const void* delta,
                     long long delta_ld, const void* norm_w, float eps, void* r_out,
                     long long r_ld, const void* W, long long w_ld, void* y, long long y_ld,
                     int M, int N, int K);

/*
 * dkv_gemv_glu: the LlamaMLP gate/up projection and SwiGLU product of a decode step in one
 * launch (reference: transformers' LlamaMLP under custom_llama.py:93-323): W holds the gate and
 * up weight rows interleaved (row 2j gate row j, row 2j + 1 up row j; 2F rows of K), and
 * h[m][j] = silu(g) * u with g, u the two projections of x row m each rounded to dtype and
 * silu(g) rounded before the product (bit-identical to dkv_gemv then dkv_silu_mul of the
 * de-interleaved halves). With norm_w the rows are first normalised as in dkv_gemv_rmsnorm
 * (delta / r_out as there; M * K * 2 <= 64 KiB), without it x is used as it is. M <= 8,
 * K % 8 == 0; DKV_E_UNSUPPORTED otherwise.
 */
int dkv_gemv_glu(void* stream, int dtype, const void* x, long long x_ld, const void* delta,
                 long long delta_ld, const void* norm_w, float eps, void* r_out, long long r_ld,
                 const void* W, long long w_ld, void* h, long long h_ld, int M, int F, int K);

#ifdef __cplusplus
}
#endif
#endif /* DYNAKV_AMD_H */
