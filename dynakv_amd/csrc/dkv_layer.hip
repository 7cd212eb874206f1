// One decode step of one attention layer in one host call (two launches): cutoff head, K+V
// append, RoPE of the query, routed decode attention.
//
// Reference behaviour: the decode branch of CustomAttention.forward
// (src/dynakv/kernels/compressed_attention.py:312-357): q RoPE (:314), cutoff-head replay
// (:321-327), update_sp for K and V (:330-334), cache length (:335) and
// compressed_decode_attention (:336-348), which routes on the post-append length
// (router.py:20-59). Every argument that does not change between steps (weights, cache
// buffers, strides, workspaces) sits in a DkvDecodeLayer the caller fills once; the call takes
// only what changes per step. The host keeps the capacity bookkeeping: it calls this only when
// the cache has room for one more token (seq + 1 <= table capacity, every row's upper bound +
// R <= flat capacity) and the RoPE table covers seq + 1 positions.
#include "dkv_internal.h"

extern "C" int dkv_decode_layer(void* stream, const DkvDecodeLayer* L, void* q,
                                const void* k_coef, const void* v_coef, void* out, int seq,
                                int pos) {
  // pos == -1: q arrives rotated by the caller (the HF decoder's position embeddings)
  if (!L || !q || !k_coef || !v_coef || !out || seq < 0 || pos < -1) return DKV_E_ARG;
  // cutoff logits, counts, the K+V appends and the q rotation in one launch
  int rc = dkv_layer_cutoff_append_rope(stream, L, k_coef, v_coef, q, seq, pos);
  if (rc != DKV_OK) return rc;
  const int S = seq + 1;
  const int route = S < L->switch_tokens ? DKV_ROUTE_FUSED : DKV_ROUTE_TWO_STAGE;
  const long long q_sb = L->q_sb ? L->q_sb : (long long)L->Hq * L->Dh;
  return dkv_decode_splitk(stream, route, L->dtype, q, q_sb, L->Dh,
                           L->k_basis, L->k_unit, L->k_sr, L->v_basis, L->v_unit, L->v_sr,
                           L->flat_k, L->flat_k_ld, L->flat_v, L->flat_v_ld, L->lens_k,
                           L->offs_k, L->tab_k_sb, L->tab_k_ss, L->lens_v, L->offs_v,
                           L->tab_v_sb, L->tab_v_ss, L->rope, L->rope_tiles, L->split_ws,
                           L->split_ws_floats, out, (long long)L->Hq * L->Dh, L->Dh, L->dtype,
                           L->B, L->Hq, L->G, L->G, S, L->R, L->Dh, 0);
}
