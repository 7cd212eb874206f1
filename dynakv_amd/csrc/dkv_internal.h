// Entry points shared between the library's source files (not part of the C ABI).
#pragma once
#include "dkv_common.h"

// dkv_cutoff.hip: the decode step's cutoff head, K+V append at position seq and RoPE of q at
// position pos, in one launch, from a layer's argument block.
int dkv_layer_cutoff_append_rope(void* stream, const DkvDecodeLayer* L, const void* k_coef,
                                 const void* v_coef, void* q, int seq, int pos);
