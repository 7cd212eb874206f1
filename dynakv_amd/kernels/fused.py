"""Short-cache route: fused flash-decode over the packed cache.

Drop-in for the reference ``src/dynakv/kernels/fused.py:144-170``
(``fused_attention_dispatch``; kernel ``:28-142``). Semantics kept: K is reconstructed from the
first ``len`` coefficients per token, rotate-half RoPE is applied at the cache row index with
``inv_freq_i = exp(-(2i/Dh) ln theta)``, tokens with ``len_K == 0`` get a score of ``-inf``,
``len_V == 0`` tokens contribute a zero V but still count in the softmax, and the output is
``acc / l`` without clamping, in ``q``'s dtype.
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from . import joint as _joint
from .decode import splitk_attention, splitk_layout


def fused_attention_dispatch(q, k_flat, k_up, v_flat, v_up, l_k, o_k, l_v, o_v, theta):
    q = q.squeeze(2)
    batch, num_heads, head_dim = q.shape
    layout = splitk_layout(q, k_up, v_up, k_flat, v_flat) if l_k.shape[1] > 0 else None
    if layout is not None:
        return splitk_attention(q, k_flat, v_flat, layout, l_k, o_k, l_v, o_v,
                                theta=theta, route=_lib.DKV_ROUTE_FUSED)
    out = _joint.joint_attention(q, k_flat, k_up, v_flat, v_up, l_k, o_k, l_v, o_v,
                                 theta=theta, route=_lib.DKV_ROUTE_FUSED)
    if out is not None:
        return out
    return _fused_vector(q, k_flat, k_up, v_flat, v_up, l_k, o_k, l_v, o_v, theta)


def _fused_vector(q, k_flat, k_up, v_flat, v_up, l_k, o_k, l_v, o_v, theta):
    """Reference-semantics vector kernels: fp32 scores with -inf masking, then the V pass."""
    lib = _lib.load()
    batch, num_heads, head_dim = q.shape
    seq_len = l_k.shape[1]
    if q.stride(2) != 1:
        q = q.contiguous()
    k_up = k_up if k_up.stride(2) == 1 else k_up.contiguous()
    v_up = v_up if v_up.stride(2) == 1 else v_up.contiguous()
    scores = torch.empty((batch, num_heads, seq_len), dtype=torch.float32, device=q.device)
    out = torch.empty((batch, num_heads, head_dim), dtype=q.dtype, device=q.device)
    st = _lib.stream_of(q)
    cdt = _lib.dtype_code(k_flat.dtype)
    rc = lib.dkv_scores(
        st, 1, _lib.dtype_code(q.dtype), cdt, _lib.DKV_F32,
        q.data_ptr(), q.stride(0), q.stride(1),
        k_up.data_ptr(), k_up.stride(0), k_up.stride(1), k_up.shape[0],
        k_flat.data_ptr(), k_flat.stride(0),
        l_k.data_ptr(), l_k.stride(0), l_k.stride(1), o_k.data_ptr(), o_k.stride(0), o_k.stride(1),
        scores.data_ptr(), scores.stride(0), scores.stride(1), scores.stride(2),
        batch, num_heads, seq_len, k_up.shape[1], head_dim, math.log(theta))
    _lib.check(rc, "dkv_scores")
    rc = lib.dkv_av(
        st, 1, _lib.DKV_F32, _lib.dtype_code(v_flat.dtype), _lib.dtype_code(q.dtype),
        scores.data_ptr(), scores.stride(0), scores.stride(1), scores.stride(2),
        v_up.data_ptr(), v_up.stride(0), v_up.stride(1), v_up.shape[0],
        v_flat.data_ptr(), v_flat.stride(0),
        l_v.data_ptr(), l_v.stride(0), l_v.stride(1), o_v.data_ptr(), o_v.stride(0), o_v.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1),
        batch, num_heads, seq_len, v_up.shape[1], head_dim)
    _lib.check(rc, "dkv_av")
    return out
