"""Long-cache route: QK scores (``abx_sparse``) and softmax-weighted V (``avx``).

Drop-in for the reference ``src/dynakv/kernels/two_stage.py``:

* ``abx_sparse`` (``:159-189``, kernel ``:48-157``) returns ``(B, Hq, S)`` scores in ``a``'s
  dtype: ``((len > 0) ? q . RoPE_s(x_s @ b[h // hpg]) : -1e4) / sqrt(Dh)`` rounded to that dtype.
* ``avx`` (``:283-324``, kernel ``:207-281``) returns
  ``((sum_s e^{z_s - m} x_s) @ v_up[h // grp]) / max(sum_s e^{z_s - m}, 1e-6)``.
* ``two_stage_attention`` is what the router's long route runs: the split-K kernel with exactly
  these semantics (scores rounded to the query dtype before the softmax, the clamp in the
  denominator) when the inputs fit it, else ``abx_sparse`` followed by ``avx``.

Both raise ``ValueError`` when ``offsets`` is ``None``, as the reference does.
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from . import joint as _joint
from .decode import splitk_attention, splitk_layout


def abx_sparse(a: torch.Tensor, b: torch.Tensor, x_flat: torch.Tensor, l_vec: torch.Tensor,
               offsets: torch.Tensor = None, theta: float = 10000.0) -> torch.Tensor:
    batch, num_heads_total, head_dim = a.shape
    b_batch, seq_len = l_vec.shape
    rank_per_head_groups = b.shape[1]
    if offsets is None:
        raise ValueError("offsets are required for the variable-length key cache")
    if seq_len > 0 and _joint.scores_eligible(a, b, x_flat):
        return _joint.joint_scores(a, b, x_flat, l_vec, offsets, theta=theta, mode=0,
                                   out_dtype=a.dtype)
    lib = _lib.load()
    if a.stride(2) != 1:
        a = a.contiguous()
    if b.stride(2) != 1:
        b = b.contiguous()
    out = torch.empty((batch, num_heads_total, seq_len), dtype=a.dtype, device=a.device)
    rc = lib.dkv_scores(
        _lib.stream_of(a), 0, _lib.dtype_code(a.dtype), _lib.dtype_code(x_flat.dtype),
        _lib.dtype_code(a.dtype),
        a.data_ptr(), a.stride(0), a.stride(1),
        b.data_ptr(), b.stride(0), b.stride(1), b.shape[0],
        x_flat.data_ptr(), x_flat.stride(0),
        l_vec.data_ptr(), l_vec.stride(0), l_vec.stride(1),
        offsets.data_ptr(), offsets.stride(0), offsets.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        batch, num_heads_total, seq_len, rank_per_head_groups, head_dim, math.log(theta))
    _lib.check(rc, "abx_sparse")
    return out


def avx(a: torch.Tensor, x_flat: torch.Tensor, v_up: torch.Tensor, l_vec: torch.Tensor,
        offsets: torch.Tensor = None) -> torch.Tensor:
    if a.ndim == 4:
        a = a.squeeze(2)
    batch, num_heads, seq_len = a.shape
    num_kv_heads, rank_total, head_dim = v_up.shape
    if offsets is None:
        raise ValueError("offsets are required for the variable-length value cache")
    if _joint.av_eligible(v_up, x_flat, num_heads, seq_len):
        return _joint.joint_av(a, v_up, x_flat, l_vec, offsets, mode=0, out_dtype=a.dtype)
    lib = _lib.load()
    if v_up.stride(2) != 1:
        v_up = v_up.contiguous()
    out = torch.empty((batch, num_heads, head_dim), dtype=a.dtype, device=a.device)
    rc = lib.dkv_av(
        _lib.stream_of(a), 0, _lib.dtype_code(a.dtype), _lib.dtype_code(x_flat.dtype),
        _lib.dtype_code(a.dtype),
        a.data_ptr(), a.stride(0), a.stride(1), a.stride(2),
        v_up.data_ptr(), v_up.stride(0), v_up.stride(1), num_kv_heads,
        x_flat.data_ptr(), x_flat.stride(0),
        l_vec.data_ptr(), l_vec.stride(0), l_vec.stride(1),
        offsets.data_ptr(), offsets.stride(0), offsets.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1),
        batch, num_heads, seq_len, rank_total, head_dim)
    _lib.check(rc, "avx")
    return out


def two_stage_attention(*, q, k_flat, k_up, v_flat, v_up, key_lengths, key_offsets,
                        value_lengths, value_offsets, theta: float) -> torch.Tensor:
    """The router's long route (reference ``router.py:49-59``)."""
    q3 = q.squeeze(2).contiguous()
    layout = splitk_layout(q3, k_up, v_up, k_flat, v_flat) if key_lengths.shape[1] > 0 else None
    if layout is not None:
        return splitk_attention(q3, k_flat, v_flat, layout, key_lengths, key_offsets,
                                value_lengths, value_offsets, theta=theta,
                                route=_lib.DKV_ROUTE_TWO_STAGE)
    out = _joint.joint_attention(q3, k_flat, k_up, v_flat, v_up, key_lengths, key_offsets,
                                 value_lengths, value_offsets, theta=theta,
                                 route=_lib.DKV_ROUTE_TWO_STAGE)
    if out is not None:
        return out
    scores = abx_sparse(q3, k_up, k_flat, key_lengths, offsets=key_offsets, theta=theta)
    return avx(scores, v_flat, v_up, value_lengths, value_offsets)
