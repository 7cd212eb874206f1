"""Host side of the gfx950 split-K decode-attention kernel.

``splitk_attention`` launches ``dkv_decode_splitk`` (split-K attention, then the merge and V
projection) on torch's current stream. It is used
by both router routes when the inputs fit the kernel and, directly, by the native multi-group
layout (per-head spectral bases, one packed cache row per (batch, KV group)):
``grouped_decode_attention``.

Two device buffers are cached per (device, stream): the RoPE cos/sin table (per theta; extended
as the cache grows, so decode steps do not rebuild it) and the split-record workspace.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .. import _lib

SPLITK_MAX_RANK = 128
SPLITK_HEAD_DIM = 128
SPLITK_MAX_HPG = 16

_ROPE_CACHE: dict = {}  # (device, stream, theta) -> (table, tiles)
_WS_CACHE: dict = {}    # (device, stream) -> zeroed fp32 workspace


def rope_table(device: torch.device, stream: int, theta: float, seq_len: int):
    """RoPE table with at least ceil(seq_len / 16) tile rows for ``theta`` (cached, grown by
    doubling; a replaced table stays allocated, ``_lib.retire``)."""
    lib = _lib.load()
    need = max(1, (seq_len + 15) // 16)
    key = (device.index, stream, float(theta))
    ent = _ROPE_CACHE.get(key)
    if ent is None or ent[1] < need:
        tiles = max(need, 2 * ent[1] if ent else 0, 64)
        t = torch.empty(int(lib.dkv_rope_table_floats(tiles)), dtype=torch.float32,
                        device=device)
        _lib.check(lib.dkv_rope_table(stream, t.data_ptr(), 0, tiles, math.log(theta)),
                   "dkv_rope_table")
        if ent is not None:
            _lib.retire(ent[0])
        ent = (t, tiles)
        _ROPE_CACHE[key] = ent
    return ent


def workspace(device: torch.device, stream: int, floats: int) -> torch.Tensor:
    """Split-K workspace of at least ``floats`` floats (cached per device and stream). It is
    zero-filled when allocated: its leading merge counters must start at zero, and every call
    leaves them zero. It grows at least twofold; a replaced workspace stays allocated
    (``_lib.retire``: graphs captured with it keep using it)."""
    key = (device.index, stream)
    t = _WS_CACHE.get(key)
    if t is None or t.numel() < floats:
        old = t
        grow = 2 * old.numel() if old is not None else 0
        t = torch.zeros(max(int(floats), grow, 1 << 16), dtype=torch.float32, device=device)
        _lib.retire(old)
        _WS_CACHE[key] = t
    return t


@dataclass(frozen=True)
class UnitLayout:
    """How query heads map onto the kernel's work units (one unit per KV basis)."""

    n_kv: int          # distinct bases (work units per batch row)
    k_unit: int        # element stride between consecutive bases in k_up
    v_unit: int
    k_basis: torch.Tensor
    v_basis: torch.Tensor


# Largest row stride (elements) of a flat buffer the split kernel addresses: each workgroup's
# buffer resource starts at its own row and covers at most 0x3ffffff0 elements, of which a row
# needs its stride plus one 16-byte window (dkv_splitk.hip FLAT_LD_MAX).
FLAT_LD_MAX = 0x3FFFFFE8


def flat_ok(t: torch.Tensor) -> bool:
    """A packed flat buffer the split kernel can read: 2-D, unit element stride, row stride at
    most ``FLAT_LD_MAX`` (the limit is per row; the number of rows is free up to 2^31 - 1)."""
    return (t.dim() == 2 and t.stride(1) == 1 and 0 < t.stride(0) <= FLAT_LD_MAX
            and t.shape[0] < 2**31)


def _basis_ok(t: torch.Tensor) -> bool:
    return (t.dim() == 3 and t.stride(2) == 1 and t.stride(1) % 8 == 0
            and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0)


def splitk_layout(q3: torch.Tensor, k_up: torch.Tensor, v_up: torch.Tensor,
                  k_flat: torch.Tensor, v_flat: torch.Tensor) -> UnitLayout | None:
    """Unit layout for the split-K kernel, or ``None`` when the inputs need the vector path.

    Bases of shape ``(Hb, R, Dh)`` with ``Hb < Hq`` are shared by ``Hq / Hb`` consecutive query
    heads (the reference's ``HEADS_PER_GROUP``); ``Hb == Hq`` with a zero head stride (an
    ``expand``) is one shared basis; otherwise every query head is its own unit.
    """
    dt = q3.dtype
    if dt not in (torch.float16, torch.bfloat16) or q3.device.type != "cuda":
        return None
    if not (k_flat.dtype == v_flat.dtype == k_up.dtype == v_up.dtype == dt):
        return None
    if k_up.dim() != 3 or v_up.shape != k_up.shape:
        return None
    hb, r, dh = k_up.shape
    B, hq, qdh = q3.shape
    if dh != SPLITK_HEAD_DIM or qdh != dh or r > SPLITK_MAX_RANK or r <= 0 or hq % hb:
        return None
    if not (flat_ok(k_flat) and flat_ok(v_flat)):
        return None
    if hb == hq and k_up.stride(0) == 0 and v_up.stride(0) == 0:
        n_kv = 1
    else:
        n_kv = hb
    if hq // n_kv > SPLITK_MAX_HPG:
        return None
    kb, vb = k_up, v_up
    if not _basis_ok(kb):
        kb = kb.contiguous()
        if n_kv == 1 and hb == hq:
            kb = kb[:1]
    if not _basis_ok(vb):
        vb = vb.contiguous()
        if n_kv == 1 and hb == hq:
            vb = vb[:1]
    return UnitLayout(n_kv, kb.stride(0), vb.stride(0), kb, vb)


def splitk_attention(q3: torch.Tensor, k_flat: torch.Tensor, v_flat: torch.Tensor,
                     layout: UnitLayout, lens_k: torch.Tensor, offs_k: torch.Tensor,
                     lens_v: torch.Tensor, offs_v: torch.Tensor, *, theta: float, route: int,
                     groups: int = 1, split_len: int = 0,
                     out: torch.Tensor | None = None,
                     out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Run the split-K kernel. ``q3``: (B, Hq, 128); tables: (B*groups, S) int32.

    The output is in ``q3``'s dtype (the reference's contract) unless ``out_dtype=torch.float32``
    asks for the merged result before that rounding."""
    lib = _lib.load()
    B, hq, dh = q3.shape
    if q3.stride(2) != 1:
        q3 = q3.contiguous()
    S = lens_k.shape[1]
    R = layout.k_basis.shape[1]
    for t in (lens_k, offs_k, lens_v, offs_v):
        if t.dtype != torch.int32:
            raise ValueError("length/offset tables must be int32")
    if offs_k.stride() != lens_k.stride() or offs_v.stride() != lens_v.stride():
        lens_k, offs_k = lens_k.contiguous(), offs_k.contiguous()
        lens_v, offs_v = lens_v.contiguous(), offs_v.contiguous()
    odt = out_dtype if out_dtype is not None else (out.dtype if out is not None else q3.dtype)
    if odt not in (q3.dtype, torch.float32):
        raise ValueError("out_dtype must be the query dtype or float32")
    if out is None:
        out = torch.empty((B, hq, dh), dtype=odt, device=q3.device)
    elif out.dtype != odt or out.stride(2) != 1:
        raise ValueError("out must have unit last stride and the requested dtype")
    k_flat, v_flat = _lib.flat_operand(k_flat), _lib.flat_operand(v_flat)
    st = _lib.stream_of(q3)
    nfl = lib.dkv_splitk_workspace_floats(B, hq, layout.n_kv, S, R, split_len)
    ws = workspace(q3.device, st, int(nfl))
    rope, rope_tiles = rope_table(q3.device, st, theta, S)
    rc = lib.dkv_decode_splitk(
        st, route, _lib.dtype_code(q3.dtype),
        q3.data_ptr(), q3.stride(0), q3.stride(1),
        layout.k_basis.data_ptr(), layout.k_unit, layout.k_basis.stride(1),
        layout.v_basis.data_ptr(), layout.v_unit, layout.v_basis.stride(1),
        k_flat.data_ptr(), k_flat.stride(0), v_flat.data_ptr(), v_flat.stride(0),
        lens_k.data_ptr(), offs_k.data_ptr(), lens_k.stride(0), lens_k.stride(1),
        lens_v.data_ptr(), offs_v.data_ptr(), lens_v.stride(0), lens_v.stride(1),
        rope.data_ptr(), rope_tiles, ws.data_ptr(), ws.numel(),
        out.data_ptr(), out.stride(0), out.stride(1), _lib.dtype_code(out.dtype),
        B, hq, layout.n_kv, groups, S, R, dh, split_len)
    _lib.check(rc, "dkv_decode_splitk")
    return out


def grouped_decode_attention(q: torch.Tensor, k_flat: torch.Tensor, v_flat: torch.Tensor,
                             lens_k: torch.Tensor, offs_k: torch.Tensor,
                             lens_v: torch.Tensor, offs_v: torch.Tensor,
                             k_basis: torch.Tensor, v_basis: torch.Tensor, *, theta: float,
                             route: str = "long_two_stage", split_len: int = 0,
                             out: torch.Tensor | None = None,
                             out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Per-head spectral layout: one packed row per (batch b, KV group g), row = b*G + g.

    ``q``: (B, Hq, Dh) or (B, Hq, 1, Dh); ``k_basis``/``v_basis``: (G, R, Dh) with the basis of
    group g shared by query heads ``g*Hq/G ... (g+1)*Hq/G - 1``; tables ``(B*G, S)``.
    ``route`` is a router decision string and selects the route semantics.
    """
    q3 = q.squeeze(2) if q.dim() == 4 else q
    G = k_basis.shape[0]
    B = q3.shape[0]
    if lens_k.shape[0] != B * G:
        raise ValueError(f"tables have {lens_k.shape[0]} rows, expected B*G = {B * G}")
    layout = splitk_layout(q3, k_basis, v_basis, k_flat, v_flat)
    if layout is None or layout.n_kv != G:
        raise NotImplementedError("grouped_decode_attention needs f16/bf16, Dh=128, R<=128, "
                                  "Hq/G <= 16 and one basis per group")
    rt = _lib.DKV_ROUTE_FUSED if route == "short_fused" else _lib.DKV_ROUTE_TWO_STAGE
    return splitk_attention(q3, k_flat, v_flat, layout, lens_k, offs_k, lens_v, offs_v,
                            theta=theta, route=rt, groups=G, split_len=split_len, out=out,
                            out_dtype=out_dtype)


def dense_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           S: int, *, split_len: int = 0, out: torch.Tensor | None = None,
                           out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Dense GQA decode attention over an uncompressed cache (``dkv_decode_dense``): the
    end-to-end comparison's baseline, the attention of the reference's uncompressed model.

    ``q``: (B, Hq, 128) or (B, Hq, 1, 128), rotated. ``k_cache`` / ``v_cache``: (B * Hkv, ld)
    with unit last stride; row b * Hkv + g holds token t's rotated key (value) at elements
    t * 128 .. t * 128 + 127; tokens 0 .. S-1 are attended."""
    lib = _lib.load()
    q3 = q.squeeze(2) if q.dim() == 4 else q
    if q3.stride(2) != 1 or q3.data_ptr() % 16 or q3.stride(0) % 8 or q3.stride(1) % 8:
        q3 = q3.contiguous()
    B, hq, dh = q3.shape
    if k_cache.shape != v_cache.shape or k_cache.dim() != 2 or k_cache.shape[0] % max(B, 1):
        raise ValueError("k_cache / v_cache must be (B * Hkv, ld) of the same shape")
    if k_cache.dtype != q3.dtype or v_cache.dtype != q3.dtype:
        raise ValueError("cache and query dtypes differ")
    if k_cache.stride(1) != 1 or v_cache.stride(1) != 1 or k_cache.stride(0) != v_cache.stride(0):
        raise ValueError("cache rows must be contiguous with one row stride for K and V")
    hkv = k_cache.shape[0] // B
    odt = out_dtype if out_dtype is not None else (out.dtype if out is not None else q3.dtype)
    if odt not in (q3.dtype, torch.float32):
        raise ValueError("out_dtype must be the query dtype or float32")
    if out is None:
        out = torch.empty((B, hq, dh), dtype=odt, device=q3.device)
    elif out.dtype != odt or out.stride(2) != 1:
        raise ValueError("out must have unit last stride and the requested dtype")
    st = _lib.stream_of(q3)
    nfl = lib.dkv_dense_workspace_floats(B, hq, hkv, S, split_len)
    ws = workspace(q3.device, st, int(nfl))
    rc = lib.dkv_decode_dense(
        st, _lib.dtype_code(q3.dtype), q3.data_ptr(), q3.stride(0), q3.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), S, ws.data_ptr(), ws.numel(),
        out.data_ptr(), out.stride(0), out.stride(1), _lib.dtype_code(out.dtype),
        B, hq, hkv, dh, split_len)
    _lib.check(rc, "dkv_decode_dense")
    return out


def dense_append_(y: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *,
                  q_pos: int, k_pos: int, heads: int, kv_heads: int, theta: float) -> None:
    """One decode step's cache write of the dense baseline (``dkv_dense_append``): ``y`` (B, W)
    rows of the fused q/k/v projection (``heads`` query heads, then ``kv_heads`` key heads, then
    ``kv_heads`` value heads of 128); the query heads are rotated in place at ``q_pos``, the key
    heads rotated at ``k_pos`` into ``k_cache`` (B * kv_heads, ld) at token ``k_pos``, the value
    heads copied into ``v_cache``."""
    lib = _lib.load()
    if y.dim() != 2 or y.stride(1) != 1:
        raise ValueError("y must be (B, W) with unit last stride")
    if k_cache.stride(1) != 1 or v_cache.stride(1) != 1 or k_cache.stride(0) != v_cache.stride(0):
        raise ValueError("cache rows must be contiguous with one row stride for K and V")
    if not (y.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("y and cache dtypes differ")
    _lib.check(lib.dkv_dense_append(_lib.stream_of(y), _lib.dtype_code(y.dtype), y.data_ptr(),
                                    y.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
                                    k_cache.stride(0), int(q_pos), int(k_pos), y.shape[0],
                                    int(heads), int(kv_heads), math.log(theta)),
               "dkv_dense_append")
