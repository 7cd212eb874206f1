"""Prefill attention over the compressed cache (host side of ``dkv_prefill.hip``).

Reference: the prefill branch of ``CustomAttention.forward``
(src/dynakv/kernels/compressed_attention.py:359-386) with ``kv_down_up`` (:130-191):
``update_sp`` packs the prompt, ``get_origin_states`` re-expands the cache, ``k_up`` / ``v_up``
project it back to head space, RoPE at positions ``0..S-1`` rotates K, and causal attention
runs over the result.

``reconstruct_kv`` does the re-expansion (``dkv_decompress``), the projection through the
per-head bases (one batched library GEMM per matrix) and the RoPE of K (``dkv_rope_dense``);
``prefill_attention`` is the causal GQA attention kernel; ``compressed_prefill_attention``
chains them for the per-head layout (cache rows ``b*G + g``).
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from .decode import rope_table


def _extent(t: torch.Tensor) -> int:
    """Elements addressable from ``t.data_ptr()`` by its strides: the byte range of the kernel's
    buffer resource over ``t`` is this count times the element size."""
    return _lib.view_extent(t)


def rope_dense_(x: torch.Tensor, *, theta: float, pos0: int = 0) -> torch.Tensor:
    """In place: rotate-half RoPE over the last dim (128) of ``x`` (..., S, 128) at positions
    ``pos0 + s``."""
    if x.shape[-1] != 128 or x.stride(-1) != 1:
        raise ValueError("rope_dense_ needs (..., S, 128) with unit last stride")
    if x.dim() < 2:
        raise ValueError("rope_dense_ needs a token dimension")
    S = x.shape[-2]
    lead = x.shape[:-2]
    rows = int(math.prod(lead)) if lead else 1
    x2 = x.reshape(rows, S, 128)
    if x2.data_ptr() != x.data_ptr():
        raise ValueError("rope_dense_ needs a tensor whose leading dims flatten without a copy")
    lib = _lib.load()
    _lib.check(lib.dkv_rope_dense(_lib.stream_of(x), _lib.dtype_code(x.dtype), x2.data_ptr(),
                                  x2.stride(0), x2.stride(1), rows, S, int(pos0),
                                  math.log(theta)), "dkv_rope_dense")
    return x


def rope_apply_(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """In place: ``x = x * cos + rotate_half(x) * sin`` in x's dtype, each product and the sum
    rounded as the reference's ``apply_rotary_pos_emb_`` computes it
    (``compressed_attention.py:18-22``). ``x`` (B, H, S, 128); ``cos`` / ``sin`` (B or 1, S, 128)
    as ``LlamaRotaryEmbedding`` returns them (the decoder's position embeddings)."""
    if x.dim() != 4 or x.shape[-1] != 128 or x.stride(-1) != 1:
        raise ValueError("rope_apply_ needs x (B, H, S, 128) with unit last stride")
    B, H, S, _ = x.shape
    cos, sin = cos.to(x.dtype), sin.to(x.dtype)
    if cos.dim() == 2:
        cos, sin = cos.unsqueeze(0), sin.unsqueeze(0)
    if cos.shape != sin.shape or cos.shape[0] not in (1, B) or cos.shape[1:] != (S, 128):
        raise ValueError(f"cos/sin {tuple(cos.shape)} do not match x {tuple(x.shape)}")
    if cos.stride() != sin.stride() or cos.stride(-1) != 1:
        cos, sin = cos.contiguous(), sin.contiguous()
    cs_sb = 0 if cos.shape[0] == 1 else cos.stride(0)
    lib = _lib.load()
    _lib.check(lib.dkv_rope_apply(_lib.stream_of(x), _lib.dtype_code(x.dtype), x.data_ptr(),
                                  x.stride(0), x.stride(1), x.stride(2), cos.data_ptr(),
                                  sin.data_ptr(), cs_sb, cos.stride(1), B, H, S),
               "dkv_rope_apply")
    return x


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = True,
                      scale: float | None = None, out: torch.Tensor | None = None,
                      out_dtype: torch.dtype | None = None,
                      kstart: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA attention: ``q`` (B, Hq, Sq, 128), ``k``/``v`` (B, Hkv, Sk, 128) ->
    (B, Hq, Sq, 128) in q's dtype (or ``out_dtype=torch.float32``: the result before that
    rounding). With ``causal`` the queries are the last ``Sq`` positions. ``kstart`` (B,) int32
    on the device: keys before ``kstart[b]`` are masked (left padding); a query with no key left
    gets 0."""
    B, Hq, Sq, Dh = q.shape
    _, Hkv, Sk, _ = k.shape
    if v.shape != k.shape or k.shape[0] != B or k.shape[3] != Dh:
        raise ValueError("k and v must be (B, Hkv, Sk, Dh) matching q")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("prefill_attention runs in float16 or bfloat16")
    for t in (q, k, v):
        if t.stride(-1) != 1:
            raise ValueError("unit last stride required")
    odt = out_dtype if out_dtype is not None else (out.dtype if out is not None else q.dtype)
    if odt not in (q.dtype, torch.float32):
        raise ValueError("out_dtype must be the query dtype or float32")
    if out is None:
        out = torch.empty((B, Hq, Sq, Dh), dtype=odt, device=q.device)
    elif out.dtype != odt or out.stride(-1) != 1:
        raise ValueError("out must have unit last stride and the requested dtype")
    scale = 1.0 / math.sqrt(Dh) if scale is None else float(scale)
    if kstart is not None:
        if kstart.shape != (B,) or kstart.device != q.device:
            raise ValueError("kstart must be (B,) on q's device")
        kstart = kstart.to(torch.int32).contiguous()
    lib = _lib.load()
    rc = lib.dkv_prefill_attention(
        _lib.stream_of(q), _lib.dtype_code(q.dtype),
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2), _extent(k),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), _extent(v),
        out.data_ptr(), _lib.dtype_code(out.dtype), out.stride(0), out.stride(1), out.stride(2),
        B, Hq, Hkv, Sq, Sk, Dh, 1 if causal else 0, scale,
        None if kstart is None else kstart.data_ptr())
    _lib.check(rc, "dkv_prefill_attention")
    return out


def _rotate_k(k: torch.Tensor, theta: float, k_rope) -> None:
    """RoPE of dense K (B, G, S, 128) at positions 0..S-1: the kernels' own rotation (fp32
    angles), or ``k_rope = (cos, sin)`` tables (S or B x S rows) applied as the reference's
    ``apply_rotary_pos_emb_`` does (its prefill rotates K by ``calc_cos_sin``,
    ``compressed_attention.py:193-200,375-378``)."""
    if k_rope is None:
        rope_dense_(k, theta=theta, pos0=0)
    else:
        rope_apply_(k, *k_rope)


def recon_kv(ck: torch.Tensor, cv: torch.Tensor, k_basis: torch.Tensor, v_basis: torch.Tensor,
             *, batch: int, theta: float, pos0: int = 0):
    """Dense K (rotated at positions ``pos0 + t``) and V ``(B, G, S, 128)`` from masked
    coefficient rows ``ck`` / ``cv`` ``(B*G, S, R)`` in one launch (``dkv_recon_kv``), or ``None``
    when the operands do not fit it (the caller then takes the library-GEMM path)."""
    G, R, Dh = k_basis.shape
    rows, S, Rc = ck.shape
    dt = ck.dtype
    if (dt not in (torch.float16, torch.bfloat16) or Dh != 128 or Rc != R or R % 8 or R > 128
            or cv.shape != ck.shape or cv.stride() != ck.stride() or ck.stride(2) != 1
            or not (cv.dtype == k_basis.dtype == v_basis.dtype == dt)
            or v_basis.shape != k_basis.shape or rows != batch * G):
        return None
    kb, vb = k_basis.contiguous(), v_basis.contiguous()
    if (ck.stride(0) % 8 or ck.stride(1) % 8 or ck.data_ptr() % 16 or cv.data_ptr() % 16
            or kb.data_ptr() % 16 or vb.data_ptr() % 16):
        return None
    k = torch.empty((batch, G, S, Dh), dtype=dt, device=ck.device)
    v = torch.empty_like(k)
    lib = _lib.load()
    st = _lib.stream_of(ck)
    rope, tiles = rope_table(ck.device, st, theta, int(pos0) + S)
    _lib.check(lib.dkv_recon_kv(st, _lib.dtype_code(dt), ck.data_ptr(),
                                cv.data_ptr(), ck.stride(0), ck.stride(1), kb.data_ptr(),
                                vb.data_ptr(), kb.stride(0), kb.stride(1), k.data_ptr(),
                                v.data_ptr(), S * Dh, Dh, rows, G, S, R, int(pos0),
                                rope.data_ptr(), tiles), "dkv_recon_kv")
    return k, v


def reconstruct_kv(cache, layer_idx: int, k_basis: torch.Tensor, v_basis: torch.Tensor, *,
                   batch: int, theta: float, k_rope=None):
    """Dense head-space K (RoPE'd at positions 0..S-1) and V ``(B, G, S, Dh)`` of a per-head
    cache (rows ``b*G + g``, bases ``(G, R, Dh)``)."""
    G, R, Dh = k_basis.shape
    dk, dv = cache.get_origin_states(R, layer_idx)  # (B*G, S, R), zero past each length
    rows, S, _ = dk.shape
    if rows != batch * G:
        raise ValueError(f"cache has {rows} rows, expected batch * G = {batch * G}")
    if k_rope is None:
        kv = recon_kv(dk, dv, k_basis, v_basis, batch=batch, theta=theta)
        if kv is not None:
            return kv
    k = torch.matmul(dk.view(batch, G, S, R), k_basis.contiguous())
    v = torch.matmul(dv.view(batch, G, S, R), v_basis.contiguous())
    _rotate_k(k, theta, k_rope)
    return k, v


def compressed_prefill_attention(q: torch.Tensor, cache, layer_idx: int, k_basis: torch.Tensor,
                                 v_basis: torch.Tensor, *, theta: float,
                                 out_dtype: torch.dtype | None = None, k_rope=None,
                                 kstart: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's prefill attention for the per-head layout: ``q`` (B, Hq, Sq, 128)
    already RoPE'd at its positions (the last ``Sq`` of the cache)."""
    k, v = reconstruct_kv(cache, layer_idx, k_basis, v_basis, batch=q.shape[0], theta=theta,
                          k_rope=k_rope)
    return prefill_attention(q, k, v, causal=True, out_dtype=out_dtype, kstart=kstart)


def coef_prefill_attention(q: torch.Tensor, ck: torch.Tensor, cv: torch.Tensor,
                           k_basis: torch.Tensor, v_basis: torch.Tensor, *, theta: float,
                           out_dtype: torch.dtype | None = None, k_rope=None,
                           kstart: torch.Tensor | None = None) -> torch.Tensor:
    """``compressed_prefill_attention`` from the masked coefficient rows themselves, ``ck`` /
    ``cv`` (B*G, S, R) zero past each token's count -- exactly what decompressing the packed
    cache returns -- so a prefill can attend before (or without) its appends."""
    G, R, Dh = k_basis.shape
    rows, S, _ = ck.shape
    batch = q.shape[0]
    if rows != batch * G or cv.shape != ck.shape:
        raise ValueError(f"coefficient rows {tuple(ck.shape)}, expected ({batch * G}, S, {R})")
    kv = recon_kv(ck, cv, k_basis, v_basis, batch=batch, theta=theta) if k_rope is None else None
    if kv is not None:
        k, v = kv
    else:
        k = torch.matmul(ck.view(batch, G, S, R), k_basis.contiguous())
        v = torch.matmul(cv.view(batch, G, S, R), v_basis.contiguous())
        _rotate_k(k, theta, k_rope)
    return prefill_attention(q, k, v, causal=True, out_dtype=out_dtype, kstart=kstart)
