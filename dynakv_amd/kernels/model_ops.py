"""Fused element-wise stages of the end-to-end decoder (host side of ``dkv_model.hip``).

The reference runs DynaKV inside HF's Llama decoder layer (``custom_llama.py:93-323`` on
transformers' ``LlamaDecoderLayer``): ``hidden = residual + sublayer(...)``, ``LlamaRMSNorm``
(fp32 statistics, normalised value rounded to the model dtype, times the weight in that dtype)
and ``LlamaMLP`` (``down(silu(gate(h)) * up(h))``). ``add_rmsnorm_`` is the residual add fused
with the following norm, ``silu_mul`` the activation product of one concatenated gate/up GEMM,
``linear`` the decoder's projections: a weight-streaming kernel for decode-sized inputs (at most
8 rows), torch's library GEMM otherwise.
"""

from __future__ import annotations

import torch

from .. import _lib


def _rows(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1:
        raise ValueError("rows need a unit last stride")
    r = t.reshape(-1, t.shape[-1])
    if r.data_ptr() != t.data_ptr():
        raise ValueError("leading dims must flatten without a copy")
    return r


def add_rmsnorm_(x: torch.Tensor, delta: torch.Tensor | None, w: torch.Tensor, eps: float,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """``x += delta`` in place (rounded to x's dtype) when ``delta`` is given, then returns
    ``rmsnorm(x) * w`` (a new tensor of x's shape, or ``out``)."""
    xr = _rows(x)
    H = xr.shape[1]
    if out is None:
        out = torch.empty_like(x)
    orr = _rows(out)
    dr = _rows(delta) if delta is not None else None
    if dr is not None and dr.shape != xr.shape:
        raise ValueError("delta must have x's shape")
    if w.shape != (H,) or not w.is_contiguous() or w.dtype != x.dtype:
        raise ValueError("w must be a contiguous (H,) vector of x's dtype")
    lib = _lib.load()
    rc = lib.dkv_add_rmsnorm(_lib.stream_of(x), _lib.dtype_code(x.dtype), xr.data_ptr(),
                             xr.stride(0), dr.data_ptr() if dr is not None else None,
                             dr.stride(0) if dr is not None else 0, w.data_ptr(), orr.data_ptr(),
                             orr.stride(0), xr.shape[0], H, float(eps))
    _lib.check(rc, "dkv_add_rmsnorm")
    return out


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """``gu`` (..., 2F) = [gate | up] -> silu(gate) * up (..., F)."""
    gr = _rows(gu)
    F2 = gr.shape[1]
    if F2 % 2:
        raise ValueError("gu must hold gate and up halves")
    F = F2 // 2
    out = torch.empty(gu.shape[:-1] + (F,), dtype=gu.dtype, device=gu.device)
    orr = out.view(-1, F)
    lib = _lib.load()
    rc = lib.dkv_silu_mul(_lib.stream_of(gu), _lib.dtype_code(gu.dtype), gr.data_ptr(),
                          gr.stride(0), orr.data_ptr(), orr.stride(0), gr.shape[0], F)
    _lib.check(rc, "dkv_silu_mul")
    return out


def silu_mul_pairs(gu: torch.Tensor) -> torch.Tensor:
    """``gu`` (..., 2F) = [g0, u0, g1, u1, ...] (the output of a gate/up weight with interleaved
    rows) -> silu(g) * u (..., F): ``silu_mul`` of the de-interleaved halves, bit for bit."""
    gr = _rows(gu)
    F2 = gr.shape[1]
    if F2 % 2:
        raise ValueError("gu must hold gate/up pairs")
    F = F2 // 2
    out = torch.empty(gu.shape[:-1] + (F,), dtype=gu.dtype, device=gu.device)
    orr = out.view(-1, F)
    lib = _lib.load()
    rc = lib.dkv_silu_mul_pairs(_lib.stream_of(gu), _lib.dtype_code(gu.dtype), gr.data_ptr(),
                                gr.stride(0), orr.data_ptr(), orr.stride(0), gr.shape[0], F)
    _lib.check(rc, "dkv_silu_mul_pairs")
    return out


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, w)`` (no bias): ``dkv_gemv`` when x has at most 8 rows (decode), the
    library GEMM otherwise. With weights streamed from HBM (as in a decode step, where no
    matrix is reused before the others evict it) the kernel measured on MI355X: the Llama-3-8B
    attention projections ~8-14 us against ~18 us, gate/up 5.9 TB/s against 3.7, down on par.
    x larger than 64 KiB (down with 3+ rows) goes to the library GEMM: unstaged, the kernel is
    slower there."""
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    N = w.shape[0] if w.dim() == 2 else 0
    if (1 <= M <= 8 and M * K * 2 <= 64 * 1024 and x.dtype == w.dtype
            and x.dtype in (torch.bfloat16, torch.float16) and w.dim() == 2 and w.shape[1] == K
            and w.stride(1) == 1 and K % 8 == 0 and x.is_cuda):
        xr = x.reshape(M, K)
        if xr.stride(1) == 1 and xr.data_ptr() % 16 == 0 and xr.stride(0) % 8 == 0 \
                and w.data_ptr() % 16 == 0 and w.stride(0) % 8 == 0:
            y = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=x.device)
            rc = _lib.load().dkv_gemv(_lib.stream_of(x), _lib.dtype_code(x.dtype),
                                      xr.data_ptr(), xr.stride(0), w.data_ptr(), w.stride(0),
                                      y.data_ptr(), N, M, N, K)
            _lib.check(rc, "dkv_gemv")
            return y
    return torch.nn.functional.linear(x, w)


def rmsnorm_linear(x: torch.Tensor, delta: torch.Tensor | None, w_norm: torch.Tensor,
                   eps: float, w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``r = x + delta`` (or ``x``), ``y = F.linear(rmsnorm(r) * w_norm, w)``; returns
    ``(y, r)``. ``x`` is consumed: it may be updated in place and returned as ``r``. One
    ``dkv_gemv_rmsnorm`` launch for one or two rows (the normalised rows are bit-identical to
    ``add_rmsnorm_``'s), else ``add_rmsnorm_`` and ``linear``: every workgroup of the fused
    kernel normalises its own copy of the rows, which costs more than the saved launch from
    about four rows on (measured on MI355X)."""
    K = x.shape[-1]
    M = x.numel() // K
    if (M <= 2 and x.is_contiguous() and (delta is None or delta.is_contiguous())
            and K % 8 == 0 and x.dtype == w.dtype == w_norm.dtype
            and x.dtype in (torch.bfloat16, torch.float16) and w.dim() == 2 and w.shape[1] == K
            and w.stride(1) == 1 and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0
            and x.data_ptr() % 16 == 0 and (delta is None or delta.data_ptr() % 16 == 0)
            and x.is_cuda and M >= 1):
        N = w.shape[0]
        y = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=x.device)
        r = torch.empty_like(x) if delta is not None else x
        rc = _lib.load().dkv_gemv_rmsnorm(
            _lib.stream_of(x), _lib.dtype_code(x.dtype), x.data_ptr(), K,
            delta.data_ptr() if delta is not None else None, K, w_norm.data_ptr(), float(eps),
            r.data_ptr() if delta is not None else None, K, w.data_ptr(), w.stride(0),
            y.data_ptr(), N, M, N, K)
        _lib.check(rc, "dkv_gemv_rmsnorm")
        return y, r
    h = add_rmsnorm_(x, delta, w_norm, eps)
    return linear(h, w), x


def rmsnorm_glu(x: torch.Tensor, delta: torch.Tensor | None, w_norm: torch.Tensor, eps: float,
                w_gu: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``r = x + delta`` (or ``x``), ``h = silu(g) * u`` with ``g``/``u`` the gate/up
    projections of ``rmsnorm(r) * w_norm`` by ``w_gu``, whose rows interleave them (row 2j gate
    j, row 2j + 1 up j); returns ``(h, r)`` like ``rmsnorm_linear``. One ``dkv_gemv_glu``
    launch for one or two rows (norm folded in as well), ``add_rmsnorm_`` and one
    ``dkv_gemv_glu`` up to eight rows, else ``add_rmsnorm_``, the library GEMM and
    ``silu_mul_pairs`` of its interleaved output (the roundings of torch's ``silu(g) * u``)."""
    K = x.shape[-1]
    M = x.numel() // K
    N = w_gu.shape[0]
    F = N // 2
    ok_w = (w_gu.dim() == 2 and w_gu.shape[1] == K and N % 2 == 0 and w_gu.stride(1) == 1
            and w_gu.stride(0) % 8 == 0 and w_gu.data_ptr() % 16 == 0 and w_gu.dtype == x.dtype
            and x.dtype in (torch.bfloat16, torch.float16) and K % 8 == 0 and x.is_cuda)
    lib = _lib.load()
    if ok_w and M <= 2 and x.is_contiguous() and (delta is None or delta.is_contiguous()) \
            and w_norm.dtype == x.dtype and x.data_ptr() % 16 == 0 \
            and (delta is None or delta.data_ptr() % 16 == 0) and M >= 1:
        h = torch.empty(x.shape[:-1] + (F,), dtype=x.dtype, device=x.device)
        r = torch.empty_like(x) if delta is not None else x
        rc = lib.dkv_gemv_glu(_lib.stream_of(x), _lib.dtype_code(x.dtype), x.data_ptr(), K,
                              delta.data_ptr() if delta is not None else None, K,
                              w_norm.data_ptr(), float(eps),
                              r.data_ptr() if delta is not None else None, K, w_gu.data_ptr(),
                              w_gu.stride(0), h.data_ptr(), F, M, F, K)
        _lib.check(rc, "dkv_gemv_glu")
        return h, r
    y = add_rmsnorm_(x, delta, w_norm, eps)
    if ok_w and 1 <= M <= 8 and y.is_contiguous():
        h = torch.empty(y.shape[:-1] + (F,), dtype=y.dtype, device=y.device)
        rc = lib.dkv_gemv_glu(_lib.stream_of(y), _lib.dtype_code(y.dtype), y.data_ptr(), K,
                              None, 0, None, 0.0, None, 0, w_gu.data_ptr(), w_gu.stride(0),
                              h.data_ptr(), F, M, F, K)
        _lib.check(rc, "dkv_gemv_glu")
        return h, x
    gu = torch.nn.functional.linear(y, w_gu)
    if (gu.dtype in (torch.bfloat16, torch.float16) and F % 8 == 0 and gu.is_contiguous()
            and gu.data_ptr() % 16 == 0):
        return silu_mul_pairs(gu), x
    return torch.nn.functional.silu(gu[..., 0::2]) * gu[..., 1::2], x
