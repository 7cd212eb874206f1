"""Dense masked-dimension decode attention on CPU torch (fp32) -- test infrastructure only.

Restates the reference research/CPU path ``src/dynakv/custom_attn.py``: the coefficients are kept
dense with the non-retained dimensions zeroed (hard mask, :78-83, :114-116), the whole cache is
re-projected to K/V every step with ``einsum('bsd,nd->bsn', coeffs, U)`` (:161-162 /
compressed_attention.py:169-170), K gets rotate-half RoPE at positions ``arange(S)`` with
HF-style cos/sin (:193-200, :237-240), and eager GQA attention runs with an fp32 softmax
(:242-255; transformers ``eager_attention_forward``).

Two uses: an independent formulation that pins ``oracle.attention`` (different data layout,
different RoPE code, joint basis), and the CPU baseline ``bench.py`` times.
"""

from __future__ import annotations

import torch


def hf_rotary(positions: torch.Tensor, head_dim: int, theta: float):
    """cos/sin of shape (S, Dh) in the HF layout: ``cat(freqs, freqs)``."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = positions.float()[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def decode_attention(q: torch.Tensor, ck: torch.Tensor, cv: torch.Tensor, Uk: torch.Tensor,
                     Uv: torch.Tensor, num_kv_heads: int, theta: float) -> torch.Tensor:
    """q (B, Hq, Dh) RoPE'd; ck/cv (B, S, D) hard-masked dense coefficients with D = Hkv*Dh;
    Uk/Uv (D, D) joint up-projections (``k_up``: coefficient d -> output n via ``U[n, d]``).
    Returns (B, Hq, Dh) fp32."""
    B, Hq, Dh = q.shape
    S = ck.shape[1]
    K = torch.einsum("bsd,nd->bsn", ck.float(), Uk.float())
    V = torch.einsum("bsd,nd->bsn", cv.float(), Uv.float())
    K = K.view(B, S, num_kv_heads, Dh).transpose(1, 2)
    V = V.view(B, S, num_kv_heads, Dh).transpose(1, 2)
    cos, sin = hf_rotary(torch.arange(S), Dh, theta)
    K = K * cos + rotate_half(K) * sin
    rep = Hq // num_kv_heads
    K = K.repeat_interleave(rep, dim=1)
    V = V.repeat_interleave(rep, dim=1)
    scores = torch.matmul(q.float().unsqueeze(2), K.transpose(-1, -2)) * (Dh ** -0.5)
    p = torch.softmax(scores.float(), dim=-1)
    return torch.matmul(p, V).squeeze(2)


def dense_from_packed(flat: torch.Tensor, lens: torch.Tensor, offs: torch.Tensor, R: int):
    """(rows, S, R) dense masked coefficients from a packed slot (zeros past each length)."""
    rows, S = lens.shape
    out = torch.zeros(rows, S, R, dtype=torch.float32)
    for b in range(rows):
        for s in range(S):
            n = max(0, min(int(lens[b, s]), R))
            o = int(offs[b, s])
            out[b, s, :n] = flat[b, o: o + n].float()
    return out


def block_diag_up(bases: torch.Tensor) -> torch.Tensor:
    """Joint (G*Dh, G*R) up-projection from per-group kernel bases (G, R, Dh):
    U[g*Dh + d, g*R + j] = basis[g, j, d] (inverse of the weight merge,
    compressed_attention.py:278-286)."""
    G, R, Dh = bases.shape
    U = torch.zeros(G * Dh, G * R, dtype=torch.float32)
    for g in range(G):
        U[g * Dh:(g + 1) * Dh, g * R:(g + 1) * R] = bases[g].float().t()
    return U
