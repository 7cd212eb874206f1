"""Decode attention over a packed cache, in numpy float64 -- test infrastructure only.

Restates, per (batch b, query head h), the reference kernels:

* K reconstruction from the first ``min(len, R)`` coefficients of each token
  (fused.py:80-94, two_stage.py:109-128): ``k_s = sum_j x_{s,j} * basis[h // hpg][j, :]``;
* rotate-half RoPE at the cache row index ``s`` with ``inv_freq_i = exp(-(2i/Dh) ln theta)``
  and the angle ``float32(s) * inv_freq`` formed in fp32 (fused.py:65-66, 97-102;
  two_stage.py:36-44, 130-144);
* score ``q . k' / sqrt(Dh)``;
  fused route: ``-inf`` where ``len_K == 0`` (fused.py:105-106);
  two-stage route: ``-1e4`` before the scale where ``len_K == 0``, then rounded to the query
  dtype (two_stage.py:153-157, output dtype :169);
* softmax over the cache and ``out = sum_s p_s v_s / D`` with ``v_s`` reconstructed from the first
  ``min(len_V, R)`` V coefficients (zero for ``len_V == 0``);
  ``D = sum p`` (fused.py:140), ``D = max(sum p, 1e-6)`` (two_stage.py:271).

Where the reference fused kernel would produce NaN because its first 64-token tile has no
``len_K > 0`` token (``exp(-inf - -inf)``), this restatement excludes those tokens and is NaN only
when every token is excluded; the build follows this restatement.
"""

from __future__ import annotations

import math

import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bfloat16, returned as float32."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return round_bf16(x)
    raise ValueError(dtype)


def inv_freq_f32(head_dim: int, theta: float) -> np.ndarray:
    """``exp(-(2i/Dh) * ln theta)`` evaluated in fp32 (fused.py:65-66)."""
    log_theta = np.float32(math.log(theta))
    f = (np.arange(head_dim // 2, dtype=np.float32) * np.float32(2)) / np.float32(head_dim)
    return np.exp(-f * log_theta).astype(np.float32)


def rope_cos_sin(positions: np.ndarray, head_dim: int, theta: float):
    """cos/sin (float64) of the fp32 angles ``float32(pos) * inv_freq``."""
    inv = inv_freq_f32(head_dim, theta)
    ang = (np.asarray(positions).astype(np.float32)[:, None] * inv[None, :]).astype(np.float32)
    a = ang.astype(np.float64)
    return np.cos(a), np.sin(a)


def apply_rope(k: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE on rows of ``k`` (S, Dh)."""
    h = k.shape[-1] // 2
    k0, k1 = k[..., :h], k[..., h:]
    return np.concatenate([k0 * cos - k1 * sin, k1 * cos + k0 * sin], axis=-1)


def gather_padded(flat_row: np.ndarray, lens_row: np.ndarray, offs_row: np.ndarray, R: int):
    """(S, R) float64: row s holds the first min(len, R) coefficients of token s, zero after."""
    lens_row = np.asarray(lens_row).astype(np.int64)
    offs_row = np.asarray(offs_row).astype(np.int64)
    S = lens_row.shape[0]
    X = np.zeros((S, R), dtype=np.float64)
    n = np.clip(lens_row, 0, R)
    mask = np.arange(R)[None, :] < n[:, None]
    idx = offs_row[:, None] + np.arange(R)[None, :]
    X[mask] = np.asarray(flat_row, dtype=np.float64)[idx[mask]]
    return X


def decode_attention(q, k_flat, k_up, v_flat, v_up, lens_k, offs_k, lens_v, offs_v, theta,
                     route: str = "short_fused", q_dtype: str = "float32",
                     row_of=None, basis_of=None) -> np.ndarray:
    """Decode attention of every (b, h); returns float64 (B, Hq, Dh).

    q: (B, Hq, Dh) already RoPE'd. k_flat/v_flat: (rows, cap). k_up/v_up: (Hb, R, Dh).
    Tables: (rows, S). By default row b serves batch b and basis ``h // (Hq // Hb)`` serves head
    h (the reference layout); ``row_of(b, h)`` / ``basis_of(h)`` override this for the per-head
    (batch, group) row layout.
    """
    q = np.asarray(q, dtype=np.float64)
    B, Hq, Dh = q.shape
    Hb, R, _ = k_up.shape
    hpg = Hq // Hb
    if row_of is None:
        row_of = lambda b, h: b  # noqa: E731
    if basis_of is None:
        basis_of = lambda h: h // hpg  # noqa: E731
    S = lens_k.shape[1]
    cos, sin = rope_cos_sin(np.arange(S), Dh, theta)
    scale = np.float32(1.0) / np.sqrt(np.float32(Dh))
    out = np.zeros((B, Hq, Dh), dtype=np.float64)
    cache = {}
    for b in range(B):
        for h in range(Hq):
            row, bi = row_of(b, h), basis_of(h)
            key = (row, bi)
            if key not in cache:
                Xk = gather_padded(np.asarray(k_flat[row], np.float64), lens_k[row], offs_k[row], R)
                Xv = gather_padded(np.asarray(v_flat[row], np.float64), lens_v[row], offs_v[row], R)
                K = apply_rope(Xk @ np.asarray(k_up[bi], np.float64), cos, sin)
                cache[key] = (K, Xv)
            K, Xv = cache[key]
            dot = K @ q[b, h]
            has = np.asarray(lens_k[row]) > 0
            if route == "short_fused":
                z = np.where(has, dot * float(scale), -np.inf)
            else:
                z = np.where(has, dot, -1.0e4) * float(scale)
                z = round_to(z, q_dtype).astype(np.float64)
            if S == 0 or not np.isfinite(z).any():
                p = np.zeros(S)
                m_ok = False
            else:
                p = np.exp(z - z[np.isfinite(z)].max())
                m_ok = True
            l = p.sum()
            acc = p @ Xv
            if route == "short_fused":
                den = l if m_ok else 0.0
                with np.errstate(invalid="ignore", divide="ignore"):
                    a = acc / den
            else:
                a = acc / max(l, 1e-6)
            out[b, h] = a @ np.asarray(v_up[bi], np.float64)
    return out


def scores_two_stage(q, k_flat, k_up, lens_k, offs_k, theta, out_dtype="float32") -> np.ndarray:
    """abx semantics (two_stage.py:48-157): (B, Hq, S) scores rounded to ``out_dtype``."""
    q = np.asarray(q, dtype=np.float64)
    B, Hq, Dh = q.shape
    Hb, R, _ = k_up.shape
    hpg = Hq // Hb
    S = lens_k.shape[1]
    cos, sin = rope_cos_sin(np.arange(S), Dh, theta)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(Dh)))
    out = np.zeros((B, Hq, S), dtype=np.float32)
    for b in range(B):
        Xk = gather_padded(np.asarray(k_flat[b], np.float64), lens_k[b], offs_k[b], R)
        for h in range(Hq):
            K = apply_rope(Xk @ np.asarray(k_up[h // hpg], np.float64), cos, sin)
            z = np.where(np.asarray(lens_k[b]) > 0, K @ q[b, h], -1.0e4) * scale
            out[b, h] = round_to(z, out_dtype)
    return out


def av_two_stage(scores, v_flat, v_up, lens_v, offs_v, clamp=True) -> np.ndarray:
    """avx semantics (two_stage.py:207-281) on given scores: float64 (B, Hq, Dh)."""
    sc = np.asarray(scores, dtype=np.float64)
    B, Hq, S = sc.shape
    Hb, R, Dh = v_up.shape
    grp = Hq // Hb
    out = np.zeros((B, Hq, Dh), dtype=np.float64)
    for b in range(B):
        Xv = gather_padded(np.asarray(v_flat[b], np.float64), lens_v[b], offs_v[b], R)
        for h in range(Hq):
            z = sc[b, h]
            fin = np.isfinite(z)
            if not fin.any():
                out[b, h] = np.nan if not clamp else 0.0
                continue
            p = np.where(fin, np.exp(z - z[fin].max()), 0.0)
            l = p.sum()
            a = (p @ Xv) / (max(l, 1e-6) if clamp else l)
            out[b, h] = a @ np.asarray(v_up[h // grp], np.float64)
    return out
