"""Prefill attention over the reconstructed cache in numpy -- test infrastructure only.

Restates the prefill branch of the reference's attention module
(src/dynakv/kernels/compressed_attention.py:359-386, kv_down_up :130-191):

* ``reconstruct``: dense K / V of a per-head cache row = its zero-padded coefficients
  (get_origin_states, compressed_cache.py:70-81) times the group's basis (the k_up / v_up
  einsum, :160-165), rounded to the compute dtype (the einsum's output dtype);
* ``rope_dense``: rotate-half RoPE of K at positions ``pos0 + s`` (calc_cos_sin, :193-200) with
  the angle formed in fp32 as ``float32(pos) * inv_freq`` (the decode kernels' convention),
  evaluated in float64 and rounded to the compute dtype;
* ``attention``: softmax(scale * q k^T) v per query head over its KV group (GQA), causal with
  the queries at the last ``Sq`` key positions (eager_attention_forward / SDPA with the causal
  mask, :373-383), in float64.
"""

from __future__ import annotations

import numpy as np

from .attention import apply_rope, round_to, rope_cos_sin


def reconstruct(coef: np.ndarray, basis: np.ndarray, dtype: str) -> np.ndarray:
    """coef (..., S, R) zero-padded coefficients, basis (R, Dh) -> rounded (..., S, Dh)."""
    return round_to(np.asarray(coef, np.float64) @ np.asarray(basis, np.float64), dtype).astype(
        np.float64)


def rope_dense(x: np.ndarray, theta: float, dtype: str, pos0: int = 0) -> np.ndarray:
    """x (..., S, 128) -> RoPE'd and rounded to dtype."""
    S = x.shape[-2]
    cos, sin = rope_cos_sin(np.arange(pos0, pos0 + S), x.shape[-1], theta)
    return round_to(apply_rope(np.asarray(x, np.float64), cos, sin), dtype).astype(np.float64)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool = True,
              scale: float | None = None, kstart=None) -> np.ndarray:
    """q (B, Hq, Sq, D), k/v (B, Hkv, Sk, D) -> (B, Hq, Sq, D) float64. ``kstart`` (B,): keys
    before ``kstart[b]`` are masked (a left-padded prompt: the reference's
    ``create_causal_mask(attention_mask, ...)``, custom_llama.py:161-168); a query with no key
    left gets 0."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    hpg = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    out = np.zeros((B, Hq, Sq, D))
    off = Sk - Sq
    for b in range(B):
        for h in range(Hq):
            s = q[b, h] @ k[b, h // hpg].T * scale  # (Sq, Sk)
            mask = np.zeros((Sq, Sk), dtype=bool)
            if causal:
                mask |= np.arange(Sk)[None, :] > (off + np.arange(Sq))[:, None]
            if kstart is not None:
                mask |= np.arange(Sk)[None, :] < int(kstart[b])
            s = np.where(mask, -np.inf, s)
            live = ~mask.all(axis=-1)
            m = np.where(live, np.where(mask, -np.inf, s).max(axis=-1), 0.0)
            p = np.where(mask, 0.0, np.exp(s - m[:, None]))
            den = np.where(live, p.sum(axis=-1), 1.0)
            out[b, h] = (p / den[:, None]) @ v[b, h // hpg]
    return out
