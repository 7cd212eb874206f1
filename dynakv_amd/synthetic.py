"""Seeded synthetic workloads for the decode path (the benchmark configurations).

All generators are deterministic given the seed. Bases are random orthogonal matrices from the QR
decomposition of a N(0,1) matrix; the kernel basis of a group is ``U^T`` (rank x dim), so a
token's reconstruction is ``k = U x`` for coefficients ``x``. Because ``U`` is orthogonal and
pre-RoPE K/V are N(0, I), the coefficients ``x = U^T k`` are N(0, I) as well and are drawn
directly. Retained counts ``r`` are prefixes of the coefficient vector, as the reference's cutoff
head produces (flip(cumsum(softmax)) >= 0.1 keeps a prefix, compressed_attention.py:99-100).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch


def random_orthogonal(n: int, rng: np.random.Generator) -> np.ndarray:
    q, r = np.linalg.qr(rng.standard_normal((n, n)))
    return q * np.sign(np.diag(r))[None, :]


def beta_lengths(shape, mean: float, R: int, rng: np.random.Generator,
                 concentration: float = 4.0) -> np.ndarray:
    """r = clip(round(R * Beta(a, b)), 1, R) with a / (a + b) = mean."""
    a = mean * concentration
    b = (1.0 - mean) * concentration
    x = rng.beta(a, b, size=shape)
    return np.clip(np.rint(R * x), 1, R).astype(np.int32)


@dataclass
class PackedCase:
    """A per-head layout case: rows = B * G, row b*G + g holds group g of batch b."""

    B: int
    G: int
    Hq: int
    S: int
    R: int
    Dh: int
    theta: float
    q: np.ndarray        # (B, Hq, Dh) float32
    k_basis: np.ndarray  # (G, R, Dh) float32
    v_basis: np.ndarray
    k_coef: np.ndarray   # (rows, S, R) float32 dense coefficients
    v_coef: np.ndarray
    k_len: np.ndarray    # (rows, S) int32
    v_len: np.ndarray


def make_case(B: int, G: int, Hq: int, S: int, R: int = 128, Dh: int = 128, *,
              theta: float = 500000.0, mean: float | None = 0.3, uniform: tuple | None = None,
              force_first: int = 0, force_frac: float = 0.0, seed: int = 0,
              zero_len_frac: float = 0.0) -> PackedCase:
    rng = np.random.default_rng(seed)
    rows = B * G
    kb = np.stack([random_orthogonal(max(R, Dh), rng)[:Dh, :R].T for _ in range(G)])
    vb = np.stack([random_orthogonal(max(R, Dh), rng)[:Dh, :R].T for _ in range(G)])
    k_coef = rng.standard_normal((rows, S, R)).astype(np.float32)
    v_coef = rng.standard_normal((rows, S, R)).astype(np.float32)

    def lens():
        if uniform is not None:
            lo, hi = uniform
            L = rng.integers(lo, hi + 1, size=(rows, S)).astype(np.int32)
        else:
            L = beta_lengths((rows, S), mean, R, rng)
        if force_first:
            L[:, :force_first] = R
        if force_frac > 0:
            L[rng.random((rows, S)) < force_frac] = R
        if zero_len_frac > 0:
            L[rng.random((rows, S)) < zero_len_frac] = 0
        return L

    k_len, v_len = lens(), lens()
    q = rng.standard_normal((B, Hq, Dh)).astype(np.float32)
    return PackedCase(B, G, Hq, S, R, Dh, theta, q, kb.astype(np.float32), vb.astype(np.float32),
                      k_coef, v_coef, k_len, v_len)


# ---------------------------------------------------------------------------------------------
# Device-side generation for benchmark sizes (no host round trip of the coefficients)
# ---------------------------------------------------------------------------------------------
def device_lengths(rows: int, S: int, R: int, mean: float, gen: torch.Generator, device,
                   force_first: int = 0, force_frac: float = 0.0,
                   concentration: float = 4.0) -> torch.Tensor:
    a = torch.full((rows, S), mean * concentration, device=device)
    b = torch.full((rows, S), (1.0 - mean) * concentration, device=device)
    # Beta(a, b) = Ga / (Ga + Gb), gammas drawn with the seeded generator
    ga = torch._standard_gamma(a, generator=gen) if hasattr(torch, "_standard_gamma") else None
    if ga is None:  # pragma: no cover
        raise RuntimeError("torch._standard_gamma unavailable")
    gb = torch._standard_gamma(b, generator=gen)
    x = ga / (ga + gb)
    L = torch.clamp(torch.round(R * x), 1, R).to(torch.int32)
    if force_first:
        L[:, :force_first] = R
    if force_frac > 0:
        mask = torch.rand((rows, S), generator=gen, device=device) < force_frac
        L[mask] = R
    return L


def log_uniform_lengths(n: int, lo: int, hi: int, rng: np.random.Generator) -> np.ndarray:
    return np.exp(rng.uniform(math.log(lo), math.log(hi), size=n)).astype(np.int64)
