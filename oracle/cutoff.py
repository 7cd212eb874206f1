"""Cutoff head (per-token retained-dimension count) in numpy -- test infrastructure only.

Restates ``KVProcessor.kv_process_fused`` (src/dynakv/kernels/compressed_attention.py:84-119) for
one matrix (K or V), per group g of G (G = 1 is the reference's joint head; the per-head form
applies the same formula to each group's D dims with its own W_g, b_g):

* logits = round(b_g + x_g @ W_g) in the compute dtype (torch.addmm, :92-93; the product is
  accumulated exactly here, in float64);
* p = round(softmax(logits)) in the compute dtype (:99; softmax of the rounded logits in
  float64);
* c_m = round(p_0 + ... + p_m) in the compute dtype (:99, cumsum of the rounded p);
* mask_j = c_{D-1-j} >= round(threshold) (:99-100: flip, then the compare in the compute dtype);
* mask[low_rank:] = 0 (:106-107); len = sum(mask) (:113-114); out = x * mask (:116-117),
  so a masked negative value becomes -0.0 as in the reference's product.

Since c is non-decreasing, mask is a prefix of length #{m : c_m >= thr}; ``cutoff`` also
returns c so that tests can tell rows whose length hinges on the last bit of a prefix sum
(``ambiguous_rows``) from rows whose length is fixed by the arithmetic.
"""

from __future__ import annotations

import numpy as np

from .attention import round_to


def cutoff(x, W, b, dtype: str, threshold: float = 0.1, low_rank: int | None = None):
    """x: (M, G*D); W: (G, D, D) with logits = x_g @ W_g; b: (G, D).

    Returns (out (M, G*D) float32, lens (M, G) int64, logits (M, G, D), c (M, G, D), thr)."""
    x = np.asarray(x, dtype=np.float64)
    W = np.asarray(W, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    G, D, _ = W.shape
    M = x.shape[0]
    xg = x.reshape(M, G, D)
    logits = np.einsum("mgk,gkn->mgn", xg, W) + b[None]
    logits = round_to(logits, dtype).astype(np.float64)
    lens, c, thr = lengths_from_logits(logits, dtype, threshold, low_rank)[:3]
    keep = (np.arange(D)[None, None, :] < lens[..., None]).astype(np.float32)
    out = (xg.astype(np.float32) * keep).reshape(M, G * D)
    return out, lens.astype(np.int64), logits, c, thr


def lengths_from_logits(logits, dtype: str, threshold: float = 0.1, low_rank: int | None = None):
    """Lengths from already-rounded logits (..., D): softmax, prefix sums and threshold.

    Returns (lens, c, thr, tie) where ``tie`` flags rows whose length an implementation that
    follows the same steps in fp32 may legitimately report differently: a probability within
    1e-6 (relative) of a rounding tie of the compute dtype can round either way, which moves
    the later prefix sums by up to one unit of that probability, and a prefix sum within that
    distance (plus fp32 accumulation slack) of the tie just below the threshold can then round
    to either side of it."""
    logits = np.asarray(logits, dtype=np.float64)
    D = logits.shape[-1]
    z = logits - logits.max(axis=-1, keepdims=True)
    e = np.exp(z)
    p_exact = e / e.sum(axis=-1, keepdims=True)
    p = round_to(p_exact, dtype).astype(np.float64)
    eta = 1e-6
    p_tie = round_to(p_exact * (1 + eta), dtype) != round_to(p_exact * (1 - eta), dtype)
    step = np.abs(round_to(p_exact * (1 + eta), dtype).astype(np.float64) - p)
    step = np.maximum(step, np.abs(round_to(p_exact * (1 - eta), dtype).astype(np.float64) - p))
    slack = np.cumsum(np.where(p_tie, np.maximum(step, np.abs(p) * 2.0 ** -7), 0.0), axis=-1)
    c_exact = np.cumsum(p, axis=-1)
    c = round_to(c_exact, dtype).astype(np.float64)
    thr = float(round_to(np.float32(threshold), dtype))
    d = slack + 1e-6 * np.abs(c_exact) + 1e-12
    lo_c = round_to(c_exact - d, dtype).astype(np.float64)
    hi_c = round_to(c_exact + d, dtype).astype(np.float64)
    tie = ((lo_c < thr) & (hi_c >= thr)).any(axis=-1)
    lens = (c >= thr).sum(axis=-1)
    lr = D if low_rank is None or low_rank < 0 else min(int(low_rank), D)
    lens = np.minimum(lens, lr)
    return lens, c, thr, tie


def ambiguous_rows(c: np.ndarray, thr: float, tol: float) -> np.ndarray:
    """(M, G) bool: some prefix sum lies within ``tol`` of the threshold, so a last-bit
    difference in the logits, the softmax or the summation order can move the length."""
    return (np.abs(c - thr) <= tol).any(axis=-1)


def length_bounds(c: np.ndarray, thr: float, tol: float, low_rank: int | None = None):
    """Smallest and largest length reachable when every prefix sum moves by at most ``tol``."""
    D = c.shape[-1]
    lr = D if low_rank is None or low_rank < 0 else min(int(low_rank), D)
    lo = np.minimum((c >= thr + tol).sum(axis=-1), lr)
    hi = np.minimum((c >= thr - tol).sum(axis=-1), lr)
    return lo, hi


def cutoff_loops(x, W, b, dtype: str, threshold: float = 0.1, low_rank: int | None = None):
    """Scalar-loop restatement of the same steps for tiny inputs (checks ``cutoff``)."""
    x = np.asarray(x, dtype=np.float64)
    W = np.asarray(W, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    G, D, _ = W.shape
    M = x.shape[0]
    rd = lambda v: float(round_to(np.float64(v), dtype))  # noqa: E731
    thr = rd(threshold)
    lr = D if low_rank is None or low_rank < 0 else min(int(low_rank), D)
    out = np.zeros((M, G * D), dtype=np.float32)
    lens = np.zeros((M, G), dtype=np.int64)
    for m in range(M):
        for g in range(G):
            lg = []
            for n in range(D):
                acc = b[g, n]
                for k in range(D):
                    acc += x[m, g * D + k] * W[g, k, n]
                lg.append(rd(acc))
            mx = max(lg)
            ex = [np.exp(v - mx) for v in lg]
            tot = sum(ex)
            p = [rd(v / tot) for v in ex]
            run, cs = 0.0, []
            for v in p:
                run += v
                cs.append(rd(run))
            flipped = cs[::-1]
            mask = [1 if flipped[j] >= thr else 0 for j in range(D)]
            for j in range(lr, D):
                mask[j] = 0
            lens[m, g] = sum(mask)
            for j in range(D):
                out[m, g * D + j] = np.float32(x[m, g * D + j]) * np.float32(mask[j])
    return out, lens
