"""Packed-cache layout and growth policy in numpy -- test infrastructure only.

Restates one slot (one layer's K or V cache) of the reference
``src/dynakv/kernels/compressed_cache.py``:

* first call sizes the flat buffer to ``max_b sum_t r[b,t]`` and the tables to the call's
  token count, pointers and upper bounds zero (:110-130);
* the sequence tables grow to ``max(cap + 1024, seq + new)`` (:135-145);
* a decode step adds ``new * MAX_DIM`` to the upper bound check, a prefill step the largest row
  total (:148-153); when ``max(ub) + added`` exceeds the flat capacity the true pointers are read
  and, if still too small, the flat buffer grows to ``max(cap + 1024 * (MAX_DIM // 2),
  max(ptr) + added)`` keeping each row's prefix (:156-168);
* decode append (the kernel, :7-34): ``off = ptr; ptr += r; lens = r; offs = off``, copy the
  first ``min(r, MAX_DIM)`` values;
* prefill append (:182-209): offsets ``ptr + exclusive_cumsum(r)``, values placed back to back,
  ``ptr += sum(min(r, MAX_DIM))``, ``ub = ptr``;
* ``seq += new`` and, for decode, ``ub += added`` (:211-214).
"""

from __future__ import annotations

import numpy as np

EXPAND_SEQ_STEP = 1024


class PackedSlot:
    def __init__(self):
        self.flat = None     # (B, capF)
        self.lens = None     # (B, capS) int32
        self.offs = None     # (B, capS) int32
        self.ptr = None      # (B,) int64 (values fit int32)
        self.seq = 0
        self.ub = None       # list[int]
        self.syncs = 0

    # -- growth ----------------------------------------------------------------------------
    def _ensure(self, new_states: np.ndarray, new_len: np.ndarray, max_dim: int, decode: bool):
        B, new_s = new_len.shape
        if self.flat is None:
            init = int(new_len.sum(axis=1).max())
            self.flat = np.zeros((B, init), dtype=new_states.dtype)
            self.lens = np.zeros((B, new_s), dtype=np.int32)
            self.offs = np.zeros((B, new_s), dtype=np.int32)
            self.ptr = np.zeros(B, dtype=np.int64)
            self.ub = [0] * B
            self.seq = 0
        if self.seq + new_s > self.lens.shape[1]:
            cap = max(self.lens.shape[1] + EXPAND_SEQ_STEP, self.seq + new_s)
            nl = np.zeros((B, cap), dtype=np.int32)
            no = np.zeros((B, cap), dtype=np.int32)
            nl[:, : self.seq] = self.lens[:, : self.seq]
            no[:, : self.seq] = self.offs[:, : self.seq]
            self.lens, self.offs = nl, no
        added = new_s * max_dim if decode else int(new_len.sum(axis=1).max())
        if max(self.ub) + added > self.flat.shape[1]:
            real = [int(p) for p in self.ptr]
            self.syncs += 1
            self.ub = real
            if max(real) + added > self.flat.shape[1]:
                cap = max(self.flat.shape[1] + EXPAND_SEQ_STEP * (max_dim // 2), max(real) + added)
                nf = np.zeros((B, cap), dtype=self.flat.dtype)
                for b in range(B):
                    nf[b, : real[b]] = self.flat[b, : real[b]]
                self.flat = nf
        return added

    # -- appends ---------------------------------------------------------------------------
    def append_decode(self, states: np.ndarray, new_len: np.ndarray, max_dim: int) -> None:
        """states (B, 1, MAX_DIM) or (B, MAX_DIM); new_len (B, 1)."""
        new_len = np.asarray(new_len).reshape(-1, 1)
        states = np.asarray(states).reshape(new_len.shape[0], -1)
        added = self._ensure(states, new_len, max_dim, True)
        for b in range(new_len.shape[0]):
            r = int(new_len[b, 0])
            off = int(self.ptr[b])
            self.ptr[b] = off + r
            self.lens[b, self.seq] = r
            self.offs[b, self.seq] = off
            n = min(r, max_dim)
            if n > 0:
                self.flat[b, off: off + n] = states[b, :n]
        self.seq += 1
        self.ub = [p + added for p in self.ub]

    def append_prefill(self, states: np.ndarray, new_len: np.ndarray, max_dim: int) -> None:
        """states (B, S, MAX_DIM); new_len (B, S)."""
        new_len = np.asarray(new_len)
        B, new_s = new_len.shape
        self._ensure(states, new_len, max_dim, False)
        for b in range(B):
            start = int(self.ptr[b])
            lens_b = new_len[b].astype(np.int64)
            excl = np.concatenate([[0], np.cumsum(lens_b)[:-1]])
            self.lens[b, self.seq: self.seq + new_s] = lens_b
            self.offs[b, self.seq: self.seq + new_s] = start + excl
            pos = start
            for t in range(new_s):
                n = max(0, min(int(lens_b[t]), max_dim))
                self.flat[b, pos: pos + n] = states[b, t, :n]
                pos += n
            self.ptr[b] = pos
        self.seq += new_s
        self.ub = [int(p) for p in self.ptr]

    # -- views -----------------------------------------------------------------------------
    def tables(self):
        return self.lens[:, : self.seq], self.offs[:, : self.seq]

    def decompress(self, max_dim: int) -> np.ndarray:
        """Dense (B, seq, max_dim), tokens read back to back from element 0 (reference :36-56)."""
        B = self.flat.shape[0]
        out = np.zeros((B, self.seq, max_dim), dtype=self.flat.dtype)
        for b in range(B):
            pos = 0
            for t in range(self.seq):
                n = max(0, min(int(self.lens[b, t]), max_dim))
                out[b, t, :n] = self.flat[b, pos: pos + n]
                pos += n
        return out


def pack_rows(coeffs: np.ndarray, lens: np.ndarray, max_dim: int):
    """One-shot packing of (B, S, MAX_DIM) coefficients into a fresh slot: (flat, lens, offs, ptr).

    Same result as ``PackedSlot().append_prefill`` (checked in the tests), vectorised per row:
    the first ``min(r, MAX_DIM)`` values of each token, back to back, offsets the exclusive
    prefix sum of the lengths.
    """
    coeffs = np.asarray(coeffs)
    lens = np.asarray(lens).astype(np.int64)
    B, S = lens.shape
    clen = np.clip(lens, 0, max_dim)
    totals = clen.sum(axis=1)
    cap = int(lens.sum(axis=1).max()) if B else 0
    flat = np.zeros((B, cap), dtype=coeffs.dtype)
    ar = np.arange(coeffs.shape[2])[None, :]
    for b in range(B):
        mask = ar < clen[b][:, None]
        vals = coeffs[b][mask]
        flat[b, : vals.size] = vals
    offs = np.zeros((B, S), dtype=np.int64)
    offs[:, 1:] = np.cumsum(lens, axis=1)[:, :-1]
    return flat, lens.astype(np.int32), offs.astype(np.int32), totals.astype(np.int64)
