"""One-call decode step of an attention layer over the per-head compressed cache.

The reference's decode branch (src/dynakv/kernels/compressed_attention.py:312-357) runs, per
layer and step, the cutoff head, the K and V appends, the router and the attention call, each
a separate Python-level operation. ``DecodeLayerPlan`` gathers everything that stays fixed
between steps (weights, cache buffers, strides, workspaces) into one ``DkvDecodeLayer``
argument block, so a step is a single ``dkv_decode_layer`` call with the step's q, the K/V
coefficients and the position. The plan reads the cache's capacities when it is built; a step
that would need the cache to grow (or a longer RoPE table) reports ``can_step() == False`` and
the caller takes the regular path (``update_sp`` and the attention call) for it and rebuilds
the plan after.
"""

from __future__ import annotations

import ctypes
import math

import torch

from .. import _lib
from . import cutoff as _cutoff
from .decode import rope_table, workspace
from .router import KernelPolicy


class DecodeLayerPlan:
    def __init__(self, cache, layer_idx: int, head: _cutoff.CutoffHead, k_basis: torch.Tensor,
                 v_basis: torch.Tensor, *, batch: int, heads: int, theta: float,
                 policy: KernelPolicy | None = None):
        self.cache = cache
        self.layer = layer_idx
        self.head = head
        self.policy = policy or KernelPolicy()
        G, R, Dh = k_basis.shape
        if head.groups != G or head.D != R:
            raise ValueError("cutoff head and bases disagree on groups / rank")
        self.B, self.G, self.R, self.Dh, self.Hq = batch, G, R, Dh, heads
        self.k_basis = k_basis.contiguous()
        self.v_basis = v_basis.contiguous()
        self.theta = theta
        self.args = None
        self._build()

    def _build(self):
        ck = self.cache.key_cache_sp[self.layer]
        cv = self.cache.value_cache_sp[self.layer]
        fk, lk, ok, pk = ck[0], ck[1], ck[2], ck[3]
        fv, lv, ov, pv = cv[0], cv[1], cv[2], cv[3]
        dev = fk.device
        if not (_lib.flat_covers_rows(fk) and _lib.flat_covers_rows(fv)):
            raise ValueError("the cache's flat buffers must hold rows * ld elements")
        st = _lib.stream_of(fk)
        lib = _lib.load()
        B, G, R, Dh, Hq = self.B, self.G, self.R, self.Dh, self.Hq
        self.cap_seq = min(lk.shape[1], lv.shape[1])
        self.cap_flat = min(fk.shape[1], fv.shape[1])
        self.rope, tiles = rope_table(dev, st, self.theta, self.cap_seq)
        self.rope_positions = tiles * 16
        units = B * G
        bound = 16384 + units * max(1, -(-256 // units)) * (Hq // G) * (Dh + 2)
        need = int(lib.dkv_splitk_workspace_floats(B, Hq, G, self.cap_seq, R, 0))
        self.split_ws = workspace(dev, st, max(bound, need))
        nb = int(lib.dkv_cutoff_workspace_bytes(B, G, R))
        self.cut_ws = _cutoff._workspace(dev, st, nb)
        dt = fk.dtype
        self.coef = torch.empty((2, B, G * R), dtype=dt, device=dev)
        self.lens = torch.empty((2, B * G), dtype=torch.int32, device=dev)
        h = self.head
        a = _lib.DecodeLayerArgs()
        a.dtype, a.B, a.G, a.Hq, a.R, a.Dh = _lib.dtype_code(dt), B, G, Hq, R, Dh
        a.low_rank = -1 if h.low_rank is None else int(h.low_rank)
        a.switch_tokens = int(self.policy.switch_tokens)
        a.threshold, a.log_theta = float(h.threshold), math.log(self.theta)
        a.wt_k, a.wt_v = h.wt_k.data_ptr(), h.wt_v.data_ptr()
        a.b_k, a.b_v = h.b_k.data_ptr(), h.b_v.data_ptr()
        a.cut_ws, a.cut_ws_bytes = self.cut_ws.data_ptr(), self.cut_ws.numel()
        a.coef_k, a.coef_v = self.coef[0].data_ptr(), self.coef[1].data_ptr()
        a.len_k, a.len_v = self.lens[0].data_ptr(), self.lens[1].data_ptr()
        a.flat_k, a.flat_k_ld = fk.data_ptr(), fk.stride(0)
        a.lens_k, a.offs_k = lk.data_ptr(), ok.data_ptr()
        a.tab_k_sb, a.tab_k_ss, a.ptr_k = lk.stride(0), lk.stride(1), pk.data_ptr()
        a.flat_v, a.flat_v_ld = fv.data_ptr(), fv.stride(0)
        a.lens_v, a.offs_v = lv.data_ptr(), ov.data_ptr()
        a.tab_v_sb, a.tab_v_ss, a.ptr_v = lv.stride(0), lv.stride(1), pv.data_ptr()
        a.k_basis, a.k_unit, a.k_sr = self.k_basis.data_ptr(), self.k_basis.stride(0), self.k_basis.stride(1)
        a.v_basis, a.v_unit, a.v_sr = self.v_basis.data_ptr(), self.v_basis.stride(0), self.v_basis.stride(1)
        a.rope, a.rope_tiles = self.rope.data_ptr(), tiles
        a.split_ws, a.split_ws_floats = self.split_ws.data_ptr(), self.split_ws.numel()
        self.args = a
        self._ptr = ctypes.byref(a)
        self._slots = (ck, cv)
        # the tensors the argument block points at must stay the cache's own
        self._bufs = (fk, lk, ok, pk, fv, lv, ov, pv)

    def can_step(self) -> bool:
        ck, cv = self.cache.key_cache_sp[self.layer], self.cache.value_cache_sp[self.layer]
        now = (ck[0], ck[1], ck[2], ck[3], cv[0], cv[1], cv[2], cv[3])
        if any(a is not b for a, b in zip(now, self._bufs)) or ck is not self._slots[0]:
            return False
        seq = ck[4]
        return (seq + 1 <= self.cap_seq and seq + 1 <= self.rope_positions
                and max(ck[5]) + self.R <= self.cap_flat and max(cv[5]) + self.R <= self.cap_flat)

    def rebuild(self):
        self._build()

    def step(self, q: torch.Tensor, k_coef: torch.Tensor, v_coef: torch.Tensor,
             pos: int) -> torch.Tensor:
        """q (B, Hq, Dh) with contiguous heads (any batch stride), rotated in place at ``pos``
        (``pos == -1``: q arrives rotated, e.g. by the HF decoder's position embeddings); k/v_coef
        (B, G*R) with unit element stride and one shared row stride (views into one projection
        output are fine). Returns the attention output (B, Hq, Dh) contiguous in the cache
        dtype."""
        ck, cv = self._slots
        seq = ck[4]
        B, Hq, Dh = self.B, self.Hq, self.Dh
        if (q.shape != (B, Hq, Dh) or q.stride(2) != 1 or q.stride(1) != Dh
                or k_coef.shape != (B, self.G * self.R) or v_coef.shape != k_coef.shape
                or k_coef.stride(1) != 1 or v_coef.stride(1) != 1
                or (B > 1 and k_coef.stride(0) != v_coef.stride(0))):
            raise ValueError("q / coefficient layout not supported by the layer step")
        a = self.args
        a.q_sb = q.stride(0) if B > 1 else Hq * Dh
        a.coef_ld = k_coef.stride(0) if B > 1 else self.G * self.R
        out = torch.empty((B, Hq, Dh), dtype=q.dtype, device=q.device)
        rc = _lib.load().dkv_decode_layer(_lib.stream_of(q), self._ptr, q.data_ptr(),
                                          k_coef.data_ptr(), v_coef.data_ptr(), out.data_ptr(),
                                          seq, pos)
        _lib.check(rc, "dkv_decode_layer")
        R = self.R
        for c in (ck, cv):
            c[4] = seq + 1
            c[5] = [u + R for u in c[5]]
        return out
