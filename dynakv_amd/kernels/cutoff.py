"""Cutoff head on the GPU: per-token retained-dimension counts and masked coefficients.

Drop-in for the reference's ``KVProcessor.kv_process_fused``
(src/dynakv/kernels/compressed_attention.py:84-119), which the decode step replays under a
CUDA graph before appending to the cache (:321-334):

    logits = addmm(b, x, W)                      # (B*S, D) in the compute dtype
    mask   = softmax(logits).cumsum(-1).flip(-1) >= 0.1
    mask[..., low_rank:] = 0
    len    = mask.sum(-1, dtype=int32);  out = x * mask

``CutoffHead(Wk, bk, Wv, bv)`` holds the weights like the reference's module attributes and
``kv_process_fused(key_states, value_states)`` returns the reference's tuple
``(k_out, v_out, len_k, len_v, 1, 1)``. ``groups=G`` applies the formula per group of
``D = hidden / G`` dims with per-group weights ``(G, D, D)`` / ``(G, D)`` (the per-head layout,
row = b*G + g in the cache); ``len`` then has shape ``(B, S, G)``.

Both matrices run in one ``dkv_cutoff_kv`` call (two kernels on the current stream). The
weights are copied once, transposed (input dimension contiguous), when the head is built;
``refresh()`` re-reads them after an in-place update.
"""

from __future__ import annotations

import torch

from .. import _lib

_WS_CACHE: dict = {}  # (device, stream) -> uint8 workspace


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Scratch of the two-step cutoff (cached per device and stream, grown at least twofold; a
    replaced buffer stays allocated, ``_lib.retire``)."""
    key = (device.index, stream)
    t = _WS_CACHE.get(key)
    if t is None or t.numel() < nbytes:
        old = t
        grow = 2 * old.numel() if old is not None else 0
        t = torch.empty(max(int(nbytes), grow, 1 << 16), dtype=torch.uint8, device=device)
        _lib.retire(old)
        _WS_CACHE[key] = t
    return t


def _rows(x: torch.Tensor) -> torch.Tensor:
    """Rows with unit element stride, a row stride of whole 16-byte units and a 16-byte aligned
    start (the kernel's operand loads); copies otherwise."""
    if x.stride(-1) != 1 or x.stride(0) % 8 != 0 or x.data_ptr() % 16 != 0:
        x = x.clone(memory_format=torch.contiguous_format)
    return x


def _prep_weight(W: torch.Tensor, groups: int) -> torch.Tensor:
    """(G, D, D) transposed copy: wt[g][n][k] = W_g[k][n]."""
    if W.dim() == 2:
        if groups != 1:
            raise ValueError("2-D weights are the joint head; pass (G, D, D) for groups > 1")
        W = W.unsqueeze(0)
    if W.dim() != 3 or W.shape[0] != groups or W.shape[1] != W.shape[2]:
        raise ValueError(f"weight must be (G, D, D) with G={groups}, got {tuple(W.shape)}")
    return W.transpose(1, 2).contiguous()


def _prep_bias(b: torch.Tensor, groups: int, D: int) -> torch.Tensor:
    b = b.reshape(groups, D)
    return b.contiguous()


class CutoffHead:
    """K and V cutoff heads of one attention layer (reference ``KVProcessor`` weights)."""

    def __init__(self, Wk: torch.Tensor, bk: torch.Tensor, Wv: torch.Tensor, bv: torch.Tensor, *,
                 groups: int = 1, low_rank: int | None = None, threshold: float = 0.1):
        self.groups = int(groups)
        self.threshold = float(threshold)
        self._src = (Wk, bk, Wv, bv)
        self.low_rank = low_rank
        self.refresh()

    def refresh(self) -> None:
        Wk, bk, Wv, bv = self._src
        G = self.groups
        self.wt_k = _prep_weight(Wk.detach(), G)
        self.wt_v = _prep_weight(Wv.detach(), G)
        self.D = self.wt_k.shape[1]
        if self.wt_v.shape != self.wt_k.shape:
            raise ValueError("K and V weights differ in shape")
        self.b_k = _prep_bias(bk.detach(), G, self.D)
        self.b_v = _prep_bias(bv.detach(), G, self.D)
        dt = self.wt_k.dtype
        if not (self.wt_v.dtype == self.b_k.dtype == self.b_v.dtype == dt):
            raise ValueError("cutoff-head weights and biases must share one dtype")

    def kv_process_fused(self, key_states: torch.Tensor, value_states: torch.Tensor):
        """Reference ``kv_process_fused``: ``(k_out, v_out, len_k, len_v, 1, 1)``."""
        k_out, len_k, v_out, len_v = cutoff_kv(
            key_states, value_states, self.wt_k, self.b_k, self.wt_v, self.b_v,
            groups=self.groups, low_rank=self.low_rank, threshold=self.threshold)
        return k_out, v_out, len_k, len_v, 1, 1


def cutoff_kv(key_states: torch.Tensor, value_states: torch.Tensor, wt_k: torch.Tensor,
              b_k: torch.Tensor, wt_v: torch.Tensor, b_v: torch.Tensor, *, groups: int = 1,
              low_rank: int | None = None, threshold: float = 0.1):
    """Cutoff of K and V with prepared (transposed) weights ``wt_*`` (G, D, D), biases (G, D).

    Returns ``(k_out, len_k, v_out, len_v)``: masked states shaped like the inputs and int32
    lengths ``(..., )`` for one group or ``(..., G)`` for several."""
    if key_states.shape != value_states.shape:
        raise ValueError("key and value states differ in shape")
    dt = key_states.dtype
    if (dt not in (torch.float16, torch.bfloat16) or value_states.dtype != dt
            or wt_k.dtype != dt or wt_v.dtype != dt):
        raise ValueError("cutoff head runs in float16 or bfloat16 (inputs and weights alike)")
    G, D = wt_k.shape[0], wt_k.shape[1]
    hidden = key_states.shape[-1]
    if hidden != G * D:
        raise ValueError(f"states have {hidden} dims, weights cover {G} x {D}")
    lead = key_states.shape[:-1]
    xk = _rows(key_states.reshape(-1, hidden))
    xv = _rows(value_states.reshape(-1, hidden))
    if xv.stride(0) != xk.stride(0):
        xk = xk.clone(memory_format=torch.contiguous_format)
        xv = xv.clone(memory_format=torch.contiguous_format)
    M = xk.shape[0]
    dev = key_states.device
    out = torch.empty((2, M, hidden), dtype=dt, device=dev)  # one allocation each for the
    lens = torch.empty((2, M, G), dtype=torch.int32, device=dev)  # outputs and the lengths
    out_k, out_v, len_k, len_v = out[0], out[1], lens[0], lens[1]
    if M > 0:
        lib = _lib.load()
        st = _lib.stream_of(key_states)
        nb = int(lib.dkv_cutoff_workspace_bytes(M, G, D))
        ws = _workspace(dev, st, nb)
        lr = -1 if low_rank is None else int(low_rank)
        rc = lib.dkv_cutoff_kv(st, _lib.dtype_code(dt), xk.data_ptr(), xv.data_ptr(), xk.stride(0),
                               wt_k.data_ptr(), wt_v.data_ptr(), b_k.data_ptr(), b_v.data_ptr(),
                               float(threshold), lr, out_k.data_ptr(), out_v.data_ptr(),
                               out_k.stride(0), len_k.data_ptr(), len_v.data_ptr(), len_k.stride(0),
                               ws.data_ptr(), ws.numel(), M, G, D)
        _lib.check(rc, "dkv_cutoff_kv")
    out_k = out_k.reshape(*lead, hidden)
    out_v = out_v.reshape(*lead, hidden)
    if G == 1:
        len_k = len_k.reshape(*lead)
        len_v = len_v.reshape(*lead)
    else:
        len_k = len_k.reshape(*lead, G)
        len_v = len_v.reshape(*lead, G)
    return out_k, len_k, out_v, len_v
