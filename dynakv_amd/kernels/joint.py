"""Decode attention for the reference's joint layout on MFMA (``dkv_joint_scores`` /
``dkv_joint_av``).

The reference ships its bases joint: one packed coefficient row per batch element with ranks up
to 1024 shared by every KV head, and ``k_up`` / ``v_up`` repeated to one ``(R, 128)`` basis per
query head (``compressed_attention.py:278-286``). Its router sends that layout to ``abx_sparse``
+ ``avx`` (``two_stage.py:48-324``) or to the fused kernel (``fused.py:28-170``). Those inputs do
not fit the per-head split kernel (rank above 128), so they run here: the scores kernel
reconstructs K on MFMA with the basis streamed through LDS in rank chunks and writes the route's
scores; the V kernel runs the online softmax and P.X^V on MFMA per token split, then one launch
merges the splits and projects through the V basis. Results are those of ``dkv_scores`` /
``dkv_av`` (the vector kernels) to fp32 accuracy.

A basis repeated over the query heads of a group (the reference's ``repeat_interleave``) is
detected once per tensor and reduced to its distinct bases, so each KV head's keys are
reconstructed once, not once per query head.
"""

from __future__ import annotations

import weakref

import torch

from .. import _lib
from .decode import FLAT_LD_MAX, rope_table

_BASIS_CACHE: dict = {}  # id(basis) -> (weakref to it, (ptr, shape, strides, version), factor)
_BT_CACHE: dict = {}  # id(k_up) -> (weakref to it, (ptr, shape, strides, version, heads), copy)
_WS_CACHE: dict = {}


def _workspace(device: torch.device, stream: int, floats: int) -> torch.Tensor:
    """Record workspace of the V pass (its own buffer: the split kernel's workspace keeps
    arrival counters in its first words). Grown at least twofold; a replaced buffer stays
    allocated (``_lib.retire``)."""
    key = (device.index, stream)
    t = _WS_CACHE.get(key)
    if t is None or t.numel() < floats:
        old = t
        grow = 2 * old.numel() if old is not None else 0
        t = torch.empty(max(int(floats), grow, 1 << 16), dtype=torch.float32, device=device)
        _lib.retire(old)
        _WS_CACHE[key] = t
    return t


def _sort_workspace(device: torch.device, stream: int, ints: int) -> torch.Tensor:
    """The scores call's sorted token tables (calls on one stream run in order, so they
    share one buffer). Grown at least twofold; a replaced buffer stays allocated."""
    key = ("sort", device.index, stream)
    t = _WS_CACHE.get(key)
    if t is None or t.numel() < ints:
        old = t
        grow = 2 * old.numel() if old is not None else 0
        t = torch.empty(max(int(ints), grow, 1 << 12), dtype=torch.int32, device=device)
        _lib.retire(old)
        _WS_CACHE[key] = t
    return t


def _remember(cache: dict, t: torch.Tensor, key, value) -> None:
    """Cache ``value`` for tensor object ``t``; the entry goes when ``t`` is collected. ``value``
    must not refer to ``t`` (no view of it: a view keeps its base alive through ``_base``), or
    the entry would keep ``t`` alive for good."""
    if id(t) not in cache:
        weakref.finalize(t, cache.pop, id(t), None)
    cache[id(t)] = (weakref.ref(t), key, value)


def _key(t: torch.Tensor, *extra):
    return (t.data_ptr(), tuple(t.shape), tuple(t.stride()), t._version, *extra)


def _repeat_factor(basis: torch.Tensor, n_heads: int) -> int:
    """k > 1 when every group of k consecutive entries of ``basis`` (Hb, R, Dh) repeats its first
    (k the largest of 8, 4, 2 that does so), else 1. Cached per tensor object and in-place
    version, so the comparison runs once per basis; the cache holds only the integer."""
    ent = _BASIS_CACHE.get(id(basis))
    key = _key(basis, n_heads)
    if ent is not None and ent[0]() is basis and ent[1] == key:
        return ent[2]
    Hb = basis.shape[0]
    factor = 1
    for k in (8, 4, 2):
        if Hb % k == 0 and Hb // k >= 1 and n_heads % (Hb // k) == 0 and n_heads // (Hb // k) <= 8:
            v = basis.reshape(Hb // k, k, *basis.shape[1:])
            if torch.equal(v, v[:, :1].expand_as(v)):
                factor = k
                break
    _remember(_BASIS_CACHE, basis, key, factor)
    return factor


def _distinct(basis: torch.Tensor, n_heads: int) -> torch.Tensor:
    """The distinct bases of ``basis`` (Hb, R, Dh) -- a view of its first entry of every repeated
    group -- when its entries repeat in groups (``_repeat_factor``), else ``basis`` itself."""
    k = _repeat_factor(basis, n_heads)
    if k == 1:
        return basis
    return basis.reshape(basis.shape[0] // k, k, *basis.shape[1:])[:, 0]


def _transposed(k_up: torch.Tensor, n_heads: int) -> torch.Tensor:
    """(nb, R/32, Dh, 32) contiguous copy of the distinct bases (nb, R, Dh) of ``k_up``
    (transposed in 32-rank chunks, each chunk contiguous), cached per ``k_up`` object and
    in-place version. The copy is its own storage, so the cache does not keep ``k_up`` alive."""
    ent = _BT_CACHE.get(id(k_up))
    key = _key(k_up, n_heads)
    if ent is not None and ent[0]() is k_up and ent[1] == key:
        return ent[2]
    basis = _distinct(k_up, n_heads)
    nb, R, Dh = basis.shape
    bt = basis.reshape(nb, R // 32, 32, Dh).transpose(2, 3).clone(
        memory_format=torch.contiguous_format)
    _remember(_BT_CACHE, k_up, key, bt)
    return bt


def _flat_ok(t: torch.Tensor) -> bool:
    return t.dim() == 2 and t.stride(1) == 1 and 0 < t.stride(0) <= FLAT_LD_MAX


def scores_eligible(q3: torch.Tensor, k_up: torch.Tensor, k_flat: torch.Tensor) -> bool:
    """Inputs ``dkv_joint_scores`` takes (else the vector kernel runs)."""
    dt = q3.dtype
    if dt not in (torch.bfloat16, torch.float16) or k_up.dtype != dt or k_flat.dtype != dt:
        return False
    if q3.dim() != 3 or q3.shape[2] != 128 or k_up.dim() != 3 or k_up.shape[2] != 128:
        return False
    R = k_up.shape[1]
    Hq, Hb = q3.shape[1], k_up.shape[0]
    if R % 32 or R > 1024 or Hb <= 0 or Hq % Hb or not _flat_ok(k_flat):
        return False
    return Hq // Hb <= 8 or Hq // _distinct(k_up, Hq).shape[0] <= 8


def av_eligible(v_up: torch.Tensor, v_flat: torch.Tensor, n_heads: int, S: int) -> bool:
    dt = v_up.dtype
    return (dt in (torch.bfloat16, torch.float16) and v_flat.dtype == dt and v_up.dim() == 3
            and v_up.shape[2] == 128 and v_up.shape[1] <= 1024 and v_up.shape[0] > 0
            and n_heads % v_up.shape[0] == 0 and _flat_ok(v_flat) and S > 0
            and v_up.data_ptr() % 4 == 0 and v_up.stride(0) % 2 == 0 and v_up.stride(1) % 2 == 0)


def joint_scores(q3: torch.Tensor, k_up: torch.Tensor, k_flat: torch.Tensor,
                 lens: torch.Tensor, offs: torch.Tensor, *, theta: float, mode: int,
                 out_dtype: torch.dtype) -> torch.Tensor:
    """Scores (B, Hq, S) of the route ``mode`` (0: abx_sparse, 1: fused) on MFMA."""
    B, Hq, Dh = q3.shape
    S = lens.shape[1]
    if q3.stride(2) != 1:
        q3 = q3.contiguous()
    bt = _transposed(k_up, Hq)
    k_flat = _lib.flat_operand(k_flat)
    st = _lib.stream_of(q3)
    rope, tiles = rope_table(q3.device, st, theta, S)
    out = torch.empty((B, Hq, S), dtype=out_dtype, device=q3.device)
    lib = _lib.load()
    ws = _sort_workspace(q3.device, st, int(lib.dkv_joint_scores_workspace_ints(B, S)))
    rc = lib.dkv_joint_scores(
        st, mode, _lib.dtype_code(q3.dtype), _lib.dtype_code(out_dtype),
        q3.data_ptr(), q3.stride(0), q3.stride(1),
        bt.data_ptr(), bt.stride(0), bt.stride(1), bt.shape[0],  # head and chunk strides
        k_flat.data_ptr(), k_flat.stride(0),
        lens.data_ptr(), lens.stride(0), lens.stride(1),
        offs.data_ptr(), offs.stride(0), offs.stride(1),
        rope.data_ptr(), tiles, ws.data_ptr(), ws.numel(),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        B, Hq, S, k_up.shape[1], Dh)
    _lib.check(rc, "dkv_joint_scores")
    return out


def joint_av(scores: torch.Tensor, v_up: torch.Tensor, v_flat: torch.Tensor,
             lens: torch.Tensor, offs: torch.Tensor, *, mode: int,
             out_dtype: torch.dtype) -> torch.Tensor:
    """The V pass (B, Hq, Dh) of the route ``mode`` (0: avx, 1: fused) on MFMA."""
    B, Hq, S = scores.shape
    lib = _lib.load()
    st = _lib.stream_of(scores)
    R = v_up.shape[1]
    if v_up.stride(2) != 1:
        v_up = v_up.contiguous()
    v_up = _distinct(v_up, Hq)  # the merge projects all query heads of a basis together
    v_flat = _lib.flat_operand(v_flat)
    ws = _workspace(scores.device, st, int(lib.dkv_joint_av_workspace_floats(B, Hq, S, R)))
    out = torch.empty((B, Hq, 128), dtype=out_dtype, device=scores.device)
    rc = lib.dkv_joint_av(
        st, mode, _lib.dtype_code(scores.dtype), _lib.dtype_code(v_flat.dtype),
        _lib.dtype_code(out_dtype),
        scores.data_ptr(), scores.stride(0), scores.stride(1), scores.stride(2),
        v_up.data_ptr(), v_up.stride(0), v_up.stride(1), v_up.shape[0],
        v_flat.data_ptr(), v_flat.stride(0),
        lens.data_ptr(), lens.stride(0), lens.stride(1),
        offs.data_ptr(), offs.stride(0), offs.stride(1),
        ws.data_ptr(), ws.numel(),
        out.data_ptr(), out.stride(0), out.stride(1),
        B, Hq, S, R, 128)
    _lib.check(rc, "dkv_joint_av")
    return out


def joint_attention(q3, k_flat, k_up, v_flat, v_up, l_k, o_k, l_v, o_v, *, theta: float,
                    route: int) -> torch.Tensor | None:
    """The router's attention for the joint layout, or ``None`` when an input needs the
    vector kernels. route: ``_lib.DKV_ROUTE_FUSED`` or ``_lib.DKV_ROUTE_TWO_STAGE``."""
    S = l_k.shape[1]
    if S == 0 or not scores_eligible(q3, k_up, k_flat):
        return None
    if not av_eligible(v_up, v_flat, q3.shape[1], S):
        return None
    if route == _lib.DKV_ROUTE_FUSED:
        sc = joint_scores(q3, k_up, k_flat, l_k, o_k, theta=theta, mode=1,
                          out_dtype=torch.float32)
        return joint_av(sc, v_up, v_flat, l_v, o_v, mode=1, out_dtype=q3.dtype)
    sc = joint_scores(q3, k_up, k_flat, l_k, o_k, theta=theta, mode=0, out_dtype=q3.dtype)
    return joint_av(sc, v_up, v_flat, l_v, o_v, mode=0, out_dtype=q3.dtype)


def joint_flops(lens_k: torch.Tensor, R: int, n_basis: int, B: int) -> float:
    """MFMA flops of the scores kernel as launched: 2 * 128 dims * 32 ranks per processed chunk,
    per token slot and basis head. A workgroup takes 512 tokens (256 when the basis heads pair
    up), sorts them by chunk count and runs each block of 16 sorted tokens up to its own
    longest token's chunk count."""
    S = lens_k.shape[1]
    tok = 256 if n_basis % 2 == 0 else 512
    groups = (S + tok - 1) // tok
    pad = groups * tok - S
    L = torch.nn.functional.pad(lens_k.clamp(0, R), (0, pad)).view(B, groups, tok)
    chunks = ((L + 31) // 32).sort(dim=2).values.view(B, groups, tok // 16, 16)[..., -1]
    return float(chunks.sum().item()) * 16 * 2 * 128 * 32 * n_basis


__all__ = ["joint_attention", "joint_scores", "joint_av", "scores_eligible", "av_eligible",
           "joint_flops"]
