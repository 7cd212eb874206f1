"""The reference's basis and checkpoint formats, converted to this build's kernel layouts.

Formats (written by the reference's scripts; read here without executing anything from the
files: ``torch.load(weights_only=True)`` and safetensors):

* PCA bases (``scripts/pca_initialization.py:99-102``): ``L{layer}_{k|v}_U.pt`` holds
  ``U`` as a ``(1, D, D)`` float32 tensor whose columns are the covariance eigenvectors in
  descending eigenvalue order; ``L{layer}_{k|v}_Ut.pt`` holds ``U^T`` the same way. The
  attention module loads them as ``k_up = U`` and ``k_down = U^T`` (``custom_attn.py:41-63``,
  ``compressed_attention.py:36-46``: a 3-D tensor is indexed ``[0]``).
* Checkpoint parameters of each converted attention block (``custom_attn.py:33-63``,
  ``scripts/modify_model.py:43-57``): ``Wk, bk, Wv, bv`` (the cutoff heads, ``(D, D)`` and
  ``(1, D)``) and ``k_down, k_up, v_down, v_up`` (``(D, D)``), under
  ``model.layers.{i}.self_attn.<name>`` in the safetensors files.

Layouts (the one-time merge of ``compressed_attention.py:263-292``):

* the coefficient projection: ``k_proj.weight <- k_down @ k_proj.weight`` (and the bias), so
  the projection emits spectral coefficients;
* the reference's kernel basis ``B = k_up[:, :R].view(Hkv, Dh, R).transpose(1, 2)`` -- one
  ``(R, Dh)`` basis per KV head, i.e. ``B[h, r, d] = k_up[h*Dh + d, r]`` -- repeated over the
  ``Hq/Hkv`` query heads of the group for the reference kernels; this build's grouped kernels
  take the unrepeated ``(Hkv, R, Dh)`` tensor;
* the per-head layout (one cache row per (batch, KV head), rank 128 per head) needs ``k_up``
  block-diagonal in ``Dh x Dh`` blocks: ``per_head_bases`` extracts the blocks
  ``(Hkv, Dh, Dh)`` and rejects a ``U`` with mass off the diagonal blocks.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch


def load_basis_file(path: str, dtype: torch.dtype | None = None) -> torch.Tensor:
    """One PCA basis file as ``(D, D)`` (a leading unit dimension is dropped, as the
    reference's loader does)."""
    value = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(value, torch.Tensor):
        raise ValueError(f"{path}: expected a tensor, found {type(value).__name__}")
    if value.ndim == 3:
        value = value[0]
    if value.ndim != 2 or value.shape[0] != value.shape[1]:
        raise ValueError(f"{path}: expected (D, D) or (1, D, D), found {tuple(value.shape)}")
    return value.to(dtype) if dtype is not None else value


def load_pca_layer(pca_dir: str, layer: int, dtype: torch.dtype | None = None) -> dict:
    """``{"k_up", "k_down", "v_up", "v_down"}`` of one layer from a PCA directory."""
    out = {}
    for kind in ("k", "v"):
        for direction, name in (("U", "up"), ("Ut", "down")):
            path = os.path.join(pca_dir, f"L{layer}_{kind}_{direction}.pt")
            if not os.path.isfile(path):
                raise FileNotFoundError(path)
            out[f"{kind}_{name}"] = load_basis_file(path, dtype)
    return out


def kernel_basis(up: torch.Tensor, n_kv_heads: int, head_dim: int,
                 rank: int | None = None) -> torch.Tensor:
    """The reference's ``B`` before the repeat over query heads: ``(Hkv, R, Dh)`` with
    ``B[h, r, d] = up[h*Dh + d, r]`` (``compressed_attention.py:279-283``)."""
    D = up.shape[0]
    if D != n_kv_heads * head_dim:
        raise ValueError(f"basis has {D} rows, expected {n_kv_heads} x {head_dim}")
    R = D if rank is None else int(rank)
    return up[:, :R].reshape(n_kv_heads, head_dim, R).transpose(1, 2).contiguous()


def repeat_for_query_heads(basis: torch.Tensor, n_heads: int) -> torch.Tensor:
    """``(Hq, R, Dh)``: each KV head's basis repeated for its query heads (the reference's
    ``repeat_interleave``, ``compressed_attention.py:283,286``)."""
    return basis.repeat_interleave(n_heads // basis.shape[0], dim=0).contiguous()


def per_head_bases(up: torch.Tensor, n_kv_heads: int, head_dim: int,
                   atol: float = 0.0) -> torch.Tensor:
    """``(Hkv, Dh, Dh)`` per-head bases (rank-major, ``[h, r, d] = up[h*Dh + d, h*Dh + r]``)
    from a block-diagonal ``up``; raises if any entry off the diagonal blocks exceeds
    ``atol``."""
    D = up.shape[0]
    if D != n_kv_heads * head_dim:
        raise ValueError(f"basis has {D} rows, expected {n_kv_heads} x {head_dim}")
    blocks = up.reshape(n_kv_heads, head_dim, n_kv_heads, head_dim)
    idx = torch.arange(n_kv_heads)
    diag = blocks[idx, :, idx, :]  # (Hkv, Dh [d], Dh [r])
    off = blocks.clone()
    off[idx, :, idx, :] = 0
    if off.abs().max() > atol:
        raise ValueError("basis is not block-diagonal per KV head: use the joint layout")
    return diag.transpose(1, 2).contiguous()


def block_diagonal(bases: torch.Tensor) -> torch.Tensor:
    """Inverse of ``per_head_bases``: the joint ``(D, D)`` basis of per-head ``(Hkv, R, Dh)``."""
    H, R, Dh = bases.shape
    up = torch.zeros(H * Dh, H * R, dtype=bases.dtype)
    for h in range(H):
        up[h * Dh:(h + 1) * Dh, h * R:(h + 1) * R] = bases[h].t()
    return up


def merge_projection(weight: torch.Tensor, down: torch.Tensor,
                     bias: torch.Tensor | None = None):
    """``down @ weight`` (and ``down @ bias``): the projection then emits coefficients
    (``compressed_attention.py:267-274``)."""
    w = torch.matmul(down.to(weight.dtype), weight)
    b = None if bias is None else torch.matmul(down.to(bias.dtype), bias)
    return w, b


CHECKPOINT_NAMES = ("Wk", "bk", "Wv", "bv", "k_down", "k_up", "v_down", "v_up")


@dataclass
class LayerParams:
    """The DynaKV parameters of one attention block."""

    Wk: torch.Tensor
    bk: torch.Tensor
    Wv: torch.Tensor
    bv: torch.Tensor
    k_down: torch.Tensor
    k_up: torch.Tensor
    v_down: torch.Tensor
    v_up: torch.Tensor


def load_checkpoint_layer(files: list[str], layer: int,
                          prefix: str = "model.layers.{i}.self_attn.") -> LayerParams:
    """One block's parameters from safetensors shards (reference names)."""
    from safetensors import safe_open

    want = {prefix.format(i=layer) + n: n for n in CHECKPOINT_NAMES}
    got = {}
    for f in files:
        with safe_open(f, framework="pt") as sf:
            for key in sf.keys():
                if key in want:
                    got[want[key]] = sf.get_tensor(key)
    missing = [n for n in CHECKPOINT_NAMES if n not in got]
    if missing:
        raise KeyError(f"layer {layer}: missing {missing}")
    return LayerParams(**got)
