"""The reference's file formats driving the kernels on the GPU.

Synthetic PCA basis files (``L{i}_{k,v}_{U,Ut}.pt``, scripts/pca_initialization.py:99-102) and
checkpoint tensors (``Wk, bk, Wv, bv, k_down, k_up, v_down, v_up`` in safetensors,
custom_attn.py:33-63, modify_model.py:43-57) are written to disk, loaded with
``dynakv_amd.formats``, merged into the K/V projections (``merge_projection``,
compressed_attention.py:263-292) and turned into kernel bases (``kernel_basis`` for the
reference's joint layout, ``per_head_bases`` for the per-head one). Hidden states then go through
the merged projection, the cutoff head, the packed cache and decode attention on the device, and
the output is compared with the oracle evaluated on the same packed tables.

Two identities pin the format handling independently of the oracle: the merged projection
reconstructs the original K/V projection through the loaded basis (``up @ (down @ W) = W`` for
an orthogonal basis -- a transposed or mis-indexed basis fails it), and the kernel basis of a
block-diagonal ``U`` equals its per-head blocks.
"""
import numpy as np
import pytest
import torch

from dynakv_amd import formats as F
from dynakv_amd.kernels.compressed_cache import CustomDynamicCache
from dynakv_amd.kernels.cutoff import CutoffHead
from dynakv_amd.kernels.decode import grouped_decode_attention
from dynakv_amd.kernels.router import KernelPolicy, compressed_decode_attention
from oracle import attention as A

from helpers import assert_close

HKV, DH, HQ = 8, 128, 32
D = HKV * DH


def _orth(n, g):
    q, r = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    return (q * torch.sign(torch.diagonal(r))).float()


def _write(tmp_path, layer, joint: bool, g):
    """PCA files and one safetensors shard of layer ``layer``; returns what was written."""
    from safetensors.torch import save_file

    def basis():
        if joint:
            return _orth(D, g)
        return torch.block_diag(*[_orth(DH, g) for _ in range(HKV)])

    Uk, Uv = basis(), basis()
    for kind, U in (("k", Uk), ("v", Uv)):
        torch.save(U.unsqueeze(0), tmp_path / f"L{layer}_{kind}_U.pt")
        torch.save(U.T.contiguous().unsqueeze(0), tmp_path / f"L{layer}_{kind}_Ut.pt")
    # cutoff heads: small weights, bias ramping over the rank (a prefix of ~half is kept);
    # per-head checkpoints carry the weights block-diagonal
    def cut_w():
        if joint:
            return torch.randn(D, D, generator=g) * (0.5 / D ** 0.5)
        return torch.block_diag(*[torch.randn(DH, DH, generator=g) * (0.5 / DH ** 0.5)
                                  for _ in range(HKV)])

    ramp = torch.arange(D if joint else DH, dtype=torch.float32) * (6.0 / (D if joint else DH))
    bias = (ramp if joint else ramp.repeat(HKV)).view(1, D)
    tensors = {"Wk": cut_w(), "bk": bias.clone(), "Wv": cut_w(), "bv": bias.clone(),
               "k_down": Uk.T.contiguous(), "k_up": Uk, "v_down": Uv.T.contiguous(), "v_up": Uv}
    save_file({f"model.layers.{layer}.self_attn.{n}": t.contiguous() for n, t in tensors.items()},
              str(tmp_path / "model-00001-of-00001.safetensors"))
    return Uk, Uv


def _load(tmp_path, layer, dtype):
    pca = F.load_pca_layer(str(tmp_path), layer, dtype=torch.float32)
    ck = F.load_checkpoint_layer([str(tmp_path / "model-00001-of-00001.safetensors")], layer)
    assert torch.equal(ck.k_up, pca["k_up"]) and torch.equal(ck.v_down, pca["v_down"])
    return pca, ck


def _project(dev, dtype, pca, hidden, S, B, g):
    """K/V projections of a random model, merged with the loaded k_down / v_down; returns the
    coefficient rows (B, S, D) of random hidden states and checks the merge identity."""
    Wk = torch.randn(D, hidden, generator=g) * 0.05
    Wv = torch.randn(D, hidden, generator=g) * 0.05
    Wk_c, _ = F.merge_projection(Wk, pca["k_down"])
    Wv_c, _ = F.merge_projection(Wv, pca["v_down"])
    # up @ (down @ W) == W: the loaded basis reconstructs the original projection
    for W, Wc, up in ((Wk, Wk_c, pca["k_up"]), (Wv, Wv_c, pca["v_up"])):
        err = (up.double() @ Wc.double() - W.double()).abs().max().item()
        assert err < 1e-5, err
    h = (torch.randn(B, S, hidden, generator=g)).to(dev, dtype)
    kc = h @ Wk_c.to(dev, dtype).T
    vc = h @ Wv_c.to(dev, dtype).T
    return kc, vc


def _oracle_inputs(cache, layer, S):
    fk, lk, ok = (cache.key_cache_sp[layer][i] for i in range(3))
    fv, lv, ov = (cache.value_cache_sp[layer][i] for i in range(3))
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    i = lambda t: t[:, :S].cpu().numpy()  # noqa: E731
    return f(fk), i(lk), i(ok), f(fv), i(lv), i(ov)


@pytest.mark.gpu
@pytest.mark.parametrize("S0", [300, 700])
def test_joint_layout_from_reference_files(dev, tmp_path, S0):
    """The reference's shipped layout: a 1024x1024 basis and cutoff head per layer, coefficients
    of rank up to 1024 in one packed row per batch element, k_up repeated to (32, 1024, 128)."""
    print(f"[gpu] formats joint S0={S0}", flush=True)
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(S0)
    _write(tmp_path, 2, True, g)
    pca, ck = _load(tmp_path, 2, dtype)
    B = 2
    kc, vc = _project(dev, dtype, pca, 256, S0 + 1, B, g)
    head = CutoffHead(ck.Wk.to(dev, dtype), ck.bk.to(dev, dtype), ck.Wv.to(dev, dtype),
                      ck.bv.to(dev, dtype), groups=1, low_rank=D)
    k_out, v_out, len_k, len_v, _, _ = head.kv_process_fused(kc, vc)
    frac = len_k.float().mean().item() / D
    assert 0.05 < frac < 0.95, frac
    cache = CustomDynamicCache()
    cache.update_sp(k_out[:, :S0].contiguous(), len_k[:, :S0].contiguous(),
                    v_out[:, :S0].contiguous(), len_v[:, :S0].contiguous(), D, 0, D)
    fk, fv, lk, lv, ok, ov = cache.update_sp(
        k_out[:, S0:].contiguous(), len_k[:, S0:].contiguous(), v_out[:, S0:].contiguous(),
        len_v[:, S0:].contiguous(), D, 0, D)
    L = cache.get_seq_length_sp(0)
    kb = F.kernel_basis(pca["k_up"], HKV, DH)
    vb = F.kernel_basis(pca["v_up"], HKV, DH)
    k_up = F.repeat_for_query_heads(kb, HQ).to(dev, dtype)
    v_up = F.repeat_for_query_heads(vb, HQ).to(dev, dtype)
    q = (torch.randn(B, HQ, 1, DH, generator=g)).to(dev, dtype)
    got = compressed_decode_attention(q=q, k_flat=fk, k_up=k_up, v_flat=fv, v_up=v_up,
                                      key_lengths=lk, key_offsets=ok, value_lengths=lv,
                                      value_offsets=ov, theta=500000.0, cache_length=L)
    route = KernelPolicy().select(L)
    hk, hlk, hok, hv, hlv, hov = _oracle_inputs(cache, 0, L)
    ref = A.decode_attention(q[:, :, 0].float().cpu().numpy(), hk,
                             k_up.float().cpu().numpy(), hv, v_up.float().cpu().numpy(),
                             hlk, hok, hlv, hov, 500000.0, route=route, q_dtype="bfloat16")
    assert_close(got, ref, f"joint from files S={L} {route}")


@pytest.mark.gpu
@pytest.mark.parametrize("S0", [300, 700])
def test_per_head_layout_from_reference_files(dev, tmp_path, S0):
    """Block-diagonal bases and cutoff weights from the same file formats, converted to the
    per-head layout (rank 128 per KV head, one packed row per (batch, KV head)) and attended by
    the split kernel (grouped_decode_attention)."""
    print(f"[gpu] formats per-head S0={S0}", flush=True)
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(1000 + S0)
    _write(tmp_path, 5, False, g)
    pca, ck = _load(tmp_path, 5, dtype)
    kb = F.per_head_bases(pca["k_up"], HKV, DH)
    vb = F.per_head_bases(pca["v_up"], HKV, DH)
    # the per-head bases are the diagonal blocks of the joint kernel basis
    assert torch.equal(kb, torch.stack([F.kernel_basis(pca["k_up"], HKV, DH)[h, h * DH:(h + 1) * DH]
                                        for h in range(HKV)]))
    B = 2
    kc, vc = _project(dev, dtype, pca, 256, S0 + 1, B, g)
    blocks = lambda W: torch.stack([W[h * DH:(h + 1) * DH, h * DH:(h + 1) * DH]  # noqa: E731
                                    for h in range(HKV)])
    head = CutoffHead(blocks(ck.Wk).to(dev, dtype), ck.bk.to(dev, dtype),
                      blocks(ck.Wv).to(dev, dtype), ck.bv.to(dev, dtype), groups=HKV)
    k_out, v_out, len_k, len_v, _, _ = head.kv_process_fused(kc, vc)  # lens (B, S, G)
    rows = lambda x: x.view(B, S0 + 1, HKV, DH).transpose(1, 2).reshape(B * HKV, S0 + 1, DH)  # noqa: E731
    lrows = lambda l: l.view(B, S0 + 1, HKV).transpose(1, 2).reshape(B * HKV, S0 + 1)  # noqa: E731
    rk, rv, lk_all, lv_all = rows(k_out), rows(v_out), lrows(len_k), lrows(len_v)
    cache = CustomDynamicCache()
    cache.update_sp(rk[:, :S0].contiguous(), lk_all[:, :S0].contiguous(),
                    rv[:, :S0].contiguous(), lv_all[:, :S0].contiguous(), DH, 0, DH)
    fk, fv, lk, lv, ok, ov = cache.update_sp(
        rk[:, S0:].contiguous(), lk_all[:, S0:].contiguous(), rv[:, S0:].contiguous(),
        lv_all[:, S0:].contiguous(), DH, 0, DH)
    L = cache.get_seq_length_sp(0)
    route = KernelPolicy().select(L)
    q = (torch.randn(B, HQ, DH, generator=g)).to(dev, dtype)
    kbd, vbd = kb.to(dev, dtype), vb.to(dev, dtype)
    got = grouped_decode_attention(q, fk, fv, lk, ok, lv, ov, kbd, vbd, theta=500000.0,
                                   route=route, out_dtype=torch.float32)
    hk, hlk, hok, hv, hlv, hov = _oracle_inputs(cache, 0, L)
    hpg = HQ // HKV
    ref = A.decode_attention(q.float().cpu().numpy(), hk, kbd.float().cpu().numpy(), hv,
                             vbd.float().cpu().numpy(), hlk, hok, hlv, hov, 500000.0,
                             route=route, q_dtype="bfloat16",
                             row_of=lambda b, h: b * HKV + h // hpg, basis_of=lambda h: h // hpg)
    assert_close(got, ref, f"per-head from files S={L} {route}")
