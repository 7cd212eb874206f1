"""The reference's PCA-basis and checkpoint formats (scripts/pca_initialization.py:99-102,
custom_attn.py:33-63, modify_model.py:43-57) and the kernel layouts built from them
(compressed_attention.py:263-292)."""
import numpy as np
import pytest
import torch

from dynakv_amd import formats as F


def _orthogonal(n, seed):
    q, _ = np.linalg.qr(np.random.default_rng(seed).standard_normal((n, n)))
    return torch.from_numpy(q).float()


def test_pca_files_round_trip(tmp_path):
    D = 64
    U = _orthogonal(D, 1)
    Uv = _orthogonal(D, 2)
    # the reference's writer: (1, D, D) tensors, U and U^T
    torch.save(U.unsqueeze(0), tmp_path / "L3_k_U.pt")
    torch.save(U.T.contiguous().unsqueeze(0), tmp_path / "L3_k_Ut.pt")
    torch.save(Uv.unsqueeze(0), tmp_path / "L3_v_U.pt")
    torch.save(Uv.T.contiguous(), tmp_path / "L3_v_Ut.pt")  # 2-D is accepted too
    got = F.load_pca_layer(str(tmp_path), 3, dtype=torch.bfloat16)
    assert got["k_up"].shape == (D, D) and got["k_up"].dtype == torch.bfloat16
    assert torch.equal(got["k_up"], U.to(torch.bfloat16))
    assert torch.equal(got["k_down"], U.T.to(torch.bfloat16))
    assert torch.equal(got["v_down"], Uv.T.to(torch.bfloat16))
    with pytest.raises(FileNotFoundError):
        F.load_pca_layer(str(tmp_path), 4)


def test_basis_file_rejects_non_square(tmp_path):
    torch.save(torch.zeros(1, 4, 5), tmp_path / "bad.pt")
    with pytest.raises(ValueError):
        F.load_basis_file(str(tmp_path / "bad.pt"))


@pytest.mark.parametrize("rank", [None, 96])
def test_kernel_basis_reconstructs_k(rank):
    """K = up[:, :R] @ c (the reference's einsum over the coefficients) equals, per KV head h,
    sum_r c_r B[h, r, :] with B the kernel layout."""
    Hkv, Dh = 4, 32
    D = Hkv * Dh
    up = _orthogonal(D, 5)
    B = F.kernel_basis(up, Hkv, Dh, rank)
    R = D if rank is None else rank
    assert B.shape == (Hkv, R, Dh)
    c = torch.randn(7, R)
    k_ref = (c @ up[:, :R].T).reshape(7, Hkv, Dh)
    k_got = torch.einsum("tr,hrd->thd", c, B)
    assert torch.allclose(k_got, k_ref, atol=1e-5)
    Bq = F.repeat_for_query_heads(B, 4 * Hkv)
    assert Bq.shape == (4 * Hkv, R, Dh)
    assert all(torch.equal(Bq[h], B[h // 4]) for h in range(4 * Hkv))


def test_per_head_bases_round_trip_and_rejection():
    Hkv, Dh = 8, 16
    bases = torch.stack([_orthogonal(Dh, 10 + h).T for h in range(Hkv)])  # (H, R, Dh)
    up = F.block_diagonal(bases)
    assert up.shape == (Hkv * Dh, Hkv * Dh)
    back = F.per_head_bases(up, Hkv, Dh)
    assert torch.equal(back, bases)
    # agrees with the joint kernel layout on the diagonal blocks
    B = F.kernel_basis(up, Hkv, Dh)
    for h in range(Hkv):
        assert torch.equal(B[h, h * Dh:(h + 1) * Dh], bases[h])
    up2 = up.clone()
    up2[0, Dh] = 0.5
    with pytest.raises(ValueError):
        F.per_head_bases(up2, Hkv, Dh)


def test_merge_projection_emits_coefficients():
    D, Din = 32, 48
    W = torch.randn(D, Din)
    bias = torch.randn(D)
    down = _orthogonal(D, 7).T
    w2, b2 = F.merge_projection(W, down, bias)
    x = torch.randn(5, Din)
    c = x @ w2.T + b2
    assert torch.allclose(c, (x @ W.T + bias) @ down.T, atol=1e-5)


def test_checkpoint_layer_from_safetensors(tmp_path):
    from safetensors.torch import save_file

    D = 32
    tensors = {}
    for i in range(2):
        for n in F.CHECKPOINT_NAMES:
            shape = (1, D) if n in ("bk", "bv") else (D, D)
            tensors[f"model.layers.{i}.self_attn.{n}"] = torch.full(shape, float(i * 10 + len(n)))
    tensors["model.layers.0.self_attn.q_proj.weight"] = torch.zeros(4, 4)
    save_file(tensors, str(tmp_path / "model.safetensors"))
    p = F.load_checkpoint_layer([str(tmp_path / "model.safetensors")], 1)
    assert p.Wk.shape == (D, D) and p.bk.shape == (1, D)
    assert float(p.k_up[0, 0]) == 10 + len("k_up")
    with pytest.raises(KeyError):
        F.load_checkpoint_layer([str(tmp_path / "model.safetensors")], 2)
