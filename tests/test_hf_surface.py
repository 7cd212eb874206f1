"""The transformers-level surface (dynakv_amd/hf.py) on the CPU: ``get_model_class`` and the
``DYNAKV_PHYSICAL_KERNELS`` switch (reference src/dynakv/__init__.py:6-17, custom_llama.py:11-16),
the ``dynakv`` import alias, the DynaKV parameter names a reference checkpoint loads into
(compressed_attention.py:24-45), and the one-time merge of ``k_down`` / ``v_down`` into the K/V
projections with the layout it selects (compressed_attention.py:263-292). No kernel runs here."""
import sys

import pytest
import torch
from transformers import LlamaConfig

from dynakv_amd import formats as F

CFG = dict(hidden_size=512, num_attention_heads=4, num_key_value_heads=2, head_dim=128,
           intermediate_size=1024, vocab_size=1000, num_hidden_layers=2, rope_theta=500000.0)


def test_get_model_class(monkeypatch):
    import dynakv_amd
    from dynakv_amd import hf

    monkeypatch.delenv(hf.PHYSICAL_ENV, raising=False)
    with pytest.raises(ValueError, match="DYNAKV_PHYSICAL_KERNELS"):
        dynakv_amd.get_model_class("llama")
    monkeypatch.setenv(hf.PHYSICAL_ENV, "1")
    for name in ("llama", "Llama3", "llama-3", "llama_3"):
        assert dynakv_amd.get_model_class(name) is hf.CustomLlamaForCausalLM
    with pytest.raises(ValueError, match="Unsupported model type"):
        dynakv_amd.get_model_class("mistral")
    with pytest.raises(ValueError, match="Qwen3"):
        dynakv_amd.get_model_class("qwen")


def test_reference_import_paths(monkeypatch):
    from dynakv_amd import hf

    saved = {k: v for k, v in sys.modules.items() if k == "dynakv" or k.startswith("dynakv.")}
    try:
        hf.install_reference_alias()
        monkeypatch.setenv(hf.PHYSICAL_ENV, "1")
        import dynakv
        from dynakv.custom_llama import CustomLlamaForCausalLM
        from dynakv.kernels.compressed_attention import CustomAttention
        from dynakv.kernels.compressed_cache import CustomDynamicCache
        from dynakv.kernels.router import KernelPolicy, compressed_decode_attention  # noqa: F401

        assert dynakv.get_model_class("llama") is CustomLlamaForCausalLM
        assert CustomAttention is hf.CustomAttention
        assert CustomDynamicCache().get_seq_length_sp(0) == 0
        assert KernelPolicy().select(499) == "short_fused"
    finally:
        for k in [k for k in sys.modules if k == "dynakv" or k.startswith("dynakv.")]:
            del sys.modules[k]
        sys.modules.update(saved)


def test_checkpoint_names_load():
    """A reference checkpoint's DynaKV tensors (model.layers.{i}.self_attn.{Wk,...}) load by name."""
    from dynakv_amd.hf import CustomAttention, CustomLlamaForCausalLM

    torch.manual_seed(0)
    model = CustomLlamaForCausalLM(LlamaConfig(**CFG))
    assert all(isinstance(layer.self_attn, CustomAttention) for layer in model.model.layers)
    D = 2 * 128
    names = dict(model.named_parameters())
    sd = {}
    for i in range(2):
        for n in F.CHECKPOINT_NAMES:
            key = f"model.layers.{i}.self_attn.{n}"
            assert key in names, key
            shape = (1, D) if n in ("bk", "bv") else (D, D)
            assert names[key].shape == shape
            sd[key] = torch.randn(shape)
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected
    assert torch.equal(model.model.layers[1].self_attn.v_up.data, sd["model.layers.1.self_attn.v_up"])


def _orth(n, g):
    q, r = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    return (q * torch.sign(torch.diagonal(r))).float()


@pytest.mark.parametrize("joint", [False, True])
def test_merge_and_layout(joint):
    """After the first forward's merge, k_proj = k_down @ k_proj (so up @ k_proj reproduces the
    original projection), k_down is the identity (a second merge changes nothing), and the
    layout follows the block structure of the bases and cutoff weights."""
    from dynakv_amd.hf import CustomAttention

    g = torch.Generator().manual_seed(7)
    cfg = LlamaConfig(**CFG)
    attn = CustomAttention(cfg, 0)
    G, Dh = 2, 128
    D = G * Dh
    if joint:
        Uk, Uv = _orth(D, g), _orth(D, g)
        Wk, Wv = torch.randn(D, D, generator=g), torch.randn(D, D, generator=g)
    else:
        Uk = torch.block_diag(*[_orth(Dh, g) for _ in range(G)])
        Uv = torch.block_diag(*[_orth(Dh, g) for _ in range(G)])
        Wk = torch.block_diag(*[torch.randn(Dh, Dh, generator=g) for _ in range(G)])
        Wv = torch.block_diag(*[torch.randn(Dh, Dh, generator=g) for _ in range(G)])
    with torch.no_grad():
        attn.k_up.copy_(Uk)
        attn.k_down.copy_(Uk.T)
        attn.v_up.copy_(Uv)
        attn.v_down.copy_(Uv.T)
        attn.Wk.copy_(Wk)
        attn.Wv.copy_(Wv)
    k0 = attn.k_proj.weight.detach().clone()
    v0 = attn.v_proj.weight.detach().clone()
    attn._merge()
    assert attn.per_head is (not joint)
    for W0, proj, U in ((k0, attn.k_proj, Uk), (v0, attn.v_proj, Uv)):
        err = (U.double() @ proj.weight.double() - W0.double()).abs().max().item()
        assert err < 1e-5, err
    assert torch.equal(attn.k_down.data, torch.eye(D)) and torch.equal(attn.v_down.data, torch.eye(D))
    if joint:
        assert attn.k_rep.shape == (4, D, Dh)
        assert torch.equal(attn.k_basis, F.kernel_basis(Uk, G, Dh))
        assert attn.cutoff.groups == 1 and attn.cutoff.D == D
    else:
        # per-head bases [h, r, d] = U[h*Dh + d, h*Dh + r]
        for h in range(G):
            blk = Uk[h * Dh:(h + 1) * Dh, h * Dh:(h + 1) * Dh]
            assert torch.equal(attn.k_basis[h], blk.T)
        assert attn.cutoff.groups == G and attn.cutoff.D == Dh
        # cutoff weights per group: the diagonal blocks, transposed for the kernel
        assert torch.equal(attn.cutoff.wt_k[1], Wk[Dh:, Dh:].T)


def test_cache_constructor_attributes():
    """CustomDynamicCache keeps the reference constructor's values under its names
    (compressed_cache.py:59-68), although transformers 5 makes max_batch_size / max_cache_len
    read-only properties of its Cache class."""
    from dynakv_amd.kernels.compressed_cache import CustomDynamicCache

    c = CustomDynamicCache(max_batch_size=4, max_cache_len=1024, dtype=torch.bfloat16)
    assert (c.max_batch_size, c.max_cache_len, c.dtype) == (4, 1024, torch.bfloat16)
    d = CustomDynamicCache()
    assert d.max_batch_size is None and d.max_cache_len is None
    assert d.key_cache_sp == [] and d.value_cache_sp == [] and d.get_seq_length_sp(0) == 0
