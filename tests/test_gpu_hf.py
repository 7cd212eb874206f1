"""The transformers model classes (dynakv_amd/hf.py) on the GPU against a float32 forward.

A tiny HF-shaped Llama (hidden 512, 2 layers, 4 query / 2 KV heads of 128, FFN 1024, vocab
1000) gets the weights of a ``RandomLlama``: the same q/o/MLP/norm weights, the K/V projections
already merged with the per-head bases (so ``k_down`` / ``v_down`` are the identity, whose merge
is exact), ``k_up`` / ``v_up`` the block-diagonal joint form of the per-head bases and ``Wk`` /
``Wv`` the block-diagonal cutoff weights -- the checkpoint layout a per-head DynaKV model ships in
(reference compressed_attention.py:24-45, custom_llama.py:250-323). ``CustomAttention`` detects
the per-head layout from the block structure (coefficient prefill attention, packed appends,
one-call decode layers and the split-K decode attention). Its logits at every prompt position
and over 12 greedy decode steps are compared with a float32 forward of the same weights that
keeps the retained lengths the model's cutoff heads produced (read back from its cache) and the
reference's rotations: q by the decoder's position embeddings (cos / sin rounded to bf16, as
``LlamaRotaryEmbedding`` returns them in the model dtype), the prefill keys by the layer's rotary
embedding at 0..L-1 likewise (calc_cos_sin, compressed_attention.py:193-200,375-378), the keys of
the decode attention by plain theta at their row index in fp32 (the decode kernels,
two_stage.py:28-46). ``generate`` is checked against the greedy tokens of the same model's
step-by-step forward.
"""
import pytest
import torch

from dynakv_amd import formats as F
from dynakv_amd.model import LlamaShape, RandomLlama

SHAPE = LlamaShape(hidden=512, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=1024, vocab=1000)


def _hf_model(model, dev, monkeypatch):
    from transformers import LlamaConfig

    from dynakv_amd import hf

    monkeypatch.setenv(hf.PHYSICAL_ENV, "1")
    s = model.shape
    cfg = LlamaConfig(hidden_size=s.hidden, num_attention_heads=s.heads,
                      num_key_value_heads=s.kv_heads, head_dim=s.head_dim,
                      intermediate_size=s.ffn, vocab_size=s.vocab, num_hidden_layers=s.layers,
                      rope_theta=s.theta, rms_norm_eps=s.eps, tie_word_embeddings=False)
    cls = hf.get_model_class("llama")
    # built with bf16 as the default dtype, as from_pretrained(dtype=bf16) builds a model (the
    # rotary inv_freq buffers stay float32; .to(bf16) would round them)
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        m = cls(cfg).to(device=dev).eval()
    finally:
        torch.set_default_dtype(old)
    assert m.model.rotary_emb.inv_freq.dtype == torch.float32
    D = s.kv_heads * s.head_dim
    eye = torch.eye(D, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        m.model.embed_tokens.weight.copy_(model.embed)
        m.lm_head.weight.copy_(model.lm_head)
        m.model.norm.weight.copy_(model.norm)
        for lw, layer in zip(model.layers, m.model.layers):
            a = layer.self_attn
            layer.input_layernorm.weight.copy_(lw.ln1)
            layer.post_attention_layernorm.weight.copy_(lw.ln2)
            a.q_proj.weight.copy_(lw.wq)
            a.k_proj.weight.copy_(lw.wk_c)
            a.v_proj.weight.copy_(lw.wv_c)
            a.o_proj.weight.copy_(lw.wo)
            a.k_down.copy_(eye)
            a.v_down.copy_(eye)
            a.k_up.copy_(F.block_diagonal(lw.k_basis.cpu()).to(dev))
            a.v_up.copy_(F.block_diagonal(lw.v_basis.cpu()).to(dev))
            cw_k, cb_k, cw_v, cb_v = lw.cutoff._src
            a.Wk.copy_(torch.block_diag(*cw_k))
            a.bk.copy_(cb_k.reshape(1, D))
            a.Wv.copy_(torch.block_diag(*cw_v))
            a.bv.copy_(cb_v.reshape(1, D))
            layer.mlp.gate_proj.weight.copy_(lw.w_gate)
            layer.mlp.up_proj.weight.copy_(lw.w_up)
            layer.mlp.down_proj.weight.copy_(lw.w_down)
    return m


def _close(got, ref, what, rel=0.03):
    err = (got.float() - ref.float()).abs().max().item()
    scale = ref.float().abs().max().item()
    print(f"[parity] {what}: max_abs={err:.3e} |ref|max={scale:.3e}", flush=True)
    assert err <= rel * scale, what


def _reference_logits(model, tokens, lens_k, lens_v, S0, dev):
    """float32 forward over all positions with the reference's rotations (see the module
    docstring); lens_*: per layer (B*G, L) retained dims; positions >= S0 are decode steps."""
    import math

    import numpy as np
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    from oracle.attention import rope_cos_sin

    s = model.shape
    f = lambda t: t.detach().to(dev).float()  # noqa: E731
    tokens = tokens.to(dev)
    B, L = tokens.shape
    G, Dh, hpg = s.kv_heads, s.head_dim, s.heads // s.kv_heads
    cfg = LlamaConfig(hidden_size=s.hidden, num_attention_heads=s.heads,
                      num_key_value_heads=s.kv_heads, head_dim=Dh, rope_theta=s.theta)
    x = f(model.embed)[tokens]
    cos_h, sin_h = LlamaRotaryEmbedding(cfg).to(dev)(x.to(torch.bfloat16),
                                                     torch.arange(L, device=dev)[None])
    cos_h, sin_h = cos_h.float()[0], sin_h.float()[0]  # (L, 128), bf16 values
    c, sn = rope_cos_sin(np.arange(L), Dh, s.theta)
    cos_k = torch.from_numpy(np.concatenate([c, c], -1)).float().to(dev)
    sin_k = torch.from_numpy(np.concatenate([sn, sn], -1)).float().to(dev)

    def rope(t, cos, sin):
        return t * cos + torch.cat([-t[..., 64:], t[..., :64]], -1) * sin

    def rms(t, w):
        return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + s.eps) * w

    ar = torch.arange(Dh, device=dev)
    causal = torch.ones(L, L, dtype=torch.bool, device=dev).triu(1)
    decode_row = (torch.arange(L, device=dev) >= S0)[:, None]
    for i, lw in enumerate(model.layers):
        h = rms(x, f(lw.ln1))
        q = (h @ f(lw.wq).T).view(B, L, s.heads, Dh).transpose(1, 2)
        kc = (h @ f(lw.wk_c).T).view(B, L, G, Dh).transpose(1, 2)
        vc = (h @ f(lw.wv_c).T).view(B, L, G, Dh).transpose(1, 2)
        kc = kc * (ar < lens_k[i].to(dev).view(B, G, L, 1)).float()
        vc = vc * (ar < lens_v[i].to(dev).view(B, G, L, 1)).float()
        k = torch.einsum("bgsr,grd->bgsd", kc, f(lw.k_basis)).repeat_interleave(hpg, dim=1)
        v = torch.einsum("bgsr,grd->bgsd", vc, f(lw.v_basis)).repeat_interleave(hpg, dim=1)
        q = rope(q, cos_h, sin_h)
        sc_pf = q @ rope(k, cos_h, sin_h).transpose(-1, -2)
        sc_dec = q @ rope(k, cos_k, sin_k).transpose(-1, -2)
        sc = torch.where(decode_row, sc_dec, sc_pf) / math.sqrt(Dh)
        a = torch.softmax(sc.masked_fill(causal, float("-inf")), -1) @ v
        x = x + a.transpose(1, 2).reshape(B, L, s.hidden) @ f(lw.wo).T
        h2 = rms(x, f(lw.ln2))
        x = x + (torch.nn.functional.silu(h2 @ f(lw.w_gate).T) * (h2 @ f(lw.w_up).T)) @ f(
            lw.w_down).T
    return rms(x, f(model.norm)) @ f(model.lm_head).T


@pytest.mark.gpu
@pytest.mark.parametrize("S", [40, 494])
def test_hf_model_matches_float32_forward(dev, monkeypatch, S):
    """Prefill logits at every position and 12 greedy decode steps against the float32 forward
    (S=494: the decode steps cross the 500-token switch from the short route to the long one)."""
    print(f"[gpu] hf model S={S}", flush=True)
    from dynakv_amd.hf import CustomAttention
    from dynakv_amd.kernels.compressed_cache import CustomDynamicCache

    model = RandomLlama(SHAPE, device=dev, seed=11, std=0.05)
    hfm = _hf_model(model, dev, monkeypatch)
    B, steps = 2, 12
    g = torch.Generator(device=dev).manual_seed(S)
    prompt = torch.randint(0, SHAPE.vocab, (B, S), generator=g, device=dev)
    with torch.no_grad():
        cache = CustomDynamicCache()
        out = hfm(input_ids=prompt, past_key_values=cache, use_cache=True)
        assert all(isinstance(layer.self_attn, CustomAttention) and layer.self_attn.per_head
                   for layer in hfm.model.layers)
        got = [out.logits.float()]
        toks = [got[0][:, -1:].argmax(-1)]
        for t in range(steps):
            got.append(hfm(input_ids=toks[-1], past_key_values=cache, use_cache=True).logits.float())
            toks.append(got[-1].argmax(-1))
        L = S + steps
        assert cache.get_seq_length() == L
        lk = [c[1][:, :L] for c in cache.key_cache_sp]
        lv = [c[1][:, :L] for c in cache.value_cache_sp]
        frac = torch.stack(lk).float().mean().item() / SHAPE.head_dim
        print(f"[gpu] hf model: mean retained fraction {frac:.3f}", flush=True)
        tokens = torch.cat([prompt] + toks[:-1], dim=1)
        ref = _reference_logits(model, tokens, lk, lv, S, dev)
    got = torch.cat(got, dim=1)  # (B, L, V): the prompt positions, then the decoded ones
    _close(got[:, :S], ref[:, :S], f"prefill logits S={S}", rel=0.05)
    for t in range(steps):
        _close(got[:, S + t], ref[:, S + t], f"decode step {t + 1} S={S}", rel=0.05)


@pytest.mark.gpu
def test_hf_generate_uses_compressed_cache(dev, monkeypatch):
    """transformers' greedy ``generate`` over the compressed cache gives the tokens of the same
    model's own step-by-step greedy forward."""
    print("[gpu] hf generate", flush=True)
    from dynakv_amd.kernels.compressed_cache import CustomDynamicCache

    model = RandomLlama(SHAPE, device=dev, seed=12, std=0.05)
    hfm = _hf_model(model, dev, monkeypatch)
    B, S, new = 2, 24, 8
    g = torch.Generator(device=dev).manual_seed(5)
    prompt = torch.randint(0, SHAPE.vocab, (B, S), generator=g, device=dev)
    with torch.no_grad():
        out = hfm.generate(prompt, max_new_tokens=new, do_sample=False, pad_token_id=0)
        assert out.shape == (B, S + new)
        assert torch.equal(out[:, :S], prompt)
        cache = CustomDynamicCache()
        logits = hfm(input_ids=prompt, past_key_values=cache, use_cache=True).logits
        toks = [logits[:, -1:].argmax(-1)]
        for _ in range(new - 1):
            logits = hfm(input_ids=toks[-1], past_key_values=cache, use_cache=True).logits
            toks.append(logits.argmax(-1))
    want = torch.cat(toks, dim=1)
    print(f"[parity] generate {out[:, S:].tolist()} vs {want.tolist()}", flush=True)
    assert torch.equal(out[:, S:], want)
