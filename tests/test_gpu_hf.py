"""The transformers model classes (dynakv_amd/hf.py) on the GPU against ``CompressedLlama``.

A tiny HF-shaped Llama (hidden 512, 2 layers, 4 query / 2 KV heads of 128, FFN 1024, vocab
1000) gets the weights of a ``RandomLlama``: the same q/o/MLP/norm weights, the K/V projections
already merged with the per-head bases (so ``k_down`` / ``v_down`` are the identity, whose merge
is exact), ``k_up`` / ``v_up`` the block-diagonal joint form of the per-head bases and ``Wk`` /
``Wv`` the block-diagonal cutoff weights -- the checkpoint layout a per-head DynaKV model ships in
(reference compressed_attention.py:24-45, custom_llama.py:250-323). ``CustomAttention`` detects
the per-head layout from the block structure, so prefill and decode run the same kernels as
``CompressedLlama`` (coefficient prefill attention, packed appends, one-call decode layers and
the split-K decode attention). The logits are compared position by position (teacher forcing on
the same tokens); the remaining differences come from HF's own RMSNorm / linear / residual
rounding, so the bound is relative to the logit scale. ``generate`` is checked against the
greedy tokens of the same model's teacher-forced forward.
"""
import pytest
import torch

from dynakv_amd import formats as F
from dynakv_amd.model import CompressedLlama, LlamaShape, RandomLlama

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
    m = cls(cfg).to(device=dev, dtype=torch.bfloat16).eval()
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


@pytest.mark.gpu
@pytest.mark.parametrize("S", [40, 494])
def test_hf_model_matches_compressed_llama(dev, monkeypatch, S):
    """Prefill logits at every position and 12 decode steps against CompressedLlama (S=494: the
    decode steps cross the 500-token switch from the short route to the long one)."""
    print(f"[gpu] hf model S={S}", flush=True)
    from dynakv_amd.hf import CustomAttention
    from dynakv_amd.kernels.compressed_cache import CustomDynamicCache

    model = RandomLlama(SHAPE, device=dev, seed=11, std=0.05)
    hfm = _hf_model(model, dev, monkeypatch)
    B, steps = 2, 12
    g = torch.Generator(device=dev).manual_seed(S)
    prompt = torch.randint(0, SHAPE.vocab, (B, S), generator=g, device=dev)
    gen = CompressedLlama(model)
    with torch.no_grad():
        x = gen.prefill(prompt)
        ref_logits = [gen.logits(x)]  # (B, S, V)
        cache = CustomDynamicCache()
        out = hfm(input_ids=prompt, past_key_values=cache, use_cache=True)
        assert all(isinstance(layer.self_attn, CustomAttention) and layer.self_attn.per_head
                   for layer in hfm.model.layers)
        got_logits = [out.logits]
        tok = ref_logits[0][:, -1:].argmax(-1)
        for t in range(steps):
            pos = S + t
            ref_logits.append(gen.logits(gen.decode(tok, pos)))
            got_logits.append(hfm(input_ids=tok, past_key_values=cache, use_cache=True).logits)
            tok = ref_logits[-1].argmax(-1)
        assert cache.get_seq_length() == S + steps
        # the same retained lengths in both caches (up to rounding-boundary flips)
        for layer in range(SHAPE.layers):
            for mine, theirs in ((cache.key_cache_sp[layer], gen.cache.key_cache_sp[layer]),
                                 (cache.value_cache_sp[layer], gen.cache.value_cache_sp[layer])):
                a = mine[1][:, : S + steps].long()
                b = theirs[1][:, : S + steps].long()
                frac = (a == b).float().mean().item()
                print(f"[parity] layer {layer} equal lengths: {frac:.4f}", flush=True)
                assert frac > 0.97, frac
    _close(got_logits[0], ref_logits[0], f"prefill logits S={S}")
    for t in range(1, steps + 1):
        _close(got_logits[t], ref_logits[t], f"decode step {t} S={S}")


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
