"""Positions and masks of the transformers surface (dynakv_amd/hf.py) on the GPU, against
transformers' own Llama and the oracle.

The reference rotates q with the decoder's position embeddings (``LlamaRotaryEmbedding`` at
``position_ids``, ``rope_scaling`` included: compressed_attention.py:314,360), the prefill K with
the layer's rotary embedding at positions 0..L-1 (calc_cos_sin, :193-200,375-378), the decode K
with plain theta inside its kernels (two_stage.py:28-46, fused.py:65-102), and masks a prompt's
padding in the prefill attention (create_causal_mask, custom_llama.py:161-168). A llama3
``rope_scaling`` config makes the scaled and the plain rotation differ, so each test below would
fail if q were rotated with the kernels' plain theta."""
import math

import numpy as np
import pytest
import torch

from dynakv_amd.kernels.prefill import prefill_attention, rope_apply_
from dynakv_amd.synthetic import random_orthogonal
from oracle import attention as A
from oracle import prefill as P

from helpers import NP_OF, assert_close, cast_np

SCALING = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
           "original_max_position_embeddings": 64}


def _config(**kw):
    from transformers import LlamaConfig

    base = dict(hidden_size=512, num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                intermediate_size=1024, vocab_size=1000, num_hidden_layers=2,
                rope_theta=500000.0, rope_scaling=dict(SCALING), tie_word_embeddings=False)
    base.update(kw)
    return LlamaConfig(**base)


def bf16_model(build):
    """``build()`` with bfloat16 as the default dtype, as ``from_pretrained(dtype=bf16)``
    constructs a model: parameters in bf16, the rotary ``inv_freq`` buffers computed in float32
    (``module.to(bf16)`` would round those too -- transformers' own behaviour)."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        return build()
    finally:
        torch.set_default_dtype(old)


def _rotate_half(x):
    return torch.cat((-x[..., 64:], x[..., :64]), dim=-1)


def _hf_rope(x, cos, sin):
    """The reference's apply_rotary_pos_emb_ (compressed_attention.py:18-22) in x's dtype."""
    return (x * cos.unsqueeze(1)) + (_rotate_half(x) * sin.unsqueeze(1))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_apply_is_the_reference_formula(dev, dtype):
    """dkv_rope_apply against the reference formula evaluated by torch in the dtype, with llama3
    scaled cos/sin: per-row positions (a left-padded batch's position ids) and one shared table
    (calc_cos_sin's positions 0..L-1); bit-exact."""
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    print(f"[gpu] rope_apply {dtype}", flush=True)
    rot = LlamaRotaryEmbedding(_config()).to(dev)
    g = torch.Generator(device=dev).manual_seed(3)
    B, H, S = 3, 5, 77
    x = (torch.randn(B, H, S, 128, generator=g, device=dev) * 3).to(dtype)
    mask = torch.ones(B, S, dtype=torch.long, device=dev)
    mask[0, :9] = 0
    mask[2, :30] = 0
    pos = (mask.cumsum(-1) - 1).clamp(min=0)
    for positions in (pos, torch.arange(S, device=dev).unsqueeze(0) + 4000):
        cos, sin = rot(x, positions)
        want = _hf_rope(x, cos, sin)
        got = rope_apply_(x.clone(), cos, sin)
        assert torch.equal(got, want)
    # a strided view (one head of a (B, S, H, 128) projection) rotates in place
    y = (torch.randn(B, S, H, 128, generator=g, device=dev)).to(dtype)
    cos, sin = rot(y, pos)
    want = _hf_rope(y.transpose(1, 2), cos, sin)
    rope_apply_(y.transpose(1, 2), cos, sin)
    assert torch.equal(y.transpose(1, 2), want)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_attention_left_padding(dev, dtype):
    """dkv_prefill_attention with kstart (keys before each row's first real token masked)
    against the oracle: rows padded by 0, 37 (inside a key tile), 64 (a whole tile), 190, and a
    row of padding only (every query gets 0)."""
    print(f"[gpu] prefill left padding {dtype}", flush=True)
    rng = np.random.default_rng(17)
    B, Hq, Hkv, S = 5, 8, 2, 200
    kstart = [0, 37, 64, 190, 200]
    q = cast_np(rng.standard_normal((B, Hq, S, 128)).astype(np.float32), dtype)
    k = cast_np(rng.standard_normal((B, Hkv, S, 128)).astype(np.float32), dtype)
    v = cast_np(rng.standard_normal((B, Hkv, S, 128)).astype(np.float32), dtype)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    ks = torch.tensor(kstart, dtype=torch.int32, device=dev)
    got = prefill_attention(t(q), t(k), t(v), causal=True, out_dtype=torch.float32, kstart=ks)
    ref = P.attention(q, k, v, causal=True, kstart=kstart)
    assert_close(got, ref, f"prefill kstart {dtype}")
    assert not got[4].any() and not got[3, :, :190].any()
    # kstart of zeros is the plain causal attention, bit for bit
    plain = prefill_attention(t(q), t(k), t(v), causal=True, out_dtype=torch.float32)
    zero = prefill_attention(t(q), t(k), t(v), causal=True, out_dtype=torch.float32,
                             kstart=torch.zeros(B, dtype=torch.int32, device=dev))
    assert torch.equal(plain, zero)


def _keep_all(attn, dev):
    """Cutoff heads that keep every dim: zero weights, the softmax mass on index 0 of each
    group (every prefix sum is ~1, so flip(cumsum) >= 0.1 keeps the whole group)."""
    D = attn.d
    with torch.no_grad():
        attn.Wk.zero_()
        attn.Wv.zero_()
        b = torch.zeros(1, D, device=dev, dtype=attn.bk.dtype)
        b[0, ::128] = 30.0
        attn.bk.copy_(b)
        attn.bv.copy_(b)


@pytest.mark.gpu
def test_hf_prefill_left_padded_matches_transformers_llama(dev, monkeypatch):
    """CustomLlamaForCausalLM with identity bases and every dim kept computes transformers'
    Llama; on a llama3 rope_scaling config and a left-padded batch its prompt logits at the real
    positions match transformers' LlamaForCausalLM (float32, eager attention, same weights)."""
    from transformers import LlamaForCausalLM

    from dynakv_amd import hf
    from dynakv_amd.kernels.compressed_cache import CustomDynamicCache

    print("[gpu] hf prefill left padded vs transformers", flush=True)
    monkeypatch.setenv(hf.PHYSICAL_ENV, "1")
    torch.manual_seed(0)
    ref = LlamaForCausalLM(_config(attn_implementation="eager")).to(dev).float().eval()
    with torch.no_grad():
        for p in ref.parameters():
            p.normal_(0.0, 0.05)
        for layer in ref.model.layers:
            layer.input_layernorm.weight.fill_(1.0)
            layer.post_attention_layernorm.weight.fill_(1.0)
        ref.model.norm.weight.fill_(1.0)
        for p in ref.parameters():  # weights representable in bf16
            p.copy_(p.to(torch.bfloat16).float())
    mine = bf16_model(lambda: hf.get_model_class("llama")(_config())).to(dev).eval()
    mine.load_state_dict({k: v.to(torch.bfloat16) for k, v in ref.state_dict().items()},
                         strict=False)
    for layer in mine.model.layers:
        _keep_all(layer.self_attn, dev)
    B, S = 3, 90
    g = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(0, 1000, (B, S), generator=g, device=dev)
    mask = torch.ones(B, S, dtype=torch.long, device=dev)
    mask[0, :7] = 0
    mask[2, :70] = 0
    with torch.no_grad():
        want = ref(input_ids=ids, attention_mask=mask).logits
        got = mine(input_ids=ids, attention_mask=mask, past_key_values=CustomDynamicCache(),
                   use_cache=True).logits.float()
        assert all(layer.self_attn.per_head for layer in mine.model.layers)
        # the same prompt without its padding mask differs (the mask is honoured)
        nomask = mine(input_ids=ids, past_key_values=CustomDynamicCache(),
                      use_cache=True).logits.float()
    real = mask.bool()
    err = (got - want).abs()[real].max().item()
    scale = want[real].abs().max().item()
    moved = (nomask - got).abs()[real].max().item()
    print(f"[parity] hf left-padded prefill vs transformers: max_abs={err:.3e} "
          f"|ref|max={scale:.3e}; without the mask the logits move by {moved:.3e}", flush=True)
    assert err <= 0.03 * scale
    assert moved > 10 * err


@pytest.mark.gpu
def test_hf_right_padding_raises(dev, monkeypatch):
    from dynakv_amd import hf

    monkeypatch.setenv(hf.PHYSICAL_ENV, "1")
    m = bf16_model(lambda: hf.get_model_class("llama")(_config(num_hidden_layers=1))).to(dev)
    ids = torch.zeros(2, 8, dtype=torch.long, device=dev)
    mask = torch.ones(2, 8, dtype=torch.long, device=dev)
    mask[1, 6:] = 0
    with pytest.raises(NotImplementedError, match="left padding"):
        m(input_ids=ids, attention_mask=mask)


def _attention_layer(dev, per_head: bool, seed: int):
    """One CustomAttention (hidden 512 = 4 heads x 128, o_proj the identity so the module's
    output is the attention output) with random projections, orthogonal bases and random cutoff
    heads: block-diagonal per KV head (per-head layout) or dense 256 x 256 (joint layout)."""
    from dynakv_amd.hf import CustomAttention

    cfg = _config(num_hidden_layers=1)
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    a = bf16_model(lambda: CustomAttention(cfg, 0))
    assert a.rotary_emb.inv_freq.dtype == torch.float32
    D = a.d
    with torch.no_grad():
        for lin in (a.q_proj, a.k_proj, a.v_proj):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 0.05)
        a.o_proj.weight.copy_(torch.eye(512))
        if per_head:
            ku = torch.block_diag(*[torch.from_numpy(random_orthogonal(128, rng)).float()
                                    for _ in range(2)])
            vu = torch.block_diag(*[torch.from_numpy(random_orthogonal(128, rng)).float()
                                    for _ in range(2)])
            wk = torch.block_diag(*[torch.randn(128, 128, generator=g) for _ in range(2)])
            wv = torch.block_diag(*[torch.randn(128, 128, generator=g) for _ in range(2)])
        else:
            ku = torch.from_numpy(random_orthogonal(D, rng)).float()
            vu = torch.from_numpy(random_orthogonal(D, rng)).float()
            wk = torch.randn(D, D, generator=g)
            wv = torch.randn(D, D, generator=g)
        a.k_up.copy_(ku)
        a.v_up.copy_(vu)
        a.Wk.copy_(wk)
        a.Wv.copy_(wv)
        a.bk.copy_(torch.randn(1, D, generator=g))
        a.bv.copy_(torch.randn(1, D, generator=g))
    return a.to(dev), cfg


def _flat_tables(slot, S):
    f, l, o = slot[0], slot[1][:, :S], slot[2][:, :S]
    return (f.float().cpu().numpy(), l.cpu().numpy(), o.cpu().numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["per_head", "joint"])
def test_attention_positions_against_oracle(dev, layout):
    """CustomAttention under a llama3 rope_scaling config, prefill of 40 tokens and 3 decode
    steps (the first per-head step on the regular path, the later ones one dkv_decode_layer call
    each with q rotated by the caller), against the oracle given q rotated by the decoder's
    position embeddings (the reference formula in bf16): prefill K rotated by the layer's rotary
    embedding at 0..L-1, decode K by plain theta at the row index, both over the coefficients the
    cache holds. The joint layout (dense 256 x 256 bases and cutoff heads) is the path a
    reference checkpoint with full PCA bases takes."""
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    from dynakv_amd.kernels.compressed_cache import CustomDynamicCache

    print(f"[gpu] attention positions {layout}", flush=True)
    per_head = layout == "per_head"
    attn, cfg = _attention_layer(dev, per_head, seed=23 if per_head else 29)
    rot = LlamaRotaryEmbedding(cfg).to(dev)
    B, S0, steps, Hq, G, Dh = 2, 40, 3, 4, 2, 128
    hpg = Hq // G
    g = torch.Generator(device=dev).manual_seed(4)
    h = torch.randn(B, S0 + steps, 512, generator=g, device=dev).to(torch.bfloat16)
    cache = CustomDynamicCache()
    outs, qrots = [], []
    with torch.no_grad():
        for t0, t1 in [(0, S0)] + [(S0 + j, S0 + j + 1) for j in range(steps)]:
            x = h[:, t0:t1]
            pe = rot(x, torch.arange(t0, t1, device=dev).unsqueeze(0))
            outs.append(attn(x, position_embeddings=pe, past_key_values=cache)[0])
            q = attn.q_proj(x).view(B, t1 - t0, Hq, Dh).transpose(1, 2)
            qrots.append(_hf_rope(q, *pe))
        assert attn.per_head == per_head
        L = S0 + steps
        fk, lk, ok = _flat_tables(cache.key_cache_sp[0], L)
        fv, lv, ov = _flat_tables(cache.value_cache_sp[0], L)
        kb = attn.k_basis.float().cpu().numpy()
        vb = attn.v_basis.float().cpu().numpy()
        R = kb.shape[1]
        # prefill: K and V reconstructed in the dtype, K rotated by the rotary embedding at
        # 0..S0-1 with the reference formula
        rows = B * G if per_head else B
        ck = np.stack([A.gather_padded(fk[r], lk[r, :S0], ok[r, :S0], R) for r in range(rows)])
        cv = np.stack([A.gather_padded(fv[r], lv[r, :S0], ov[r, :S0], R) for r in range(rows)])
        if per_head:
            ck, cv = ck.reshape(B, G, S0, R), cv.reshape(B, G, S0, R)
            K = np.stack([P.reconstruct(ck[:, gi], kb[gi], "bfloat16") for gi in range(G)], 1)
            V = np.stack([P.reconstruct(cv[:, gi], vb[gi], "bfloat16") for gi in range(G)], 1)
        else:
            K = np.stack([P.reconstruct(ck, kb[gi], "bfloat16") for gi in range(G)], 1)
            V = np.stack([P.reconstruct(cv, vb[gi], "bfloat16") for gi in range(G)], 1)
        Kt = torch.from_numpy(K).to(device=dev, dtype=torch.bfloat16)
        cos, sin = rot(Kt, torch.arange(S0, device=dev).unsqueeze(0))
        Kr = _hf_rope(Kt, cos, sin).float().cpu().numpy()
        ref = P.attention(qrots[0].float().cpu().numpy(), Kr, V, causal=True)
        assert_close(outs[0].view(B, S0, Hq, Dh).transpose(1, 2).float(), ref,
                     f"{layout} prefill", tol_abs=8e-3)
        # decode steps: the oracle over the cache as it stood after each append
        plain = None
        for j in range(steps):
            S = S0 + j + 1
            qr = qrots[j + 1][:, :, 0].float().cpu().numpy()
            if per_head:
                kw = dict(row_of=lambda b, hh: b * G + hh // hpg, basis_of=lambda hh: hh // hpg)
                kbj, vbj = kb, vb
            else:
                kw = {}
                kbj, vbj = np.repeat(kb, hpg, 0), np.repeat(vb, hpg, 0)
            ref = A.decode_attention(qr, fk, kbj, fv, vbj, lk[:, :S], ok[:, :S], lv[:, :S],
                                     ov[:, :S], cfg.rope_parameters["rope_theta"],
                                     route="short_fused", q_dtype="bfloat16", **kw)
            assert_close(outs[j + 1].view(B, Hq, Dh).float(), ref, f"{layout} decode {j}",
                         tol_abs=8e-3)
            if j == 0:
                # the kernels' plain-theta q would be a different result: the test sees drift
                qp = attn.q_proj(h[:, S - 1:S]).view(B, 1, Hq, Dh).transpose(1, 2)
                cs = A.rope_cos_sin(np.array([S - 1]), Dh, cfg.rope_parameters["rope_theta"])
                qpl = A.apply_rope(qp[:, :, 0].float().cpu().numpy().astype(np.float64),
                                   cs[0][0], cs[1][0])
                plain = A.decode_attention(qpl, fk, kbj, fv, vbj, lk[:, :S], ok[:, :S],
                                           lv[:, :S], ov[:, :S], cfg.rope_parameters["rope_theta"],
                                           route="short_fused", q_dtype="bfloat16", **kw)
                diff = float(np.abs(plain - ref).max())
                print(f"[parity] {layout}: plain-theta q would move the output by {diff:.3e}",
                      flush=True)
                assert diff > 5e-2
