"""The end-to-end model path (dynakv_amd/model.py) on a small Llama shape against a float32 torch
restatement of the same forward on the CPU: the compressed model with the retained lengths its
cutoff heads produced (read back from the cache), the dense model with every dim kept."""
import math

import pytest
import torch

from dynakv_amd.model import CompressedLlama, DenseLlama, LlamaShape, RandomLlama
from oracle.attention import rope_cos_sin

SHAPE = LlamaShape(hidden=512, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=1024, vocab=1000)


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope(x, pos0, theta):
    """x (..., S, 128) float32 at positions pos0 + s (fp32 angles, as the kernels form them)."""
    S = x.shape[-2]
    import numpy as np

    c, s = rope_cos_sin(np.arange(pos0, pos0 + S), 128, theta)
    c = torch.from_numpy(c).float().to(x.device)
    s = torch.from_numpy(s).float().to(x.device)
    x0, x1 = x[..., :64], x[..., 64:]
    return torch.cat([x0 * c - x1 * s, x1 * c + x0 * s], dim=-1)


def _reference_logits(model, tokens, lens_k=None, lens_v=None, device="cpu"):
    """float32 forward over all positions (on the CPU, or on ``device`` for the full shape);
    lens_*: per layer (B*G, S) retained dims or None (keep all)."""
    s = model.shape
    f = lambda t: t.detach().to(device).float()  # noqa: E731
    tokens = tokens.to(device)
    x = f(model.embed)[tokens]
    B, S = tokens.shape
    G, Dh, hpg = s.kv_heads, s.head_dim, s.heads // s.kv_heads
    for i, lw in enumerate(model.layers):
        h = _rms(x, f(lw.ln1), s.eps)
        q = (h @ f(lw.wq).T).view(B, S, s.heads, Dh).transpose(1, 2)
        kc = (h @ f(lw.wk_c).T).view(B, S, G, Dh).transpose(1, 2)  # (B, G, S, R)
        vc = (h @ f(lw.wv_c).T).view(B, S, G, Dh).transpose(1, 2)
        if lens_k is not None:
            ar = torch.arange(Dh, device=device)
            kc = kc * (ar < lens_k[i].view(B, G, S, 1)).float()
            vc = vc * (ar < lens_v[i].view(B, G, S, 1)).float()
        k = torch.einsum("bgsr,grd->bgsd", kc, f(lw.k_basis))
        v = torch.einsum("bgsr,grd->bgsd", vc, f(lw.v_basis))
        k = _rope(k, 0, s.theta)
        q = _rope(q, 0, s.theta)
        k = k.repeat_interleave(hpg, dim=1)
        v = v.repeat_interleave(hpg, dim=1)
        sc = q @ k.transpose(-1, -2) / math.sqrt(Dh)
        sc = sc.masked_fill(torch.ones(S, S, dtype=torch.bool, device=device).triu(1),
                            float("-inf"))
        a = torch.softmax(sc, -1) @ v
        x = x + a.transpose(1, 2).reshape(B, S, s.hidden) @ f(lw.wo).T
        h2 = _rms(x, f(lw.ln2), s.eps)
        x = x + (torch.nn.functional.silu(h2 @ f(lw.w_gate).T) * (h2 @ f(lw.w_up).T)) @ f(lw.w_down).T
    return _rms(x, f(model.norm), s.eps) @ f(model.lm_head).T


def _close(got, ref, what, rel=0.05):
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    print(f"[parity] {what}: max_abs={err:.3e} |ref|max={scale:.3e}", flush=True)
    assert err <= rel * scale, what


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["compressed", "compressed_per_op", "dense", "dense_sdpa"])
def test_model_matches_float32_forward(dev, kind):
    """compressed: the first decode step per layer takes the regular path, the later ones one
    dkv_decode_layer call; compressed_per_op: every step the regular path; dense: the
    uncompressed cache with dkv_decode_dense; dense_sdpa: the same cache through torch's SDPA."""
    print(f"[gpu] model {kind}", flush=True)
    model = RandomLlama(SHAPE, device=dev, seed=3, std=0.05)
    if kind.startswith("dense"):
        gen = DenseLlama(model, max_len=64, attention="sdpa" if kind == "dense_sdpa" else "kernel")
    else:
        gen = CompressedLlama(model, one_call_layers=(kind == "compressed"))
    g = torch.Generator(device="cpu").manual_seed(1)
    B, S = 2, 37
    tokens = torch.randint(0, SHAPE.vocab, (B, S), generator=g)
    prompt = tokens[:, :-3].to(dev)
    x = gen.prefill(prompt)
    got = [gen.logits(x).float().cpu()]
    for j in range(3):
        x = gen.decode(tokens[:, S - 3 + j:S - 2 + j].to(dev), S - 3 + j)
        got.append(gen.logits(x).float().cpu())
    got = torch.cat(got, dim=1)  # prompt positions, then the three decoded positions
    lk = lv = None
    if not kind.startswith("dense"):
        lk = [c[1][:, :S].cpu() for c in gen.cache.key_cache_sp]
        lv = [c[1][:, :S].cpu() for c in gen.cache.value_cache_sp]
        frac = torch.stack(lk).float().mean().item() / SHAPE.head_dim
        print(f"[gpu] model: mean retained fraction {frac:.3f}", flush=True)
        assert 0.3 < frac < 0.65  # the cutoff heads aim at 0.47
    ref = _reference_logits(model, tokens, lk, lv)
    _close(got, ref, kind)


@pytest.mark.gpu
def test_full_shape_keep_all_dims_matches_dense(dev):
    """Config 5 at its full Llama-3-8B shape (hidden 4096, 32 layers, 32/8 heads, FFN 14336,
    vocab 128256, bf16 weights N(0, 0.02)). With every layer's cutoff heads set to keep all 128
    dims the compressed model computes the dense model's function (orthogonal bases: k = U U^T k)
    and differs only by rounding (bf16 coefficients instead of bf16 keys, fp32-reconstructed K
    and V in the kernels). Its logits at the prompt's last position and over three decode steps
    must match the dense model's."""
    from dynakv_amd.kernels.cutoff import CutoffHead

    print("[gpu] model full shape, r = 128 everywhere, against the dense model", flush=True)
    shape = LlamaShape()
    model = RandomLlama(shape, device=dev, seed=11)
    G, Dh = shape.kv_heads, shape.head_dim
    zero = torch.zeros(G, Dh, Dh, device=dev, dtype=model.dtype)
    bias = torch.zeros(G, Dh, device=dev, dtype=model.dtype)
    # softmax mass on index 0: every prefix sum is ~1, so flip(cumsum) >= 0.1 keeps all dims
    bias[:, 0] = 30.0
    for lw in model.layers:
        lw.cutoff = CutoffHead(zero, bias, zero, bias, groups=G)
    g = torch.Generator(device="cpu").manual_seed(5)
    B, S = 2, 64
    tokens = torch.randint(0, shape.vocab, (B, S + 3), generator=g)
    outs = {}
    for kind in ("compressed", "dense"):
        gen = CompressedLlama(model) if kind == "compressed" else DenseLlama(model, max_len=128)
        x = gen.prefill(tokens[:, :S].to(dev))
        lg = [gen.logits(x[:, -1:]).float()]
        for j in range(3):
            x = gen.decode(tokens[:, S + j:S + j + 1].to(dev), S + j)
            lg.append(gen.logits(x).float())
        outs[kind] = torch.cat(lg, dim=1).cpu()  # (B, 4, vocab)
        if kind == "compressed":
            for slots in (gen.cache.key_cache_sp, gen.cache.value_cache_sp):
                for c in slots:
                    assert int(c[1][:, : S + 3].min()) == Dh  # every dim retained
        del gen
        torch.cuda.empty_cache()
    # float32 forward of the same weights over all S + 3 positions (compressed form, all dims
    # kept); positions S-1 .. S+2 are the prompt's last and the three decoded ones
    with torch.no_grad():
        ref = _reference_logits(model, tokens, device=dev)[:, S - 1:].float().cpu()
    scale = ref.abs().amax().item()
    errs = {k: (v - ref).abs().amax().item() for k, v in outs.items()}
    top1 = {k: (v.argmax(-1) == ref.argmax(-1)).float().mean().item() for k, v in outs.items()}
    between = (outs["compressed"] - outs["dense"]).abs().amax().item()
    print(f"[parity] full shape r=128 against float32: compressed max_abs={errs['compressed']:.3e} "
          f"dense max_abs={errs['dense']:.3e} (|ref|max={scale:.3f}); compressed vs dense "
          f"{between:.3e}; top-1 agreement with float32 {top1}", flush=True)
    # the compressed cache adds no error beyond the dense bf16 model's own rounding
    assert errs["compressed"] <= 1.25 * errs["dense"] + 0.01 * scale, errs
    assert errs["compressed"] <= 0.1 * scale, errs


@pytest.mark.gpu
def test_config5_workload_against_float32_forward(dev):
    """Config 5 at its stated workload: the full Llama-3-8B shape with the cutoff heads as
    RandomLlama builds them (mean retention ~0.47), a 2048-token prompt and 24 greedy decode
    steps; the first decode step grows every layer's packed caches (flat and tables), the later
    ones run one dkv_decode_layer call per layer. The logits at the prompt's last position and at
    every decoded one are checked against the float32 forward of the same weights with the
    retained lengths read back from the cache; every layer's K and V tables, pointers, upper
    bounds and buffer capacities bit-exact against the oracle's packing and growth model
    (compressed_cache.py:96-214) fed the same lengths; the flat buffers zero past each row's
    pointer, and layer 0's packed prompt kept bit for bit across its growth."""
    import numpy as np

    from oracle.packing import PackedSlot

    print("[gpu] config 5 workload: full shape, retention 0.47, prompt 2048, 24 steps",
          flush=True)
    shape = LlamaShape()
    model = RandomLlama(shape, device=dev, seed=7)
    gen = CompressedLlama(model)
    B, S, steps = 1, 2048, 24
    G, Dh = shape.kv_heads, shape.head_dim
    g = torch.Generator(device="cpu").manual_seed(9)
    prompt = torch.randint(0, shape.vocab, (B, S), generator=g)
    with torch.no_grad():
        x = gen.prefill(prompt.to(dev))
        lg = [gen.logits(x[:, -1:]).float()]
        fk0 = gen.cache.key_cache_sp[0][0].clone()
        ptr0 = gen.cache.key_cache_sp[0][3].clone()
        cap0 = gen.cache.key_cache_sp[0][0].shape[1]
        toks = [lg[-1].argmax(-1)]
        for j in range(steps):
            x = gen.decode(toks[-1], S + j)
            lg.append(gen.logits(x).float())
            toks.append(lg[-1].argmax(-1))
    got = torch.cat(lg, dim=1).cpu()  # (B, steps + 1, vocab)
    L = S + steps
    assert gen.cache.get_seq_length_sp(0) == L
    assert gen.cache.key_cache_sp[0][0].shape[1] > cap0, "the decode steps grew the flat buffer"
    lk = [c[1][:, :L].cpu() for c in gen.cache.key_cache_sp]
    lv = [c[1][:, :L].cpu() for c in gen.cache.value_cache_sp]
    frac = torch.stack(lk).float().mean().item() / Dh
    print(f"[gpu] config 5: mean retained fraction {frac:.3f}", flush=True)
    assert 0.35 < frac < 0.6
    # packing: the oracle's slot model fed the read-back lengths (prefill, then one token a step)
    for slots, lens in ((gen.cache.key_cache_sp, lk), (gen.cache.value_cache_sp, lv)):
        for i, c in enumerate(slots):
            ln = lens[i].numpy()
            slot = PackedSlot()
            slot.append_prefill(np.zeros((B * G, S, Dh), np.float32), ln[:, :S], Dh)
            for j in range(steps):
                slot.append_decode(np.zeros((B * G, Dh), np.float32), ln[:, S + j:S + j + 1], Dh)
            ol, oo = slot.tables()
            assert np.array_equal(c[1][:, :L].cpu().numpy(), ol), f"layer {i} lens"
            assert np.array_equal(c[2][:, :L].cpu().numpy(), oo), f"layer {i} offsets"
            assert np.array_equal(c[3].cpu().numpy(), slot.ptr), f"layer {i} pointers"
            assert list(c[5]) == list(slot.ub), f"layer {i} upper bounds"
            assert c[0].shape == slot.flat.shape, f"layer {i} flat capacity"
            assert c[1].shape == slot.lens.shape and c[2].shape == slot.offs.shape
            assert c[4] == slot.seq
            tail = torch.arange(c[0].shape[1], device=dev)[None, :] >= c[3][:, None].long()
            assert not (c[0] * tail).any(), f"layer {i}: elements past the row pointers"
    # the packed prompt of layer 0 survives the growth bit for bit
    fk = gen.cache.key_cache_sp[0][0]
    for r in range(B * G):
        n = int(ptr0[r])
        assert torch.equal(fk[r, :n], fk0[r, :n])
    tokens = torch.cat([prompt, torch.cat(toks[:-1], dim=1).cpu()], dim=1)  # (B, L)
    del gen
    torch.cuda.empty_cache()
    with torch.no_grad():
        ref = _reference_logits(model, tokens, [t.to(dev) for t in lk], [t.to(dev) for t in lv],
                                device=dev)[:, S - 1:].float().cpu()
    err = (got - ref).abs().amax().item()
    scale = ref.abs().amax().item()
    corr = torch.corrcoef(torch.stack([got.flatten(), ref.flatten()]))[0, 1].item()
    print(f"[parity] config 5 workload vs float32: max_abs={err:.3e} |ref|max={scale:.3e} "
          f"corr={corr:.5f}", flush=True)
    assert err <= 0.1 * scale
    assert corr > 0.99
