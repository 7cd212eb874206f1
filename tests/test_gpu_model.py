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
    c = torch.from_numpy(c).float()
    s = torch.from_numpy(s).float()
    x0, x1 = x[..., :64], x[..., 64:]
    return torch.cat([x0 * c - x1 * s, x1 * c + x0 * s], dim=-1)


def _reference_logits(model, tokens, lens_k=None, lens_v=None):
    """float32 CPU forward over all positions; lens_*: per layer (B*G, S) retained dims or None
    (keep all)."""
    s = model.shape
    f = lambda t: t.detach().float().cpu()  # noqa: E731
    x = f(model.embed)[tokens]
    B, S = tokens.shape
    G, Dh, hpg = s.kv_heads, s.head_dim, s.heads // s.kv_heads
    for i, lw in enumerate(model.layers):
        h = _rms(x, f(lw.ln1), s.eps)
        q = (h @ f(lw.wq).T).view(B, S, s.heads, Dh).transpose(1, 2)
        kc = (h @ f(lw.wk_c).T).view(B, S, G, Dh).transpose(1, 2)  # (B, G, S, R)
        vc = (h @ f(lw.wv_c).T).view(B, S, G, Dh).transpose(1, 2)
        if lens_k is not None:
            ar = torch.arange(Dh)
            kc = kc * (ar < lens_k[i].view(B, G, S, 1)).float()
            vc = vc * (ar < lens_v[i].view(B, G, S, 1)).float()
        k = torch.einsum("bgsr,grd->bgsd", kc, f(lw.k_basis))
        v = torch.einsum("bgsr,grd->bgsd", vc, f(lw.v_basis))
        k = _rope(k, 0, s.theta)
        q = _rope(q, 0, s.theta)
        k = k.repeat_interleave(hpg, dim=1)
        v = v.repeat_interleave(hpg, dim=1)
        sc = q @ k.transpose(-1, -2) / math.sqrt(Dh)
        sc = sc.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
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
@pytest.mark.parametrize("kind", ["compressed", "compressed_per_op", "dense"])
def test_model_matches_float32_forward(dev, kind):
    """compressed: the first decode step per layer takes the regular path, the later ones one
    dkv_decode_layer call; compressed_per_op: every step the regular path."""
    print(f"[gpu] model {kind}", flush=True)
    model = RandomLlama(SHAPE, device=dev, seed=3, std=0.05)
    if kind == "dense":
        gen = DenseLlama(model, max_len=64)
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
    if kind != "dense":
        lk = [c[1][:, :S].cpu() for c in gen.cache.key_cache_sp]
        lv = [c[1][:, :S].cpu() for c in gen.cache.value_cache_sp]
        frac = torch.stack(lk).float().mean().item() / SHAPE.head_dim
        print(f"[gpu] model: mean retained fraction {frac:.3f}", flush=True)
        assert 0.3 < frac < 0.65  # the cutoff heads aim at 0.47
    ref = _reference_logits(model, tokens, lk, lv)
    _close(got, ref, kind)
