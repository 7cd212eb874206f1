"""The one-call decode layer step (``dkv_decode_layer`` through ``DecodeLayerPlan``: cutoff
logits, then counts + K/V appends + q RoPE in one launch, then the routed attention) against
the same step taken operation by operation (``kv_process_fused``, ``update_sp``,
``rope_dense_``, ``grouped_decode_attention``): the cache tables, pointers and stored
coefficients, the rotated query and the attention output are bit-identical."""
import pytest
import torch

from dynakv_amd.kernels.compressed_cache import CustomDynamicCache
from dynakv_amd.kernels.cutoff import CutoffHead
from dynakv_amd.kernels.decode import grouped_decode_attention
from dynakv_amd.kernels.layer import DecodeLayerPlan
from dynakv_amd.kernels.prefill import rope_dense_
from dynakv_amd.kernels.router import KernelPolicy
from dynakv_amd.model import ramp_for_retention


def _basis(G, R, g, dev, dtype):
    a = torch.randn(G, R, R, generator=g)
    q, r = torch.linalg.qr(a)
    return (q * torch.sign(torch.diagonal(r, dim1=-2, dim2=-1)).unsqueeze(-2)).transpose(1, 2) \
        .contiguous().to(dtype).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,S0,steps", [(2, 37, 3), (3, 600, 2),
                                         (20, 37, 2),   # a second, partial 16-row tile
                                         (33, 40, 2),   # three tiles, the last of one row
                                         (5, 496, 4),   # across the 500-token route switch
                                         (7, 254, 3),   # past 256 tokens: one split -> several
                                         (12, 1, 3)])   # a one-token prompt
def test_layer_step_matches_per_op_path(dev, dtype, B, S0, steps):
    print(f"[gpu] layer step {dtype} B={B} S0={S0}", flush=True)
    G, R, Hq, theta = 8, 128, 32, 500000.0
    g = torch.Generator(device="cpu").manual_seed(B * 1009 + S0)
    ramp = ramp_for_retention(R, 0.47) * torch.arange(R, dtype=torch.float32) / R
    head = CutoffHead((0.05 * torch.randn(G, R, R, generator=g)).to(dtype).to(dev),
                      ramp.expand(G, R).contiguous().to(dtype).to(dev),
                      (0.05 * torch.randn(G, R, R, generator=g)).to(dtype).to(dev),
                      ramp.expand(G, R).contiguous().to(dtype).to(dev), groups=G)
    kb, vb = _basis(G, R, g, dev, dtype), _basis(G, R, g, dev, dtype)
    policy = KernelPolicy()
    # identical prompt caches (the prompt's coefficients through the cutoff head, packed)
    x0k = torch.randn(B, S0, G * R, generator=g).to(dtype).to(dev)
    x0v = torch.randn(B, S0, G * R, generator=g).to(dtype).to(dev)
    caches = []
    for _ in range(2):
        c = CustomDynamicCache()
        ko, vo, lk, lv, _, _ = head.kv_process_fused(x0k, x0v)
        rk = ko.view(B, S0, G, R).transpose(1, 2).reshape(B * G, S0, R).contiguous()
        rv = vo.view(B, S0, G, R).transpose(1, 2).reshape(B * G, S0, R).contiguous()
        c.update_sp(rk, lk.view(B, S0, G).transpose(1, 2).reshape(B * G, S0).contiguous(), rv,
                    lv.view(B, S0, G).transpose(1, 2).reshape(B * G, S0).contiguous(), R, 0, R)
        caches.append(c)

    def per_op(cache, q, kc, vc, pos):
        ko, vo, lk, lv, _, _ = head.kv_process_fused(kc.view(B, 1, G * R), vc.view(B, 1, G * R))
        rk = ko.view(B, G, R).reshape(B * G, 1, R).contiguous()
        rv = vo.view(B, G, R).reshape(B * G, 1, R).contiguous()
        fk, fv, tk, tv, ok, ov = cache.update_sp(rk, lk.view(B * G, 1).contiguous(), rv,
                                                 lv.view(B * G, 1).contiguous(), R, 0, R)
        rope_dense_(q.view(B * Hq, 1, 128), theta=theta, pos0=pos)
        L = cache.get_seq_length_sp(0)
        return grouped_decode_attention(q, fk, fv, tk, ok, tv, ov, kb, vb, theta=theta,
                                        route=policy.select(L))

    def inputs():
        return (torch.randn(B, Hq, 128, generator=g).to(dtype).to(dev),
                torch.randn(B, G * R, generator=g).to(dtype).to(dev),
                torch.randn(B, G * R, generator=g).to(dtype).to(dev))

    # the first decode step grows the flat buffers (sized exactly at prefill, as the reference
    # sizes them): both caches take it operation by operation, as the model does
    q, kc, vc = inputs()
    for c in caches:
        per_op(c, q.clone(), kc, vc, S0)
    plan = DecodeLayerPlan(caches[0], 0, head, kb, vb, batch=B, heads=Hq, theta=theta,
                           policy=policy)
    for st in range(1, steps + 1):
        pos = S0 + st
        q, kc, vc = inputs()
        assert plan.can_step()
        qa = q.clone()
        out_a = plan.step(qa, kc, vc, pos)
        qb = q.clone()
        out_b = per_op(caches[1], qb, kc, vc, pos)
        assert torch.equal(qa, qb), "rotated query"
        for name, ca, cb in (("K", caches[0].key_cache_sp[0], caches[1].key_cache_sp[0]),
                             ("V", caches[0].value_cache_sp[0], caches[1].value_cache_sp[0])):
            assert ca[4] == cb[4], f"{name} length"
            n = ca[4]
            assert torch.equal(ca[1][:, :n], cb[1][:, :n]), f"{name} lens"
            assert torch.equal(ca[2][:, :n], cb[2][:, :n]), f"{name} offs"
            assert torch.equal(ca[3], cb[3]), f"{name} ptr"
            used = int(ca[3].max())
            for r in range(B * G):
                u = int(ca[3][r])
                assert torch.equal(ca[0][r, :u], cb[0][r, :u]), f"{name} row {r}"
            assert used > 0
        assert torch.equal(out_a, out_b), "attention output"
    print(f"[parity] layer step: {steps} steps bit-identical", flush=True)
