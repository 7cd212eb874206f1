"""The dense GQA decode kernel (the uncompressed baseline) against a float64 softmax attention.

The reference's uncompressed model attends every cached token's rotated key and value at full
width (transformers' Llama attention, scripts/benchmark_throughput.py:17-77); the check here is
the mathematics of that attention on the same inputs: softmax(q . k / sqrt(128)) v per query
head over its KV head's tokens, in float64 on the CPU."""
import math

import pytest
import torch

from dynakv_amd.kernels.decode import dense_decode_attention


def _case(B, Hkv, hpg, S, cap, dtype, dev, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn((B, Hkv * hpg, 128), generator=g) * scale).to(dtype)
    k = torch.randn((B * Hkv, cap * 128), generator=g).to(dtype)
    v = torch.randn((B * Hkv, cap * 128), generator=g).to(dtype)
    return q, k, v


def _reference(q, k, v, S):
    B, Hq, dh = q.shape
    rows = k.shape[0]
    Hkv = rows // B
    hpg = Hq // Hkv
    kk = k[:, :S * dh].double().reshape(B, Hkv, S, dh)
    vv = v[:, :S * dh].double().reshape(B, Hkv, S, dh)
    qq = q.double().reshape(B, Hkv, hpg, dh)
    s = torch.einsum("bgjd,bgtd->bgjt", qq, kk) / math.sqrt(dh)
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bgjt,bgtd->bgjd", p, vv).reshape(B, Hq, dh)


CASES = {
    # name: (B, Hkv, hpg, S, capacity, dtype, seed)
    "llama_b1_2k_bf16": (1, 8, 4, 2048, 2200, torch.bfloat16, 1),
    "llama_b4_2k_bf16": (4, 8, 4, 2111, 2200, torch.bfloat16, 2),
    "llama_b2_fp16": (2, 8, 4, 777, 800, torch.float16, 3),
    "S1": (3, 8, 4, 1, 8, torch.bfloat16, 4),
    "S17": (2, 4, 4, 17, 40, torch.float16, 5),
    "hpg1": (2, 8, 1, 300, 300, torch.bfloat16, 6),
    "hpg8": (2, 2, 8, 500, 512, torch.float16, 7),
    "hpg16": (1, 2, 16, 1000, 1024, torch.bfloat16, 8),
    "long_8k": (2, 8, 4, 8195, 8200, torch.bfloat16, 9),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_dense_decode_matches_float64(dev, name):
    B, Hkv, hpg, S, cap, dtype, seed = CASES[name]
    print(f"[gpu] dense decode {name}", flush=True)
    q, k, v = _case(B, Hkv, hpg, S, cap, dtype, dev, seed)
    got = dense_decode_attention(q.to(dev), k.to(dev), v.to(dev), S, out_dtype=torch.float32)
    ref = _reference(q, k, v, S)
    err = (got.double().cpu() - ref).abs()
    rel = err / ref.abs().clamp_min(1e-3)
    print(f"[gpu]   max_abs={err.max().item():.3e} max_rel={rel.max().item():.3e}", flush=True)
    assert err.max().item() <= 2e-3, name
    # the stored dtype output is the fp32 result rounded once
    got16 = dense_decode_attention(q.to(dev), k.to(dev), v.to(dev), S)
    assert got16.dtype == dtype
    assert torch.equal(got16, got.to(dtype))


@pytest.mark.gpu
def test_dense_decode_peaked_softmax(dev):
    """Large scores (a near one-hot softmax) exercise the running-maximum rescale."""
    print("[gpu] dense decode peaked", flush=True)
    q, k, v = _case(2, 8, 4, 1500, 1500, torch.bfloat16, dev, 21, scale=6.0)
    got = dense_decode_attention(q.to(dev), k.to(dev), v.to(dev), 1500, out_dtype=torch.float32)
    ref = _reference(q, k, v, 1500)
    assert (got.double().cpu() - ref).abs().max().item() <= 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize("split_len", [64, 128, 640, 4096])
def test_dense_decode_split_invariance(dev, split_len):
    print(f"[gpu] dense decode split_len={split_len}", flush=True)
    q, k, v = _case(2, 8, 4, 3001, 3100, torch.bfloat16, dev, 31)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    a = dense_decode_attention(qd, kd, vd, 3001, split_len=split_len, out_dtype=torch.float32)
    ref = _reference(q, k, v, 3001)
    assert (a.double().cpu() - ref).abs().max().item() <= 2e-3


@pytest.mark.gpu
def test_dense_decode_many_units_separate_merge(dev):
    """More units than arrival counters (16384): the separate merge kernel runs."""
    print("[gpu] dense decode separate merge", flush=True)
    B, Hkv, hpg, S = 2050, 8, 1, 20
    q, k, v = _case(B, Hkv, hpg, S, S, torch.float16, dev, 41)
    got = dense_decode_attention(q.to(dev), k.to(dev), v.to(dev), S, split_len=64,
                                 out_dtype=torch.float32)
    ref = _reference(q, k, v, S)
    assert (got.double().cpu() - ref).abs().max().item() <= 2e-3


@pytest.mark.gpu
def test_dense_decode_rejects_bad_arguments(dev):
    from dynakv_amd import _lib

    q, k, v = _case(1, 8, 4, 64, 64, torch.bfloat16, dev, 51)
    with pytest.raises(ValueError):
        dense_decode_attention(q.to(dev), k.to(dev), v.to(dev), 65)  # S past the row length
    with pytest.raises(ValueError):
        dense_decode_attention(q.to(dev), k.to(dev), v.to(dev), 64, split_len=100)
    lib = _lib.load()
    assert lib.dkv_decode_dense(None, _lib.DKV_BF16, None, 0, 0, None, None, 0, 1, None, 0,
                                None, 0, 0, _lib.DKV_BF16, 1, 32, 8, 128, 0) == _lib.DKV_E_ARG


def _random_dense(i: int):
    """Case i of a seeded sweep: KV heads, query heads per KV head 1-16, batch, 1-6000 tokens
    (log-uniform) in a buffer of up to 64 extra token slots, dtype."""
    g = torch.Generator().manual_seed(12000 + i)
    r = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))  # noqa: E731
    Hkv = [1, 2, 4, 8][r(0, 3)]
    hpg = [1, 2, 3, 4, 6, 8, 16][r(0, 6)]
    B = r(1, 4)
    S = max(1, int(math.exp(float(torch.rand(1, generator=g)) * math.log(6000))))
    cap = S + r(0, 64)
    dtype = torch.bfloat16 if r(0, 1) else torch.float16
    return B, Hkv, hpg, S, cap, dtype


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(12))
def test_random_dense_shapes_match_float64(dev, i):
    B, Hkv, hpg, S, cap, dtype = _random_dense(i)
    print(f"[gpu] dense decode random {i}: B={B} Hkv={Hkv} hpg={hpg} S={S} cap={cap} {dtype}",
          flush=True)
    q, k, v = _case(B, Hkv, hpg, S, cap, dtype, dev, seed=13000 + i)
    got = dense_decode_attention(q.to(dev), k.to(dev), v.to(dev), S, out_dtype=torch.float32)
    ref = _reference(q, k, v, S)
    err = (got.double().cpu() - ref).abs()
    assert err.max().item() <= 2e-3, i
    got16 = dense_decode_attention(q.to(dev), k.to(dev), v.to(dev), S)
    assert torch.equal(got16, got.to(dtype))
