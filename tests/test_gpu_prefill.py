"""The gfx950 prefill path (dkv_rope_dense, dkv_prefill_attention, and the whole reconstruct +
attend chain over a per-head cache) against the oracle (reference
compressed_attention.py:359-386)."""
import zlib

import numpy as np
import pytest
import torch

from dynakv_amd.kernels.compressed_cache import CustomDynamicCache
from dynakv_amd.kernels.prefill import compressed_prefill_attention, prefill_attention, rope_dense_
from dynakv_amd.synthetic import random_orthogonal
from oracle import prefill as P

from helpers import NP_OF, assert_close, cast_np

CASES = {
    # name: (B, Hq, Hkv, Sq, Sk, causal, dtype)
    "S1": (1, 32, 8, 1, 1, True, torch.bfloat16),
    "S17_gqa": (2, 32, 8, 17, 17, True, torch.float16),
    "S64": (1, 8, 2, 64, 64, True, torch.bfloat16),
    "S100_mha": (1, 4, 4, 100, 100, True, torch.float16),
    "chunk_Sq50_Sk300": (2, 8, 2, 50, 300, True, torch.bfloat16),
    "noncausal": (1, 8, 2, 33, 129, False, torch.bfloat16),
    "S1024": (1, 32, 8, 1024, 1024, True, torch.bfloat16),
    # 9 (query block, batch, KV head) units: the work items go out in the ungrouped order
    "S300_units9": (1, 6, 3, 300, 300, True, torch.float16),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_prefill_attention_matches_oracle(dev, name):
    B, Hq, Hkv, Sq, Sk, causal, dtype = CASES[name]
    print(f"[gpu] prefill attention {name}", flush=True)
    rng = np.random.default_rng(zlib.crc32(name.encode()) % 997)
    q = cast_np(rng.standard_normal((B, Hq, Sq, 128)).astype(np.float32), dtype)
    k = cast_np(rng.standard_normal((B, Hkv, Sk, 128)).astype(np.float32), dtype)
    v = cast_np(rng.standard_normal((B, Hkv, Sk, 128)).astype(np.float32), dtype)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    got = prefill_attention(t(q), t(k), t(v), causal=causal, out_dtype=torch.float32)
    low = prefill_attention(t(q), t(k), t(v), causal=causal)
    torch.cuda.synchronize()
    ref = P.attention(q, k, v, causal=causal)
    # the bar applies to the result before the output rounding; the stored output is exactly
    # that result rounded to the dtype
    assert_close(got, ref, name)
    assert torch.equal(low, got.to(dtype))


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [0.3, 0.01])
def test_prefill_attention_custom_scale(dev, scale):
    """A positive scale other than 1/sqrt(128): the kernel takes each tile's maximum of the
    unscaled scores and applies the scale there and inside the exponent, so a sharp (0.3) and a
    flat (0.01) softmax check that fold against the oracle; scales <= 0 are rejected."""
    print(f"[gpu] prefill attention scale {scale}", flush=True)
    B, Hq, Hkv, S = 2, 8, 2, 200
    dtype = torch.bfloat16
    rng = np.random.default_rng(31)
    q = cast_np(rng.standard_normal((B, Hq, S, 128)).astype(np.float32), dtype)
    k = cast_np(rng.standard_normal((B, Hkv, S, 128)).astype(np.float32), dtype)
    v = cast_np(rng.standard_normal((B, Hkv, S, 128)).astype(np.float32), dtype)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    got = prefill_attention(t(q), t(k), t(v), causal=True, scale=scale, out_dtype=torch.float32)
    ref = P.attention(q, k, v, causal=True, scale=scale)
    assert_close(got, ref, f"scale {scale}")
    with pytest.raises(NotImplementedError):
        prefill_attention(t(q), t(k), t(v), causal=True, scale=-scale)


@pytest.mark.gpu
def test_prefill_attention_strided_views(dev):
    """(B, S, H, D) activations viewed as (B, H, S, D) without a copy."""
    print("[gpu] prefill attention strided", flush=True)
    B, Hq, Hkv, S = 2, 8, 2, 80
    dtype = torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(3)
    q = torch.randn(B, S, Hq, 128, generator=g).to(dev, dtype)
    k = torch.randn(B, S, Hkv, 128, generator=g).to(dev, dtype)
    v = torch.randn(B, S, Hkv, 128, generator=g).to(dev, dtype)
    got = prefill_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                            out_dtype=torch.float32)
    ref = P.attention(q.transpose(1, 2).float().cpu().numpy(), k.transpose(1, 2).float().cpu().numpy(),
                      v.transpose(1, 2).float().cpu().numpy())
    assert_close(got.float(), ref, "strided")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_dense_matches_oracle(dev, dtype):
    print(f"[gpu] rope dense {dtype}", flush=True)
    rng = np.random.default_rng(7)
    x = cast_np(rng.standard_normal((3, 4, 700, 128)).astype(np.float32), dtype)
    xt = torch.from_numpy(x).to(device=dev, dtype=dtype)
    rope_dense_(xt, theta=500000.0, pos0=5)
    got = xt.float().cpu().numpy()
    ref = P.rope_dense(x, 500000.0, NP_OF[dtype], pos0=5)
    # fp32 rotation vs the float64 one: one unit in the last place of the result, plus the fp32
    # slack of the angle (inv_freq from the device's expf, |angle| < 705) and of the products
    mant = 10 if dtype == torch.float16 else 7
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -14))) - mant)
    pair = np.abs(x[..., :64]) + np.abs(x[..., 64:])
    pair = np.concatenate([pair, pair], axis=-1)
    slack = (705 * 2.0 ** -22 + 2.0 ** -21) * pair
    err = np.abs(got - ref)
    assert (err <= ulp + slack).all(), float((err - ulp - slack).max())
    assert (got == ref).mean() > 0.95


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_compressed_prefill_matches_oracle(dev, dtype):
    """Prompt packed into a per-head cache, re-expanded, projected, RoPE'd and attended."""
    print(f"[gpu] compressed prefill {dtype}", flush=True)
    B, G, Hq, S, R = 2, 8, 32, 200, 128
    rng = np.random.default_rng(11)
    theta = 500000.0
    lens = rng.integers(0, R + 1, size=(B * G, S)).astype(np.int32)
    coef = cast_np(rng.standard_normal((B * G, S, R)).astype(np.float32), dtype)
    vcoef = cast_np(rng.standard_normal((B * G, S, R)).astype(np.float32), dtype)
    vlens = rng.integers(0, R + 1, size=(B * G, S)).astype(np.int32)
    kb = cast_np(np.stack([random_orthogonal(R, rng).T for _ in range(G)]).astype(np.float32), dtype)
    vb = cast_np(np.stack([random_orthogonal(R, rng).T for _ in range(G)]).astype(np.float32), dtype)
    q = cast_np(rng.standard_normal((B, Hq, S, 128)).astype(np.float32), dtype)
    t = lambda a, dt=dtype: torch.from_numpy(a).to(device=dev, dtype=dt)  # noqa: E731
    cache = CustomDynamicCache()
    cache.update_sp(t(coef), t(lens, torch.int32), t(vcoef), t(vlens, torch.int32), R, 0, R)
    got = compressed_prefill_attention(t(q), cache, 0, t(kb), t(vb), theta=theta,
                                       out_dtype=torch.float32)
    torch.cuda.synchronize()
    # oracle: zero-padded coefficients, projection rounded to dtype, RoPE rounded, attention
    keep_k = np.arange(R)[None, None, :] < lens[..., None]
    keep_v = np.arange(R)[None, None, :] < vlens[..., None]
    ck = (coef * keep_k).reshape(B, G, S, R)
    cv = (vcoef * keep_v).reshape(B, G, S, R)
    nd = NP_OF[dtype]
    K = np.stack([P.reconstruct(ck[:, g], kb[g], nd) for g in range(G)], axis=1)
    V = np.stack([P.reconstruct(cv[:, g], vb[g], nd) for g in range(G)], axis=1)
    K = P.rope_dense(K, theta, nd)
    ref = P.attention(q, K, V, causal=True)
    assert_close(got.float(), ref, f"compressed prefill {dtype}")


def _oracle_heads(q, k, v, picks, scale=None):
    """The oracle for sampled (b, h) pairs only: (len(picks), Sq, D)."""
    Hq, Hkv = q.shape[1], k.shape[1]
    out = []
    for b, h in picks:
        kv = h // (Hq // Hkv)
        out.append(P.attention(q[b:b + 1, h:h + 1], k[b:b + 1, kv:kv + 1],
                               v[b:b + 1, kv:kv + 1], causal=True, scale=scale)[0, 0])
    return np.stack(out)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scores", ["normal", "wide_rising"])
def test_prefill_attention_bench_shape(dev, dtype, scores):
    """The shape bench times (B=4, S=2048, 32 query / 8 KV heads, causal) against the oracle on
    sampled (b, h) pairs spread over the batch rows, KV heads and query slots of a group (one
    per XCD-balanced work unit class). "wide_rising": keys whose norm grows with the position
    and queries scaled by 3, so later tiles' maxima exceed the running one by more than the
    2^8 the kernel defers its rescale by -- the rescale path runs for most query blocks, and
    peaked rows check P's hi + lo split at large values."""
    print(f"[gpu] prefill attention bench shape {dtype} {scores}", flush=True)
    B, Hq, Hkv, S = 4, 32, 8, 2048
    rng = np.random.default_rng(2048 + (scores == "wide_rising"))
    q = rng.standard_normal((B, Hq, S, 128)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, S, 128)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, 128)).astype(np.float32)
    if scores == "wide_rising":
        q *= 3.0
        k *= (1.0 + 3.0 * np.arange(S, dtype=np.float32) / S)[None, None, :, None]
    q, k, v = cast_np(q, dtype), cast_np(k, dtype), cast_np(v, dtype)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    got = prefill_attention(t(q), t(k), t(v), causal=True, out_dtype=torch.float32)
    low = prefill_attention(t(q), t(k), t(v), causal=True)
    torch.cuda.synchronize()
    picks = [(0, 0), (1, 13), (2, 22), (3, 31), (3, 4), (0, 27)]
    ref = _oracle_heads(q, k, v, picks)
    g = torch.stack([got[b, h] for b, h in picks])
    assert_close(g, ref, f"bench shape {dtype} {scores}")
    assert torch.equal(low, got.to(dtype))
    assert torch.isfinite(got).all()


def _random_prefill(i: int):
    """Case i of a seeded sweep over prefill attention: KV heads and query heads per KV head,
    batch, key length (1 to 1500, log-uniform), a prompt (Sq = Sk) or a chunk of the last Sq
    positions, causal or not, left padding (kstart) on some causal cases, dtype and scale."""
    rng = np.random.default_rng(8000 + i)
    Hkv = int(rng.choice([1, 2, 4, 8]))
    Hq = Hkv * int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 4))
    Sk = int(np.exp(rng.uniform(0, np.log(1500))))
    Sq = Sk if rng.random() < 0.6 else int(rng.integers(1, Sk + 1))
    while B * Hq * Sq * Sk > 1.5e7:  # keeps the float64 oracle to about a second
        Sq = max(1, Sq // 2)
    causal = bool(rng.random() < 0.8)
    kstart = [int(rng.integers(0, Sk + 1)) for _ in range(B)] if causal and rng.random() < 0.4 \
        else None
    dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float16
    scale = None if rng.random() < 0.7 else float(rng.uniform(0.01, 0.3))
    return B, Hq, Hkv, Sq, Sk, causal, kstart, dtype, scale


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(16))
def test_random_prefill_shapes_against_oracle(dev, i):
    B, Hq, Hkv, Sq, Sk, causal, kstart, dtype, scale = _random_prefill(i)
    print(f"[gpu] prefill attention random {i}: B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} "
          f"causal={causal} kstart={kstart} {dtype} scale={scale}", flush=True)
    rng = np.random.default_rng(9000 + i)
    q = cast_np(rng.standard_normal((B, Hq, Sq, 128)).astype(np.float32), dtype)
    k = cast_np(rng.standard_normal((B, Hkv, Sk, 128)).astype(np.float32), dtype)
    v = cast_np(rng.standard_normal((B, Hkv, Sk, 128)).astype(np.float32), dtype)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    ks = None if kstart is None else torch.tensor(kstart, dtype=torch.int32, device=dev)
    got = prefill_attention(t(q), t(k), t(v), causal=causal, scale=scale,
                            out_dtype=torch.float32, kstart=ks)
    low = prefill_attention(t(q), t(k), t(v), causal=causal, scale=scale, kstart=ks)
    torch.cuda.synchronize()
    ref = P.attention(q, k, v, causal=causal, scale=scale, kstart=kstart)
    assert_close(got, ref, f"prefill random {i}")
    assert torch.equal(low, got.to(dtype))
