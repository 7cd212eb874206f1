"""Pins the prefill-attention oracle (oracle/prefill.py) against closed forms, RoPE identities and
torch's own scaled_dot_product_attention (float64, CPU)."""
import numpy as np
import pytest
import torch

from oracle import prefill as P


def test_single_key_returns_its_value():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 4, 1, 128))
    k = rng.standard_normal((1, 1, 1, 128))
    v = rng.standard_normal((1, 1, 1, 128))
    out = P.attention(q, k, v)
    assert np.allclose(out, np.broadcast_to(v, out.shape))


def test_zero_query_gives_causal_prefix_means():
    rng = np.random.default_rng(1)
    S = 9
    v = rng.standard_normal((1, 1, S, 128))
    out = P.attention(np.zeros((1, 2, S, 128)), rng.standard_normal((1, 1, S, 128)), v)
    means = np.cumsum(v[0, 0], axis=0) / np.arange(1, S + 1)[:, None]
    assert np.allclose(out[0, 0], means) and np.allclose(out[0, 1], means)


@pytest.mark.parametrize("causal,Sq,Sk", [(True, 12, 12), (True, 5, 12), (False, 7, 10)])
def test_matches_torch_sdpa(causal, Sq, Sk):
    rng = np.random.default_rng(2)
    B, Hq, Hkv, D = 2, 8, 2, 128
    q = rng.standard_normal((B, Hq, Sq, D))
    k = rng.standard_normal((B, Hkv, Sk, D))
    v = rng.standard_normal((B, Hkv, Sk, D))
    out = P.attention(q, k, v, causal=causal)
    kt = torch.from_numpy(k).repeat_interleave(Hq // Hkv, dim=1)
    vt = torch.from_numpy(v).repeat_interleave(Hq // Hkv, dim=1)
    mask = None
    if causal:  # queries at the last Sq positions
        mask = torch.ones(Sq, Sk, dtype=torch.bool).tril(diagonal=Sk - Sq)
    ref = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q), kt, vt,
                                                           attn_mask=mask)
    assert np.allclose(out, ref.numpy(), atol=1e-10)


def test_rope_dense_identities():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 6, 128))
    y = P.rope_dense(x, 500000.0, "float32")
    # position 0 is the identity; rotations keep each (i, i+64) pair's norm
    assert np.allclose(y[0, 0], x[0, 0], atol=1e-6)
    nx = x[..., :64] ** 2 + x[..., 64:] ** 2
    ny = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert np.allclose(nx, ny, rtol=1e-5)
    # relative positions: <R_m a, R_n b> depends on m - n only (positions 2,5 vs 10,13)
    a = rng.standard_normal(128)
    b = rng.standard_normal(128)
    A = P.rope_dense(np.stack([a] * 14)[None], 10000.0, "float32")[0]
    B = P.rope_dense(np.stack([b] * 14)[None], 10000.0, "float32")[0]
    assert abs(A[2] @ B[5] - A[10] @ B[13]) < 1e-3


def test_reconstruct_is_the_projection():
    rng = np.random.default_rng(4)
    c = rng.standard_normal((3, 5, 16))
    U = rng.standard_normal((16, 128))
    assert np.allclose(P.reconstruct(c, U, "float32"), (c @ U).astype(np.float32), rtol=1e-6)


def test_left_padding_closed_forms():
    """kstart[b]: keys before it are masked. kstart 0 is the plain causal attention; a query at
    the first real position attends only that key (its value comes back); queries before it have
    no key left and give 0."""
    rng = np.random.default_rng(5)
    B, Hq, Hkv, S, D = 2, 4, 2, 10, 128
    q = rng.standard_normal((B, Hq, S, D))
    k = rng.standard_normal((B, Hkv, S, D))
    v = rng.standard_normal((B, Hkv, S, D))
    assert np.array_equal(P.attention(q, k, v, kstart=[0, 0]), P.attention(q, k, v))
    out = P.attention(q, k, v, kstart=[3, 0])
    assert np.array_equal(out[0, :, :3], np.zeros((Hq, 3, D)))
    for h in range(Hq):
        assert np.allclose(out[0, h, 3], v[0, h // 2, 3])
    assert np.allclose(out[1], P.attention(q, k, v)[1])
    # every key masked: all zeros
    assert not np.any(P.attention(q, k, v, kstart=[S, S]))


@pytest.mark.parametrize("Sq", [10, 4])
def test_left_padding_matches_torch_sdpa(Sq):
    """Real queries (at or past each row's first real key) against torch SDPA in float64 with
    the padding and causal masks built as one boolean mask."""
    rng = np.random.default_rng(6)
    B, Hq, Hkv, Sk, D = 3, 4, 2, 10, 128
    kstart = [2, 0, 5]
    q = rng.standard_normal((B, Hq, Sq, D))
    k = rng.standard_normal((B, Hkv, Sk, D))
    v = rng.standard_normal((B, Hkv, Sk, D))
    out = P.attention(q, k, v, kstart=kstart)
    kt = torch.from_numpy(k).repeat_interleave(Hq // Hkv, dim=1)
    vt = torch.from_numpy(v).repeat_interleave(Hq // Hkv, dim=1)
    qpos = torch.arange(Sk - Sq, Sk)
    for b in range(B):
        keys = torch.arange(Sk)
        mask = (keys[None, :] <= qpos[:, None]) & (keys[None, :] >= kstart[b])
        live = mask.any(dim=1)
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[b:b + 1, :, live]), kt[b:b + 1], vt[b:b + 1],
            attn_mask=mask[live])
        assert np.allclose(out[b][:, live.numpy()], ref[0].numpy(), atol=1e-10)
        assert not np.any(out[b][:, ~live.numpy()])
