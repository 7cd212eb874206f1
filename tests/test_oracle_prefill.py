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
