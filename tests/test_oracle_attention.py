"""Pins the attention oracle (oracle/attention.py) on CPU: agreement with the independent
masked-dimension formulation (oracle/masked_dim.py), closed forms, and brute force."""
import math

import numpy as np
import pytest
import torch

from dynakv_amd.synthetic import make_case
from oracle import attention as A
from oracle import masked_dim as M
from oracle.packing import pack_rows


def _pack(case):
    fk, lk, ok, _ = pack_rows(case.k_coef, case.k_len, case.R)
    fv, lv, ov, _ = pack_rows(case.v_coef, case.v_len, case.R)
    return fk, lk, ok, fv, lv, ov


def _oracle_grouped(case, route="short_fused", q_dtype="float32"):
    fk, lk, ok, fv, lv, ov = _pack(case)
    hpg = case.Hq // case.G
    return A.decode_attention(case.q, fk, case.k_basis, fv, case.v_basis, lk, ok, lv, ov,
                              case.theta, route=route, q_dtype=q_dtype,
                              row_of=lambda b, h: b * case.G + h // hpg,
                              basis_of=lambda h: h // hpg)


@pytest.mark.parametrize("seed,S,G,Hq", [(0, 37, 2, 8), (1, 200, 4, 8), (2, 5, 1, 4)])
def test_packed_oracle_matches_masked_dim(seed, S, G, Hq):
    case = make_case(B=2, G=G, Hq=Hq, S=S, uniform=(1, 128), seed=seed)
    ref = _oracle_grouped(case)
    # dense masked joint coefficients: (B, S, G*R), block-diagonal joint basis
    B, R = case.B, case.R
    def dense(coef, L):
        d = np.zeros((B, S, G * R), np.float32)
        for b in range(B):
            for g in range(G):
                for s in range(S):
                    n = L[b * G + g, s]
                    d[b, s, g * R: g * R + n] = coef[b * G + g, s, :n]
        return torch.from_numpy(d)
    ck, cv = dense(case.k_coef, case.k_len), dense(case.v_coef, case.v_len)
    Uk = M.block_diag_up(torch.from_numpy(case.k_basis))
    Uv = M.block_diag_up(torch.from_numpy(case.v_basis))
    got = M.decode_attention(torch.from_numpy(case.q), ck, cv, Uk, Uv, G, case.theta).numpy()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 2e-5, err


def test_single_token_returns_its_value():
    case = make_case(B=1, G=1, Hq=2, S=1, uniform=(1, 128), seed=3)
    out = _oracle_grouped(case)
    n = case.v_len[0, 0]
    v0 = case.v_coef[0, 0, :n].astype(np.float64) @ case.v_basis[0, :n].astype(np.float64)
    np.testing.assert_allclose(out[0, 0], v0, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(out[0, 1], v0, rtol=1e-10, atol=1e-10)


def test_zero_query_gives_mean_value():
    case = make_case(B=1, G=1, Hq=1, S=9, uniform=(1, 128), seed=4)
    case.q[:] = 0
    out = _oracle_grouped(case)
    V = np.stack([case.v_coef[0, s, : case.v_len[0, s]].astype(np.float64)
                  @ case.v_basis[0, : case.v_len[0, s]].astype(np.float64) for s in range(9)])
    np.testing.assert_allclose(out[0, 0], V.mean(0), rtol=1e-10, atol=1e-12)


def test_identity_basis_at_position_zero_is_plain_attention():
    # one token at position 0: no rotation; out = v. Two tokens with identical K at positions 0
    # and 1 differ only by the rotation of position 1: check the score against a hand rotation.
    Dh = 8
    theta = 10000.0
    k = np.arange(1, Dh + 1, dtype=np.float64)
    cos, sin = A.rope_cos_sin(np.array([1]), Dh, theta)
    h = Dh // 2
    rot = np.concatenate([k[:h] * cos[0] - k[h:] * sin[0], k[h:] * cos[0] + k[:h] * sin[0]])
    inv = [math.exp(-(2 * i / Dh) * math.log(theta)) for i in range(h)]
    hand = np.array([k[i] * math.cos(inv[i]) - k[i + h] * math.sin(inv[i]) for i in range(h)] +
                    [k[i + h] * math.cos(inv[i]) + k[i] * math.sin(inv[i]) for i in range(h)])
    np.testing.assert_allclose(rot, hand, rtol=1e-6)
    # the oracle with an identity basis, Dh=8
    q = np.random.default_rng(0).standard_normal((1, 1, Dh)).astype(np.float32)
    flat = np.concatenate([k, k]).astype(np.float32)[None, :]
    lens = np.array([[Dh, Dh]], np.int32)
    offs = np.array([[0, Dh]], np.int32)
    I = np.eye(Dh, dtype=np.float32)[None]
    vflat = np.concatenate([np.ones(Dh), 2 * np.ones(Dh)]).astype(np.float32)[None, :]
    out = A.decode_attention(q, flat, I, vflat, I, lens, offs, lens, offs, theta)
    z = np.array([q[0, 0] @ k, q[0, 0] @ rot]) / math.sqrt(Dh)
    p = np.exp(z - z.max())
    p /= p.sum()
    np.testing.assert_allclose(out[0, 0], (p[0] * 1 + p[1] * 2) * np.ones(Dh), rtol=1e-6)


def test_rope_preserves_norm_and_first_pair_angle():
    cos, sin = A.rope_cos_sin(np.arange(50), 128, 500000.0)
    k = np.random.default_rng(1).standard_normal((50, 128))
    kr = A.apply_rope(k, cos, sin)
    np.testing.assert_allclose(np.linalg.norm(kr, axis=1), np.linalg.norm(k, axis=1), rtol=1e-12)
    # inv_freq_0 = 1: the (0, 64) pair rotates by exactly the position
    np.testing.assert_allclose(cos[:, 0], np.cos(np.arange(50)), atol=1e-6)
    np.testing.assert_allclose(sin[:, 0], np.sin(np.arange(50)), atol=1e-6)


def test_brute_force_scalar_loops():
    case = make_case(B=1, G=2, Hq=4, S=6, R=16, Dh=8, uniform=(0, 16), seed=7)
    case.k_len[:, 0] = np.maximum(case.k_len[:, 0], 1)
    out = _oracle_grouped(case)
    inv = A.inv_freq_f32(8, case.theta)
    for h in range(4):
        g = h // 2
        zs, vs = [], []
        for s in range(6):
            rk, rv = case.k_len[g, s], case.v_len[g, s]
            k = [sum(float(case.k_coef[g, s, j]) * float(case.k_basis[g, j, d]) for j in range(rk))
                 for d in range(8)]
            ang = [float(np.float32(s) * inv[i]) for i in range(4)]
            kr = [k[i] * math.cos(ang[i]) - k[i + 4] * math.sin(ang[i]) for i in range(4)] + \
                 [k[i + 4] * math.cos(ang[i]) + k[i] * math.sin(ang[i]) for i in range(4)]
            dot = sum(float(case.q[0, h, d]) * kr[d] for d in range(8))
            # the reference scales by 1/sqrt(Dh) evaluated in fp32 (fused.py:58)
            zs.append(dot * float(np.float32(1) / np.sqrt(np.float32(8))) if rk > 0 else -math.inf)
            vs.append([sum(float(case.v_coef[g, s, j]) * float(case.v_basis[g, j, d])
                           for j in range(rv)) for d in range(8)])
        m = max(z for z in zs if z != -math.inf)
        p = [math.exp(z - m) if z != -math.inf else 0.0 for z in zs]
        o = [sum(p[s] * vs[s][d] for s in range(6)) / sum(p) for d in range(8)]
        np.testing.assert_allclose(out[0, h], o, rtol=1e-9, atol=1e-12)


def test_routes_agree_in_fp32_without_empty_tokens():
    case = make_case(B=1, G=2, Hq=8, S=40, uniform=(1, 128), seed=8)
    a = _oracle_grouped(case, "short_fused")
    b = _oracle_grouped(case, "long_two_stage", "float32")
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)


def test_two_stage_rounds_scores_to_query_dtype():
    case = make_case(B=1, G=1, Hq=4, S=30, uniform=(1, 128), seed=9)
    a = _oracle_grouped(case, "long_two_stage", "float32")
    b = _oracle_grouped(case, "long_two_stage", "bfloat16")
    d = np.abs(a - b).max()
    assert 1e-6 < d < 5e-2  # rounding is applied, and only perturbs


def test_empty_keys_route_semantics():
    case = make_case(B=1, G=1, Hq=2, S=5, uniform=(1, 128), seed=10)
    case.k_len[:] = 0
    fused = _oracle_grouped(case, "short_fused")
    assert np.isnan(fused).all()
    two = _oracle_grouped(case, "long_two_stage", "bfloat16")
    # every score is round(-1e4/sqrt(128)): equal weights -> mean of V (two_stage.py:153-157)
    V = np.stack([case.v_coef[0, s, : case.v_len[0, s]].astype(np.float64)
                  @ case.v_basis[0, : case.v_len[0, s]].astype(np.float64) for s in range(5)])
    np.testing.assert_allclose(two[0, 0], V.mean(0), rtol=1e-9, atol=1e-12)


def test_zero_length_value_counts_in_denominator():
    case = make_case(B=1, G=1, Hq=1, S=2, uniform=(1, 128), seed=11)
    case.q[:] = 0
    case.v_len[0, 1] = 0
    out = _oracle_grouped(case)
    v0 = (case.v_coef[0, 0, : case.v_len[0, 0]].astype(np.float64)
          @ case.v_basis[0, : case.v_len[0, 0]].astype(np.float64))
    np.testing.assert_allclose(out[0, 0], v0 / 2, rtol=1e-10, atol=1e-12)


def test_two_stage_split_functions_compose():
    case = make_case(B=1, G=1, Hq=4, S=25, uniform=(0, 128), seed=12)
    fk, lk, ok, fv, lv, ov = _pack(case)
    sc = A.scores_two_stage(case.q, fk, case.k_basis, lk, ok, case.theta, "float16")
    av = A.av_two_stage(sc, fv, case.v_basis, lv, ov)
    full = A.decode_attention(case.q, fk, case.k_basis, fv, case.v_basis, lk, ok, lv, ov,
                              case.theta, route="long_two_stage", q_dtype="float16")
    np.testing.assert_allclose(av, full, rtol=1e-9, atol=1e-12)


def test_round_bf16_known_values():
    x = np.array([1.0, 1.00390625, 1.005859375, -3.0e-3, 65504.0], np.float32)
    r = A.round_bf16(x)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 1.5*2^-8 -> 1 + 2^-7
    assert r[0] == 1.0 and r[1] == 1.0 and r[2] == np.float32(1.0078125)
    assert abs(r[3] - x[3]) <= abs(x[3]) * 2 ** -8
    assert r[4] == 65536.0


def test_gather_padded_matches_loop():
    rng = np.random.default_rng(13)
    flat = rng.standard_normal(500)
    lens = rng.integers(0, 40, size=20)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]])
    X = A.gather_padded(flat, lens, offs, 32)
    for s in range(20):
        n = min(lens[s], 32)
        np.testing.assert_array_equal(X[s, :n], flat[offs[s]: offs[s] + n])
        assert not X[s, n:].any()
