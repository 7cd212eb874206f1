"""Reference-semantics vector kernels (abx_sparse, avx, fused with an fp32 cache, and the joint
R=1024 layout the reference ships) against the oracle."""
import math

import numpy as np
import pytest
import torch

from dynakv_amd.kernels.fused import fused_attention_dispatch
from dynakv_amd.kernels.router import compressed_decode_attention
from dynakv_amd.kernels.two_stage import abx_sparse, avx
from dynakv_amd.synthetic import make_case
from oracle import attention as A
from oracle.packing import pack_rows

from helpers import NP_OF, assert_close, cast_np, packed_from_case


def _joint_case(B, S, R, n_basis, Hq=32, Dh=128, dtype=torch.bfloat16, seed=0, len_lo=0):
    """Reference joint layout: one packed row per batch element, per-token r in [len_lo, R]."""
    rng = np.random.default_rng(seed)
    coef_k = cast_np(rng.standard_normal((B, S, R)), dtype)
    coef_v = cast_np(rng.standard_normal((B, S, R)), dtype)
    lk = rng.integers(len_lo, R + 1, size=(B, S)).astype(np.int32)
    lv = rng.integers(len_lo, R + 1, size=(B, S)).astype(np.int32)
    fk, lk, ok, _ = pack_rows(coef_k, lk, R)
    fv, lv, ov, _ = pack_rows(coef_v, lv, R)
    kb = cast_np(rng.standard_normal((n_basis, R, Dh)) / math.sqrt(R), dtype)
    vb = cast_np(rng.standard_normal((n_basis, R, Dh)) / math.sqrt(R), dtype)
    q = cast_np(rng.standard_normal((B, Hq, Dh)), dtype)
    return dict(q=q, fk=fk, lk=lk, ok=ok, fv=fv, lv=lv, ov=ov, kb=kb, vb=vb)


def _dev(h, dev, dtype):
    t = lambda x, dt=dtype: torch.from_numpy(np.ascontiguousarray(x)).to(dev, dt)  # noqa: E731
    return dict(q=t(h["q"]), fk=t(h["fk"]), fv=t(h["fv"]), kb=t(h["kb"]), vb=t(h["vb"]),
                lk=t(h["lk"], torch.int32), ok=t(h["ok"], torch.int32),
                lv=t(h["lv"], torch.int32), ov=t(h["ov"], torch.int32))


ULP_REL = {torch.float32: 1e-5, torch.float16: 2 ** -9, torch.bfloat16: 2 ** -7}


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("R,n_basis", [(1024, 8), (128, 32), (100, 4)])
def test_abx_sparse_matches_oracle(dev, dtype, R, n_basis):
    print(f"[gpu] abx_sparse dtype={dtype} R={R} n_basis={n_basis}", flush=True)
    h = _joint_case(2, 45, R, n_basis, dtype=dtype, seed=R + n_basis)
    d = _dev(h, dev, dtype)
    theta = 500000.0
    got = abx_sparse(d["q"], d["kb"], d["fk"], d["lk"], offsets=d["ok"], theta=theta)
    assert got.dtype == dtype and got.shape == (2, 32, 45)
    ref = A.scores_two_stage(h["q"], h["fk"], h["kb"], h["lk"], h["ok"], theta, NP_OF[dtype])
    g = got.float().cpu().numpy()
    # same rounding target; allow two units in the last place of the output dtype
    tol = 2 * ULP_REL[dtype] * np.abs(ref) + 1e-4
    assert (np.abs(g - ref) <= tol).all(), float(np.abs(g - ref).max())
    masked = h["lk"] == 0
    if masked.any():
        np.testing.assert_array_equal(g[:, :, :][np.broadcast_to(masked[:, None, :], g.shape)],
                                      ref[np.broadcast_to(masked[:, None, :], ref.shape)])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("R,n_basis", [(1024, 8), (128, 32)])
def test_avx_matches_oracle(dev, dtype, R, n_basis):
    print(f"[gpu] avx dtype={dtype} R={R} n_basis={n_basis}", flush=True)
    h = _joint_case(2, 300, R, n_basis, dtype=dtype, seed=3 + R)
    d = _dev(h, dev, dtype)
    sc = cast_np(np.random.default_rng(5).standard_normal((2, 32, 300)) * 2, dtype)
    got = avx(torch.from_numpy(sc).to(dev, dtype), d["fv"], d["vb"], d["lv"], offsets=d["ov"])
    ref = A.av_two_stage(sc, h["fv"], h["vb"], h["lv"], h["ov"], clamp=True)
    assert_close(got, ref, f"avx {dtype}")


@pytest.mark.gpu
def test_config1_fp32_fused_per_group(dev):
    """Config 1: B=1, 32/8 heads, S=257, fp32, per-KV-head 128x128 bases, r ~ U{8..128};
    one fused_attention_dispatch call per KV group with the group's basis expanded to its 4
    heads (the per-head mapping of the reference call)."""
    print("[gpu] config1 fp32 fused", flush=True)
    case = make_case(B=1, G=8, Hq=32, S=257, uniform=(8, 128), seed=1)
    p = packed_from_case(case, torch.float32, dev)
    h = p["host"]
    outs = []
    for g in range(8):
        q = p["q"][:, 4 * g: 4 * g + 4, None, :]
        kb = p["k_basis"][g: g + 1].expand(4, 128, 128)
        vb = p["v_basis"][g: g + 1].expand(4, 128, 128)
        outs.append(fused_attention_dispatch(
            q, p["k_flat"][g: g + 1], kb, p["v_flat"][g: g + 1], vb,
            p["lens_k"][g: g + 1], p["offs_k"][g: g + 1],
            p["lens_v"][g: g + 1], p["offs_v"][g: g + 1], case.theta))
    got = torch.cat(outs, dim=1)
    from helpers import oracle_grouped
    ref = oracle_grouped(case, h, "short_fused", "float32")
    assert_close(got, ref, "config1 fp32", tol_abs=1e-4, tol_rel=1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("S", [60, 500])
def test_joint_layout_router_both_routes(dev, S):
    """The reference's shipped layout: joint R=1024, k_up (32, 1024, 128) repeat-interleaved from
    8 KV-head bases; the router picks fused below 500 tokens and two-stage at 500."""
    print(f"[gpu] joint layout router S={S}", flush=True)
    dtype = torch.bfloat16
    h = _joint_case(2, S, 1024, 8, dtype=dtype, seed=S, len_lo=1)
    d = _dev(h, dev, dtype)
    k_up = d["kb"].repeat_interleave(4, dim=0).contiguous()
    v_up = d["vb"].repeat_interleave(4, dim=0).contiguous()
    got = compressed_decode_attention(
        q=d["q"][:, :, None, :], k_flat=d["fk"], k_up=k_up, v_flat=d["fv"], v_up=v_up,
        key_lengths=d["lk"], key_offsets=d["ok"], value_lengths=d["lv"], value_offsets=d["ov"],
        theta=500000.0, cache_length=S)
    route = "short_fused" if S < 500 else "long_two_stage"
    kup = np.repeat(h["kb"], 4, axis=0)
    vup = np.repeat(h["vb"], 4, axis=0)
    ref = A.decode_attention(h["q"], h["fk"], kup, h["fv"], vup, h["lk"], h["ok"], h["lv"],
                             h["ov"], 500000.0, route=route, q_dtype="bfloat16")
    assert_close(got, ref, f"joint S={S}")
