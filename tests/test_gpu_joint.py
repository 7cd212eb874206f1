"""The joint-layout MFMA kernels (dkv_joint_scores / dkv_joint_av, dynakv_amd/kernels/joint.py)
against the vector kernels of the same semantics (dkv_scores / dkv_av, themselves checked against
the oracle in test_gpu_generic.py) and against the oracle directly.

Reference: abx_sparse / avx (two_stage.py:48-324) and the fused route (fused.py:28-170) on the
reference's shipped layout: one packed row per batch element, ranks up to 1024, k_up / v_up
repeated over query heads. Cases cover every rank chunk count (token counts 0..R), token counts
not a multiple of the 512-token scores block or the 16-token V tile, a packed buffer that ends
exactly at the last coefficient (the last window read past the end), repeated and distinct
bases (1, 4 and 8 query heads per basis), fp16 and bf16.
"""
import math

import numpy as np
import pytest
import torch

from dynakv_amd import _lib
from dynakv_amd.kernels import joint as J
from oracle import attention as A
from oracle.packing import pack_rows

from helpers import assert_close, cast_np

THETA = 500000.0


def _case(B, S, R, n_basis, Hq=32, dtype=torch.bfloat16, seed=0, len_lo=0, exact_end=False):
    rng = np.random.default_rng(seed)
    coef_k = cast_np(rng.standard_normal((B, S, R)), dtype)
    coef_v = cast_np(rng.standard_normal((B, S, R)), dtype)
    lk = rng.integers(len_lo, R + 1, size=(B, S)).astype(np.int32)
    lv = rng.integers(len_lo, R + 1, size=(B, S)).astype(np.int32)
    if S > 2:
        lk[:, 0], lk[:, 1], lv[:, 0], lv[:, 1] = R, 0, 0, R
    if exact_end:  # the longest rows last, so the buffer can end at the last row's last value
        lk = lk[np.argsort(lk.sum(1), kind="stable")]
        lv = lv[np.argsort(lv.sum(1), kind="stable")]
    fk, lk, ok, _ = pack_rows(coef_k, lk, R)
    fv, lv, ov, _ = pack_rows(coef_v, lv, R)
    if exact_end:
        fk = np.ascontiguousarray(fk[:, : int(lk[-1].sum())])
        fv = np.ascontiguousarray(fv[:, : int(lv[-1].sum())])
    kb = cast_np(rng.standard_normal((n_basis, R, 128)) / math.sqrt(R), dtype)
    vb = cast_np(rng.standard_normal((n_basis, R, 128)) / math.sqrt(R), dtype)
    q = cast_np(rng.standard_normal((B, Hq, 128)), dtype)
    return dict(q=q, fk=fk, lk=lk, ok=ok, fv=fv, lv=lv, ov=ov, kb=kb, vb=vb)


def _dev(h, dev, dtype):
    t = lambda x, dt=dtype: torch.from_numpy(np.ascontiguousarray(x)).to(dev, dt)  # noqa: E731
    return {k: t(v, torch.int32 if k in ("lk", "ok", "lv", "ov") else dtype) for k, v in h.items()}


def _generic_scores(d, k_up, mode, out_dtype):
    q = d["q"]
    B, Hq, _ = q.shape
    S = d["lk"].shape[1]
    out = torch.empty((B, Hq, S), dtype=out_dtype, device=q.device)
    rc = _lib.load().dkv_scores(
        _lib.stream_of(q), mode, _lib.dtype_code(q.dtype), _lib.dtype_code(d["fk"].dtype),
        _lib.dtype_code(out_dtype), q.data_ptr(), q.stride(0), q.stride(1),
        k_up.data_ptr(), k_up.stride(0), k_up.stride(1), k_up.shape[0],
        d["fk"].data_ptr(), d["fk"].stride(0),
        d["lk"].data_ptr(), d["lk"].stride(0), d["lk"].stride(1),
        d["ok"].data_ptr(), d["ok"].stride(0), d["ok"].stride(1),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        B, Hq, S, k_up.shape[1], 128, math.log(THETA))
    _lib.check(rc, "dkv_scores")
    return out


def _generic_av(sc, d, v_up, mode, out_dtype):
    B, Hq, S = sc.shape
    out = torch.empty((B, Hq, 128), dtype=out_dtype, device=sc.device)
    rc = _lib.load().dkv_av(
        _lib.stream_of(sc), mode, _lib.dtype_code(sc.dtype), _lib.dtype_code(d["fv"].dtype),
        _lib.dtype_code(out_dtype), sc.data_ptr(), sc.stride(0), sc.stride(1), sc.stride(2),
        v_up.data_ptr(), v_up.stride(0), v_up.stride(1), v_up.shape[0],
        d["fv"].data_ptr(), d["fv"].stride(0),
        d["lv"].data_ptr(), d["lv"].stride(0), d["lv"].stride(1),
        d["ov"].data_ptr(), d["ov"].stride(0), d["ov"].stride(1),
        out.data_ptr(), out.stride(0), out.stride(1), B, Hq, S, v_up.shape[1], 128)
    _lib.check(rc, "dkv_av")
    return out


ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,S,R,n_basis,repeat,Hq", [
    (2, 777, 1024, 8, 4, 32),   # the reference's repeated k_up (32 bases -> 8 distinct)
    (3, 513, 512, 4, 1, 32),    # 8 query heads per basis
    (1, 40, 32, 32, 1, 32),     # one rank chunk, one query head per basis
    (2, 1100, 1024, 8, 1, 32),  # 4 query heads per basis, blocks of 256 tokens x 2 bases
    (2, 700, 256, 3, 1, 12),    # an odd number of bases: one basis per workgroup
    (1, 300, 512, 1, 1, 8),     # a single basis for 8 query heads
])
def test_scores_match_vector_kernel(dev, dtype, B, S, R, n_basis, repeat, Hq):
    print(f"[gpu] joint scores {dtype} B={B} S={S} R={R} nb={n_basis} rep={repeat} Hq={Hq}",
          flush=True)
    h = _case(B, S, R, n_basis, Hq=Hq, dtype=dtype, seed=S + R, exact_end=True)
    d = _dev(h, dev, dtype)
    k_up = d["kb"].repeat_interleave(repeat, dim=0).contiguous() if repeat > 1 else d["kb"]
    for mode, odt in ((0, dtype), (1, torch.float32)):
        got = J.joint_scores(d["q"], k_up, d["fk"], d["lk"], d["ok"], theta=THETA, mode=mode,
                             out_dtype=odt)
        ref = _generic_scores(d, k_up, mode, odt)
        g, r = got.float(), ref.float()
        fin = torch.isfinite(r)
        assert torch.equal(torch.isfinite(g), fin)
        err = (g[fin] - r[fin]).abs()
        # fp32-faithful K' and products: mode 0 results are the same rounding target (allow two
        # units in the last place), mode 1 agrees to fp32 accumulation-order differences
        tol = (2 * ULP[dtype] * r[fin].abs() + 1e-4) if mode == 0 else (1e-4 * r[fin].abs() + 1e-4)
        print(f"[parity] scores mode {mode}: max_abs={err.max().item():.3e}", flush=True)
        assert (err <= tol).all(), float(err.max())
        masked = d["lk"] == 0
        if mode == 0:
            assert torch.equal(g.masked_select(masked[:, None, :]), r.masked_select(masked[:, None, :]))


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,R,n_basis,Hq", [
    (1, 2049, 256, 2, 8),    # one token past the first window
    (2, 2348, 128, 4, 16),   # a partial second window
    (1, 4097, 64, 2, 8),     # a third window of one token
    (1, 1100, 1024, 1, 8),   # one basis per workgroup (512-token ranges), a 1536-position window
])
def test_scores_across_sort_windows(dev, B, S, R, n_basis, Hq):
    """The scores kernel takes its tokens ordered by chunk count within windows of up to 2048
    positions (joint_sort_kernel), pad entries filling each window's last range. Fused-route
    scores (fp32) against the float64 oracle at window edges: a token given the wrong slot,
    offset or position is off by O(1). The slack covers the rotation angle: the kernels compose
    R(16T) R(n) by angle addition from exact table rows, the reference rounds float32(p) *
    inv_freq once (half a unit in the last place of an angle below S rad, inv_freq <= 1), so
    each rotated pair moves by at most that angle times its norm."""
    print(f"[gpu] joint scores across sort windows B={B} S={S} R={R} nb={n_basis}", flush=True)
    dtype = torch.bfloat16
    h = _case(B, S, R, n_basis, Hq=Hq, dtype=dtype, seed=3 * S + R, exact_end=True)
    d = _dev(h, dev, dtype)
    got = J.joint_scores(d["q"], d["kb"], d["fk"], d["lk"], d["ok"], theta=THETA, mode=1,
                         out_dtype=torch.float32).double().cpu().numpy()
    ref = A.scores_two_stage(h["q"], h["fk"], h["kb"], h["lk"], h["ok"], THETA,
                             out_dtype="float32").astype(np.float64)
    lk = h["lk"]
    hpg = Hq // n_basis
    scale = 1.0 / math.sqrt(128.0)
    dang = S * 2.0 ** -24 + 2.0 ** -22
    qn = np.linalg.norm(np.asarray(h["q"], np.float64), axis=-1)  # (B, Hq)
    for b in range(B):
        Xk = A.gather_padded(np.asarray(h["fk"][b], np.float64), lk[b], h["ok"][b], R)
        for hb in range(n_basis):
            kn = np.linalg.norm(Xk @ np.asarray(h["kb"][hb], np.float64), axis=-1)  # (S,)
            for hh in range(hb * hpg, (hb + 1) * hpg):
                live = lk[b] > 0
                assert np.all(np.isneginf(got[b, hh, ~live]))
                g, r = got[b, hh, live], ref[b, hh, live]
                tol = 1e-4 * np.abs(r) + 1e-4 + dang * qn[b, hh] * kn[live] * scale
                err = np.abs(g - r)
                assert np.all(err <= tol), (b, hh, float(err.max()), float((err / tol).max()))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,S,R,n_basis,Hq", [
    (2, 1000, 1024, 8, 32), (1, 17, 1024, 32, 32), (3, 1, 256, 4, 32), (2, 300, 1024, 8, 32),
    (2, 50, 97, 2, 32),      # one partial rank block (97 ranks), two chunks of 8 heads per basis
    (1, 2048, 512, 8, 32),   # many token splits: the merge's many-splits path
    (2, 400, 256, 3, 12),    # one set of 16 query heads (12 used) per workgroup
    (2, 300, 1024, 8, 48),   # three sets of 16 query heads: one set per workgroup
    # batches that are not powers of two, split counts chosen by rounds of 256 workgroups:
    (3, 2048, 256, 4, 32),   # 64 splits of 32 tokens
    (12, 1000, 256, 8, 32),  # 21 splits of 48 tokens, the last one 40
    (5, 777, 128, 4, 16),    # one head set, 49 splits of 16 tokens, the last one 9
])
def test_av_matches_vector_kernel(dev, dtype, B, S, R, n_basis, Hq):
    print(f"[gpu] joint av {dtype} B={B} S={S} R={R} nb={n_basis} Hq={Hq}", flush=True)
    h = _case(B, S, R, n_basis, Hq=Hq, dtype=dtype, seed=7 * S + R, exact_end=True)
    d = _dev(h, dev, dtype)
    rng = np.random.default_rng(S)
    for mode in (0, 1):
        sdt = dtype if mode == 0 else torch.float32
        z = rng.standard_normal((B, Hq, S)) * 2
        if mode == 1:
            z[:, :, rng.random(S) < 0.3] = -np.inf  # the fused route's masked tokens
            z[:, :, 0] = 0.5
        sc = torch.from_numpy(cast_np(z, sdt)).to(dev, sdt)
        got = J.joint_av(sc, d["vb"], d["fv"], d["lv"], d["ov"], mode=mode, out_dtype=torch.float32)
        ref = _generic_av(sc, d, d["vb"], mode, torch.float32)
        # bf16 caches: P as bf16 hi + lo (fp32-faithful); fp16 caches: P in fp16 (2^-11 per term)
        ta = 2e-4 if dtype == torch.bfloat16 else 1e-3
        assert_close(got, ref.cpu().numpy(), f"av mode {mode}", tol_abs=ta, tol_rel=2e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("route", ["short_fused", "long_two_stage"])
def test_joint_attention_against_oracle(dev, route, dtype):
    """The router's joint path end to end against the oracle (two rows, 700 tokens)."""
    print(f"[gpu] joint attention {route} {dtype}", flush=True)
    h = _case(2, 700, 1024, 8, dtype=dtype, seed=11, len_lo=0)
    d = _dev(h, dev, dtype)
    k_up = d["kb"].repeat_interleave(4, dim=0).contiguous()
    v_up = d["vb"].repeat_interleave(4, dim=0).contiguous()
    rt = _lib.DKV_ROUTE_FUSED if route == "short_fused" else _lib.DKV_ROUTE_TWO_STAGE
    got = J.joint_attention(d["q"], d["fk"], k_up, d["fv"], v_up, d["lk"], d["ok"], d["lv"],
                            d["ov"], theta=THETA, route=rt)
    assert got is not None and got.dtype == dtype
    ref = A.decode_attention(h["q"], h["fk"], np.repeat(h["kb"], 4, axis=0), h["fv"],
                             np.repeat(h["vb"], 4, axis=0), h["lk"], h["ok"], h["lv"], h["ov"],
                             THETA, route=route,
                             q_dtype="bfloat16" if dtype == torch.bfloat16 else "float16")
    assert_close(got, ref, f"joint {route} {dtype}")


@pytest.mark.gpu
def test_distinct_basis_detection(dev):
    """A k_up repeated over query heads is reduced to its distinct bases (once per tensor and
    in-place version); a basis whose copies differ is kept whole."""
    kb = torch.randn(8, 64, 128, device=dev, dtype=torch.bfloat16)
    rep = kb.repeat_interleave(4, dim=0).contiguous()
    got = J._distinct(rep, 32)
    assert got.shape == (8, 64, 128) and torch.equal(got, kb)
    assert J._BASIS_CACHE[id(rep)][2] == 4
    rep[5, 0, 0] += 1  # in place: the copies differ now
    assert J._distinct(rep, 32).shape[0] == 32


def _pack_rows_dev(x: torch.Tensor, lens: torch.Tensor):
    """Packed rows of x (rows, S, R) keeping the first lens[row, t] values of each token:
    (flat (rows, cap), offs (rows, S)) with exclusive-prefix offsets, on the device."""
    rows, S, R = x.shape
    keep = torch.arange(R, device=x.device)[None, None, :] < lens[..., None]
    tot = lens.sum(dim=1)
    cap = int(tot.max().item()) + 8
    offs = torch.zeros_like(lens)
    offs[:, 1:] = torch.cumsum(lens, dim=1, dtype=torch.int32)[:, :-1]
    pos = torch.cumsum(keep.reshape(rows, -1), dim=1, dtype=torch.int32) - 1
    flat = torch.zeros((rows, cap), dtype=x.dtype, device=x.device)
    ridx = torch.arange(rows, device=x.device)[:, None].expand(rows, S * R)
    km = keep.reshape(rows, -1)
    flat[ridx[km], pos[km].long()] = x.reshape(rows, -1)[km]
    return flat, offs.contiguous()


@pytest.mark.gpu
@pytest.mark.parametrize("route", ["short_fused", "long_two_stage"])
def test_joint_matches_split_kernel_at_config3_shape(dev, route):
    """Size-independent cross-check at the config-3 shape (B=16, S=8192, 8 KV heads x rank 128,
    32 query heads, mean retention 0.29 with 5% full tokens, bf16): a per-head cache and the
    joint cache holding the same coefficients (token t's joint row is the heads' rows side by
    side, each padded with zeros to 128 ranks; the joint K/V bases block-diagonal) give the
    same attention, the per-head one through the split kernel (itself checked against the
    oracle) and the joint one through dkv_joint_scores / dkv_joint_av."""
    from dynakv_amd.kernels.decode import grouped_decode_attention
    from dynakv_amd.synthetic import device_lengths

    print(f"[gpu] joint vs split kernel at config 3, {route}", flush=True)
    B, S, G, R, Hq, dt = 16, 8192, 8, 128, 32, torch.bfloat16
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    lk = device_lengths(B * G, S, R, 0.29, gen, dev, 4, 0.05).view(B, G, S)
    lv = device_lengths(B * G, S, R, 0.29, gen, dev, 4, 0.05).view(B, G, S)
    ar = torch.arange(R, device=dev)
    xk = torch.randn((B, G, S, R), generator=gen, device=dev).to(dt) * (ar < lk[..., None])
    xv = torch.randn((B, G, S, R), generator=gen, device=dev).to(dt) * (ar < lv[..., None])

    def bases():
        a = torch.randn((G, R, R), generator=gen, device=dev)
        qm, rm = torch.linalg.qr(a)
        return (qm * torch.sign(torch.diagonal(rm, dim1=-2, dim2=-1)).unsqueeze(-2)).to(dt)

    kb, vb = bases(), bases()
    q = torch.randn((B, Hq, 128), generator=gen, device=dev).to(dt)
    # per-head layout: row b*G + g
    fk, ok = _pack_rows_dev(xk.reshape(B * G, S, R), lk.reshape(B * G, S))
    fv, ov = _pack_rows_dev(xv.reshape(B * G, S, R), lv.reshape(B * G, S))
    rt = "short_fused" if route == "short_fused" else "long_two_stage"
    want = grouped_decode_attention(q, fk, fv, lk.reshape(B * G, S).contiguous(), ok,
                                    lv.reshape(B * G, S).contiguous(), ov, kb, vb, theta=THETA,
                                    route=rt, out_dtype=torch.float32)
    del fk, fv, ok, ov
    # joint layout: one row per batch element, count = the last head's end
    hk = torch.arange(G, device=dev)[None, :, None] * R
    jk = (hk + lk).amax(dim=1).to(torch.int32)
    jv = (hk + lv).amax(dim=1).to(torch.int32)
    xjk = xk.permute(0, 2, 1, 3).reshape(B, S, G * R)
    xjv = xv.permute(0, 2, 1, 3).reshape(B, S, G * R)
    del xk, xv
    fjk, ojk = _pack_rows_dev(xjk, jk)
    del xjk
    fjv, ojv = _pack_rows_dev(xjv, jv)
    del xjv
    k_up = torch.zeros((G, G * R, 128), dtype=dt, device=dev)
    v_up = torch.zeros((G, G * R, 128), dtype=dt, device=dev)
    for h in range(G):
        k_up[h, R * h:R * (h + 1)] = kb[h]
        v_up[h, R * h:R * (h + 1)] = vb[h]
    mode = 1 if route == "short_fused" else 0
    sc = J.joint_scores(q, k_up, fjk, jk, ojk, theta=THETA, mode=mode,
                        out_dtype=torch.float32 if mode == 1 else dt)
    got = J.joint_av(sc, v_up, fjv, jv, ojv, mode=mode, out_dtype=torch.float32)
    torch.cuda.synchronize()
    err = (got - want).abs()
    scale = want.abs().max().item()
    print(f"[parity] joint vs split {route}: max_abs={err.max().item():.3e} |ref|max={scale:.3e}",
          flush=True)
    if mode == 1:
        # both fp32-faithful: accumulation-order differences only
        assert err.max().item() <= 1e-4 * max(scale, 1.0)
    else:
        # scores rounded to bf16 by both routes; a score on a rounding tie may round apart
        assert err.max().item() <= 2e-3 and (err.norm() / want.norm()).item() <= 1e-2


def _random_joint(i: int):
    """Case i of a seeded sweep over the joint layout: bases (1, 2, 4, 8) and query heads per
    basis (1 to 8), rank (32 to 1024, multiples of the 32-rank chunk), batch, cache length (1
    to 1500 tokens, log-uniform), counts from 0 or 1 up to the rank, dtype and route."""
    rng = np.random.default_rng(3000 + i)
    n_basis = int(rng.choice([1, 2, 4, 8]))
    hpb = int(rng.choice([1, 2, 3, 4, 5, 8]))
    R = 32 * int(rng.integers(1, 33))
    B = int(rng.integers(1, 4))
    S = int(np.exp(rng.uniform(0, np.log(1500))))
    S = max(1, min(S, 400000 // (B * R)))  # keeps the oracle's reconstruction to seconds
    dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float16
    route = ["short_fused", "long_two_stage"][int(rng.integers(0, 2))]
    # exact_end only past two tokens, where the first token's full rank keeps the buffer
    # non-empty
    return dict(B=B, S=S, R=R, n_basis=n_basis, Hq=n_basis * hpb, len_lo=int(rng.integers(0, 2)),
                exact_end=bool(rng.random() < 0.5) and S > 2), dtype, route


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(16))
def test_random_joint_shapes_against_oracle(dev, i):
    kw, dtype, route = _random_joint(i)
    print(f"[gpu] joint random shape {i}: {kw} {dtype} route={route}", flush=True)
    h = _case(**kw, dtype=dtype, seed=4000 + i)
    d = _dev(h, dev, dtype)
    hpb = kw["Hq"] // kw["n_basis"]
    k_up = d["kb"].repeat_interleave(hpb, dim=0).contiguous()
    v_up = d["vb"].repeat_interleave(hpb, dim=0).contiguous()
    rt = _lib.DKV_ROUTE_FUSED if route == "short_fused" else _lib.DKV_ROUTE_TWO_STAGE
    got = J.joint_attention(d["q"], d["fk"], k_up, d["fv"], v_up, d["lk"], d["ok"], d["lv"],
                            d["ov"], theta=THETA, route=rt)
    assert got is not None and got.dtype == dtype
    # the same two launches with an fp32 output: the bar applies to that result (a stored
    # fp16/bf16 value of magnitude 1-2 carries up to 2^-8 of rounding by itself), and the stored
    # output is its rounding, bit for bit
    mode = 1 if route == "short_fused" else 0
    sc = J.joint_scores(d["q"], k_up, d["fk"], d["lk"], d["ok"], theta=THETA, mode=mode,
                        out_dtype=torch.float32 if mode == 1 else dtype)
    got32 = J.joint_av(sc, v_up, d["fv"], d["lv"], d["ov"], mode=mode, out_dtype=torch.float32)
    assert torch.equal(got, got32.to(dtype))
    ref = A.decode_attention(h["q"], h["fk"], np.repeat(h["kb"], hpb, axis=0), h["fv"],
                             np.repeat(h["vb"], hpb, axis=0), h["lk"], h["ok"], h["lv"], h["ov"],
                             THETA, route=route,
                             q_dtype="bfloat16" if dtype == torch.bfloat16 else "float16")
    assert_close(got32, ref, f"joint random shape {i} {route}")
