"""The gfx950 split-K kernel (both routes) against the oracle, per-head layout (row = b*G + g)."""
import numpy as np
import pytest
import torch

from dynakv_amd.kernels.decode import grouped_decode_attention
from dynakv_amd.kernels.router import compressed_decode_attention
from dynakv_amd.synthetic import make_case

from helpers import NP_OF, assert_close, oracle_grouped, packed_from_case

ROUTES = ["short_fused", "long_two_stage"]


def _run(p, case, route, split_len=0, out_dtype=torch.float32):
    """fp32 output by default: the north-star bar applies to the merged result; the stored
    q-dtype output is its rounding (test_output_is_rounded_fp32_result)."""
    return grouped_decode_attention(
        p["q"], p["k_flat"], p["v_flat"], p["lens_k"], p["offs_k"], p["lens_v"], p["offs_v"],
        p["k_basis"], p["v_basis"], theta=case.theta, route=route, split_len=split_len,
        out_dtype=out_dtype)


CASES = {
    # name: (make_case kwargs, dtype)
    "cfg1_shape_f16": (dict(B=1, G=8, Hq=32, S=257, uniform=(8, 128), seed=11), torch.float16),
    "cfg1_shape_bf16": (dict(B=1, G=8, Hq=32, S=257, uniform=(8, 128), seed=12), torch.bfloat16),
    "cfg2_shape_f16": (dict(B=4, G=8, Hq=32, S=480, mean=0.47, seed=13), torch.float16),
    "cfg3_shape_bf16_B2": (dict(B=2, G=8, Hq=32, S=8192, mean=0.29, force_first=4,
                                force_frac=0.05, seed=14), torch.bfloat16),
    "S1": (dict(B=3, G=8, Hq=32, S=1, uniform=(1, 128), seed=15), torch.float16),
    "S17_zero_lens": (dict(B=2, G=8, Hq=32, S=17, uniform=(0, 128), seed=16), torch.bfloat16),
    "zero_len_frac": (dict(B=2, G=4, Hq=16, S=700, mean=0.3, zero_len_frac=0.2, seed=17), torch.float16),
    "R64": (dict(B=2, G=8, Hq=32, S=333, R=64, uniform=(1, 64), seed=18), torch.bfloat16),
    "R40": (dict(B=2, G=2, Hq=8, S=129, R=40, uniform=(1, 40), seed=19), torch.float16),
    "hpg1": (dict(B=2, G=8, Hq=8, S=200, uniform=(1, 128), seed=20), torch.bfloat16),
    "hpg16": (dict(B=2, G=2, Hq=32, S=200, uniform=(1, 128), seed=21), torch.float16),
    "r_max_all": (dict(B=1, G=8, Hq=32, S=96, uniform=(128, 128), seed=22), torch.bfloat16),
}


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("name", list(CASES))
def test_splitk_matches_oracle(dev, name, route):
    kw, dtype = CASES[name]
    print(f"[gpu] splitk {name} route={route}", flush=True)
    case = make_case(**kw)
    p = packed_from_case(case, dtype, dev)
    got = _run(p, case, route)
    ref = oracle_grouped(case, p["host"], route, NP_OF[dtype])
    assert_close(got, ref, f"{name} {route}")


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
def test_split_length_invariance(dev, route):
    print(f"[gpu] splitk split invariance route={route}", flush=True)
    case = make_case(B=2, G=8, Hq=32, S=3000, mean=0.29, force_first=4, force_frac=0.05, seed=30)
    p = packed_from_case(case, torch.bfloat16, dev)
    ref = oracle_grouped(case, p["host"], route, "bfloat16")
    outs = [_run(p, case, route, sl) for sl in (64, 192, 320, 512, 1024, 3008)]
    for o in outs:
        assert_close(o, ref, f"split {route}")
    # fp32 results of different split lengths differ by summation order and, on the two-stage
    # route, by the bf16 rounding of a score sitting on a rounding boundary (the RoPE angles of a
    # token come from a recurrence seeded at the first tile of its wave, so their last bits
    # depend on the split layout)
    tol = 2e-5 if route == "short_fused" else 2e-3
    for o in outs[1:]:
        d = (o - outs[0]).abs().max().item()
        assert d <= tol * outs[0].abs().max().item(), d


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("S,split_len", [(976, 320), (1009, 256), (4097, 256), (250, 128)])
def test_tile_pair_edges_against_oracle(dev, route, S, split_len):
    """Splits of 256+ tokens run their waves on pairs of consecutive tiles (the second tile's
    keys rotated by R(16 + n) under the first tile's query operand). Edge cases of that mapping
    against the oracle: a last split of a single tile (976 = 3 x 320 + 16), a ragged last tile
    (1009), a one-token last split (4097 = 16 x 256 + 1), and a cache short enough for single
    tiles (250 tokens in 128-token splits)."""
    print(f"[gpu] splitk tile-pair edges S={S} split_len={split_len} route={route}", flush=True)
    case = make_case(B=2, G=8, Hq=32, S=S, mean=0.29, force_first=4, force_frac=0.05,
                     seed=40 + S % 97)
    p = packed_from_case(case, torch.bfloat16, dev)
    got = _run(p, case, route, split_len)
    ref = oracle_grouped(case, p["host"], route, "bfloat16")
    assert_close(got, ref, f"tile pairs S={S} split_len={split_len} {route}")


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
def test_more_units_than_cus_automatic_splits(dev, route):
    """288 units (B=36 x 8 KV groups) at 4100 tokens: the chooser splits each unit in two
    (rounds of 256 workgroups); sampled batch rows against the oracle."""
    from dynakv_amd import _lib
    print(f"[gpu] splitk 288 units route={route}", flush=True)
    case = make_case(B=36, G=8, Hq=32, S=4100, mean=0.29, force_first=4, force_frac=0.05,
                     seed=88)
    assert -(-case.S // _lib.load().dkv_splitk_choose_split(case.B, case.G, case.S)) == 2
    p = packed_from_case(case, torch.bfloat16, dev)
    got = _run(p, case, route)
    rows = [0, 17, 35]
    ref = oracle_grouped(case, p["host"], route, "bfloat16", batches=rows)
    assert_close(got[rows], ref, f"288 units {route}")


HPG_CASES = {
    # name: (G, Hq, S, split_len, dtype): the kernel's instances for at most 4, 8 and 16 query
    # heads per KV group, with and without tile pairs (splits of 256+ tokens), at group sizes
    # that fill them and at sizes that leave head slots empty (2, 3, 6, 12)
    "hpg8_pairs_bf16": (4, 32, 1000, 320, torch.bfloat16),
    "hpg8_single_f16": (4, 32, 700, 0, torch.float16),
    "hpg8_one_group_bf16": (1, 8, 600, 256, torch.bfloat16),
    "hpg6_pairs_bf16": (4, 24, 900, 320, torch.bfloat16),
    "hpg3_f16": (8, 24, 500, 0, torch.float16),
    "hpg2_pairs_bf16": (8, 16, 1500, 320, torch.bfloat16),
    "hpg12_bf16": (2, 24, 700, 0, torch.bfloat16),
}


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("name", list(HPG_CASES))
def test_heads_per_group_instances(dev, name, route):
    G, Hq, S, split_len, dtype = HPG_CASES[name]
    print(f"[gpu] splitk heads per group {name} route={route}", flush=True)
    case = make_case(B=2, G=G, Hq=Hq, S=S, mean=0.29, force_first=4, force_frac=0.05,
                     seed=60 + Hq + S % 89)
    p = packed_from_case(case, dtype, dev)
    got = _run(p, case, route, split_len)
    ref = oracle_grouped(case, p["host"], route, NP_OF[dtype])
    assert_close(got, ref, f"{name} {route}")


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
def test_keys_beyond_fp16_range_bf16(dev, route):
    """bf16 keys whose values lie far past fp16's range (coefficients scaled by 2^17, |K'| up to
    ~6e5) with the queries scaled by 2^-17: the scores are those of the unscaled case (the power
    of two commutes with every rounding), so a kernel that narrowed K' or q to fp16 would give
    inf/NaN scores here while the reference's fp32 dot product stays finite."""
    print(f"[gpu] splitk keys beyond fp16 range route={route}", flush=True)
    case = make_case(B=2, G=8, Hq=32, S=700, mean=0.29, force_first=4, force_frac=0.05, seed=33)
    case.k_coef = case.k_coef * np.float32(2.0 ** 17)
    case.q = case.q * np.float32(2.0 ** -17)
    p = packed_from_case(case, torch.bfloat16, dev)
    assert p["k_flat"].float().abs().max().item() > 4 * 65504
    got = _run(p, case, route)
    assert torch.isfinite(got).all()
    ref = oracle_grouped(case, p["host"], route, "bfloat16")
    assert_close(got, ref, f"keys beyond fp16 range {route}")


@pytest.mark.gpu
def test_all_keys_empty_in_one_row(dev):
    print("[gpu] splitk empty-key row", flush=True)
    case = make_case(B=2, G=2, Hq=8, S=150, uniform=(1, 128), seed=31)
    case.k_len[1, :] = 0  # row (b=0, g=1): every key excluded
    for route, dtype in (("short_fused", torch.float16), ("long_two_stage", torch.bfloat16)):
        p = packed_from_case(case, dtype, dev)
        got = _run(p, case, route).float().cpu().numpy()
        ref = oracle_grouped(case, p["host"], route, NP_OF[dtype])
        if route == "short_fused":
            assert np.isnan(got[0, 4:8]).all() and np.isfinite(got[0, :4]).all()
            assert_close(got[:, :4], ref[:, :4], "fused finite part")
            assert_close(got[1], ref[1], "fused other batch")
        else:
            assert_close(got, ref, "two-stage with empty row")


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
def test_full_config3_size_rows_against_oracle(dev, route):
    """Config 3 at full size (B=16, S=8192, bf16): every batch row against the oracle, and
    properties of the whole output (finite, linear in V)."""
    print(f"[gpu] splitk full config3 route={route}", flush=True)
    case = make_case(B=16, G=8, Hq=32, S=8192, mean=0.29, force_first=4, force_frac=0.05, seed=32)
    p = packed_from_case(case, torch.bfloat16, dev)
    got = _run(p, case, route)
    assert torch.isfinite(got.float()).all()
    ref = oracle_grouped(case, p["host"], route, "bfloat16")
    assert_close(got, ref, "config3 all 16 rows")
    # linearity in the V coefficients: doubling every V coefficient doubles the output (exact
    # in binary floating point up to the final rounding)
    p2 = dict(p)
    p2["v_flat"] = p["v_flat"] * 2
    got2 = _run(p2, case, route)
    d = (got2 / 2 - got).abs().max().item()
    assert d <= 1e-6 * got.abs().max().item(), d


@pytest.mark.gpu
def test_reference_api_per_group_equals_native(dev):
    """Per-head mode through the reference surface: one compressed_decode_attention call per KV
    group with q[:, 4g:4g+4] and the group's basis (as B_g[None] and as an expand) equals the
    one-launch native call."""
    print("[gpu] reference API per group", flush=True)
    case = make_case(B=2, G=8, Hq=32, S=620, mean=0.47, seed=33)
    p = packed_from_case(case, torch.float16, dev)
    B, G = case.B, case.G
    native = _run(p, case, "long_two_stage")
    for mode in ("slice", "expand"):
        outs = []
        for g in range(G):
            rows = [b * G + g for b in range(B)]
            kb = p["k_basis"][g: g + 1]
            vb = p["v_basis"][g: g + 1]
            if mode == "expand":
                kb, vb = kb.expand(4, 128, 128), vb.expand(4, 128, 128)
            outs.append(compressed_decode_attention(
                q=p["q"][:, 4 * g: 4 * g + 4, None, :].contiguous(), k_flat=p["k_flat"][rows],
                k_up=kb, v_flat=p["v_flat"][rows], v_up=vb,
                key_lengths=p["lens_k"][rows], key_offsets=p["offs_k"][rows],
                value_lengths=p["lens_v"][rows], value_offsets=p["offs_v"][rows],
                theta=case.theta, cache_length=case.S))
        per_group = torch.cat(outs, dim=1)
        assert per_group.dtype == torch.float16
        assert torch.equal(per_group, native.to(torch.float16)), mode


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_output_is_rounded_fp32_result(dev, dtype):
    """The q-dtype output (the reference contract) is exactly the round-to-nearest of the fp32
    merge result."""
    print(f"[gpu] splitk output rounding {dtype}", flush=True)
    case = make_case(B=2, G=8, Hq=32, S=900, mean=0.3, seed=34)
    p = packed_from_case(case, dtype, dev)
    for route in ROUTES:
        f32 = _run(p, case, route)
        low = _run(p, case, route, out_dtype=None)
        assert low.dtype == dtype
        assert torch.equal(low, f32.to(dtype)), route


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
def test_more_units_than_merge_counters(dev, route):
    """16400 units (batch 2050 x 8 KV groups) exceed the fused merge's 16384 arrival
    counters: the split records are merged by the separate merge kernel instead. Rows spread
    over the batch against the oracle."""
    print(f"[gpu] splitk standalone merge route={route}", flush=True)
    case = make_case(B=2050, G=8, Hq=8, S=70, R=16, uniform=(0, 16), seed=41)
    p = packed_from_case(case, torch.float16, dev)
    got = _run(p, case, route, split_len=64)
    rows = [0, 1, 1024, 2049]
    ref = oracle_grouped(case, p["host"], route, "float16", batches=rows)
    assert_close(got[rows], ref, f"standalone merge {route}")


@pytest.mark.gpu
@pytest.mark.parametrize("route", ROUTES)
def test_flat_buffers_beyond_32bit_range(dev, route):
    """Flat buffers of 3 rows with a row stride of 0x16000000 elements (2.06 GiB per buffer,
    rows * stride >= 2^30): each workgroup addresses its own row, so the fast path takes them.
    Results equal the same cache in compact buffers, and match the oracle."""
    print(f"[gpu] splitk flat buffers past 2^30 elements route={route}", flush=True)
    from dynakv_amd.kernels.decode import splitk_layout

    case = make_case(B=3, G=1, Hq=4, S=300, uniform=(1, 128), seed=42)
    p = packed_from_case(case, torch.bfloat16, dev)
    LD = 0x16000000
    big = {}
    for name in ("k_flat", "v_flat"):
        t = torch.empty((3, LD), dtype=torch.bfloat16, device=dev)
        t[:, : p[name].shape[1]] = p[name]
        big[name] = t
    assert big["k_flat"].shape[0] * big["k_flat"].stride(0) >= 2**30
    assert splitk_layout(p["q"], p["k_basis"], p["v_basis"], big["k_flat"], big["v_flat"]) is not None
    compact = _run(p, case, route)
    pb = dict(p, **big)
    got = _run(pb, case, route)
    assert torch.equal(got, compact)
    ref = oracle_grouped(case, p["host"], route, "bfloat16")
    assert_close(got, ref, f"large buffers {route}")
    del big, pb
    torch.cuda.empty_cache()


def _random_shape(i: int):
    """Case i of a seeded sweep over the kernel's argument space: KV groups, query heads per
    group (every instance, with empty head slots), batch, cache length (1 to 4000 tokens,
    log-uniform), rank, retained-count distribution, dtype, route and split length (automatic
    or an explicit multiple of 64)."""
    rng = np.random.default_rng(1000 + i)
    G = int(rng.choice([1, 2, 4, 8]))
    hpg = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 16]))
    B = int(rng.integers(1, 7))
    S = int(np.exp(rng.uniform(0, np.log(4000))))
    while B * G * S > 60000 and B > 1:  # keeps each oracle run to about a second
        B -= 1
    S = max(1, min(S, 60000 // (B * G)))
    R = int(rng.choice([128, 128, 128, 120, 96, 64, 40, 8]))
    kw = dict(B=B, G=G, Hq=G * hpg, S=S, R=R, seed=2000 + i)
    if rng.random() < 0.5:
        kw["mean"] = float(rng.uniform(0.05, 0.95))
    else:
        kw["uniform"] = (0 if S >= 64 else 1, R)
    if S >= 64 and rng.random() < 0.5:
        kw.update(force_first=4, force_frac=0.05)
        if rng.random() < 0.5:
            kw["zero_len_frac"] = 0.2
    dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float16
    route = ROUTES[int(rng.integers(0, 2))]
    split_len = 0 if rng.random() < 0.5 else 64 * int(rng.integers(1, 17))
    return kw, dtype, route, split_len


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(24))
def test_random_shapes_against_oracle(dev, i):
    kw, dtype, route, split_len = _random_shape(i)
    print(f"[gpu] splitk random shape {i}: {kw} {dtype} route={route} split_len={split_len}",
          flush=True)
    case = make_case(**kw)
    p = packed_from_case(case, dtype, dev)
    got = _run(p, case, route, split_len)
    ref = oracle_grouped(case, p["host"], route, NP_OF[dtype])
    assert_close(got, ref, f"random shape {i} {route}")
