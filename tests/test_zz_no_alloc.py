"""The no-allocation split-K entry point (dkv_decode_splitk_noalloc) against dkv_decode_splitk.

Both are called through the C ABI on the same inputs; the fp32 results must be bit-identical
(same kernels, same split layout, same merge order). Two calls in a row on one GPU, the second
with a smaller input: the shared scratch array keeps the first call's records and must not leak
into the second call's result.
"""
import ctypes as C

import pytest
import torch

from dynakv_amd import _lib
from dynakv_amd.kernels.decode import rope_table, splitk_layout
from dynakv_amd.synthetic import make_case

from helpers import packed_from_case


def _args(p, case, dev, route):
    """Common argument list (up to, not including, the workspace) and the output tensor."""
    q3 = p["q"]
    layout = splitk_layout(q3, p["k_basis"], p["v_basis"], p["k_flat"], p["v_flat"])
    assert layout is not None and layout.n_kv == case.G
    st = _lib.stream_of(q3)
    rope, tiles = rope_table(dev, st, case.theta, case.S)
    out = torch.full((case.B, case.Hq, case.Dh), float("nan"), dtype=torch.float32, device=dev)
    lk, ok, lv, ov = p["lens_k"], p["offs_k"], p["lens_v"], p["offs_v"]
    head = [st, route, _lib.dtype_code(q3.dtype), q3.data_ptr(), q3.stride(0), q3.stride(1),
            layout.k_basis.data_ptr(), layout.k_unit, layout.k_basis.stride(1),
            layout.v_basis.data_ptr(), layout.v_unit, layout.v_basis.stride(1),
            p["k_flat"].data_ptr(), p["k_flat"].stride(0), p["v_flat"].data_ptr(),
            p["v_flat"].stride(0), lk.data_ptr(), ok.data_ptr(), lk.stride(0), lk.stride(1),
            lv.data_ptr(), ov.data_ptr(), lv.stride(0), lv.stride(1), rope.data_ptr(), tiles]
    tail = [out.data_ptr(), out.stride(0), out.stride(1), _lib.DKV_F32,
            case.B, case.Hq, case.G, case.G, case.S, case.R, case.Dh, 0]
    return head, tail, out, layout


def _both(dev, case, dtype, route):
    lib = _lib.load()
    p = packed_from_case(case, dtype, dev)
    head, tail, out_ref, layout = _args(p, case, dev, route)
    nfl = lib.dkv_splitk_workspace_floats(case.B, case.Hq, case.G, case.S, case.R, 0)
    assert 0 < nfl <= _lib.DKV_NOALLOC_SCRATCH_FLOATS
    ws = torch.zeros(int(nfl), dtype=torch.float32, device=dev)
    _lib.check(lib.dkv_decode_splitk(*head, ws.data_ptr(), ws.numel(), *tail),
               "dkv_decode_splitk")
    _, tail2, out_na, _ = _args(p, case, dev, route)
    _lib.check(lib.dkv_decode_splitk_noalloc(*head, *tail2), "dkv_decode_splitk_noalloc")
    torch.cuda.synchronize()
    return out_ref, out_na


@pytest.mark.gpu
@pytest.mark.parametrize("route", [_lib.DKV_ROUTE_TWO_STAGE, _lib.DKV_ROUTE_FUSED])
def test_noalloc_matches_workspace_entry(dev, route):
    # first call: a config-3 shaped cache (bf16, two splits per unit); second: smaller batch,
    # shorter cache, fp16 (one split per unit for most units, fewer records)
    calls = [
        (dict(B=4, G=8, Hq=32, S=4100, mean=0.29, force_first=4, force_frac=0.05, seed=71),
         torch.bfloat16),
        (dict(B=2, G=8, Hq=32, S=300, mean=0.47, seed=72), torch.float16),
    ]
    for i, (kw, dtype) in enumerate(calls):
        print(f"[gpu] noalloc call {i} route={route} {kw}", flush=True)
        case = make_case(**kw)
        ref, got = _both(dev, case, dtype, route)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref), (got - ref).abs().max().item()


@pytest.mark.gpu
def test_noalloc_rejects_calls_beyond_the_scratch(dev):
    print("[gpu] noalloc size limit", flush=True)
    lib = _lib.load()
    # B = 2048 rows of 8 units with 16 heads per unit: one split each, records alone exceed 4 MiB
    B, Hq, Hkv, S, R = 2048, 128, 8, 64, 128
    need = lib.dkv_splitk_workspace_floats(B, Hq, Hkv, S, R, 0)
    assert need > _lib.DKV_NOALLOC_SCRATCH_FLOATS
    fake = C.c_void_p(256)  # never dereferenced: the size check comes before any launch
    rc = lib.dkv_decode_splitk_noalloc(
        None, _lib.DKV_ROUTE_TWO_STAGE, _lib.DKV_BF16, fake, Hq * 128, 128, fake, R * 128, 128,
        fake, R * 128, 128, fake, 1024, fake, 1024, fake, fake, S, 1, fake, fake, S, 1, fake,
        (S + 15) // 16, fake, Hq * 128, 128, _lib.DKV_BF16, B, Hq, Hkv, Hkv, S, R, 128, 0)
    assert rc == _lib.DKV_E_SCRATCH
    with pytest.raises(ValueError, match="no-allocation scratch"):
        _lib.check(rc, "dkv_decode_splitk_noalloc")
