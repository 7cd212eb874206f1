"""Decode calls captured in a HIP graph (torch.cuda.CUDAGraph) and replayed, as a serving loop
runs its decode step (the reference replays its cutoff head under a CUDA graph,
compressed_attention.py:321-334).

Each graph is replayed several times. Between the replays the test runs eager calls of a larger
shape on the capturing stream (they grow that stream's cached workspace and RoPE table, so the
buffers the graph captured are replaced in the caches) and eager work on the default stream,
with host synchronisations. Every replay must equal the eager result bit for bit: the split
kernel resets its arrival counters itself (nothing is cleared by a memset), its merge reads the
split records in split order whichever split arrives last, and replaced cached buffers stay
allocated (``_lib.retire``)."""
import pytest
import torch

from dynakv_amd import _lib
from dynakv_amd.kernels.cutoff import CutoffHead
from dynakv_amd.kernels.decode import (dense_decode_attention, grouped_decode_attention,
                                       rope_table, splitk_layout)
from dynakv_amd.synthetic import make_case

from helpers import packed_from_case

REPLAYS = 4

CASES = {
    # name: (make_case kwargs, dtype, route): several splits per unit merged by the last split
    # to arrive, the short route, one split per unit (merged in its workgroup's LDS)
    "multi_split_bf16": (dict(B=2, G=8, Hq=32, S=3000, mean=0.29, force_first=4,
                              force_frac=0.05, seed=51), torch.bfloat16, "long_two_stage"),
    "short_route_f16": (dict(B=4, G=8, Hq=32, S=480, mean=0.47, seed=52), torch.float16,
                        "short_fused"),
    "single_split_bf16": (dict(B=1, G=8, Hq=32, S=200, uniform=(1, 128), seed=53),
                          torch.bfloat16, "short_fused"),
}


def _outputs(x):
    return list(x) if isinstance(x, (tuple, list)) else [x]


def _replay_matches_eager(dev, call, grow, between):
    """Warm ``call`` up on a side stream, take its eager result, capture it there, then replay:
    before each replay ``grow`` (eager, same stream) and ``between`` (eager, default stream) run
    and the captured outputs are overwritten with NaN / -1, so each replay must write them."""
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(2):
            call()
        want = [t.clone() for t in _outputs(call())]
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        got = _outputs(call())
    torch.cuda.synchronize(dev)
    for r in range(REPLAYS):
        with torch.cuda.stream(side):
            grow(r)
        between(r)
        for t in got:
            t.fill_(float("nan") if t.is_floating_point() else -1)
        torch.cuda.synchronize(dev)
        g.replay()
        torch.cuda.synchronize(dev)
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), f"replay {r}, output {i}"
    del g


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_split_kernel_graph_replays(dev, name):
    kw, dtype, route = CASES[name]
    print(f"[gpu] graph replay split kernel {name}", flush=True)
    case = make_case(**kw)
    p = packed_from_case(case, dtype, dev)
    # a longer cache of the same layout, run with 64-token splits: its eager calls need a
    # larger RoPE table and more split records than the captured call
    big_case = make_case(**{**kw, "S": 2 * kw["S"] + 2049, "seed": kw["seed"] + 100})
    big = packed_from_case(big_case, dtype, dev)
    other_case = make_case(B=1, G=8, Hq=32, S=77, uniform=(0, 128), seed=7)
    other = packed_from_case(other_case, dtype, dev)

    def run(pk, c, split_len=0):
        return grouped_decode_attention(
            pk["q"], pk["k_flat"], pk["v_flat"], pk["lens_k"], pk["offs_k"], pk["lens_v"],
            pk["offs_v"], pk["k_basis"], pk["v_basis"], theta=c.theta, route=route,
            split_len=split_len)

    _replay_matches_eager(dev, lambda: run(p, case), lambda r: run(big, big_case, 64),
                          lambda r: run(other, other_case))


@pytest.mark.gpu
def test_dense_decode_graph_replays(dev):
    print("[gpu] graph replay dense decode kernel", flush=True)
    g = torch.Generator(device="cpu").manual_seed(5)
    B, Hkv, hpg, S = 2, 8, 4, 1500

    def cache(S_):
        return (torch.randn(B * Hkv, S_ * 128, generator=g).to(dev, torch.bfloat16),
                torch.randn(B * Hkv, S_ * 128, generator=g).to(dev, torch.bfloat16))

    k, v = cache(S)
    kb, vb = cache(4 * S)
    q = torch.randn(B, Hkv * hpg, 128, generator=g).to(dev, torch.bfloat16)
    _replay_matches_eager(dev, lambda: dense_decode_attention(q, k, v, S),
                          lambda r: dense_decode_attention(q, kb, vb, 4 * S),
                          lambda r: dense_decode_attention(q, k, v, S - 100))


@pytest.mark.gpu
@pytest.mark.parametrize("G,D", [(8, 128), (1, 1024)])
def test_cutoff_head_graph_replays(dev, G, D):
    print(f"[gpu] graph replay cutoff head G={G} D={D}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(9 + G)
    W = [(torch.randn(G, D, D, generator=g) * 3 / D ** 0.5).to(dev, torch.bfloat16)
         for _ in range(2)]
    b = [torch.randn(G, D, generator=g).to(dev, torch.bfloat16) for _ in range(2)]
    head = CutoffHead(W[0] if G > 1 else W[0][0], b[0], W[1] if G > 1 else W[1][0], b[1],
                      groups=G)

    def x(M):
        return [torch.randn(M, 1, G * D, generator=g).to(dev, torch.bfloat16) for _ in range(2)]

    xs, xbig = x(16), x(300)
    _replay_matches_eager(dev, lambda: head.kv_process_fused(xs[0], xs[1])[:4],
                          lambda r: head.kv_process_fused(xbig[0], xbig[1]),
                          lambda r: head.kv_process_fused(xbig[1], xbig[0]))


@pytest.mark.gpu
def test_noalloc_entry_graph_replays(dev):
    """dkv_decode_splitk_noalloc (for callers that cannot allocate, graph capture among them)
    captured and replayed: between the replays an eager call of another shape leaves its records
    and counters in the shared scratch array (on the capturing stream: calls that overlap on one
    GPU would race for it), and every replay equals the eager call."""
    print("[gpu] graph replay no-allocation entry point", flush=True)
    lib = _lib.load()
    case = make_case(B=2, G=8, Hq=32, S=2500, mean=0.29, force_first=4, force_frac=0.05, seed=61)
    p = packed_from_case(case, torch.bfloat16, dev)
    other_case = make_case(B=1, G=8, Hq=32, S=300, mean=0.47, seed=62)
    po = packed_from_case(other_case, torch.bfloat16, dev)

    def call(pk, c):
        q3 = pk["q"]
        lay = splitk_layout(q3, pk["k_basis"], pk["v_basis"], pk["k_flat"], pk["v_flat"])
        st = _lib.stream_of(q3)
        rope, tiles = rope_table(dev, st, c.theta, c.S)
        out = torch.empty((c.B, c.Hq, c.Dh), dtype=torch.float32, device=dev)
        lk, ok, lv, ov = pk["lens_k"], pk["offs_k"], pk["lens_v"], pk["offs_v"]
        rc = lib.dkv_decode_splitk_noalloc(
            st, _lib.DKV_ROUTE_TWO_STAGE, _lib.dtype_code(q3.dtype), q3.data_ptr(), q3.stride(0),
            q3.stride(1), lay.k_basis.data_ptr(), lay.k_unit, lay.k_basis.stride(1),
            lay.v_basis.data_ptr(), lay.v_unit, lay.v_basis.stride(1), pk["k_flat"].data_ptr(),
            pk["k_flat"].stride(0), pk["v_flat"].data_ptr(), pk["v_flat"].stride(0),
            lk.data_ptr(), ok.data_ptr(), lk.stride(0), lk.stride(1), lv.data_ptr(),
            ov.data_ptr(), lv.stride(0), lv.stride(1), rope.data_ptr(), tiles, out.data_ptr(),
            out.stride(0), out.stride(1), _lib.DKV_F32, c.B, c.Hq, c.G, c.G, c.S, c.R, c.Dh, 0)
        _lib.check(rc, "dkv_decode_splitk_noalloc")
        return out

    _replay_matches_eager(dev, lambda: call(p, case), lambda r: call(po, other_case),
                          lambda r: None)
