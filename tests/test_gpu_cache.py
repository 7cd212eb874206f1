"""Packed cache on the GPU against the packing oracle: decode appends (single and K+V launch),
prefill packing (multi-chunk), growth/reallocation, re-expansion. Bit-exact: buffers (including
capacity), lengths, offsets, pointers, host bookkeeping."""
import numpy as np
import pytest
import torch

from dynakv_amd.kernels.compressed_cache import CustomDynamicCache
from oracle.packing import PackedSlot

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _cmp_slot(dev_slot, ref: PackedSlot, what):
    flat, lens, offs, ptr, seq, ub = dev_slot
    assert tuple(flat.shape) == ref.flat.shape, (what, flat.shape, ref.flat.shape)
    assert tuple(lens.shape) == ref.lens.shape and tuple(offs.shape) == ref.offs.shape, what
    np.testing.assert_array_equal(flat.float().cpu().numpy(), ref.flat.astype(np.float32), what)
    np.testing.assert_array_equal(lens.cpu().numpy(), ref.lens, what)
    np.testing.assert_array_equal(offs.cpu().numpy(), ref.offs, what)
    np.testing.assert_array_equal(ptr.cpu().numpy().astype(np.int64), ref.ptr, what)
    assert seq == ref.seq and list(ub) == list(ref.ub), (what, ub, ref.ub)


def _rounded(x, dtype):
    return torch.from_numpy(x).to(dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("max_dim,B", [(16, 3), (128, 5)])
def test_prefill_then_decode_matches_oracle(dev, dtype, max_dim, B):
    print(f"[gpu] cache prefill+decode dtype={dtype} max_dim={max_dim} B={B}", flush=True)
    rng = np.random.default_rng(max_dim + B)
    cache = CustomDynamicCache()
    rk, rv = PackedSlot(), PackedSlot()
    n_pre = 300  # more than one 256-token chunk of the prefill kernel
    ks = rng.standard_normal((B, n_pre, max_dim)).astype(np.float32)
    vs = rng.standard_normal((B, n_pre, max_dim)).astype(np.float32)
    kl = rng.integers(0, max_dim + 1, size=(B, n_pre)).astype(np.int32)
    vl = rng.integers(1, max_dim + 1, size=(B, n_pre)).astype(np.int32)
    tk, tv = _rounded(ks, dtype), _rounded(vs, dtype)
    cache.update_sp(tk.to(dev), torch.from_numpy(kl).to(dev), tv.to(dev),
                    torch.from_numpy(vl).to(dev), max_dim, 0, max_dim)
    rk.append_prefill(tk.float().numpy(), kl, max_dim)
    rv.append_prefill(tv.float().numpy(), vl, max_dim)
    _cmp_slot(cache.key_cache_sp[0], rk, "K after prefill")
    _cmp_slot(cache.value_cache_sp[0], rv, "V after prefill")
    for step in range(40):
        kd = _rounded(rng.standard_normal((B, 1, max_dim)).astype(np.float32), dtype)
        vd = _rounded(rng.standard_normal((B, 1, max_dim)).astype(np.float32), dtype)
        kdl = rng.integers(0, max_dim + 1, size=(B, 1)).astype(np.int32)
        vdl = rng.integers(0, max_dim + 1, size=(B, 1)).astype(np.int32)
        out = cache.update_sp(kd.to(dev), torch.from_numpy(kdl).to(dev), vd.to(dev),
                              torch.from_numpy(vdl).to(dev), max_dim, 0, max_dim)
        rk.append_decode(kd.float().numpy(), kdl, max_dim)
        rv.append_decode(vd.float().numpy(), vdl, max_dim)
        if step in (0, 1, 39):
            _cmp_slot(cache.key_cache_sp[0], rk, f"K step {step}")
            _cmp_slot(cache.value_cache_sp[0], rv, f"V step {step}")
    lk, ok = rk.tables()
    np.testing.assert_array_equal(out[2].cpu().numpy(), lk)
    np.testing.assert_array_equal(out[4].cpu().numpy(), ok)
    assert cache.get_seq_length_sp(0) == n_pre + 40 == cache.get_seq_length(0)
    dk, dv = cache.get_origin_states(max_dim, 0)
    np.testing.assert_array_equal(dk.float().cpu().numpy(), rk.decompress(max_dim).astype(np.float32))
    np.testing.assert_array_equal(dv.float().cpu().numpy(), rv.decompress(max_dim).astype(np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_from_empty_and_reset(dev, dtype):
    print(f"[gpu] cache decode-from-empty dtype={dtype}", flush=True)
    rng = np.random.default_rng(7)
    cache = CustomDynamicCache()
    ref = PackedSlot()
    B, D = 4, 64
    for layer in (0, 2):  # lazy creation of a non-contiguous layer slot
        for _ in range(30):
            x = _rounded(rng.standard_normal((B, 1, D)).astype(np.float32), dtype)
            l = rng.integers(1, D + 1, size=(B, 1)).astype(np.int32)
            cache.update_sp(x.to(dev), torch.from_numpy(l).to(dev), x.to(dev),
                            torch.from_numpy(l).to(dev), D, layer, torch.full((B, 1), D, device=dev))
            if layer == 0:
                ref.append_decode(x.float().numpy(), l, D)
    _cmp_slot(cache.key_cache_sp[0], ref, "K layer 0")
    assert cache.key_cache_sp[1] is None and cache.get_seq_length_sp(1) == 0
    assert cache.get_seq_length_sp(2) == 30 and cache.get_seq_length_sp(7) == 0
    cache.reset()
    assert cache.key_cache_sp == [] and cache.get_seq_length_sp(0) == 0


@pytest.mark.gpu
def test_single_slot_append_path(dev):
    """The one-slot launch (used when K and V slots are out of step) matches too."""
    print("[gpu] cache single-slot append", flush=True)
    rng = np.random.default_rng(3)
    cache = CustomDynamicCache()
    ref = PackedSlot()
    B, D = 2, 32
    for _ in range(10):
        x = _rounded(rng.standard_normal((B, 1, D)).astype(np.float32), torch.float16)
        l = rng.integers(0, D + 1, size=(B, 1)).astype(np.int32)
        cache._update_layer_cache(cache.key_cache_sp, 0, x.to(dev), torch.from_numpy(l).to(dev), D,
                                  is_decode=True)
        ref.append_decode(x.float().numpy(), l, D)
    _cmp_slot(cache.key_cache_sp[0], ref, "K single")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_bulk_prefill_append_equals_per_layer(dev, dtype):
    """update_sp_prefill_many (one host synchronisation for all layers) leaves the caches
    exactly as one update_sp per layer does, and attention from the masked coefficient rows
    equals attention from the packed cache."""
    from dynakv_amd.kernels.prefill import coef_prefill_attention, compressed_prefill_attention
    print(f"[gpu] bulk prefill append {dtype}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(77)
    B, G, R, S, layers = 2, 4, 128, 300, 3
    items = []
    for i in range(layers):
        lk = torch.randint(1, R + 1, (B * G, S), generator=g, dtype=torch.int32)
        lv = torch.randint(1, R + 1, (B * G, S), generator=g, dtype=torch.int32)
        ks = torch.randn(B * G, S, R, generator=g) * (torch.arange(R) < lk[..., None])
        vs = torch.randn(B * G, S, R, generator=g) * (torch.arange(R) < lv[..., None])
        items.append((i, ks.to(dtype).to(dev), lk.to(dev), vs.to(dtype).to(dev), lv.to(dev)))
    a, b = CustomDynamicCache(), CustomDynamicCache()
    for i, ks, lk, vs, lv in items:
        a.update_sp(ks, lk, vs, lv, R, i, R)
    b.update_sp_prefill_many(items, R)
    assert b.device_syncs == 1

    def same(tag):
        for i in range(layers):
            for sa, sb in ((a.key_cache_sp[i], b.key_cache_sp[i]),
                           (a.value_cache_sp[i], b.value_cache_sp[i])):
                assert tuple(sa[0].shape) == tuple(sb[0].shape), tag
                assert tuple(sa[1].shape) == tuple(sb[1].shape), tag
                for t in range(4):
                    assert torch.equal(sa[t], sb[t]), (tag, i, t)
                assert sa[4] == sb[4] and list(sa[5]) == list(sb[5]), tag

    same("prefill")
    kb = torch.linalg.qr(torch.randn(G, R, R, generator=g))[0].to(dtype).to(dev)
    vb = torch.linalg.qr(torch.randn(G, R, R, generator=g))[0].to(dtype).to(dev)
    q = torch.randn(B, 2 * G, S, 128, generator=g).to(dtype).to(dev)
    i, ks, _, vs, _ = items[1]
    o1 = compressed_prefill_attention(q, a, 1, kb, vb, theta=500000.0)
    o2 = coef_prefill_attention(q, ks, vs, kb, vb, theta=500000.0)
    assert torch.equal(o1, o2)
    # decode appends on both: the first grows every slot (flat and tables) out of the bulk
    # prefill's shared buffers
    for step in range(3):
        for i in range(layers):
            lk = torch.randint(0, R + 1, (B * G, 1), generator=g, dtype=torch.int32).to(dev)
            lv = torch.randint(0, R + 1, (B * G, 1), generator=g, dtype=torch.int32).to(dev)
            ks = torch.randn(B * G, 1, R, generator=g).to(dtype).to(dev)
            vs = torch.randn(B * G, 1, R, generator=g).to(dtype).to(dev)
            for c in (a, b):
                c.update_sp(ks, lk, vs, lv, R, i, R)
        same(f"decode {step}")
    # a second prompt onto the slots that now hold tokens: the appends start at each row's
    # pointer (K and V slots in one launch on the bulk path, one launch per slot on the other)
    items2 = []
    for i in range(layers):
        S2 = 70
        lk = torch.randint(0, R + 1, (B * G, S2), generator=g, dtype=torch.int32)
        lv = torch.randint(0, R + 1, (B * G, S2), generator=g, dtype=torch.int32)
        ks = torch.randn(B * G, S2, R, generator=g) * (torch.arange(R) < lk[..., None])
        vs = torch.randn(B * G, S2, R, generator=g) * (torch.arange(R) < lv[..., None])
        items2.append((i, ks.to(dtype).to(dev), lk.to(dev), vs.to(dtype).to(dev), lv.to(dev)))
    for i, ks, lk, vs, lv in items2:
        a.update_sp(ks, lk, vs, lv, R, i, R)
    b.update_sp_prefill_many(items2, R)
    same("second prompt")


def _random_ops(i: int):
    """Case i of a seeded sweep over cache operation sequences: rows, row width (8 to 1024),
    dtype, a first prompt of 1-600 tokens or decode from empty, then up to three rounds of
    1-60 decode steps, each round possibly followed by another prompt onto the filled rows;
    retained counts uniform, all zero or all full for a row-step at random."""
    rng = np.random.default_rng(10000 + i)
    B = int(rng.integers(1, 7))
    max_dim = int(rng.choice([8, 16, 40, 64, 100, 128, 128, 256, 1024]))
    dtype = DTYPES[int(rng.integers(0, 3))]
    ops = []
    if rng.random() < 0.75:
        ops.append(("prefill", int(np.exp(rng.uniform(0, np.log(600))))))
    for _ in range(int(rng.integers(1, 4))):
        ops.append(("decode", int(rng.integers(1, 61))))
        if rng.random() < 0.3:
            ops.append(("prefill", int(rng.integers(1, 200))))
    return B, max_dim, dtype, ops


def _random_lengths(rng, shape, max_dim):
    L = rng.integers(0, max_dim + 1, size=shape).astype(np.int32)
    u = rng.random(shape)
    L[u < 0.05] = 0
    L[u > 0.95] = max_dim
    return L


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(12))
def test_random_op_sequences_match_oracle(dev, i):
    B, max_dim, dtype, ops = _random_ops(i)
    print(f"[gpu] cache random ops {i}: B={B} max_dim={max_dim} {dtype} {ops}", flush=True)
    rng = np.random.default_rng(11000 + i)
    cache = CustomDynamicCache()
    rk, rv = PackedSlot(), PackedSlot()
    total = 0
    for kind, n in ops:
        steps = [n] if kind == "prefill" else [1] * n
        for S in steps:
            kx = _rounded(rng.standard_normal((B, S, max_dim)).astype(np.float32), dtype)
            vx = _rounded(rng.standard_normal((B, S, max_dim)).astype(np.float32), dtype)
            kl = _random_lengths(rng, (B, S), max_dim)
            vl = _random_lengths(rng, (B, S), max_dim)
            cache.update_sp(kx.to(dev), torch.from_numpy(kl).to(dev), vx.to(dev),
                            torch.from_numpy(vl).to(dev), max_dim, 0, max_dim)
            if S > 1:
                rk.append_prefill(kx.float().numpy(), kl, max_dim)
                rv.append_prefill(vx.float().numpy(), vl, max_dim)
            else:
                rk.append_decode(kx.float().numpy(), kl, max_dim)
                rv.append_decode(vx.float().numpy(), vl, max_dim)
            total += S
        _cmp_slot(cache.key_cache_sp[0], rk, f"K after {kind} {n}")
        _cmp_slot(cache.value_cache_sp[0], rv, f"V after {kind} {n}")
    assert cache.get_seq_length_sp(0) == total
    dk, dv = cache.get_origin_states(max_dim, 0)
    np.testing.assert_array_equal(dk.float().cpu().numpy(), rk.decompress(max_dim).astype(np.float32))
    np.testing.assert_array_equal(dv.float().cpu().numpy(), rv.decompress(max_dim).astype(np.float32))
