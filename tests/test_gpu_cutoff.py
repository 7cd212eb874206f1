"""The gfx950 cutoff head (dkv_cutoff_kv) against the oracle (reference
compressed_attention.py:84-119): rounded logits within one unit in the last place, lengths
equal wherever the arithmetic fixes them (and inside the reachable range where a prefix sum
sits on the threshold), masked outputs bit-exact for the lengths produced, and the result
feeding the cache append."""
import zlib

import numpy as np
import pytest
import torch

from dynakv_amd.kernels import cutoff as CK
from dynakv_amd.kernels.compressed_cache import CustomDynamicCache
from oracle import cutoff as C

from helpers import NP_OF, cast_np

ULP_AT_THR = {torch.float16: 2.0 ** -14, torch.bfloat16: 2.0 ** -11}  # ulp of 0.1 (exponent -4)

CASES = {
    # name: (G, D, M, dtype, low_rank, weight scale)
    "joint_bf16_decode": (1, 1024, 16, torch.bfloat16, None, 3.0),
    "joint_f16_M5": (1, 1024, 5, torch.float16, None, 3.0),
    "perhead_bf16_decode": (8, 128, 16, torch.bfloat16, None, 3.0),
    "perhead_f16_M33": (8, 128, 33, torch.float16, None, 2.0),
    "perhead_bf16_prefill": (8, 128, 512, torch.bfloat16, None, 3.0),
    "G2_D64_f16": (2, 64, 7, torch.float16, None, 4.0),
    "joint_low_rank": (1, 1024, 16, torch.bfloat16, 300, 3.0),
    "D256_M1": (1, 256, 1, torch.float16, 100, 3.0),
}


def _inputs(G, D, M, dtype, scale, seed):
    rng = np.random.default_rng(seed)
    x = cast_np(rng.standard_normal((M, G * D)).astype(np.float32), dtype)
    W = cast_np((rng.standard_normal((G, D, D)) * scale / np.sqrt(D)).astype(np.float32), dtype)
    b = cast_np(rng.standard_normal((G, D)).astype(np.float32), dtype)
    return x, W, b


def _dev_rows(x, dtype, dev, pad):
    """Device rows with row stride G*D + pad (a view into a wider buffer when pad > 0)."""
    M, H = x.shape
    big = torch.zeros((M, H + pad), dtype=dtype, device=dev)
    big[:, :H] = torch.from_numpy(x).to(dtype)
    return big[:, :H]


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy()


def _check(name, got_out, got_len, x, W, b, dtype, low_rank, logits_dev):
    nd = NP_OF[dtype]
    ref_out, ref_len, ref_logits, c, thr = C.cutoff(x, W, b, nd, low_rank=low_rank)
    G, D = W.shape[0], W.shape[1]
    M = x.shape[0]
    # logits: the kernel accumulates in fp32 in another order, so a rounded logit may land one
    # unit in the last place away from the exact sum's rounding, plus the fp32 accumulation
    # error where the sum cancels (bounded by 2^-20 of the sum of absolute terms)
    lg = logits_dev.float().cpu().numpy().reshape(M, G, D)
    mant = 10 if dtype == torch.float16 else 7
    e = np.floor(np.log2(np.maximum(np.abs(ref_logits), 2.0 ** -14)))
    ulp = 2.0 ** (e - mant)
    abs_terms = np.einsum("mgk,gkn->mgn", np.abs(x.reshape(M, G, D)), np.abs(W)) + np.abs(b)[None]
    tol = ulp + 2.0 ** -20 * abs_terms
    assert (np.abs(lg - ref_logits) <= tol).all(), f"{name}: logits outside 1 ulp + fp32 slack"
    # lengths: the softmax / prefix-sum / threshold steps restated on the kernel's own logits
    # give the length exactly, except on rows where a rounding tie lets an fp32 implementation
    # of the same steps go either way (tie rows: then it must still be a length the oracle's
    # prefix sums allow within a few units in the last place)
    L = got_len.cpu().numpy().reshape(M, G).astype(np.int64)
    lens_k, ck, _, tie = C.lengths_from_logits(lg, nd, low_rank=low_rank)
    assert (L[~tie] == lens_k[~tie]).all(), f"{name}: length differs on a row without a tie"
    if tie.size >= 16:
        assert tie.mean() < 0.05, f"{name}: {tie.mean():.3f} of rows on a rounding tie"
    tol = 4 * ULP_AT_THR[dtype]
    lo, hi = C.length_bounds(ck, thr, tol, low_rank)
    assert ((L >= lo) & (L <= hi)).all(), f"{name}: length outside the reachable range"
    # masked copy: bit-exact for the lengths the kernel produced (x * 1 or x * 0, so -0.0 for
    # masked negatives)
    keep = np.arange(D)[None, None, :] < L[..., None]
    want = (x.reshape(M, G, D).astype(np.float32) * keep).reshape(M, G * D)
    want_t = torch.from_numpy(want).to(dtype)
    gb, wb = _bits(got_out.reshape(M, G * D)), _bits(want_t)
    bad = np.argwhere(gb != wb)
    assert bad.size == 0, (f"{name}: masked output differs at {len(bad)} places, first "
                           f"{bad[:4].tolist()}: got {gb[tuple(bad[0])]:#06x} want "
                           f"{wb[tuple(bad[0])]:#06x}")
    return (L == ref_len).mean(), tie.mean()


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_cutoff_matches_oracle(dev, name):
    G, D, M, dtype, low_rank, scale = CASES[name]
    print(f"[gpu] cutoff {name}", flush=True)
    seed = zlib.crc32(name.encode()) % 100000
    xk, Wk, bk = _inputs(G, D, M, dtype, scale, seed=seed)
    xv, Wv, bv = _inputs(G, D, M, dtype, scale, seed=seed + 1)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    head = CK.CutoffHead(t(Wk) if G > 1 else t(Wk[0]), t(bk), t(Wv) if G > 1 else t(Wv[0]), t(bv),
                         groups=G, low_rank=low_rank)
    pad = 64 if M % 2 else 0  # odd M: rows inside a wider buffer (row stride G*D + 64)
    ks = _dev_rows(xk, dtype, dev, pad)
    vs = _dev_rows(xv, dtype, dev, pad)
    k_out, v_out, len_k, len_v, _, _ = head.kv_process_fused(ks, vs)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(dev).cuda_stream
    ws = CK._WS_CACHE[(dev.index, st)]
    n = M * G * D * 2
    lgk = ws[:n].view(dtype)
    lgv = ws[n:2 * n].view(dtype)
    fk, tk = _check(name + " K", k_out, len_k, xk, Wk, bk, dtype, low_rank, lgk)
    fv, tv = _check(name + " V", v_out, len_v, xv, Wv, bv, dtype, low_rank, lgv)
    print(f"[gpu] cutoff {name}: lengths equal to the exact-arithmetic oracle on {fk:.3f} (K) / "
          f"{fv:.3f} (V); rounding-tie rows {tk:.3f} / {tv:.3f}", flush=True)
    assert len_k.dtype == torch.int32
    assert len_k.shape == ((M,) if G == 1 else (M, G))


@pytest.mark.gpu
def test_cutoff_reference_shapes_and_spread(dev):
    """Reference call shape (B, S, D) -> lengths (B, S); weights that spread the mass give
    lengths over the whole range."""
    print("[gpu] cutoff reference shapes", flush=True)
    B, S, D = 4, 3, 1024
    dtype = torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(5)
    Wk = (torch.randn(D, D, generator=g) * 4 / D ** 0.5).to(dev, dtype)
    bk = torch.randn(1, D, generator=g).to(dev, dtype)
    head = CK.CutoffHead(Wk, bk, Wk.clone(), bk.clone())
    k = torch.randn(B, S, D, generator=g).to(dev, dtype)
    k_out, v_out, len_k, len_v, a, b = head.kv_process_fused(k, k.clone())
    assert (a, b) == (1, 1)
    assert k_out.shape == (B, S, D) and len_k.shape == (B, S) and len_k.dtype == torch.int32
    assert torch.equal(len_k, len_v) and torch.equal(k_out, v_out)
    assert int(len_k.min()) >= 0 and int(len_k.max()) <= D


@pytest.mark.gpu
def test_cutoff_feeds_cache_append(dev):
    """Per-head decode step: cutoff (B, 1, G*D) -> per-head cache rows (B*G, 1, D) appended with
    the cutoff lengths; the packed payload is each row's first len values."""
    print("[gpu] cutoff -> append", flush=True)
    B, G, D = 4, 8, 128
    dtype = torch.bfloat16
    x, W, b = _inputs(G, D, B, dtype, 3.0, seed=77)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    head = CK.CutoffHead(t(W), t(b), t(W), t(b), groups=G)
    cache = CustomDynamicCache()
    for step in range(3):
        ks = t(x).reshape(B, 1, G * D)
        k_out, v_out, len_k, len_v, _, _ = head.kv_process_fused(ks, ks)
        rows_k = k_out.view(B, 1, G, D).transpose(1, 2).reshape(B * G, 1, D)
        rows_len = len_k.view(B, 1, G).transpose(1, 2).reshape(B * G, 1)
        cache.update_sp(rows_k, rows_len.contiguous(), rows_k, rows_len.contiguous(), D, 0, D)
    slot = cache.key_cache_sp[0]
    flat, lens, offs = slot[0], slot[1], slot[2]
    lens_h = lens[:, :3].cpu().numpy()
    assert (lens_h == rows_len.cpu().numpy()).all()
    fh = flat.float().cpu().numpy()
    xr = x.reshape(B, G, D).reshape(B * G, D)
    for r in range(B * G):
        L = int(lens_h[r, 0])
        for s in range(3):
            o = int(offs[r, s])
            assert (fh[r, o:o + L] == xr[r, :L]).all()


@pytest.mark.gpu
def test_cutoff_rejects_unsupported_width(dev):
    print("[gpu] cutoff unsupported width", flush=True)
    D = 96
    W = torch.zeros(D, D, dtype=torch.float16, device=dev)
    b = torch.zeros(1, D, dtype=torch.float16, device=dev)
    head = CK.CutoffHead(W, b, W, b)
    x = torch.zeros(2, D, dtype=torch.float16, device=dev)
    with pytest.raises(NotImplementedError):
        head.kv_process_fused(x, x)


def _random_cutoff(i: int):
    """Case i of a seeded sweep over the cutoff head: width D (64 to 1024), groups, rows (1 to
    600, log-uniform: decode steps and prompt chunks, so both the single-launch and the
    two-kernel paths), dtype, low_rank cap and weight scale (peaked or spread softmax)."""
    rng = np.random.default_rng(5000 + i)
    D = int(rng.choice([64, 128, 128, 256, 512, 1024]))
    G = int(rng.choice([1, 2, 4, 8])) if D <= 128 else int(rng.choice([1, 2]))
    M = int(np.exp(rng.uniform(0, np.log(600))))
    M = max(1, min(M, int(3e8 // (G * D * D))))
    dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float16
    low_rank = None if rng.random() < 0.6 else int(rng.integers(1, D + 1))
    return G, D, M, dtype, low_rank, float(rng.uniform(1.0, 5.0))


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(20))
def test_random_cutoff_shapes_against_oracle(dev, i):
    G, D, M, dtype, low_rank, scale = _random_cutoff(i)
    name = f"random {i} (G={G} D={D} M={M} {dtype} low_rank={low_rank} scale={scale:.2f})"
    print(f"[gpu] cutoff {name}", flush=True)
    xk, Wk, bk = _inputs(G, D, M, dtype, scale, seed=6000 + i)
    xv, Wv, bv = _inputs(G, D, M, dtype, scale, seed=7000 + i)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    head = CK.CutoffHead(t(Wk) if G > 1 else t(Wk[0]), t(bk), t(Wv) if G > 1 else t(Wv[0]), t(bv),
                         groups=G, low_rank=low_rank)
    pad = 64 * (i % 2)  # every other case: rows inside a wider buffer
    k_out, v_out, len_k, len_v, _, _ = head.kv_process_fused(_dev_rows(xk, dtype, dev, pad),
                                                             _dev_rows(xv, dtype, dev, pad))
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(dev).cuda_stream
    ws = CK._WS_CACHE[(dev.index, st)]
    n = M * G * D * 2
    _check(name + " K", k_out, len_k, xk, Wk, bk, dtype, low_rank, ws[:n].view(dtype))
    _check(name + " V", v_out, len_v, xv, Wv, bv, dtype, low_rank, ws[n:2 * n].view(dtype))
