"""Pins the cutoff-head oracle (oracle/cutoff.py) against closed forms, a scalar-loop restatement
and torch's own evaluation of the reference formula (compressed_attention.py:84-119)."""
import numpy as np
import pytest
import torch

from oracle import cutoff as C
from oracle.attention import round_to

DTYPES = ["bfloat16", "float16"]


def _rand(shape, rng, scale, dtype):
    return round_to(rng.standard_normal(shape) * scale, dtype).astype(np.float64)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [64, 128, 1024])
def test_uniform_logits_closed_form(dtype, D):
    # W = 0, b = 0: p = 1/D, c_m = (m+1)/D (exact in both dtypes for these D),
    # len = #{m : (m+1)/D >= thr} = D - ceil(thr * D) + 1
    x = np.ones((3, D))
    W = np.zeros((1, D, D))
    b = np.zeros((1, D))
    out, lens, logits, c, thr = C.cutoff(x, W, b, dtype)
    want = D - int(np.ceil(thr * D)) + 1
    assert (lens == want).all(), (lens, want)
    assert thr == float(round_to(np.float32(0.1), dtype))
    assert (out[:, :want] == 1).all() and (out[:, want:] == 0).all()


@pytest.mark.parametrize("dtype", DTYPES)
def test_dominant_logit_closed_form(dtype):
    # one logit far above the others at index k: p_k ~ 1, c_m ~ 0 before k and ~ 1 from k on,
    # so len = D - k
    D = 128
    for k in (0, 1, 37, 127):
        b = np.zeros((1, D))
        b[0, k] = 30.0
        out, lens, _, _, _ = C.cutoff(np.ones((1, D)), np.zeros((1, D, D)), b, dtype)
        assert lens[0, 0] == D - k, (k, lens)


@pytest.mark.parametrize("dtype", DTYPES)
def test_low_rank_and_negative_zero(dtype):
    rng = np.random.default_rng(3)
    D = 64
    x = _rand((4, D), rng, 1.0, dtype)
    W = np.zeros((1, D, D))
    b = np.zeros((1, D))
    out, lens, _, _, _ = C.cutoff(x, W, b, dtype, low_rank=20)
    assert (lens == 20).all()
    assert (out[:, :20] == x[:, :20].astype(np.float32)).all()
    neg = x[:, 20:] < 0
    # masked negatives are -0.0 as in the reference's x * mask
    assert np.signbit(out[:, 20:][neg]).all() and (out[:, 20:] == 0).all()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("G,D", [(1, 8), (2, 8), (3, 16)])
def test_matches_scalar_loops(dtype, G, D):
    rng = np.random.default_rng(G * 100 + D)
    M = 5
    x = _rand((M, G * D), rng, 1.0, dtype)
    W = _rand((G, D, D), rng, 0.7, dtype)
    b = _rand((G, D), rng, 0.5, dtype)
    out, lens, _, c, thr = C.cutoff(x, W, b, dtype, low_rank=D - 2)
    out2, lens2 = C.cutoff_loops(x, W, b, dtype, low_rank=D - 2)
    # the loop sums in a different order: any difference must sit on a rounding boundary
    amb = C.ambiguous_rows(c, thr, 4 * np.finfo(np.float16).eps * thr)
    assert ((lens == lens2) | amb).all()
    same = np.repeat(lens == lens2, D, axis=1)
    assert (out[same] == out2[same]).all()


@pytest.mark.parametrize("dtype", DTYPES)
def test_matches_torch_reference_formula(dtype):
    """torch (CPU) evaluating the reference's expressions step by step in the compute dtype:
    addmm -> softmax -> cumsum -> flip -> >= 0.1 -> sum, x * mask."""
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    rng = np.random.default_rng(11)
    M, D = 64, 128
    x = _rand((M, D), rng, 1.0, dtype)
    W = _rand((1, D, D), rng, 0.12, dtype)
    b = _rand((1, D), rng, 1.0, dtype)
    out, lens, logits, c, thr = C.cutoff(x, W, b, dtype)
    xt = torch.tensor(x, dtype=tdt)
    Wt = torch.tensor(W[0], dtype=tdt)
    bt = torch.tensor(b[0], dtype=tdt)
    lg = torch.addmm(bt.float(), xt.float(), Wt.float()).to(tdt)  # fp32 accumulate, dtype out
    mask = torch.softmax(lg.float(), dim=-1).to(tdt).float().cumsum(-1).to(tdt).flip(-1)
    hard = mask >= torch.tensor(0.1, dtype=tdt)
    tl = hard.sum(-1, dtype=torch.int32).numpy()
    tout = (xt * hard.to(tdt)).float().numpy()
    amb = C.ambiguous_rows(c, thr, 8 * thr * (2.0 ** -10 if dtype == "float16" else 2.0 ** -7))
    assert ((tl == lens[:, 0]) | amb[:, 0]).all()
    assert (tl == lens[:, 0]).mean() > 0.9
    ok = tl == lens[:, 0]
    assert (tout[ok] == out[ok]).all()
    # the prefix-mask reading of flip(cumsum) >= thr: every torch mask is a prefix
    h = hard.numpy()
    assert all(h[i, : tl[i]].all() and not h[i, tl[i]:].any() for i in range(M))


def test_length_bounds_bracket():
    rng = np.random.default_rng(5)
    c = np.sort(rng.random((10, 2, 64)), axis=-1)
    lo, hi = C.length_bounds(c, 0.1, 0.01)
    exact = (c >= 0.1).sum(-1)
    assert (lo <= exact).all() and (exact <= hi).all()
