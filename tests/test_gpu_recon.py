"""dkv_recon_kv (the compressed prefill's reconstruction of dense K and V) against float64.

K[t] = RoPE_{pos0+t}(basis_K^T c_K[t]) and V[t] = basis_V^T c_V[t] per cache row (reference
compressed_attention.py:359-386, the coefficients zero past each token's count as
get_origin_states returns them, compressed_cache.py:36-56): the kernel accumulates in fp32 and
rounds the projection to the dtype, then rotates the keys in fp32 and rounds again (the
reference's two steps), so V is within one rounding of its float64 value and K within two
roundings plus the rotation's fp32 slack (the oracle's RoPE angles,
oracle.attention.rope_cos_sin)."""
import numpy as np
import pytest
import torch

from dynakv_amd.kernels.prefill import recon_kv
from dynakv_amd.synthetic import random_orthogonal
from oracle.attention import apply_rope, rope_cos_sin

from helpers import cast_np

CASES = {
    # name: (B, G, S, R, dtype, pos0, strided_rows)
    "s1": (3, 8, 1, 128, torch.bfloat16, 0, False),
    "b1_2k_bf16_strided": (1, 8, 2048, 128, torch.bfloat16, 0, True),
    "b2_77_fp16": (2, 8, 77, 128, torch.float16, 0, False),
    "r64_bf16": (1, 2, 130, 64, torch.bfloat16, 0, False),
    "pos0_fp16": (2, 4, 40, 128, torch.float16, 37, False),
}
THETA = 500000.0


def _inputs(B, G, S, R, dtype, seed):
    rng = np.random.default_rng(seed)
    rows = B * G
    ck = rng.standard_normal((rows, S, R)).astype(np.float32)
    cv = rng.standard_normal((rows, S, R)).astype(np.float32)
    lk = rng.integers(0, R + 1, size=(rows, S))
    lv = rng.integers(0, R + 1, size=(rows, S))
    ar = np.arange(R)
    ck[ar[None, None, :] >= lk[..., None]] = 0.0
    cv[ar[None, None, :] >= lv[..., None]] = 0.0
    kb = np.stack([random_orthogonal(128, rng)[:R] for _ in range(G)]).astype(np.float32)
    vb = np.stack([random_orthogonal(128, rng)[:R] for _ in range(G)]).astype(np.float32)
    return [cast_np(a, dtype) for a in (ck, cv, kb, vb)]


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_recon_kv_matches_float64(dev, name):
    B, G, S, R, dtype, pos0, strided = CASES[name]
    print(f"[gpu] recon_kv {name}", flush=True)
    ck, cv, kb, vb = _inputs(B, G, S, R, dtype, seed=len(name) * 7 + S)
    t = lambda a: torch.from_numpy(a).to(device=dev, dtype=dtype)  # noqa: E731
    if strided:
        # the batch-1 model path: rows b*G + g as views of (S, G, R) token-major coefficients
        ckd = t(ck.reshape(G, S, R).transpose(1, 0, 2).copy()).transpose(0, 1)
        cvd = t(cv.reshape(G, S, R).transpose(1, 0, 2).copy()).transpose(0, 1)
        assert ckd.stride() == (R, G * R, 1)
    else:
        ckd, cvd = t(ck), t(cv)
    out = recon_kv(ckd, cvd, t(kb), t(vb), batch=B, theta=THETA, pos0=pos0)
    assert out is not None
    k, v = out
    assert k.shape == (B, G, S, 128) and v.shape == (B, G, S, 128)
    kref = np.empty((B * G, S, 128))
    vref = np.empty((B * G, S, 128))
    pair = np.empty((B * G, S, 128))
    cos, sin = rope_cos_sin(np.arange(pos0, pos0 + S), 128, THETA)
    for r in range(B * G):
        g = r % G
        k0 = ck[r].astype(np.float64) @ kb[g].astype(np.float64)
        kref[r] = apply_rope(k0, cos, sin)
        vref[r] = cv[r].astype(np.float64) @ vb[g].astype(np.float64)
        p = np.abs(k0[:, :64]) + np.abs(k0[:, 64:])
        pair[r] = np.concatenate([p, p], axis=-1)
    # the rotation's fp32 slack: the kernel composes R(16T) R(n) from the RoPE table's rows
    # (cos and sin of the fp32 angles 16T * inv_freq and n * inv_freq), where the oracle rounds
    # float32(pos) * inv_freq once: the angles differ by up to a unit in the last place of fp32
    # at |angle| < pos0 + S; plus the fp32 products of the composition and the rotation
    slack_k = ((pos0 + S) * 2.0 ** -22 + 2.0 ** -21) * pair
    bad = []
    for got, ref, what in ((k, kref, "K"), (v, vref, "V")):
        g64 = got.reshape(B * G, S, 128).float().cpu().numpy().astype(np.float64)
        ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
        err = np.abs(g64 - ref)
        bound = ulp * np.abs(ref) + 3e-5
        if what == "K":
            # the unrotated projection's rounding (unit roundoff on each of the pair, carried
            # through the rotation) and the slack, both again under the final rounding
            bound = bound + (1.0 + ulp) * (slack_k + ulp * pair)
        w = np.unravel_index(np.argmax(err / bound), err.shape)
        print(f"[gpu]   {what}: max_abs={err.max():.3e} worst err/bound={np.max(err / bound):.3f} "
              f"at (row, token, dim) {tuple(int(i) for i in w)}: got {g64[w]:.5f} ref {ref[w]:.5f}",
              flush=True)
        if not np.all(err <= bound):
            bad.append(what)
    assert not bad, f"{name} {bad}"


@pytest.mark.gpu
def test_recon_kv_declines_unsupported_ranks(dev):
    ck, cv, kb, vb = _inputs(1, 2, 10, 40, torch.bfloat16, seed=3)
    ckd = torch.from_numpy(ck[..., :36].copy()).to(dev, torch.bfloat16)
    kbd = torch.from_numpy(kb[:, :36].copy()).to(dev, torch.bfloat16)
    # R = 36 is not a multiple of 8: the wrapper returns None (library-GEMM path)
    assert recon_kv(ckd, ckd.clone(), kbd, kbd.clone(), batch=1, theta=THETA) is None
