"""Fused residual-add + RMSNorm and SwiGLU product (dkv_model.hip) against torch: the residual
add is bit-exact (one fp32 add of two dtype values, rounded once); the normalised output and
the activation product are within two units in the last place of the dtype, with almost all
elements identical: each is rounded twice (the normalised value or silu(g), then its product
with the weight or with up), and the first rounding can land on the neighbouring value (the
kernel sums the squares in a different order than the reference's reduction, and evaluates
e^-g with the device exp)."""
import pytest
import torch
import torch.nn.functional as F

from dynakv_amd.kernels.model_ops import add_rmsnorm_, silu_mul, silu_mul_pairs


def _ulps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units in the last place between same-sign 16-bit floats."""
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    return (ai - bi).abs()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,H", [(1, 4096), (5, 4096), (3, 1024), (2, 8192), (300, 512)])
def test_add_rmsnorm(dev, dtype, rows, H):
    print(f"[gpu] add_rmsnorm {dtype} rows={rows} H={H}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(rows * 7919 + H)
    x = torch.randn(rows, H, generator=g).to(dtype).to(dev)
    d = torch.randn(rows, H, generator=g).to(dtype).to(dev)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype).to(dev)
    eps = 1e-5
    r = (x.float() + d.float()).to(dtype)
    xs = x.clone()
    out = add_rmsnorm_(xs, d, w, eps)
    assert torch.equal(xs, r), "residual add"
    rf = r.double()
    ref = (rf * torch.rsqrt(rf.pow(2).mean(-1, keepdim=True) + eps)).to(dtype)
    ref = (ref.double() * w.double()).to(dtype)
    u = _ulps(out, ref)
    print(f"[parity] add_rmsnorm: max ulp {int(u.max())}, differing {float((u > 0).float().mean()):.4f}",
          flush=True)
    assert int(u.max()) <= 2 and float((u > 0).float().mean()) < 0.02
    # without the residual the input is left as it is
    xs2 = r.clone()
    out2 = add_rmsnorm_(xs2, None, w, eps)
    assert torch.equal(xs2, r) and torch.equal(out2, out)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,Fdim", [(1, 14336), (4, 14336), (7, 1000), (3, 8)])
def test_silu_mul(dev, dtype, rows, Fdim):
    print(f"[gpu] silu_mul {dtype} rows={rows} F={Fdim}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(rows * 31 + Fdim)
    gu = (3 * torch.randn(rows, 2 * Fdim, generator=g)).to(dtype).to(dev)
    out = silu_mul(gu)
    gate, up = gu[:, :Fdim].double(), gu[:, Fdim:].double()
    ref = ((gate / (1 + torch.exp(-gate))).to(dtype).double() * up).to(dtype)
    u = _ulps(out, ref)
    print(f"[parity] silu_mul: max ulp {int(u.max())}, differing {float((u > 0).float().mean()):.4f}",
          flush=True)
    assert int(u.max()) <= 2 and float((u > 0).float().mean()) < 0.02
    # the torch expression the model used before these kernels
    t = F.silu(gu[:, :Fdim]) * gu[:, Fdim:]
    assert int(_ulps(out, t).max()) <= 2


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (4, 1024, 4096), (3, 28672, 4096),
                                   (2, 4096, 14336), (4, 4096, 14336), (8, 130, 1024),
                                   (5, 7, 96), (8, 40, 8192)])
def test_gemv(dev, dtype, M, N, K):
    """Against a float64 product of the same inputs: error within fp32 accumulation plus one
    rounding of y."""
    from dynakv_amd import _lib
    from dynakv_amd.kernels.model_ops import linear
    print(f"[gpu] gemv {dtype} M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M * 1000003 + N * 31 + K)
    x = torch.randn(M, K, generator=g).to(dtype).to(dev)
    w = (0.02 * torch.randn(N, K, generator=g)).to(dtype).to(dev)
    y = torch.empty(M, N, dtype=dtype, device=dev)
    rc = _lib.load().dkv_gemv(_lib.stream_of(x), _lib.dtype_code(dtype), x.data_ptr(), K,
                              w.data_ptr(), K, y.data_ptr(), N, M, N, K)
    _lib.check(rc, "dkv_gemv")
    ref = x.double() @ w.double().T
    err = (y.double() - ref).abs()
    bound = ref.abs() * 2.0 ** (-8 if dtype == torch.bfloat16 else -11) + 1e-5 * (
        x.double().abs() @ w.double().abs().T)
    print(f"[parity] gemv: max err {float(err.max()):.3e}, worst ratio "
          f"{float((err / bound).max()):.3f}", flush=True)
    assert bool((err <= bound).all())
    # the model's entry point: this kernel when x can be staged in LDS, the library GEMM else
    y2 = linear(x, w)
    if M * K * 2 <= 64 * 1024:
        assert torch.equal(y2, y)
    else:
        assert bool(((y2.double() - ref).abs() <= bound).all())



@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(1, 6144, 4096), (4, 28672, 4096), (2, 128256, 4096),
                                   (8, 100, 512), (3, 40, 8192)])
@pytest.mark.parametrize("with_delta", [True, False])
def test_gemv_rmsnorm_is_norm_then_gemv(dev, dtype, M, N, K, with_delta):
    """The fused norm + projection equals add_rmsnorm_ followed by dkv_gemv bit for bit, and
    returns the updated residual; the kernel does not touch x."""
    from dynakv_amd import _lib
    from dynakv_amd.kernels.model_ops import rmsnorm_linear
    print(f"[gpu] gemv_rmsnorm {dtype} M={M} N={N} K={K} delta={with_delta}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g).to(dtype).to(dev)
    d = torch.randn(M, K, generator=g).to(dtype).to(dev) if with_delta else None
    wn = (1 + 0.1 * torch.randn(K, generator=g)).to(dtype).to(dev)
    w = (0.02 * torch.randn(N, K, generator=g)).to(dtype).to(dev)
    x0 = x.clone()
    y, r = rmsnorm_linear(x.clone(), d, wn, 1e-5, w)
    if M > 2:  # the model's entry point takes the unfused pair here; the kernel itself:
        r = torch.empty_like(x) if with_delta else x
        y = torch.empty(M, N, dtype=dtype, device=dev)
        _lib.check(_lib.load().dkv_gemv_rmsnorm(
            _lib.stream_of(x), _lib.dtype_code(dtype), x.data_ptr(), K,
            d.data_ptr() if with_delta else None, K, wn.data_ptr(), 1e-5,
            r.data_ptr() if with_delta else None, K, w.data_ptr(), K, y.data_ptr(), N, M, N, K),
            "dkv_gemv_rmsnorm")
    assert torch.equal(x, x0), "x untouched"
    xs = x.clone()
    h = add_rmsnorm_(xs, d, wn, 1e-5)
    assert torch.equal(r, xs), "residual"
    y_ref = torch.empty(M, N, dtype=dtype, device=dev)
    _lib.check(_lib.load().dkv_gemv(_lib.stream_of(h), _lib.dtype_code(dtype), h.data_ptr(), K,
                                    w.data_ptr(), K, y_ref.data_ptr(), N, M, N, K), "dkv_gemv")
    assert torch.equal(y, y_ref), "projection of the normalised rows"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,F,K,norm", [(1, 14336, 4096, True), (2, 14336, 4096, True),
                                        (4, 14336, 4096, False), (1, 136, 512, True),
                                        (3, 1000, 1024, False), (8, 64, 256, False)])
def test_gemv_glu_is_gemv_then_silu_mul(dev, dtype, M, F, K, norm):
    """The gate/up projection with the SwiGLU product in its epilogue (interleaved gate/up
    rows) equals dkv_gemv of the de-interleaved weights followed by silu_mul, bit for bit, with
    the norm folded in (one or two rows) or not."""
    from dynakv_amd import _lib
    from dynakv_amd.kernels.model_ops import rmsnorm_glu
    print(f"[gpu] gemv_glu {dtype} M={M} F={F} K={K} norm={norm}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M * 5 + F + K)
    x = torch.randn(M, K, generator=g).to(dtype).to(dev)
    d = torch.randn(M, K, generator=g).to(dtype).to(dev)
    wn = (1 + 0.1 * torch.randn(K, generator=g)).to(dtype).to(dev)
    w = (0.05 * torch.randn(2 * F, K, generator=g)).to(dtype).to(dev)  # rows interleaved
    lib = _lib.load()
    # reference: normalised rows, then the [gate | up] projection and silu_mul
    xs = x.clone()
    hn = add_rmsnorm_(xs, d, wn, 1e-5)
    w_halves = torch.cat([w[0::2], w[1::2]]).contiguous()
    gu = torch.empty(M, 2 * F, dtype=dtype, device=dev)
    _lib.check(lib.dkv_gemv(_lib.stream_of(hn), _lib.dtype_code(dtype), hn.data_ptr(), K,
                            w_halves.data_ptr(), K, gu.data_ptr(), 2 * F, M, 2 * F, K), "dkv_gemv")
    ref = silu_mul(gu)
    h = torch.empty(M, F, dtype=dtype, device=dev)
    if norm:
        r = torch.empty_like(x)
        rc = lib.dkv_gemv_glu(_lib.stream_of(x), _lib.dtype_code(dtype), x.data_ptr(), K,
                              d.data_ptr(), K, wn.data_ptr(), 1e-5, r.data_ptr(), K, w.data_ptr(),
                              K, h.data_ptr(), F, M, F, K)
        _lib.check(rc, "dkv_gemv_glu")
        assert torch.equal(r, xs), "residual"
    else:
        rc = lib.dkv_gemv_glu(_lib.stream_of(hn), _lib.dtype_code(dtype), hn.data_ptr(), K, None,
                              0, None, 0.0, None, 0, w.data_ptr(), K, h.data_ptr(), F, M, F, K)
        _lib.check(rc, "dkv_gemv_glu")
    assert torch.equal(h, ref), "silu(gate) * up in the epilogue"
    # the model's entry point agrees with the launch it makes
    h2, r2 = rmsnorm_glu(x.clone(), d, wn, 1e-5, w)
    assert torch.equal(h2, ref) and torch.equal(r2, xs)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rmsnorm_glu_many_rows_fallback(dev, dtype):
    """More than eight rows (a prompt) take the library GEMM and silu_mul_pairs of its
    interleaved output: silu_mul of the de-interleaved halves, bit for bit."""
    from dynakv_amd.kernels.model_ops import rmsnorm_glu
    print(f"[gpu] rmsnorm_glu fallback {dtype}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(99)
    M, F, K = 40, 512, 1024
    x = torch.randn(M, K, generator=g).to(dtype).to(dev)
    d = torch.randn(M, K, generator=g).to(dtype).to(dev)
    wn = (1 + 0.1 * torch.randn(K, generator=g)).to(dtype).to(dev)
    w = (0.05 * torch.randn(2 * F, K, generator=g)).to(dtype).to(dev)
    h, r = rmsnorm_glu(x.clone(), d, wn, 1e-5, w)
    xs = x.clone()
    hn = add_rmsnorm_(xs, d, wn, 1e-5)
    assert torch.equal(r, xs)
    gu = torch.nn.functional.linear(hn, w)
    ref = silu_mul(torch.cat([gu[:, 0::2], gu[:, 1::2]], dim=1).contiguous())
    assert torch.equal(h, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,Fdim", [(1, 8), (40, 1000), (300, 14336)])
def test_silu_mul_pairs_is_silu_mul_of_the_halves(dev, dtype, rows, Fdim):
    print(f"[gpu] silu_mul_pairs {dtype} rows={rows} F={Fdim}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(rows * 7 + Fdim)
    gu = (3 * torch.randn(rows, 2 * Fdim, generator=g)).to(dtype).to(dev)
    out = silu_mul_pairs(gu)
    ref = silu_mul(torch.cat([gu[:, 0::2], gu[:, 1::2]], dim=1).contiguous())
    assert torch.equal(out, ref)
    # torch's own expression stays within two units in the last place (silu by another formula)
    assert int(_ulps(out, F.silu(gu[:, 0::2]) * gu[:, 1::2]).max()) <= 2
