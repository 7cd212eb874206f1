"""Shared helpers for the GPU parity tests (not collected by pytest)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import attention as A
from oracle.packing import pack_rows

TOL_ABS = 2e-3  # north-star bar for fp16/bf16 outputs against the fp32+ oracle
TOL_REL = 1e-2  # normwise: max|a-b| / max|b|

NP_OF = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def cast_np(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Round an fp32 array to ``dtype`` and return it as float32 (what the device will hold)."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dtype).float().numpy()


def packed_from_case(case, dtype: torch.dtype, device):
    """Pack a PackedCase with the oracle (rows = B*G) and upload it. Returns a dict of device
    tensors plus the fp32 host copies the oracle uses (already rounded to dtype)."""
    kc = cast_np(case.k_coef, dtype)
    vc = cast_np(case.v_coef, dtype)
    fk, lk, ok, _ = pack_rows(kc, case.k_len, case.R)
    fv, lv, ov, _ = pack_rows(vc, case.v_len, case.R)
    kb = cast_np(case.k_basis, dtype)
    vb = cast_np(case.v_basis, dtype)
    q = cast_np(case.q, dtype)

    def dev(x, dt=dtype):
        return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dt)

    return dict(
        q=dev(q), k_flat=dev(fk), v_flat=dev(fv),
        lens_k=dev(lk, torch.int32), offs_k=dev(ok, torch.int32),
        lens_v=dev(lv, torch.int32), offs_v=dev(ov, torch.int32),
        k_basis=dev(kb), v_basis=dev(vb),
        host=dict(q=q, fk=fk, lk=lk, ok=ok, fv=fv, lv=lv, ov=ov, kb=kb, vb=vb),
    )


def oracle_grouped(case, host, route: str, q_dtype: str, batches=None) -> np.ndarray:
    """Oracle output for the per-head layout; ``batches`` restricts to some batch rows."""
    hpg = case.Hq // case.G
    bsel = list(range(case.B)) if batches is None else list(batches)
    q = host["q"][bsel]
    return A.decode_attention(
        q, host["fk"], host["kb"], host["fv"], host["vb"], host["lk"], host["ok"], host["lv"],
        host["ov"], case.theta, route=route, q_dtype=q_dtype,
        row_of=lambda b, h: bsel[b] * case.G + h // hpg, basis_of=lambda h: h // hpg)


def assert_close(got: torch.Tensor | np.ndarray, ref: np.ndarray, what: str = "",
                 tol_abs: float = TOL_ABS, tol_rel: float = TOL_REL):
    g = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    r = np.asarray(ref, dtype=np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.isfinite(g).all() == np.isfinite(r).all(), f"{what}: finite mismatch"
    fin = np.isfinite(r)
    d = np.abs(g[fin] - r[fin])
    max_abs = float(d.max()) if d.size else 0.0
    scale = float(np.abs(r[fin]).max()) if d.size else 1.0
    max_rel = max_abs / max(scale, 1e-30)
    print(f"[parity] {what}: max_abs={max_abs:.3e} max_rel={max_rel:.3e} |ref|max={scale:.3e}",
          flush=True)
    assert max_abs <= tol_abs and max_rel <= tol_rel, \
        f"{what}: max_abs={max_abs:.3e} max_rel={max_rel:.3e} (|ref|max={scale:.3e})"
    return max_abs, max_rel
