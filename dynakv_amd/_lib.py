"""ctypes binding of ``libdynakv_amd.so`` (the C ABI declared in ``include/dynakv_amd.h``).

The library is loaded lazily and only from this package's ``lib/`` directory. There is no
fallback: if the library is missing the call raises, so a GPU run can never silently take a
CPU or eager-PyTorch path.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libdynakv_amd.so"

DKV_F32, DKV_F16, DKV_BF16 = 0, 1, 2
DKV_OK, DKV_E_ARG, DKV_E_UNSUPPORTED, DKV_E_WORKSPACE, DKV_E_SCRATCH = 0, -1, -2, -3, -4
DKV_NOALLOC_SCRATCH_FLOATS = 1 << 20
DKV_E_HIP_BASE = 1000
DKV_ROUTE_FUSED, DKV_ROUTE_TWO_STAGE = 0, 1

_DTYPE_CODE = {torch.float32: DKV_F32, torch.float16: DKV_F16, torch.bfloat16: DKV_BF16}

_vp, _ll, _i, _f = C.c_void_p, C.c_longlong, C.c_int, C.c_float

# name -> (restype, argtypes); must match include/dynakv_amd.h
_SIGNATURES = {
    "dkv_version": (_i, []),
    "dkv_status_string": (C.c_char_p, [_i]),
    "dkv_flat_range_elems": (_ll, [_ll, _ll, _ll]),
    "dkv_view_extent_elems": (_ll, [_i, _vp, _vp]),
    "dkv_append_decode": (_i, [_vp, _i, _vp, _ll, _vp, _ll, _vp, _ll, _vp, _vp, _ll, _ll, _vp, _i, _i, _i]),
    "dkv_append_decode_kv": (_i, [_vp, _i, _i, _i, _i,
                                  _vp, _ll, _vp, _ll, _vp, _ll, _vp, _vp, _ll, _ll, _vp,
                                  _vp, _ll, _vp, _ll, _vp, _ll, _vp, _vp, _ll, _ll, _vp]),
    "dkv_append_prefill": (_i, [_vp, _i, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _vp, _vp, _ll, _ll,
                                _vp, _i, _i, _i, _i]),
    "dkv_append_prefill_kv": (_i, [_vp, _i, _i, _i, _i, _i,
                                   _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _vp, _vp, _ll, _ll, _vp,
                                   _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _vp, _vp, _ll, _ll, _vp]),
    "dkv_decompress": (_i, [_vp, _i, _vp, _ll, _vp, _vp, _ll, _ll, _vp, _i, _i, _i]),
    "dkv_scores": (_i, [_vp, _i, _i, _i, _i, _vp, _ll, _ll, _vp, _ll, _ll, _i, _vp, _ll,
                        _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll, _ll, _i, _i, _i, _i, _i, _f]),
    "dkv_av": (_i, [_vp, _i, _i, _i, _i, _vp, _ll, _ll, _ll, _vp, _ll, _ll, _i, _vp, _ll,
                    _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll, _i, _i, _i, _i, _i]),
    "dkv_joint_scores": (_i, [_vp, _i, _i, _i, _vp, _ll, _ll, _vp, _ll, _ll, _i, _vp, _ll,
                              _vp, _ll, _ll, _vp, _ll, _ll, _vp, _i, _vp, _ll, _vp, _ll, _ll,
                              _ll, _i, _i, _i, _i, _i]),
    "dkv_joint_scores_workspace_ints": (_ll, [_i, _i]),
    "dkv_joint_av_workspace_floats": (_ll, [_i, _i, _i, _i]),
    "dkv_joint_av": (_i, [_vp, _i, _i, _i, _i, _vp, _ll, _ll, _ll, _vp, _ll, _ll, _i, _vp, _ll,
                          _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _vp, _ll, _ll,
                          _i, _i, _i, _i, _i]),
    "dkv_splitk_workspace_floats": (_ll, [_i, _i, _i, _i, _i, _i]),
    "dkv_splitk_choose_split": (_i, [_i, _i, _i]),
    "dkv_dense_workspace_floats": (_ll, [_i, _i, _i, _i, _i]),
    "dkv_dense_choose_split": (_i, [_i, _i, _i]),
    "dkv_recon_kv": (_i, [_vp, _i, _vp, _vp, _ll, _ll, _vp, _vp, _ll, _ll, _vp, _vp, _ll, _ll,
                          _i, _i, _i, _i, _i, _vp, _i]),
    "dkv_dense_append": (_i, [_vp, _i, _vp, _ll, _vp, _vp, _ll, _i, _i, _i, _i, _i, _f]),
    "dkv_decode_dense": (_i, [_vp, _i, _vp, _ll, _ll, _vp, _vp, _ll, _i, _vp, _ll, _vp, _ll, _ll,
                              _i, _i, _i, _i, _i, _i]),
    "dkv_rope_table_floats": (_ll, [_i]),
    "dkv_rope_table": (_i, [_vp, _vp, _i, _i, _f]),
    "dkv_decode_splitk": (_i, [_vp, _i, _i, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll,
                               _vp, _ll, _vp, _ll, _vp, _vp, _ll, _ll, _vp, _vp, _ll, _ll,
                               _vp, _i, _vp, _ll, _vp, _ll, _ll, _i,
                               _i, _i, _i, _i, _i, _i, _i, _i]),
    "dkv_decode_splitk_noalloc": (_i, [_vp, _i, _i, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll,
                                       _vp, _ll, _vp, _ll, _vp, _vp, _ll, _ll, _vp, _vp, _ll, _ll,
                                       _vp, _i, _vp, _ll, _ll, _i,
                                       _i, _i, _i, _i, _i, _i, _i, _i]),
    "dkv_profile_begin": (_i, [_i]),
    "dkv_profile_end": (_i, [_vp, _vp, _vp]),
    "dkv_selftest_layouts": (_i, [_vp, _vp]),
    "dkv_cutoff_workspace_bytes": (_ll, [_i, _i, _i]),
    "dkv_rope_dense": (_i, [_vp, _i, _vp, _ll, _ll, _i, _i, _i, _f]),
    "dkv_add_rmsnorm": (_i, [_vp, _i, _vp, _ll, _vp, _ll, _vp, _vp, _ll, _i, _i, _f]),
    "dkv_silu_mul": (_i, [_vp, _i, _vp, _ll, _vp, _ll, _i, _i]),
    "dkv_silu_mul_pairs": (_i, [_vp, _i, _vp, _ll, _vp, _ll, _i, _i]),
    "dkv_gemv": (_i, [_vp, _i, _vp, _ll, _vp, _ll, _vp, _ll, _i, _i, _i]),
    "dkv_gemv_rmsnorm": (_i, [_vp, _i, _vp, _ll, _vp, _ll, _vp, _f, _vp, _ll, _vp, _ll, _vp,
                              _ll, _i, _i, _i]),
    "dkv_gemv_glu": (_i, [_vp, _i, _vp, _ll, _vp, _ll, _vp, _f, _vp, _ll, _vp, _ll, _vp, _ll,
                          _i, _i, _i]),
    "dkv_decode_layer": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "dkv_prefill_attention": (_i, [_vp, _i, _vp, _ll, _ll, _ll, _vp, _ll, _ll, _ll, _ll,
                                   _vp, _ll, _ll, _ll, _ll, _vp, _i, _ll, _ll, _ll,
                                   _i, _i, _i, _i, _i, _i, _i, _f, _vp]),
    "dkv_rope_apply": (_i, [_vp, _i, _vp, _ll, _ll, _ll, _vp, _vp, _ll, _ll, _i, _i, _i]),
    "dkv_cutoff_kv": (_i, [_vp, _i, _vp, _vp, _ll, _vp, _vp, _vp, _vp, _f, _i, _vp, _vp, _ll,
                           _vp, _vp, _ll, _vp, _ll, _i, _i, _i]),
}

class DecodeLayerArgs(C.Structure):
    """``DkvDecodeLayer`` of include/dynakv_amd.h (field order and types must match)."""

    _fields_ = [
        ("dtype", _i), ("B", _i), ("G", _i), ("Hq", _i), ("R", _i), ("Dh", _i),
        ("low_rank", _i), ("switch_tokens", _i), ("threshold", _f), ("log_theta", _f),
        ("wt_k", _vp), ("wt_v", _vp), ("b_k", _vp), ("b_v", _vp),
        ("cut_ws", _vp), ("cut_ws_bytes", _ll),
        ("coef_k", _vp), ("coef_v", _vp), ("len_k", _vp), ("len_v", _vp),
        ("flat_k", _vp), ("flat_k_ld", _ll), ("lens_k", _vp), ("offs_k", _vp),
        ("tab_k_sb", _ll), ("tab_k_ss", _ll), ("ptr_k", _vp),
        ("flat_v", _vp), ("flat_v_ld", _ll), ("lens_v", _vp), ("offs_v", _vp),
        ("tab_v_sb", _ll), ("tab_v_ss", _ll), ("ptr_v", _vp),
        ("k_basis", _vp), ("k_unit", _ll), ("k_sr", _ll),
        ("v_basis", _vp), ("v_unit", _ll), ("v_sr", _ll),
        ("rope", _vp), ("rope_tiles", _i), ("split_ws", _vp), ("split_ws_floats", _ll),
        ("q_sb", _ll), ("coef_ld", _ll),
    ]


_lock = threading.Lock()
_lib = None


class DynaKVError(RuntimeError):
    """A HIP runtime failure reported by the native library."""


def load() -> C.CDLL:
    """Load the native library (once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"dynakv_amd native library not found at {LIB_PATH}; "
                    "build it with `python -m dynakv_amd.build`")
            # torch is imported first so its HIP runtime (same SONAME) is the one the
            # library binds to; streams and pointers are then shared with torch.
            lib = C.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(status: int, what: str) -> None:
    if status == DKV_OK:
        return
    msg = load().dkv_status_string(status).decode()
    if status in (DKV_E_ARG, DKV_E_WORKSPACE, DKV_E_SCRATCH):
        raise ValueError(f"{what}: {msg}")
    if status == DKV_E_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise DynaKVError(f"{what}: {msg} (status {status})")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}") from None


def flat_covers_rows(t: torch.Tensor) -> bool:
    """The C ABI's contract for packed flat buffers (rows, ld): rows * ld elements addressable
    from the base pointer inside the tensor's storage (each kernel's buffer resource for row r
    covers the elements from row r to the buffer's end, ``dkv_flat_range_elems``)."""
    if t.dim() != 2 or t.stride(0) < 0:
        return False
    avail = t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()
    return t.shape[0] * t.stride(0) <= avail


def view_extent(t: torch.Tensor) -> int:
    """Elements addressable from ``t.data_ptr()`` by its shape and strides (one past its last
    element), from the library's own definition (``dkv_view_extent_elems``)."""
    nd = t.dim()
    shape = (C.c_longlong * max(nd, 1))(*t.shape)
    stride = (C.c_longlong * max(nd, 1))(*t.stride())
    n = int(load().dkv_view_extent_elems(nd, shape, stride))
    if n < 0:
        raise ValueError("dkv_view_extent_elems rejected the view")
    return n


def flat_operand(t: torch.Tensor) -> torch.Tensor:
    """``t`` when it meets the flat-buffer contract (``flat_covers_rows``), else a contiguous
    copy (a column slice whose storage ends inside its last row's stride: the last row's
    resource would otherwise reach past the allocation)."""
    if flat_covers_rows(t):
        return t
    # clone rather than contiguous(): a one-row view counts as contiguous whatever its stride
    return t.clone(memory_format=torch.contiguous_format)


# Cached device buffers (workspaces, RoPE tables) replaced by larger ones. They stay allocated
# for the rest of the process instead of going back to torch's allocator: a HIP graph captured
# while one of them was current holds its address and writes into it on every replay. Caches
# grow at least twofold, so these add at most the size of the buffers in use.
_RETIRED_BUFFERS: list = []


def retire(t: torch.Tensor | None) -> None:
    """Keep a superseded cached device buffer allocated (see ``_RETIRED_BUFFERS``)."""
    if t is not None:
        _RETIRED_BUFFERS.append(t)


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on t's device."""
    if t.device.type != "cuda":
        raise RuntimeError(
            f"dynakv_amd kernels need device tensors (got {t.device}); there is no CPU path")
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
