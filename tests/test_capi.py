"""The C-ABI library loads and exports every function declared in include/dynakv_amd.h, the ctypes
signatures match the header's parameter counts, and host-only calls behave (no device needed)."""
import ctypes
import os
import re

import pytest
import torch

from dynakv_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "dynakv_amd.h")


def _header_declarations():
    """name -> (return type, [parameter types]) of every dkv_ function in the header."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(int|long long|const char\*)\s+(dkv_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(3).split(",") if p.strip() and p.strip() != "void"]
        # a parameter's type: its declaration without the trailing name
        types = [" ".join(re.sub(r"\w+$", "", p).split()) for p in params]
        out[m.group(2)] = (m.group(1), types)
    return out


def _header_functions():
    return {k: len(v[1]) for k, v in _header_declarations().items()}


# ctypes type each C type of the header must be bound with
_CTYPE = {"int": ctypes.c_int, "long long": ctypes.c_longlong, "float": ctypes.c_float,
          "const char*": ctypes.c_char_p}


def _ctype_of(c: str):
    if c.endswith("*"):  # every pointer parameter crosses as a void*
        return ctypes.c_void_p
    return _CTYPE[c]


def test_header_parses():
    fns = _header_functions()
    assert "dkv_decode_splitk" in fns and "dkv_append_decode" in fns
    assert len(fns) >= 13


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _header_functions():
        assert hasattr(lib, name), name


def test_ctypes_signatures_match_header():
    """Every binding's return and parameter types are the header's, position by position (a
    long long bound as int, or a float as a pointer, would pass a count check and corrupt the
    call)."""
    decls = _header_declarations()
    assert set(decls) == set(_lib.exported_symbols())
    for name, (ret, types) in decls.items():
        res, args = _lib._SIGNATURES[name]
        assert res is _CTYPE[ret], (name, "return", ret)
        assert len(args) == len(types), name
        for i, (c, bound) in enumerate(zip(types, args)):
            assert bound is _ctype_of(c), (name, i, c, bound)


def test_header_type_parser():
    """The parser reads pointer, const and multi-word types."""
    decls = _header_declarations()
    ret, types = decls["dkv_view_extent_elems"]
    assert ret == "long long" and types == ["int", "const long long*", "const long long*"]
    ret, types = decls["dkv_status_string"]
    assert ret == "const char*" and types == ["int"]
    assert decls["dkv_prefill_attention"][1][-2:] == ["float", "const int*"]


def test_traffic_record_measured_on_this_library():
    """bench.py reports the committed HBM-traffic record only for the library version it was
    measured on, so a version bump without a new measurement would drop roofline.traffic."""
    import json
    path = os.path.join(os.path.dirname(HEADER), "..", "profiles", "splitk_config3_traffic.json")
    with open(path) as f:
        rec = json.load(f)
    assert rec["dkv_version"] == _lib.load().dkv_version()
    assert rec["bytes_per_launch"] == rec["fetch_bytes_per_launch"] + rec["write_bytes_per_launch"]


def test_host_only_entry_points():
    lib = _lib.load()
    assert lib.dkv_version() >= 100
    assert lib.dkv_status_string(-1) == b"invalid argument"
    sl = lib.dkv_splitk_choose_split(16, 8, 8292)
    # about one workgroup per CU (256): 128 units -> two splits of the 8292 tokens
    assert sl % 64 == 0 and sl == 4160
    assert lib.dkv_splitk_choose_split(1, 8, 8292) % 64 == 0
    assert lib.dkv_splitk_choose_split(1, 8, 10) == 64
    # up to 256 tokens one split per unit (two tiles per wave at most, merged in LDS), at any
    # batch; past that several splits again
    for B in (1, 4, 16):
        for S in (1, 63, 64, 100, 192, 256):
            sl = lib.dkv_splitk_choose_split(B, 8, S)
            assert sl % 64 == 0 and S <= sl < S + 64, (B, S, sl)
    assert lib.dkv_splitk_choose_split(1, 8, 600) < 600
    assert lib.dkv_rope_table_floats(10) == (17 + 10) * 128
    assert lib.dkv_splitk_workspace_floats(16, 32, 8, 8292, 128, sl) > 0


def test_chooser_above_256_units():
    """With more units than CUs the chooser weighs the rounds of workgroups against the per
    workgroup fixed cost: long caches take more splits, 2K-token caches one."""
    lib = _lib.load()
    n_splits = lambda B, S: -(-S // lib.dkv_splitk_choose_split(B, 8, S))  # noqa: E731
    assert n_splits(48, 8193) == 2 and n_splits(36, 8193) == 2 and n_splits(33, 8192) == 2
    assert n_splits(48, 2049) == 1 and n_splits(64, 2049) == 1 and n_splits(128, 8192) == 1
    for B, S in ((48, 8193), (40, 4097), (300, 9000)):
        sl = lib.dkv_splitk_choose_split(B, 8, S)
        assert sl % 64 == 0 and sl >= 128
    # below 256 units, batches that are not powers of two keep to one round of workgroups
    # where a partial second round would cost more (measured: 12 x 8 units at 8K tokens 72.9
    # us with two splits against 99.3 with three, 6 x 8 units 41.2 with five against 64.4 with
    # six), and take a second round where it pays (20 x 8 units: three splits, 105.2 against
    # 142.1 with two)
    assert n_splits(12, 8193) == 2 and n_splits(6, 8193) == 5 and n_splits(20, 8193) == 3
    for B in (1, 2, 4, 8, 16, 32):  # powers of two: one full round as before
        assert B * 8 * n_splits(B, 8192) == 256 or n_splits(B, 8192) == 8192 // 128


def test_joint_v_pass_splits_fill_one_round():
    """The joint layout's V pass runs one workgroup per CU, per (token split, head-set
    workgroup, batch row); its split count, read back from the workspace size (B * Hq * (splits
    * (4 + 1024) + ranks / 128 * 128) floats), fills one round of 256 workgroups without
    spilling into a second (measured at S = 8192, 32 query heads: B = 12 59.0 us with 21 splits
    against 91.1 with 22, B = 24 97.0 with 10 against 147.9 with 11)."""
    lib = _lib.load()

    def splits(B, Hq, S, R=1024):
        ws = lib.dkv_joint_av_workspace_floats(B, Hq, S, R)
        rest = ws // (B * Hq) - (R + 127) // 128 * 128
        assert rest % (4 + 1024) == 0
        return rest // (4 + 1024)

    wgs = lambda B, Hq: B * (1 if (Hq + 15) // 16 % 2 else (Hq + 15) // 32)  # noqa: E731
    assert splits(12, 32, 8192) == 21 and splits(24, 32, 8192) == 10 and splits(3, 32, 8192) == 74
    assert splits(16, 32, 8192) == 16 and splits(1, 32, 8192) == 256 and splits(256, 32, 8192) == 1
    for B in (1, 2, 3, 4, 8, 12, 16, 20, 24, 32, 48, 64):
        for Hq in (16, 32, 64):
            if wgs(B, Hq) <= 64:  # one round of at least four splits per unit is on offer
                assert wgs(B, Hq) * splits(B, Hq, 8192) <= 256, (B, Hq)
    # with more units, whole rounds: 96 units at 8 splits, three full rounds of 1024 tokens,
    # rather than one round of 2 splits of 4096 tokens or two of 5 splits of 1648
    assert splits(48, 64, 8192) == 8
    assert splits(1, 32, 40) == 3 and splits(5, 32, 16) == 1  # splits of at least 16 tokens


def test_argument_validation_without_device():
    lib = _lib.load()
    # invalid dtype / negative sizes are rejected before any launch
    assert lib.dkv_append_decode(None, 7, None, 0, None, 0, None, 0, None, None, 0, 0, None, 0, 1, 4) == -1
    assert lib.dkv_append_decode(None, 1, None, 0, None, 0, None, 0, None, None, 0, 0, None, 0, -1, 4) == -1
    # zero rows is a no-op
    assert lib.dkv_append_decode(None, 1, None, 0, None, 0, None, 0, None, None, 0, 0, None, 0, 0, 4) == 0
    # split-K: rank above 128 is outside the kernel
    rc = lib.dkv_decode_splitk(None, 0, 2, None, 0, 0, None, 0, 0, None, 0, 0, None, 0, None, 0,
                               None, None, 0, 0, None, None, 0, 0, None, 0, None, 0,
                               None, 0, 0, 2, 1, 32, 8, 8, 10, 256, 128, 0)
    assert rc == -2
    with pytest.raises(NotImplementedError):
        _lib.check(rc, "dkv_decode_splitk")
    # prefill attention: the scale must be positive and finite (checked before anything else)
    for scale in (0.0, -0.088, float("nan"), float("inf")):
        rc = lib.dkv_prefill_attention(None, 2, None, 0, 0, 0, None, 0, 0, 0, 0, None, 0, 0, 0, 0,
                                       None, 2, 0, 0, 0, 1, 32, 8, 16, 16, 128, 1, scale, None)
        assert rc == -2, scale


def test_no_cpu_fallback():
    from dynakv_amd.kernels.two_stage import abx_sparse

    a = torch.zeros(1, 4, 128)
    b = torch.zeros(1, 16, 128)
    x = torch.zeros(1, 64)
    l = torch.ones(1, 4, dtype=torch.int32)
    o = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU path"):
        abx_sparse(a, b, x, l, offsets=o)
    with pytest.raises(ValueError, match="offsets are required"):
        abx_sparse(a, b, x, l, offsets=None)


def test_decode_layer_struct_layout(tmp_path):
    """The ctypes mirror of DkvDecodeLayer has the C layout (offsets and size from gcc)."""
    import ctypes
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    fields = [f[0] for f in _lib.DecodeLayerArgs._fields_]
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("{n} %zu\\n", offsetof(DkvDecodeLayer, {n}));\n' for n in fields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "dynakv_amd.h"\n'
                   "int main(void) {\n" + body +
                   '  printf("__size__ %zu\\n", sizeof(DkvDecodeLayer));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    got = dict(zip(out[0::2], map(int, out[1::2])))
    for n in fields:
        assert getattr(_lib.DecodeLayerArgs, n).offset == got[n], n
    assert ctypes.sizeof(_lib.DecodeLayerArgs) == got["__size__"]
