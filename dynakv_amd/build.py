"""Build the C-ABI shared library ``dynakv_amd/lib/libdynakv_amd.so`` for gfx950.

Plain ``hipcc`` per source file (in parallel), then one link step. The library is built
in-tree so it travels with the repository snapshot to the GPU host.

Usage: ``python -m dynakv_amd.build`` (or ``dynakv_amd.build.build()``).
"""

from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libdynakv_amd.so"
OBJ_DIR = PKG_DIR / "_build"
SOURCES = ("dkv_append.hip", "dkv_generic.hip", "dkv_splitk.hip", "dkv_cutoff.hip",
           "dkv_prefill.hip", "dkv_layer.hip", "dkv_model.hip", "dkv_joint.hip", "dkv_dense.hip",
           "dkv_recon.hip")
ARCH = os.environ.get("DYNAKV_AMD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # never emit packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results and accumulators in VGPRs: the split kernel keeps its 128-register K basis in
    # the accumulation registers (as MFMA A operands) and post-processes every MFMA result with
    # VALU code, which would otherwise be copied out of accumulation registers first
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: set ROCM_PATH or put hipcc on PATH")
    return found


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link the shared library. Always rebuilds."""
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objs = [OBJ_DIR / (Path(s).stem + ".o") for s in SOURCES]
    with _cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        futs = [ex.submit(_compile, CSRC / s, o) for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[dynakv_amd] built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
