"""dynakv_amd: MI355X (gfx950) physical compressed-KV-cache decode path.

A drop-in for the reference package's ``dynakv.kernels`` (router, packed cache, fused and
two-stage decode attention) with hand-written HIP kernels behind the C ABI in
``include/dynakv_amd.h``. Import the kernels as ``dynakv_amd.kernels.router`` etc.
"""

__version__ = "0.1.0"

from . import _lib  # noqa: F401


def native_library_path():
    return _lib.LIB_PATH
