"""dynakv_amd: MI355X (gfx950) physical compressed-KV-cache decode path.

A drop-in for the reference package's ``dynakv.kernels`` (router, packed cache, fused and
two-stage decode attention) with hand-written HIP kernels behind the C ABI in
``include/dynakv_amd.h``. Import the kernels as ``dynakv_amd.kernels.router`` etc.

``get_model_class`` (reference ``dynakv/__init__.py``) and the transformers model classes live in
:mod:`dynakv_amd.hf`, imported on first use; ``dynakv_amd.hf.install_reference_alias()`` makes the
reference's ``dynakv`` import paths resolve to this package.
"""

__version__ = "0.1.0"

from . import _lib  # noqa: F401


def native_library_path():
    return _lib.LIB_PATH


def get_model_class(model_type: str):
    """The reference's ``dynakv.get_model_class`` (``src/dynakv/__init__.py:6-17``)."""
    from .hf import get_model_class as _get

    return _get(model_type)
