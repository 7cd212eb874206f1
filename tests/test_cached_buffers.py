"""Cached per-stream buffers grow at least twofold and the buffers they replace stay allocated
(a HIP graph captured with one keeps its address). CPU tensors stand in for device memory:
the caches only allocate, they launch nothing."""
import torch

from dynakv_amd import _lib
from dynakv_amd.kernels import cutoff, decode, joint


def test_split_workspace_grows_and_retires():
    dev = torch.device("cpu")
    w1 = decode.workspace(dev, 0x51, 1000)
    assert w1.numel() >= 1000 and bool((w1 == 0).all())
    assert decode.workspace(dev, 0x51, 500) is w1  # large enough: reused
    w2 = decode.workspace(dev, 0x51, w1.numel() + 1)
    assert w2 is not w1 and w2.numel() >= 2 * w1.numel() and bool((w2 == 0).all())
    assert any(t is w1 for t in _lib._RETIRED_BUFFERS)


def test_other_caches_grow_and_retire():
    dev = torch.device("cpu")
    for get in (lambda n: cutoff._workspace(dev, 0x52, n),
                lambda n: joint._workspace(dev, 0x53, n),
                lambda n: joint._sort_workspace(dev, 0x54, n)):
        a = get(10)
        b = get(a.numel() + 1)
        assert b is not a and b.numel() >= 2 * a.numel()
        assert any(t is a for t in _lib._RETIRED_BUFFERS)
