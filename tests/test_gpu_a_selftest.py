"""First GPU test: the MFMA operand layouts and unaligned/out-of-range buffer gathers the split-K
kernel is written against (runs before any parity test)."""
import pytest
import torch

from dynakv_amd import _lib


@pytest.mark.gpu
def test_selftest_layouts(dev):
    print("[gpu] dkv_selftest_layouts", flush=True)
    buf = torch.zeros(512, dtype=torch.int32, device=dev)
    rc = _lib.load().dkv_selftest_layouts(torch.cuda.current_stream(dev).cuda_stream, buf.data_ptr())
    _lib.check(rc, "dkv_selftest_layouts")
    torch.cuda.synchronize(dev)
    assert int(buf[0].item()) == 0
