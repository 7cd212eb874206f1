"""Host-side layout checks of the split-K path (no device): which flat buffers the kernel can
address. The kernel bases each workgroup's buffer resource at its own cache row, so the limit is
on the row stride alone; large batches of long caches (many rows) stay on the fast path."""
import torch

from dynakv_amd.kernels.decode import FLAT_LD_MAX, flat_ok


def _flat(rows, ld):
    return torch.empty((rows, ld), dtype=torch.bfloat16, device="meta")


def test_row_stride_limit():
    assert flat_ok(_flat(1, FLAT_LD_MAX))
    assert not flat_ok(_flat(1, FLAT_LD_MAX + 1))


def test_many_rows_of_a_long_cache_fit():
    # per-head layout, B = 64 at 32K tokens with full retention: 512 rows of 32K*128 elements,
    # 2^31 elements in all (4 GiB) -- beyond one 32-bit buffer range, fine per row
    t = _flat(64 * 8, 32768 * 128)
    assert t.shape[0] * t.stride(0) >= 2**31
    assert flat_ok(t)


def test_layout_requirements():
    assert not flat_ok(torch.empty((4, 8, 2), device="meta"))          # not 2-D
    assert not flat_ok(_flat(8, 64).t())                                # element stride != 1
    assert flat_ok(_flat(8, 64)[:, :32])                                # row stride 64, view ok
