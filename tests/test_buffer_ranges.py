"""Buffer-resource ranges on the host (no GPU): every range a kernel reads through must end inside
the memory the caller owns. A raw buffer resource returns zeros past its range without touching
memory, but a range longer than the allocation lets a load reach unmapped memory (a joint V-pass
score range four elements too long once faulted the GPU where the scores ended at a page end).

The ranges come from the library's own functions (``dkv_flat_range_elems``,
``dkv_view_extent_elems``) and the wrappers' contract checks (``_lib.flat_covers_rows``,
``_lib.flat_operand``); these tests build strided, offset and tail-aligned views on the CPU and
check that the range of every row stays inside the view's storage."""
import itertools

import pytest
import torch

from dynakv_amd import _lib
from dynakv_amd.kernels import prefill as P

CAP = 0x3FFFFFF0


def _avail(t: torch.Tensor) -> int:
    """Elements of t's storage from its base pointer to the storage's end."""
    return t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()


def _tail_aligned(rows: int, n: int, ld: int, dtype=torch.bfloat16) -> torch.Tensor:
    """(rows, n) view with row stride ld whose storage ends right after its last element."""
    base = torch.zeros((rows - 1) * ld + n, dtype=dtype)
    return base.as_strided((rows, n), (ld, 1))


def _flat_views():
    yield "whole buffer", torch.zeros(5, 300, dtype=torch.bfloat16)
    big = torch.zeros(6, 512, dtype=torch.bfloat16)
    yield "column slice", big[:, :300]
    yield "row-offset slice", big[2:5, :300]
    yield "row-offset column slice", big[1:, 8:200]
    yield "single row at the end", big[5:, :]
    yield "tail-aligned slice", _tail_aligned(4, 300, 512)
    yield "tail-aligned, fp16", _tail_aligned(3, 129, 136, torch.float16)
    yield "single tail-aligned row", _tail_aligned(1, 40, 64)


@pytest.mark.parametrize("name,t", list(_flat_views()), ids=[n for n, _ in _flat_views()])
def test_flat_row_ranges_stay_in_storage(name, t):
    """After the wrappers' contract step, every row's resource (row r to the buffer's end, as the
    split and joint kernels form it) lies inside the storage; views that break the contract
    (tail-aligned slices) are detected and copied."""
    lib = _lib.load()
    covers = _lib.flat_covers_rows(t)
    rows, n = t.shape
    ld = t.stride(0)
    assert covers == (rows * ld <= _avail(t)), name
    if "tail-aligned" in name and ld > n:
        assert not covers, "a slice ending inside its last row's stride must be copied"
    u = _lib.flat_operand(t)
    assert _lib.flat_covers_rows(u)
    assert torch.equal(u, t)
    assert (u is t) == covers
    lu, au = u.stride(0), _avail(u)
    for r in range(rows):
        rng = int(lib.dkv_flat_range_elems(rows, r, lu))
        assert rng == min((rows - r) * lu, CAP)
        assert r * lu + rng <= au, f"{name}: row {r} range reaches past the storage"
        # the row's own elements are inside its range
        assert rng >= min(n, CAP)


def test_flat_range_cap_and_degenerate_rows():
    lib = _lib.load()
    assert int(lib.dkv_flat_range_elems(4, 0, 1 << 30)) == CAP  # capped at 2^31 bytes
    assert int(lib.dkv_flat_range_elems(4, 3, 100)) == 100  # the last row: its stride only
    assert int(lib.dkv_flat_range_elems(4, 4, 100)) == 0  # no row past the end
    assert int(lib.dkv_flat_range_elems(4, 5, 100)) == 0


def _score_views():
    """(B, Hq, S) score views as the joint V pass may receive them: contiguous, head-sliced,
    batch-sliced, transposed storage, token counts not divisible by 4, tail-aligned."""
    for S in (4, 6, 13, 64, 67):
        for dt in (torch.float32, torch.bfloat16):
            yield f"contiguous S={S} {dt}", torch.zeros(3, 8, S, dtype=dt)
            big = torch.zeros(4, 10, S + 5, dtype=dt)
            yield f"sliced S={S} {dt}", big[1:, 2:, 3:3 + S]
            yield f"transposed S={S} {dt}", torch.zeros(S, 3, 8, dtype=dt).permute(1, 2, 0)
            base = torch.zeros(2 * 8 * (S + 4) - 4, dtype=dt)
            yield f"tail-aligned S={S} {dt}", base.as_strided((2, 8, S), (8 * (S + 4), S + 4, 1))


@pytest.mark.parametrize("name,t", list(_score_views()), ids=[n for n, _ in _score_views()])
def test_view_extent_stays_in_storage(name, t):
    """The extent the library computes for a strided operand (the joint V pass's score range,
    the prefill kernel's K/V ranges) is one past the view's last element: it never reaches past
    the storage, and for a tail-aligned view it ends exactly at the storage's end."""
    ext = _lib.view_extent(t)
    want = 1 + sum((s - 1) * st for s, st in zip(t.shape, t.stride()))
    assert ext == want
    assert ext <= _avail(t), name
    if name.startswith("tail-aligned"):
        assert ext == _avail(t)
    # every element of the view is inside the extent
    idx = torch.arange(t.numel()).reshape(t.shape)
    offs = sum(i * st for i, st in zip(torch.meshgrid(*[torch.arange(s) for s in t.shape],
                                                       indexing="ij"), t.stride()))
    assert int(offs.max()) == ext - 1 and idx.numel() == t.numel()


@pytest.mark.parametrize("S", [4, 8, 64, 68])
def test_vector_score_groups_never_cross_the_extent(S):
    """The joint V pass loads a lane's 4 scores in one access only for token-contiguous rows with
    4-aligned starts and S % 4 == 0; then each group of 4 lies wholly inside or wholly past the
    range that ends at the last score, so a prefetch past the last row reads zeros only."""
    base = torch.zeros(2 * 8 * (S + 4), dtype=torch.bfloat16)
    t = base.as_strided((2, 8, S), (8 * (S + 4), S + 4, 1))
    ext = _lib.view_extent(t)
    for b, h in itertools.product(range(2), range(8)):
        row = b * t.stride(0) + h * t.stride(1)
        assert row % 4 == 0
        for g in range(0, S + 16, 4):  # the prefetch runs past the row's end
            lo, hi = row + g, row + g + 4
            assert hi <= ext or lo >= ext, (b, h, g)


def test_prefill_extent_matches_library():
    q = torch.zeros(2, 4, 300, 128, dtype=torch.bfloat16)
    for view in (q, q[:, 1:3], q[1:, :, 100:], q.transpose(1, 2)):
        assert P._extent(view) == _lib.view_extent(view)
        assert P._extent(view) <= _avail(view)
    assert _lib.view_extent(torch.zeros(0, 4, 128)) == 0
