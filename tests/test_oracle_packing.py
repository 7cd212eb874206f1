"""Pins the packing oracle (oracle/packing.py) against layouts computed by hand from the
reference's arithmetic (src/dynakv/kernels/compressed_cache.py:7-34, 96-227) and against the
layout invariants, on CPU."""
import numpy as np
import pytest

from oracle.packing import PackedSlot, pack_rows
from dynakv_amd.kernels.compressed_cache import flat_capacity_after, seq_capacity_after


def _states(B, S, D, seed=0):
    return np.random.default_rng(seed).standard_normal((B, S, D)).astype(np.float32)


def test_decode_from_empty_hand_computed():
    # B=2, MAX_DIM=4. First decode: init flat = max(3,1) = 3, seq cap 1. The upper bound check
    # 0 + 1*4 > 3 reads the pointers (0, 0) and grows to max(3 + 1024*2, 0 + 4) = 2051.
    s = PackedSlot()
    x1 = _states(2, 1, 4, 1)
    s.append_decode(x1, np.array([[3], [1]]), 4)
    assert s.flat.shape == (2, 2051) and s.lens.shape == (2, 1) and s.syncs == 1
    assert s.ub == [4, 4]
    # Second decode: seq cap grows to max(1 + 1024, 2) = 1025; 4 + 4 <= 2051, no pointer read.
    x2 = _states(2, 1, 4, 2)
    s.append_decode(x2, np.array([[2], [4]]), 4)
    lens, offs = s.tables()
    assert s.lens.shape == (2, 1025) and s.syncs == 1 and s.ub == [8, 8]
    assert lens.tolist() == [[3, 2], [1, 4]]
    assert offs.tolist() == [[0, 3], [0, 1]]
    assert s.ptr.tolist() == [5, 5]
    np.testing.assert_array_equal(s.flat[0, :5], np.concatenate([x1[0, 0, :3], x2[0, 0, :2]]))
    np.testing.assert_array_equal(s.flat[1, :5], np.concatenate([x1[1, 0, :1], x2[1, 0, :4]]))
    assert not s.flat[:, 5:].any()


def test_prefill_then_decode_hand_computed():
    # prefill lens (2,3,1): flat exactly 6, offs (0,2,5), ptr 6 (quirk: capacity is exact)
    s = PackedSlot()
    x = _states(1, 3, 4, 3)
    s.append_prefill(x, np.array([[2, 3, 1]]), 4)
    lens, offs = s.tables()
    assert s.flat.shape == (1, 6) and s.lens.shape == (1, 3)
    assert offs.tolist() == [[0, 2, 5]] and s.ptr.tolist() == [6] and s.ub == [6]
    # first decode after prefill always reads the pointer and grows: max(6 + 2048, 6 + 4) = 2054;
    # the seq tables grow to max(3 + 1024, 4) = 1027
    y = _states(1, 1, 4, 4)
    s.append_decode(y, np.array([[4]]), 4)
    lens, offs = s.tables()
    assert s.flat.shape == (1, 2054) and s.lens.shape == (1, 1027) and s.syncs == 1
    assert lens.tolist() == [[2, 3, 1, 4]] and offs.tolist() == [[0, 2, 5, 6]]
    np.testing.assert_array_equal(
        s.flat[0, :10], np.concatenate([x[0, 0, :2], x[0, 1, :3], x[0, 2, :1], y[0, 0, :4]]))


def test_prefill_offsets_start_at_current_pointer():
    s = PackedSlot()
    s.append_prefill(_states(2, 2, 8, 5), np.array([[3, 4], [1, 1]]), 8)
    s.append_prefill(_states(2, 3, 8, 6), np.array([[2, 2, 2], [5, 0, 1]]), 8)
    lens, offs = s.tables()
    assert offs.tolist() == [[0, 3, 7, 9, 11], [0, 1, 2, 7, 7]]
    assert s.ptr.tolist() == [13, 8]


def test_capacity_helpers_match_oracle_policy():
    # the cache class computes capacities with these helpers; same arithmetic as the oracle
    assert seq_capacity_after(1, 1, 1) == 1025
    assert seq_capacity_after(3, 3, 1) == 1027
    assert seq_capacity_after(10, 3, 5) == 10
    assert seq_capacity_after(10, 3, 5000) == 5003
    assert flat_capacity_after(3, [0, 0], 4, 4) == 2051
    assert flat_capacity_after(6, [6], 4, 4) == 2054
    assert flat_capacity_after(100, [10, 20], 4, 4) == 100
    assert flat_capacity_after(100, [10, 20], 128, 128) == 100 + 1024 * 64


@pytest.mark.parametrize("seed", range(4))
def test_layout_invariants_random(seed):
    rng = np.random.default_rng(seed)
    B, D = 3, int(rng.integers(4, 64))
    s = PackedSlot()
    coef_hist = [[] for _ in range(B)]
    n_pre = int(rng.integers(1, 20))
    x = rng.standard_normal((B, n_pre, D)).astype(np.float32)
    L = rng.integers(0, D + 1, size=(B, n_pre))
    s.append_prefill(x, L, D)
    for b in range(B):
        coef_hist[b] += [x[b, t, : L[b, t]] for t in range(n_pre)]
    for _ in range(int(rng.integers(1, 40))):
        y = rng.standard_normal((B, 1, D)).astype(np.float32)
        l1 = rng.integers(0, D + 1, size=(B, 1))
        s.append_decode(y, l1, D)
        for b in range(B):
            coef_hist[b].append(y[b, 0, : l1[b, 0]])
    lens, offs = s.tables()
    for b in range(B):
        excl = np.concatenate([[0], np.cumsum(lens[b])[:-1]])
        np.testing.assert_array_equal(offs[b], excl)           # offs = exclusive prefix sum
        assert s.ptr[b] == lens[b].sum()                        # ptr = sum of lengths
        payload = np.concatenate(coef_hist[b]) if coef_hist[b] else np.zeros(0, np.float32)
        np.testing.assert_array_equal(s.flat[b, : s.ptr[b]], payload)  # prefixes back to back
        assert not s.flat[b, s.ptr[b]:].any()                   # zero tail
    dec = s.decompress(D)
    for b in range(B):
        for t in range(s.seq):
            n = lens[b, t]
            np.testing.assert_array_equal(dec[b, t, :n], coef_hist[b][t])
            assert not dec[b, t, n:].any()


def test_pack_rows_one_shot():
    x = _states(2, 5, 16, 9)
    L = np.array([[16, 1, 7, 0, 3], [2, 2, 2, 2, 2]])
    flat, lens, offs, ptr = pack_rows(x, L, 16)
    assert flat.shape == (2, 27) and ptr.tolist() == [27, 10]
    assert offs.tolist() == [[0, 16, 17, 24, 24], [0, 2, 4, 6, 8]]


def test_pack_rows_equals_incremental_slot():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((4, 70, 32)).astype(np.float32)
    L = rng.integers(0, 33, size=(4, 70))
    flat, lens, offs, ptr = pack_rows(x, L, 32)
    s = PackedSlot()
    s.append_prefill(x, L, 32)
    l2, o2 = s.tables()
    np.testing.assert_array_equal(flat, s.flat)
    np.testing.assert_array_equal(lens, l2)
    np.testing.assert_array_equal(offs, o2)
    np.testing.assert_array_equal(ptr, s.ptr)
