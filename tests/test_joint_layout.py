"""Host logic of the joint-layout path (dynakv_amd/kernels/joint.py) on the CPU: which inputs the
MFMA kernels take, the reduction of a repeated basis to its distinct bases, the chunk-major
transposed K basis the scores kernel reads, and the V-pass workspace size the library reports.
No kernel runs here."""
import torch

from dynakv_amd import _lib
from dynakv_amd.kernels import joint as J


def _basis(nb, R, dt=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(nb, R, 128, generator=g).to(dt)


def test_distinct_bases_of_a_repeated_basis():
    kb = _basis(8, 64)
    rep = kb.repeat_interleave(4, dim=0).contiguous()  # the reference's k_up for 32 heads
    got = J._distinct(rep, 32)
    assert got.shape == (8, 64, 128) and torch.equal(got, kb)
    assert got.data_ptr() == rep.data_ptr()  # a view of the first copy of every group
    assert J._BASIS_CACHE[id(rep)][2] == 4  # cached per object and version: the factor only
    # a repeat by 2 of 16 bases (2 query heads per basis)
    kb16 = _basis(16, 32, seed=1)
    assert J._distinct(kb16.repeat_interleave(2, dim=0).contiguous(), 32).shape[0] == 16
    # distinct bases stay whole; an in-place change invalidates the cached reduction
    assert J._distinct(kb, 8) is kb
    rep[5, 0, 0] += 1
    assert J._distinct(rep, 32).shape[0] == 32


def test_chunk_major_transpose():
    """Element B[h][32c + k][d] sits at [h][c][d][k]: each 32-rank chunk of the transposed basis
    is one contiguous (Dh, 32) block."""
    b = _basis(3, 96, dt=torch.float32)
    bt = J._transposed(b, 3)
    assert bt.shape == (3, 3, 128, 32) and bt.is_contiguous()
    h, c, d, k = 2, 1, 77, 5
    assert bt[h, c, d, k] == b[h, 32 * c + k, d]
    assert torch.equal(bt.permute(0, 1, 3, 2).reshape(3, 96, 128), b)
    assert J._transposed(b, 3) is bt
    # a repeated basis: the copy holds its distinct bases only
    rep = b.repeat_interleave(4, dim=0).contiguous()
    assert torch.equal(J._transposed(rep, 12), bt)


def test_basis_caches_release_their_tensors():
    """Neither cache keeps its key tensor alive: once the caller drops a basis (repeated or not)
    and it is collected, both entries are gone."""
    import gc

    for nrep in (1, 4):
        b = _basis(8, 64).repeat_interleave(nrep, dim=0).contiguous()
        ident = id(b)
        J._distinct(b, 8 * nrep)
        J._transposed(b, 8 * nrep)
        assert ident in J._BASIS_CACHE and ident in J._BT_CACHE
        ref = __import__("weakref").ref(b)
        del b
        gc.collect()
        assert ref() is None, "a cache entry keeps the basis alive"
        assert ident not in J._BASIS_CACHE and ident not in J._BT_CACHE


def test_eligibility():
    q = torch.zeros(2, 32, 128, dtype=torch.bfloat16)
    flat = torch.zeros(2, 4096, dtype=torch.bfloat16)
    kb = _basis(8, 1024).repeat_interleave(4, dim=0).contiguous()
    assert J.scores_eligible(q, kb, flat)
    assert J.av_eligible(kb, flat, 32, 100)
    assert not J.av_eligible(kb, flat, 32, 0)  # an empty cache keeps the vector path
    # rank not a multiple of 32, or above 1024: the vector kernels
    assert not J.scores_eligible(q, _basis(32, 100), flat)
    assert not J.scores_eligible(q, _basis(32, 1056), flat)
    # fp32 caches and mixed dtypes: the vector kernels
    assert not J.scores_eligible(q.float(), kb.float(), flat.float())
    assert not J.scores_eligible(q, kb, flat.half())
    # one basis for 16 query heads (past 8 per basis): the vector kernels; the same basis given
    # once per query head is 16 bases of one head each
    q16 = torch.zeros(1, 16, 128, dtype=torch.bfloat16)
    assert not J.scores_eligible(q16, _basis(1, 64), flat)
    assert J.scores_eligible(q16, _basis(1, 64).expand(16, 64, 128).contiguous(), flat)


def test_av_workspace_size():
    """Split records (R + 4 floats per head and split) plus one 128-float partial projection per
    head and 128-rank block."""
    lib = _lib.load()
    B, Hq, S, R = 16, 32, 8192, 1024
    n = int(lib.dkv_joint_av_workspace_floats(B, Hq, S, R))
    blocks = (R + 127) // 128
    per_head = n // (B * Hq)
    assert n % (B * Hq) == 0
    splits = (per_head - blocks * 128) // (1024 + 4)
    assert per_head == splits * (1024 + 4) + blocks * 128 and splits >= 1
    assert int(lib.dkv_joint_av_workspace_floats(B, Hq, 0, R)) == 0
    assert int(lib.dkv_joint_av_workspace_floats(B, Hq, S, 2048)) == 0
