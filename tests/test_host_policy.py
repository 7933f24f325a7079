"""Host-side policy of sparse.ops (CPU): the automatic key-centric choice.

With set_key_centric("auto") (the default) a selection takes the key-centric
plan when its runs of identical rows are short enough for the plan to group
them (under a quarter of a 128-row tile's queries): per-token rows do, rows
shared by whole query blocks do not.  The choice is a pure function of the
rows, checked here on CPU tensors."""

import torch

import sparse.ops as ops
from sparse.ops import native_sparse_attention as nsa


def _q_k(n, hq, hkv):
    return torch.empty(n, hq, 8), torch.empty(n, hkv, 8)


def test_auto_key_centric_follows_run_lengths():
    gen = torch.Generator().manual_seed(0)
    n, hkv = 4096, 2
    per_token = torch.randint(0, 64, (hkv, n, 8), generator=gen, dtype=torch.int32)
    per_block = torch.randint(0, 64, (hkv, n // 128, 8), generator=gen,
                              dtype=torch.int32).repeat_interleave(128, dim=1)
    runs_of_16 = torch.randint(0, 64, (hkv, n // 16, 8), generator=gen,
                               dtype=torch.int32).repeat_interleave(16, dim=1)
    runs_of_64 = torch.randint(0, 64, (hkv, n // 64, 8), generator=gen,
                               dtype=torch.int32).repeat_interleave(64, dim=1)
    ops.set_key_centric("auto")
    q, k = _q_k(n, 2, hkv)  # MHA: runs under 32 queries are grouped
    assert nsa._use_key_centric(q, k, per_token)
    assert nsa._use_key_centric(q, k, runs_of_16)
    assert not nsa._use_key_centric(q, k, runs_of_64)
    assert not nsa._use_key_centric(q, k, per_block)
    q16, k16 = _q_k(n, 32, hkv)  # 16 query heads per kv head: 8-query tiles
    assert nsa._use_key_centric(q16, k16, per_token)
    assert not nsa._use_key_centric(q16, k16, runs_of_16)


def test_explicit_key_centric_settings():
    q, k = _q_k(16, 2, 2)
    rows = torch.zeros(2, 16, 4, dtype=torch.int32)
    try:
        ops.set_key_centric(True)
        assert nsa._use_key_centric(q, k, rows)
        ops.set_key_centric(False)
        assert not nsa._use_key_centric(q, k, torch.arange(64, dtype=torch.int32).view(2, 8, 4))
    finally:
        ops.set_key_centric("auto")


def test_plan_cache_key_tracks_the_selection():
    # A cached plan is reused only for the same selection tensors, unchanged
    # since the plan was built (same storage, same version counter).
    import lsrm_hip as H
    rows = torch.zeros(2, 16, 4, dtype=torch.int32)
    cu_sb = torch.tensor([0, 4], dtype=torch.int32)
    cu_blk = torch.tensor([0, 4, 8, 12, 16], dtype=torch.int32)
    cu_q = torch.tensor([0, 16], dtype=torch.int32)
    key = lambda r, kc=False: H._plan_key((16, 2, 8), (16, 2, 8), r, cu_sb, cu_blk, cu_q, kc)
    k0 = key(rows)
    assert key(rows) == k0
    assert key(rows, True) != k0                      # another plan kind
    assert key(rows.clone()) != k0                    # same values, other storage
    rows[0, 0, 0] = 1                                 # in-place change of the selection
    assert key(rows) != k0
    k1 = key(rows)
    cu_blk[1] = 3                                     # in-place change of the metadata
    assert key(rows) != k1
