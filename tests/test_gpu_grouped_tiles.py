"""GPU parity of the forward and backward on per-token selection rows:
consecutive queries whose rows differ are grouped into tiles that run over
the union of their blocks with a per-query mask, or run by run (duplicated
ids, unions too large or more expensive than the runs); dK/dV gather the
queries of grouped tiles per block.  Checked against the fp32 oracle
(autograd for the gradients) at the attention tolerance, including the
LSE."""

import numpy as np
import pytest
import torch

import lsrm_hip as H
from helpers import assert_attn_close
from lsrm_hip import workloads as W
from oracle.attention import sel_attn_ref
from oracle.select3d import nearest_blocks_ref, volume_points_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _voxel_case(n=16384, hq=2, hkv=2, topk=16, seed=0, d=64):
    """cfg3-style voxel tokens (Morton-ordered cells of a 64^3 grid cut into
    runs of 32..512) with the 3D-aware per-token rows (nearest centroids)."""
    w = W.config(3, n=n, heads=hkv)
    nv = w.voxel_coords.shape[0]
    cu_blk = w.cu_block_tokens.numpy().astype(np.int64)
    cu_v = (cu_blk[w.n_image_blocks:] - cu_blk[w.n_image_blocks]).astype(np.int32)
    coords = np.concatenate([np.zeros((nv, 1), np.int64), w.voxel_coords], axis=1)
    pts = volume_points_ref(coords, 64, 1.0)
    sel = nearest_blocks_ref(pts, cu_v, np.array([0, len(cu_v) - 1]), np.array([0, nv]), topk)
    topk_idx = torch.from_numpy(np.broadcast_to(sel, (hkv, nv, topk)).copy())
    g = torch.Generator().manual_seed(seed)
    q = (0.5 * torch.randn(nv, hq, d, generator=g)).to(torch.bfloat16)
    k = (0.5 * torch.randn(nv, hkv, d, generator=g)).to(torch.bfloat16)
    v = (0.5 * torch.randn(nv, hkv, d, generator=g)).to(torch.bfloat16)
    cu_sb = torch.tensor([0, len(cu_v) - 1], dtype=torch.int32)
    cu_q = torch.tensor([0, nv], dtype=torch.int32)
    return q, k, v, topk_idx, cu_sb, torch.from_numpy(cu_v), cu_q


def _check(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, do=None):
    scale = 1.0 / 8.0
    dev_args = [t.to(DEV) for t in (q, k, v, topk_idx, cu_sb, cu_blk, cu_q)]
    o, lse = H.sel_attn_fwd(*dev_args, scale)
    qf, kf, vf = (t.float().requires_grad_(do is not None) for t in (q, k, v))
    o_ref, lse_ref = sel_attn_ref(qf, kf, vf, topk_idx, cu_sb, cu_blk, cu_q, scale)
    assert_attn_close(o, o_ref, "out")
    lse_c = lse.cpu()
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse_c), fin)
    if fin.any():
        assert float((lse_c[fin] - lse_ref[fin]).abs().max()) <= 2e-2
    if do is None:
        return
    dq, dk, dv, delta = H.sel_attn_bwd(do.to(DEV), *dev_args[:3], o, lse, *dev_args[3:], scale)
    o_ref.backward(do.float())
    assert_attn_close(dq, qf.grad, "dq")
    assert_attn_close(dk, kf.grad, "dk")
    assert_attn_close(dv, vf.grad, "dv")
    delta_ref = (o.float().cpu() * do.float()).sum(-1).transpose(0, 1)
    torch.testing.assert_close(delta.cpu(), delta_ref, rtol=1e-4, atol=1e-4)


def _grad_out(q, seed):
    g = torch.Generator().manual_seed(100 + seed)
    return (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype)


def test_3d_aware_rows_union_tiles():
    _check(*_voxel_case())


def test_3d_aware_rows_gqa():
    _check(*_voxel_case(n=8192, hq=8, hkv=2, topk=8, seed=1))


def test_rows_with_duplicate_ids_run_passes():
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _voxel_case(n=8192, topk=8, seed=2)
    topk_idx = topk_idx.clone()
    topk_idx[:, ::3, 7] = topk_idx[:, ::3, 0]   # every third query lists a block twice
    _check(q, k, v, topk_idx, cu_sb, cu_blk, cu_q)


def test_random_per_token_rows_union_or_runs():
    # Unrelated rows: unions of 128 queries exceed the runs' own keys or the
    # 256-block limit, so tiles fall back to passes per run.  Includes -1
    # padding, out-of-range ids and empty rows.
    w = W.config(2, n=6000, heads=2)
    q, k, v = W.tensors(w, "cpu")
    g = torch.Generator().manual_seed(4)
    nb = w.n_blocks
    topk_idx = torch.randint(0, nb, (w.hkv, w.n, 12), generator=g, dtype=torch.int32)
    topk_idx[:, ::5, 9:] = -1
    topk_idx[:, 1::7, 3] = nb + 5
    topk_idx[:, 2::11, :] = -1
    _check(q, k, v, topk_idx, w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens)


def test_two_batch_elements_short_runs():
    # short runs on both sides of a batch boundary are never grouped together
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _voxel_case(n=8192, topk=8, seed=3)
    nv = q.shape[0]
    half = nv // 2
    nbv = cu_blk.numel() - 1
    # batch element 1 = the same tokens again, with its own copy of the blocks
    q2 = torch.cat([q, q]); k2 = torch.cat([k, k]); v2 = torch.cat([v, v])
    cu_blk2 = torch.cat([cu_blk, cu_blk[1:] + nv])
    cu_sb2 = torch.tensor([0, nbv, 2 * nbv], dtype=torch.int32)
    cu_q2 = torch.tensor([0, nv, 2 * nv], dtype=torch.int32)
    rows2 = torch.cat([topk_idx, topk_idx], dim=1)
    _check(q2, k2, v2, rows2, cu_sb2, cu_blk2, cu_q2)
    assert half > 0


# ------------------------------------------------------------- backward --

def test_bwd_3d_aware_rows_union_tiles():
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _voxel_case(n=8192, topk=8, seed=5)
    _check(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, do=_grad_out(q, 5))


def test_bwd_3d_aware_rows_gqa():
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _voxel_case(n=4096, hq=8, hkv=2, topk=4, seed=6)
    _check(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, do=_grad_out(q, 6))


def test_bwd_duplicate_ids_and_empty_rows():
    # Repeated ids (run passes in dQ, repeated entries for dK/dV) and rows
    # that attend nothing inside grouped tiles (dQ = 0 for them).
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _voxel_case(n=4096, topk=4, seed=7)
    topk_idx = topk_idx.clone()
    topk_idx[:, ::3, 3] = topk_idx[:, ::3, 0]
    topk_idx[:, 5::13, :] = -1
    _check(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, do=_grad_out(q, 7))


def test_bwd_run_tiles_and_grouped_queries_share_blocks():
    # The first half of the queries share their block's row (long runs: run
    # tiles), the second half have per-token rows (grouped tiles), so dK/dV
    # of most blocks take rows from both reverse maps.
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _voxel_case(n=8192, topk=6, seed=8)
    topk_idx = topk_idx.clone()
    nv = q.shape[0]
    cu = cu_blk.tolist()
    for b in range(len(cu) - 1):
        s, e = cu[b], cu[b + 1]
        if e <= nv // 2:
            topk_idx[:, s:e] = topk_idx[:, s:s + 1]
    _check(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, do=_grad_out(q, 8))


def test_bwd_random_rows_two_batches():
    w = W.config(2, n=3000, heads=2)
    q, k, v = W.tensors(w, "cpu")
    g = torch.Generator().manual_seed(9)
    nb = w.n_blocks
    topk_idx = torch.randint(0, nb, (w.hkv, w.n, 6), generator=g, dtype=torch.int32)
    topk_idx[:, ::5, 4:] = -1
    topk_idx[:, 1::7, 2] = nb + 5
    # two batch elements over the same blocks and tokens
    q2, k2, v2 = torch.cat([q, q]), torch.cat([k, k]), torch.cat([v, v])
    cu_blk2 = torch.cat([w.cu_block_tokens, w.cu_block_tokens[1:] + w.n])
    cu_sb2 = torch.tensor([0, nb, 2 * nb], dtype=torch.int32)
    cu_q2 = torch.tensor([0, w.n, 2 * w.n], dtype=torch.int32)
    rows2 = torch.cat([topk_idx, topk_idx.flip(1)], dim=1).contiguous()
    _check(q2, k2, v2, rows2, cu_sb2, cu_blk2, cu_q2, do=_grad_out(q2, 9))


def test_bwd_per_token_rows_deterministic():
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _voxel_case(n=16384, topk=16, seed=10)
    do = _grad_out(q, 10).to(DEV)
    args = [t.to(DEV) for t in (q, k, v, topk_idx, cu_sb, cu_blk, cu_q)]
    o, lse = H.sel_attn_fwd(*args, 0.125)
    first = H.sel_attn_bwd(do, *args[:3], o, lse, *args[3:], 0.125)
    again = H.sel_attn_bwd(do, *args[:3], o, lse, *args[3:], 0.125)
    for x, y in zip(first, again):
        assert torch.equal(x, y)


def test_gqa16_d32_per_token_rows_fwd_bwd():
    # 16 query heads per kv head at head dim 32 (the product's grouped
    # layout): 8 queries per tile, grouped tiles of at most 7 queries.
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _voxel_case(n=4096, hq=32, hkv=2, topk=4, seed=11,
                                                         d=32)
    _check(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, do=_grad_out(q, 11))


def _mid_runs_case(n=6144, hkv=2, topk=8, seed=12, d=64):
    """Blocks of 8..40 tokens; runs of 1..40 identical rows; each new row
    either swaps one id of the previous row (neighbours share all but one)
    or is drawn afresh (they share about none), so short runs of 8 or more
    queries meet neighbours on both sides of the shared-ids rule.  Some rows
    carry -1 padding."""
    rng = np.random.default_rng(seed)
    sizes = rng.integers(8, 41, size=n // 8)
    cu = np.concatenate([[0], np.cumsum(sizes)])
    cu = cu[cu <= n]
    cu[-1] = n
    nb = len(cu) - 1
    g = torch.Generator().manual_seed(seed)
    q = (0.5 * torch.randn(n, hkv, d, generator=g)).to(torch.bfloat16)
    k = (0.5 * torch.randn(n, hkv, d, generator=g)).to(torch.bfloat16)
    v = (0.5 * torch.randn(n, hkv, d, generator=g)).to(torch.bfloat16)
    rows = np.empty((hkv, n, topk), np.int32)
    for h in range(hkv):
        cur = rng.choice(nb, topk, replace=False)
        i = 0
        while i < n:
            ln = int(rng.integers(1, 41))
            if rng.random() < 0.5:
                cur = cur.copy()
                free = np.setdiff1d(np.arange(nb), cur)
                cur[rng.integers(topk)] = rng.choice(free)
            else:
                cur = rng.choice(nb, topk, replace=False)
            r = cur.copy()
            if rng.random() < 0.2:
                r[topk - 2:] = -1
            rows[h, i:i + ln] = r
            i += ln
    return (q, k, v, torch.from_numpy(rows), torch.tensor([0, nb], dtype=torch.int32),
            torch.from_numpy(cu.astype(np.int32)), torch.tensor([0, n], dtype=torch.int32))


@pytest.mark.parametrize("key_centric,topk", [(False, 8), (True, 8), (False, 20), (False, 72)])
def test_mid_length_runs_join_by_shared_ids(key_centric, topk):
    # runs of 8..31 queries join a neighbouring short run only when their
    # rows share at least half their ids; both outcomes through the forward
    # and the backward of either plan, rows of one or two wave widths of ids
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _mid_runs_case(topk=topk)
    scale = 0.125
    dev_args = [t.to(DEV) for t in (q, k, v, topk_idx, cu_sb, cu_blk, cu_q)]
    do = _grad_out(q, 12)
    o, lse = H.sel_attn_fwd(*dev_args, scale, key_centric=key_centric)
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    o_ref, lse_ref = sel_attn_ref(qf, kf, vf, topk_idx, cu_sb, cu_blk, cu_q, scale)
    assert_attn_close(o, o_ref, "out")
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert float((lse.cpu()[fin] - lse_ref[fin]).abs().max()) <= 2e-2
    dq, dk, dv, _ = H.sel_attn_bwd(do.to(DEV), *dev_args[:3], o, lse, *dev_args[3:], scale,
                                   key_centric=key_centric)
    o_ref.backward(do.float())
    assert_attn_close(dq, qf.grad, "dq")
    assert_attn_close(dk, kf.grad, "dk")
    assert_attn_close(dv, vf.grad, "dv")
