"""GPU parity of the block-metadata builders and the 3D-aware selection,
bit-exact against the integer / float64 oracles."""

import types

import numpy as np
import pytest
import torch

import sparse.builders as B
from lsrm_hip import workloads as W
from oracle.builders import block_sort_perm_ref, compute_block_separation_ref
from oracle.select3d import nearest_blocks_ref, volume_points_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _voxels(n_per_batch=(5000, 3000), grid=64, seed=0):
    rng = np.random.default_rng(seed)
    parts = []
    for b, n in enumerate(n_per_batch):
        cells = rng.choice(grid ** 3, size=n, replace=False)
        xyz = np.stack([cells // (grid * grid), (cells // grid) % grid, cells % grid], 1)
        parts.append(np.concatenate([np.full((n, 1), b), xyz], axis=1))
    return np.concatenate(parts).astype(np.int64)


def test_volume_points_bitexact():
    c = _voxels()
    got = B.from_volcoords_to_points(torch.from_numpy(c).to(DEV),
                                     types.SimpleNamespace(volume_res=64, bbox_radius=0.9))
    ref = volume_points_ref(c, 64, 0.9)
    assert torch.equal(got.cpu().view(torch.int32), torch.from_numpy(ref).view(torch.int32))


@pytest.mark.parametrize("layout", [0, 1])
def test_block_sort_permutation_exact(layout):
    c = _voxels((4000, 2500))
    if layout == 1:   # image-like: (batch, image, row, col) on a 32 x 32 patch grid
        rng = np.random.default_rng(1)
        c = np.concatenate([c[:, :1], rng.integers(0, 4, (len(c), 1)),
                            rng.integers(0, 32, (len(c), 2))], axis=1)
        dims = (4, 32)
    else:
        dims = (64,)
    perm = B._hip.block_sort_permutation(torch.from_numpy(c).to(DEV), layout, 8, dims)
    assert perm.cpu().numpy().tolist() == block_sort_perm_ref(c, layout, 8, dims).tolist()


def test_sort_then_separate_bitexact():
    c = _voxels()
    args = types.SimpleNamespace(volume_res=64, block_size=8)
    feats = torch.arange(len(c), dtype=torch.float32)[:, None].to(DEV)
    f2, c2, idx = B.sort_volume_blocks(feats, torch.from_numpy(c).to(DEV), args)
    assert torch.equal(f2[:, 0].long().cpu(), idx.cpu())
    cs = c2.cpu().numpy()
    cu_sb, cu_blk = B.compute_block_separation(c2, 3, [8, 8, 8], 2, [64, 64, 64])
    ref_sb, ref_blk = compute_block_separation_ref(cs, 3, [8, 8, 8], 2, [64, 64, 64])
    assert cu_sb.cpu().numpy().tolist() == ref_sb.tolist()
    assert cu_blk.cpu().numpy().tolist() == ref_blk.tolist()


def test_separation_outside_grid_and_2d():
    rng = np.random.default_rng(3)
    c = np.concatenate([np.sort(rng.integers(0, 3, 900))[:, None],
                        rng.integers(-2, 40, (900, 2))], axis=1)
    cu_sb, cu_blk = B.compute_block_separation(torch.from_numpy(c).to(DEV), 2, [4, 8], 3, [32, 32])
    ref_sb, ref_blk = compute_block_separation_ref(c, 2, [4, 8], 3, [32, 32])
    assert cu_sb.cpu().numpy().tolist() == ref_sb.tolist()
    assert cu_blk.cpu().numpy().tolist() == ref_blk.tolist()


@pytest.mark.parametrize("topk", [8, 16, 24, 65, 66, 67, 72, 128])
def test_build_volume_to_volume_attn_3d_aware_bitexact(topk):
    # topk above 64 takes the two-launch selection (first k1 = min(64, topk - 3))
    c = _voxels()
    args = types.SimpleNamespace(volume_res=64, block_size=8, bbox_radius=1.0,
                                 use_3d_aware_attn=True, topk_volume=topk)
    feats = torch.zeros(len(c), 1, device=DEV)
    _, c2, _ = B.sort_volume_blocks(feats, torch.from_numpy(c).to(DEV), args)
    res = B.build_volume_to_volume_attn(c2, args)
    cs = c2.cpu().numpy()
    ref_sb, ref_blk = compute_block_separation_ref(cs, 3, [8] * 3, 2, [64] * 3)
    assert res["cu_seqblocks"].cpu().numpy().tolist() == ref_sb.tolist()
    assert res["cu_block_include_tokens"].cpu().numpy().tolist() == ref_blk.tolist()
    pts = volume_points_ref(cs, 64, 1.0)
    n0 = int((cs[:, 0] == 0).sum())
    ref = nearest_blocks_ref(pts, ref_blk, ref_sb, np.array([0, n0, len(cs)]), topk)
    got = res["block_topk"].cpu().numpy()
    assert got.shape == (2, len(cs), topk)
    assert (got[0] == ref).all() and (got[1] == ref).all()


def test_3d_aware_selection_feeds_attention():
    """The built metadata and per-token rows drive spatial_selection_attention
    (grouped union tiles) within the attention tolerance."""
    import sparse.ops as ops
    from helpers import assert_attn_close
    from oracle.attention import sel_attn_ref
    c = _voxels((6000,))
    args = types.SimpleNamespace(volume_res=64, block_size=8, bbox_radius=1.0,
                                 use_3d_aware_attn=True, topk_volume=8)
    _, c2, _ = B.sort_volume_blocks(torch.zeros(len(c), 1, device=DEV),
                                    torch.from_numpy(c).to(DEV), args)
    res = B.build_volume_to_volume_attn(c2, args)
    n = len(c)
    g = torch.Generator().manual_seed(0)
    q, k, v = ((0.5 * torch.randn(n, 2, 64, generator=g)).to(torch.bfloat16) for _ in range(3))
    cu_q = torch.tensor([0, n], dtype=torch.int32)
    out = ops.spatial_selection_attention(q.to(DEV), k.to(DEV), v.to(DEV), res["block_topk"],
                                          res["cu_seqblocks"], res["cu_block_include_tokens"],
                                          cu_q.to(DEV), cu_q.to(DEV), None, None)
    ref, _ = sel_attn_ref(q.float(), k.float(), v.float(), res["block_topk"].cpu(),
                          res["cu_seqblocks"].cpu(), res["cu_block_include_tokens"].cpu(), cu_q,
                          1.0 / 8.0)
    assert_attn_close(out, ref, "out")
