"""GPU parity of the image-side 3D-aware builders (sparse.builders:
from_imcoords_to_points, build_image_to_image_attn, build_image_to_volume_attn,
build_volume_to_image_attn, build_3D_aware_attn) against the oracles of
oracle/select3d_image.py and oracle/select3d.py, bit for bit, on a synthetic
multi-view scene; and the image-to-image rows driving
spatial_selection_attention within the attention tolerance."""

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import sparse.ops as ops
from helpers import assert_attn_close
from oracle.attention import sel_attn_ref
from oracle.select3d import nearest_blocks_to_ref, volume_points_ref
from oracle.select3d_image import image_rank_rows_ref, imcoords_points_ref
from sparse import builders

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

ARGS = SimpleNamespace(patch_size=4, block_size=2, input_image_res=(32, 32), attn_winsize=2,
                       topk_multiimage=3, image_num_per_batch=3, bbox_radius=0.5, volume_res=16,
                       topk_volume=5, use_3d_aware_attn=True)


def _look_at(pos):
    back = pos / np.linalg.norm(pos)
    right = np.cross([0.0, 1.0, 0.0], back)
    right /= np.linalg.norm(right)
    up = np.cross(back, right)
    ext = np.eye(4)
    ext[:3, 0], ext[:3, 1], ext[:3, 2], ext[:3, 3] = right, up, back, pos
    return ext


def _scene(seed, b_n=2, m_n=3, crop=False):
    """mask_input [B, M, 1, 32, 32] (4x4 blocks of 8x8 pixels per image),
    dense 16x16 surface points, cameras around the origin, and the image
    tokens: every patch (8x8 per image) of every kept block, block-major."""
    rng = np.random.default_rng(seed)
    mask = (rng.random((b_n, m_n, 1, 32, 32)) < 0.01).astype(np.float32)
    mask[1, 1] = 0.0                      # an image without kept blocks
    mask[0, 0, 0, 4, 4] = 1.0
    cams = np.zeros((b_n, m_n, 17), dtype=np.float32)
    for b in range(b_n):
        for m in range(m_n):
            ang = 0.7 * m + 0.3 * b
            ext = _look_at(np.array([2.5 * math.sin(ang), 0.4, 2.5 * math.cos(ang)]))
            cams[b, m, :16] = ext.reshape(-1)
            cams[b, m, 16] = 0.9
    sp = (0.4 * rng.standard_normal((b_n, m_n, 16, 16, 3))).astype(np.float32)
    dm = rng.random((b_n, m_n, 16, 16)).astype(np.float32)
    coords = []
    for b in range(b_n):
        for m in range(m_n):
            for by in range(4):
                for bx in range(4):
                    if mask[b, m, 0, by * 8:(by + 1) * 8, bx * 8:(bx + 1) * 8].any():
                        for r in range(2):
                            for c in range(2):
                                coords.append([b, m, by * 2 + r, bx * 2 + c])
    batch = {"mask_input": torch.from_numpy(mask), "cameras_input": torch.from_numpy(cams)}
    if crop:
        batch["crop_input"] = torch.tensor([[[5, 45, 8, 48]] * m_n] * b_n, dtype=torch.int32)
        batch["origin_size"] = torch.tensor([[64]] * b_n, dtype=torch.int32)
    dense = {"surface_points_input": torch.from_numpy(sp), "masks_input": torch.from_numpy(dm)}
    return batch, dense, np.asarray(coords, dtype=np.int32)


def _volume_coords(seed, b_n=2, n_per=150):
    rng = np.random.default_rng(seed)
    out = []
    for b in range(b_n):
        cells = rng.choice(16 ** 3, size=n_per, replace=False)
        xyz = np.stack([cells // 256, (cells // 16) % 16, cells % 16], 1)
        key = [(tuple(c // 2), tuple(c % 2)) for c in xyz]
        order = sorted(range(n_per), key=lambda i: key[i])
        out += [[b, *xyz[i]] for i in order]
    return np.asarray(out, dtype=np.int32)


def _oracle_image_rows(query_pts, cu_q, batch, dense, w2c, tan_half, crop):
    mask = batch["mask_input"].numpy()
    sp = dense["surface_points_input"].numpy()
    dm = dense["masks_input"].numpy()
    topk = ARGS.topk_multiimage * ARGS.image_num_per_batch
    rows = []
    for b in range(len(cu_q) - 1):
        images = []
        for m in range(mask.shape[1]):
            cr = None
            if crop:
                ci = batch["crop_input"][b, m].numpy().astype(np.float64)
                o = float(batch["origin_size"][b, 0])
                cr = (o - 1, ci[2], ci[0], ci[1] - ci[0] - 1)
            images.append({"mask": mask[b, m, 0], "surface": sp[b, m], "dense_mask": dm[b, m],
                           "w2c": w2c[b, m], "tan_half": float(tan_half[b, m]), "crop": cr})
        rows.append(image_rank_rows_ref(query_pts[cu_q[b]:cu_q[b + 1]], images, ARGS.patch_size,
                                        ARGS.block_size, ARGS.attn_winsize ** 2, topk,
                                        ARGS.bbox_radius * 2))
    return np.concatenate(rows)


def _cams(batch):
    cam = batch["cameras_input"].to(DEV)
    w2c = torch.inverse(cam[..., :16].reshape(*cam.shape[:2], 4, 4)).cpu().numpy()
    tan_half = torch.tan(cam[..., 16] / 2.0).cpu().numpy()
    return w2c, tan_half


def _dev(batch, dense):
    return ({k: v.to(DEV) for k, v in batch.items()}, {k: v.to(DEV) for k, v in dense.items()})


def test_image_points_bitexact():
    batch, dense, coords = _scene(1)
    _, dd = _dev(batch, dense)
    pts = builders.from_imcoords_to_points(torch.from_numpy(coords).to(DEV), dd, ARGS)
    ref = imcoords_points_ref(coords, dense["surface_points_input"].numpy(),
                              dense["masks_input"].numpy(), 8)
    assert np.array_equal(pts.cpu().numpy().view(np.int32), ref.view(np.int32))


@pytest.mark.parametrize("crop", [False, True])
def test_image_to_image_rows_bitexact(crop):
    batch, dense, coords = _scene(2, crop=crop)
    bd, dd = _dev(batch, dense)
    res = builders.build_image_to_image_attn(torch.from_numpy(coords).to(DEV), bd, dd, ARGS)
    topk = res["block_topk"].cpu().numpy()
    pts = imcoords_points_ref(coords, dense["surface_points_input"].numpy(),
                              dense["masks_input"].numpy(), 8)
    cu_q = np.concatenate([[0], np.cumsum(np.bincount(coords[:, 0], minlength=2))])
    w2c, tan_half = _cams(batch)
    ref = _oracle_image_rows(pts, cu_q, batch, dense, w2c, tan_half, crop)
    assert topk.shape == (2, coords.shape[0], 9)
    assert (ref >= 0).mean() > 0.5          # rows carry candidates from several views
    np.testing.assert_array_equal(topk[0], ref)
    np.testing.assert_array_equal(topk[1], ref)
    # block metadata: the kept blocks, 4 tokens each
    nb = int(res["cu_seqblocks"][-1])
    assert (res["cu_block_include_tokens"].diff().cpu() == 4).all() and nb * 4 == coords.shape[0]


@pytest.mark.parametrize("crop", [False, True])
def test_volume_to_image_rows_bitexact(crop):
    batch, dense, coords = _scene(3, crop=crop)
    vol = _volume_coords(4)
    bd, dd = _dev(batch, dense)
    res = builders.build_volume_to_image_attn(torch.from_numpy(coords).to(DEV),
                                              torch.from_numpy(vol).to(DEV), bd, dd, ARGS)
    vpts = volume_points_ref(vol, ARGS.volume_res, ARGS.bbox_radius)
    cu_q = np.concatenate([[0], np.cumsum(np.bincount(vol[:, 0], minlength=2))])
    w2c, tan_half = _cams(batch)
    ref = _oracle_image_rows(vpts, cu_q, batch, dense, w2c, tan_half, crop)
    assert (ref >= 0).mean() > 0.5
    np.testing.assert_array_equal(res["block_topk"][0].cpu().numpy(), ref)


def test_image_to_volume_rows_bitexact():
    batch, dense, coords = _scene(5)
    vol = _volume_coords(6)
    _, dd = _dev(batch, dense)
    res = builders.build_image_to_volume_attn(torch.from_numpy(coords).to(DEV),
                                              torch.from_numpy(vol).to(DEV), dd, ARGS)
    ipts = imcoords_points_ref(coords, dense["surface_points_input"].numpy(),
                               dense["masks_input"].numpy(), 8)
    vpts = volume_points_ref(vol, ARGS.volume_res, ARGS.bbox_radius)
    cu_q = np.concatenate([[0], np.cumsum(np.bincount(coords[:, 0], minlength=2))])
    ref = nearest_blocks_to_ref(ipts, vpts, res["cu_block_include_tokens"].cpu().numpy(),
                                res["cu_seqblocks"].cpu().numpy(), cu_q, ARGS.topk_volume)
    np.testing.assert_array_equal(res["block_topk"][1].cpu().numpy(), ref)


def test_3d_aware_maps_drive_attention():
    batch, dense, coords = _scene(7)
    vol = _volume_coords(8)
    bd, dd = _dev(batch, dense)
    maps = builders.build_3D_aware_attn(torch.from_numpy(coords).to(DEV),
                                        torch.from_numpy(vol).to(DEV), bd, dd, ARGS)
    assert set(maps) == {"img_to_img_attn", "img_to_vol_attn", "vol_to_img_attn",
                         "vol_to_vol_attn"}
    n = coords.shape[0]
    hq, hkv, d = 4, 2, 32
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(n, h, d, generator=g).to(torch.bfloat16) for h in (hq, hkv, hkv))
    m = maps["img_to_img_attn"]
    cu_q = torch.from_numpy(np.concatenate([[0], np.cumsum(np.bincount(coords[:, 0],
                                                                       minlength=2))]))
    cu_q = cu_q.to(torch.int32)
    out = ops.spatial_selection_attention(q.to(DEV), k.to(DEV), v.to(DEV), m["block_topk"],
                                          m["cu_seqblocks"], m["cu_block_include_tokens"],
                                          cu_q.to(DEV), cu_q.to(DEV), None, None)
    ref, _ = sel_attn_ref(q.float(), k.float(), v.float(), m["block_topk"].cpu(),
                          m["cu_seqblocks"].cpu(), m["cu_block_include_tokens"].cpu(), cu_q,
                          1.0 / math.sqrt(d))
    assert_attn_close(out, ref, "out")
