"""Block-metadata builders on the GPU: the drop-ins for the functions of
misc/sparse_utils.py on either side of the attention kernels.

  compute_block_separation(k_coords, DIM, block_size, batch_size, resolution)
      misc/sparse_utils.py:592-641 -> (cu_seqblocks, cu_block_include_tokens)
  sort_volume_blocks(feats, coords, args, coords_idx=None)      lines 126-152
  sort_image_blocks(feats, coords, args, coords_idx=None)       lines 95-123
  from_volcoords_to_points(volcoords, args)                     lines 644-650
  from_imcoords_to_points(imcoords, dense_points, args)         lines 653-688
  build_image_to_image_attn(imfeat_coords, batch, dense_points, args)          690-898
  build_image_to_volume_attn(imfeat_coords, volfeat_coords, dense_points, args) 901-988
  build_volume_to_image_attn(imfeat_coords, volfeat_coords, batch, dense_points,
                             args)                              lines 991-1200
  build_volume_to_volume_attn(volfeat_coords, args)             lines 1203-1280
  build_3D_aware_attn(imfeat_coords, volfeat_coords, batch, dense_points, args)
                                                                lines 1283-1298

`args` is any object with the reference's attribute names (block_size,
volume_res, bbox_radius, topk_volume, use_3d_aware_attn, input_image_res,
patch_size, attn_winsize, topk_multiimage, image_num_per_batch); `batch` holds
mask_input [B, M, C, H, W], cameras_input [B, M, >=17] (a 4x4 extrinsic, then
the field of view) and optionally crop_input / origin_size; `dense_points`
holds surface_points_input [B, M, S, S, 3] and masks_input (B*M*S*S values).  Block separation, the sort permutations, the token points and
the 3D-aware per-token selection run on the gfx950 kernels of liblsrm_hip.so;
gathering the features and coordinates by the permutation is a torch index.
The reference reads batch boundaries and the image count with .item(); so
do these (compute_block_separation also reads the block count once).
"""

from __future__ import annotations

from typing import Optional

import torch

import lsrm_hip as _hip


def compute_block_separation(k_coords: torch.Tensor, DIM: int, block_size, batch_size: int,
                             resolution):
    """k_coords [N, 1 + DIM] (batch id, then coordinates; sorted by batch and
    block) -> (cu_seqblocks [B + 1], cu_block_include_tokens [nb + 1]) int32."""
    return _hip.block_separation(k_coords, DIM, block_size, resolution, int(batch_size))


def _gather(feats, coords, idx):
    return feats[idx, :], coords[idx, :]


def sort_volume_blocks(feats: torch.Tensor, coords: torch.Tensor, args,
                       coords_idx: Optional[torch.Tensor] = None):
    """Orders volume tokens by (batch, block, in-block position) ->
    (feats, coords, coords_idx) as sparse_utils.sort_volume_blocks."""
    if coords_idx is None:
        coords_idx = _hip.block_sort_permutation(coords, 0, args.block_size, (args.volume_res,))
    feats, coords = _gather(feats, coords, coords_idx)
    return feats, coords, coords_idx


def sort_image_blocks(feats: torch.Tensor, coords: torch.Tensor, args,
                      coords_idx: Optional[torch.Tensor] = None):
    """Orders image tokens by (batch, image, block, in-block position) ->
    (feats, coords, coords_idx) as sparse_utils.sort_image_blocks."""
    if coords_idx is None:
        im_num = int(coords[:, 1].max().item()) + 1
        patch_res = args.input_image_res[1] // args.patch_size
        coords_idx = _hip.block_sort_permutation(coords, 1, args.block_size, (im_num, patch_res))
    feats, coords = _gather(feats, coords, coords_idx)
    return feats, coords, coords_idx


def from_volcoords_to_points(volcoords: torch.Tensor, args) -> torch.Tensor:
    """[N, 4] volume coordinates -> [N, 3] fp32 points (x, y, z)."""
    return _hip.volume_points(volcoords, args.volume_res, args.bbox_radius)


def build_volume_to_volume_attn(volfeat_coords: torch.Tensor, args, num_kv_heads: int = 2):
    """Block metadata (and, with args.use_3d_aware_attn, the per-token
    nearest-block selection) of volume-to-volume attention -> dict with
    block_topk ([num_kv_heads, N, topk_volume] int32 or None), cu_seqblocks,
    cu_block_include_tokens.  The reference stacks its rows for two kv heads
    (line 1273); num_kv_heads sets that count."""
    block_size = [args.block_size] * 3
    resolution = [args.volume_res] * 3
    batch_size = int(volfeat_coords[:, 0].max().item()) + 1
    cu_seqblocks, cu_block_include_tokens = compute_block_separation(
        volfeat_coords, 3, block_size, batch_size, resolution)
    block_topk = None
    if args.use_3d_aware_attn:
        counts = torch.bincount(volfeat_coords[:, 0].long(), minlength=batch_size)
        cu_seqlens = torch.zeros(batch_size + 1, dtype=torch.int32, device=volfeat_coords.device)
        cu_seqlens[1:] = torch.cumsum(counts, 0).to(torch.int32)
        points = from_volcoords_to_points(volfeat_coords, args)
        block_topk = _hip.nearest_blocks(points, cu_block_include_tokens, cu_seqblocks, cu_seqlens,
                                         args.topk_volume, num_kv_heads)
    return {"block_topk": block_topk, "cu_seqblocks": cu_seqblocks,
            "cu_block_include_tokens": cu_block_include_tokens}


def from_imcoords_to_points(imcoords: torch.Tensor, dense_points: dict, args) -> torch.Tensor:
    """[N, 4] image coordinates (batch, image, patch row, patch column) ->
    [N, 3] fp32: the dense surface point of each token's patch with the
    largest mask value (misc/sparse_utils.py:653-688)."""
    patch_res = args.input_image_res[1] // args.patch_size
    return _hip.image_points(imcoords, dense_points["surface_points_input"],
                             dense_points["masks_input"], patch_res)


def _cu_from_batch_ids(ids: torch.Tensor, batch_size: int) -> torch.Tensor:
    counts = torch.bincount(ids.long(), minlength=batch_size)[:batch_size]
    cu = torch.zeros(batch_size + 1, dtype=torch.int32, device=ids.device)
    cu[1:] = torch.cumsum(counts, 0).to(torch.int32)
    return cu


def _image_block_rows(query_points: torch.Tensor, cu_seqlens_q: torch.Tensor, batch: dict,
                      dense_points: dict, args, num_kv_heads: int) -> torch.Tensor:
    """The per-image loop of build_image_to_image_attn / build_volume_to_image_attn
    (misc/sparse_utils.py:731-896, 1032-1193) for every batch element at
    once: the kept blocks of each image mask, the camera records, then one
    lsrm_image_block_rank launch for every query token."""
    sp = dense_points["surface_points_input"]
    b_n, m_n, s = sp.shape[0], sp.shape[1], sp.shape[2]
    dev = sp.device
    mask = batch["mask_input"][:b_n, :m_n, 0].to(device=dev, dtype=torch.float32)
    bps = args.patch_size * args.block_size
    h, w = mask.shape[-2:]
    bh, bw = h // bps, w // bps
    blocks = mask[:, :, : bh * bps, : bw * bps].reshape(b_n, m_n, bh, bps, bw, bps)
    kept = (blocks != 0).any(dim=5).any(dim=3).reshape(b_n * m_n, bh * bw)
    nsel = kept.sum(dim=1).to(torch.int32)                       # [B*M]
    kept_blocks = torch.nonzero(kept)[:, 1].to(torch.int32)     # (image, block) order
    win = args.attn_winsize ** 2
    sel_off = torch.cumsum(nsel, 0) - nsel
    nsel_bm = nsel.view(b_n, m_n)
    ncols = torch.clamp(nsel_bm, max=win)
    col_off = torch.cumsum(ncols, 1) - ncols
    id_off = torch.cumsum(nsel_bm, 1) - nsel_bm
    cols_per_batch = ncols.sum(1).to(torch.int32)
    meta = torch.stack([nsel_bm, sel_off.view(b_n, m_n), col_off, id_off], dim=-1).to(torch.int32)
    cols = int(cols_per_batch.max().item()) if b_n > 0 else 0

    cam = batch["cameras_input"][:b_n, :m_n].to(device=dev, dtype=torch.float32)
    extrinsic = cam[..., :16].reshape(b_n, m_n, 4, 4)
    w2c = torch.inverse(extrinsic)
    tan_half = torch.tan(cam[..., 16] / 2.0)
    rec = torch.zeros(b_n, m_n, 18, dtype=torch.float32, device=dev)
    rec[..., :12] = w2c[..., :3, :].reshape(b_n, m_n, 12)
    rec[..., 12] = tan_half
    if "crop_input" in batch:
        crop = batch["crop_input"][:b_n, :m_n].to(device=dev)
        origin = batch["origin_size"][:b_n, 0].to(device=dev)
        rec[..., 13] = 1.0
        rec[..., 14] = (origin - 1).to(torch.float32).view(b_n, 1).expand(b_n, m_n)
        rec[..., 15] = crop[..., 2].to(torch.float32)
        rec[..., 16] = crop[..., 0].to(torch.float32)
        rec[..., 17] = ((crop[..., 1] - crop[..., 0]) - 1).to(torch.float32)
    topk_num = args.topk_multiimage * args.image_num_per_batch
    max_dist = float(torch.tensor(args.bbox_radius * 2, dtype=torch.float32))
    return _hip.image_block_rank(query_points, cu_seqlens_q, rec, meta, kept_blocks,
                                 cols_per_batch, cols, bw, s // bh, sp,
                                 dense_points["masks_input"], win, topk_num, max_dist,
                                 num_kv_heads)


def _image_block_meta(imfeat_coords: torch.Tensor, dense_points: dict, args, batch_size: int):
    resolution = [dense_points["surface_points_input"].shape[1],
                  args.input_image_res[-1] // args.block_size,
                  args.input_image_res[-1] // args.block_size]
    return compute_block_separation(imfeat_coords, 3, [1, args.block_size, args.block_size],
                                    batch_size, resolution)


def build_image_to_image_attn(imfeat_coords: torch.Tensor, batch: dict, dense_points: dict,
                              args, num_kv_heads: int = 2):
    """Image-token blocks and, with args.use_3d_aware_attn, every image
    token's nearest image blocks over all views (misc/sparse_utils.py:690-898)
    -> dict with block_topk ([num_kv_heads, N, topk_multiimage *
    image_num_per_batch] int32 or None), cu_seqblocks, cu_block_include_tokens."""
    batch_size = int(imfeat_coords[:, 0].max().item()) + 1
    cu_seqblocks, cu_block_include_tokens = _image_block_meta(imfeat_coords, dense_points, args,
                                                              batch_size)
    block_topk = None
    if args.use_3d_aware_attn:
        cu_q = _cu_from_batch_ids(imfeat_coords[:, 0], batch_size)
        points = from_imcoords_to_points(imfeat_coords, dense_points, args)
        block_topk = _image_block_rows(points, cu_q, batch, dense_points, args, num_kv_heads)
    return {"block_topk": block_topk, "cu_seqblocks": cu_seqblocks,
            "cu_block_include_tokens": cu_block_include_tokens}


def build_image_to_volume_attn(imfeat_coords: torch.Tensor, volfeat_coords: torch.Tensor,
                               dense_points: dict, args, num_kv_heads: int = 2):
    """Volume-token blocks and, with args.use_3d_aware_attn, every image
    token's topk_volume nearest volume-block centroids
    (misc/sparse_utils.py:901-988)."""
    batch_size = int(volfeat_coords[:, 0].max().item()) + 1
    cu_seqblocks, cu_block_include_tokens = compute_block_separation(
        volfeat_coords, 3, [args.block_size] * 3, batch_size, [args.volume_res] * 3)
    block_topk = None
    if args.use_3d_aware_attn:
        cu_q = _cu_from_batch_ids(imfeat_coords[:, 0], batch_size)
        impoints = from_imcoords_to_points(imfeat_coords, dense_points, args)
        volpoints = from_volcoords_to_points(volfeat_coords, args)
        block_topk = _hip.nearest_blocks_to(impoints, volpoints, cu_block_include_tokens,
                                            cu_seqblocks, cu_q, args.topk_volume, num_kv_heads)
    return {"block_topk": block_topk, "cu_seqblocks": cu_seqblocks,
            "cu_block_include_tokens": cu_block_include_tokens}


def build_volume_to_image_attn(imfeat_coords: torch.Tensor, volfeat_coords: torch.Tensor,
                               batch: dict, dense_points: dict, args, num_kv_heads: int = 2):
    """Image-token blocks and, with args.use_3d_aware_attn, every volume
    token's nearest image blocks over all views (misc/sparse_utils.py:991-1200)."""
    batch_size = int(imfeat_coords[:, 0].max().item()) + 1
    cu_seqblocks, cu_block_include_tokens = _image_block_meta(imfeat_coords, dense_points, args,
                                                              batch_size)
    block_topk = None
    if args.use_3d_aware_attn:
        cu_q = _cu_from_batch_ids(volfeat_coords[:, 0], batch_size)
        points = from_volcoords_to_points(volfeat_coords, args)
        block_topk = _image_block_rows(points, cu_q, batch, dense_points, args, num_kv_heads)
    return {"block_topk": block_topk, "cu_seqblocks": cu_seqblocks,
            "cu_block_include_tokens": cu_block_include_tokens}


def build_3D_aware_attn(imfeat_coords: torch.Tensor, volfeat_coords: torch.Tensor, batch: dict,
                        dense_points: dict, args):
    """The four maps of misc/sparse_utils.py:1283-1298."""
    return {
        "img_to_img_attn": build_image_to_image_attn(imfeat_coords, batch, dense_points, args),
        "img_to_vol_attn": build_image_to_volume_attn(imfeat_coords, volfeat_coords,
                                                      dense_points, args),
        "vol_to_img_attn": build_volume_to_image_attn(imfeat_coords, volfeat_coords, batch,
                                                      dense_points, args),
        "vol_to_vol_attn": build_volume_to_volume_attn(volfeat_coords, args),
    }
