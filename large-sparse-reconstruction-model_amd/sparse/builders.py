"""Block-metadata builders on the GPU: the drop-ins for the functions of
misc/sparse_utils.py on either side of the attention kernels.

  compute_block_separation(k_coords, DIM, block_size, batch_size, resolution)
      misc/sparse_utils.py:592-641 -> (cu_seqblocks, cu_block_include_tokens)
  sort_volume_blocks(feats, coords, args, coords_idx=None)      lines 126-152
  sort_image_blocks(feats, coords, args, coords_idx=None)       lines 95-123
  from_volcoords_to_points(volcoords, args)                     lines 644-650
  build_volume_to_volume_attn(volfeat_coords, args)             lines 1203-1280

`args` is any object with the reference's attribute names (block_size,
volume_res, bbox_radius, topk_volume, use_3d_aware_attn, input_image_res,
patch_size).  Block separation, the sort permutations, the token points and
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
