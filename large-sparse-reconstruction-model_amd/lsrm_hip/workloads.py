"""Seeded synthetic inputs for the five benchmark configurations.

Block metadata follows the reference's conventions (misc/sparse_utils.py:592-641,
compute_block_separation): tokens are sorted block-major, cu_block_include_tokens
holds cumulative block sizes, cu_seqblocks cumulative block counts per batch
element, both int32.  Block ids inside top-k rows are batch-local.

Configs (B = 1 everywhere):
  1  H=4,  D=64, N=4096,   fp32, N(0,1),      blocks U[16,128],   top-8,  self forced
  2  H=16, D=64, N=32768,  bf16, 0.5 N(0,1),  blocks U[32,256],   top-16, self forced
  3  H=24, D=64, N=131072, bf16, 0.5 N(0,1),  8 image blocks of 1024 tokens + 122880
     voxel tokens (distinct cells of a 64^3 grid in Morton order) in runs U[32,512];
     top-16 with the 8 image blocks and self forced
  4  config 2 shapes plus dO ~ N(0,1) (training path)
  5  H=4, D=64, N=524288, bf16, blocks clip(round(LogNormal(ln 64, 1)), 8, 1024),
     top-32, Q/K with a shared rank-4 component (10% of the variance) for near ties
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch


@dataclass
class Workload:
    name: str
    n: int
    hq: int
    hkv: int
    d: int
    dtype: torch.dtype
    topk: int
    cu_block_tokens: torch.Tensor      # int32 [nb + 1] (CPU)
    cu_seqblocks: torch.Tensor         # int32 [B + 1] (CPU)
    cu_seqlens: torch.Tensor           # int32 [B + 1] (CPU)
    forced_blocks: List[int] = field(default_factory=list)
    force_self: bool = True
    seed: int = 0
    qk_scale: float = 0.5              # std of Q/K/V entries
    lowrank: Optional[dict] = None     # config 5 near-tie construction
    voxel_coords: Optional[np.ndarray] = None  # cfg3: (x, y, z) cells of the voxel tokens
    n_image_tokens: int = 0            # cfg3: tokens before the voxel tokens
    n_image_blocks: int = 0

    @property
    def n_blocks(self) -> int:
        return self.cu_block_tokens.numel() - 1

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.d)


def uniform_partition(n: int, lo: int, hi: int, rng: np.random.Generator) -> np.ndarray:
    """Contiguous block sizes ~ U[lo, hi] covering n tokens; the final block is
    truncated to fit and merged into its predecessor when shorter than lo."""
    sizes = []
    total = 0
    while total < n:
        s = int(rng.integers(lo, hi + 1))
        s = min(s, n - total)
        sizes.append(s)
        total += s
    if len(sizes) > 1 and sizes[-1] < lo:
        last = sizes.pop()
        sizes[-1] += last
    return np.asarray(sizes, dtype=np.int64)


def lognormal_partition(n: int, mu: float, sigma: float, lo: int, hi: int,
                        rng: np.random.Generator) -> np.ndarray:
    """Heavy-tailed block sizes clip(round(LogNormal(mu, sigma)), lo, hi)."""
    sizes = []
    total = 0
    while total < n:
        s = int(np.clip(np.round(rng.lognormal(mu, sigma)), lo, hi))
        s = min(s, n - total)
        sizes.append(s)
        total += s
    if len(sizes) > 1 and sizes[-1] < lo:
        last = sizes.pop()
        sizes[-1] += last
    return np.asarray(sizes, dtype=np.int64)


def morton3(x: np.ndarray, y: np.ndarray, z: np.ndarray, bits: int = 6) -> np.ndarray:
    """Interleaves the bits of (x, y, z) into a 3*bits Morton code."""
    code = np.zeros_like(x, dtype=np.int64)
    for b in range(bits):
        code |= ((x >> b) & 1) << (3 * b + 2)
        code |= ((y >> b) & 1) << (3 * b + 1)
        code |= ((z >> b) & 1) << (3 * b)
    return code


def morton_voxel_runs(n_vox: int, grid: int, lo: int, hi: int,
                      rng: np.random.Generator, return_coords: bool = False):
    """Distinct random occupied cells of a grid^3 volume sorted by Morton code
    and cut into consecutive runs of U[lo, hi] tokens (spatially coherent
    blocks).  Returns the run lengths (and, with return_coords, the cells'
    integer (x, y, z) coordinates [n_vox, 3] in token order)."""
    cells = rng.choice(grid ** 3, size=n_vox, replace=False)
    x, y, z = cells // (grid * grid), (cells // grid) % grid, cells % grid
    bits = int(math.log2(grid))
    order = np.argsort(morton3(x, y, z, bits), kind="stable")
    assert order.shape[0] == n_vox
    runs = uniform_partition(n_vox, lo, hi, rng)
    if return_coords:
        return runs, np.stack([x[order], y[order], z[order]], axis=1).astype(np.int64)
    return runs


def _cu(sizes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))


def config(idx: int, n: Optional[int] = None, heads: Optional[int] = None) -> Workload:
    """Builds the metadata of config idx (1-5).  n / heads shrink the config
    for quick tests (the block-size distribution is kept)."""
    rng = np.random.default_rng(idx)
    if idx == 1:
        n = n or 4096
        sizes = uniform_partition(n, 16, 128, rng)
        return Workload("cfg1", n, heads or 4, heads or 4, 64, torch.float32, 8, _cu(sizes),
                        torch.tensor([0, len(sizes)], dtype=torch.int32),
                        torch.tensor([0, n], dtype=torch.int32), seed=1, qk_scale=1.0)
    if idx in (2, 4):
        n = n or 32768
        sizes = uniform_partition(n, 32, 256, rng)
        return Workload(f"cfg{idx}", n, heads or 16, heads or 16, 64, torch.bfloat16, 16,
                        _cu(sizes), torch.tensor([0, len(sizes)], dtype=torch.int32),
                        torch.tensor([0, n], dtype=torch.int32), seed=idx)
    if idx == 3:
        n = n or 131072
        n_img_blocks, img_len = 8, 1024
        if n < 131072:  # shrunken variant: keep 8 image blocks, scale their size
            img_len = max(32, n // 128)
        n_vox = n - n_img_blocks * img_len
        runs, vox = morton_voxel_runs(n_vox, 64, 32, 512, rng, return_coords=True)
        sizes = np.concatenate([np.full(n_img_blocks, img_len), runs])
        w = Workload("cfg3", n, heads or 24, heads or 24, 64, torch.bfloat16, 16, _cu(sizes),
                     torch.tensor([0, len(sizes)], dtype=torch.int32),
                     torch.tensor([0, n], dtype=torch.int32),
                     forced_blocks=list(range(n_img_blocks)), seed=3)
        w.voxel_coords = vox
        w.n_image_tokens = n_img_blocks * img_len
        w.n_image_blocks = n_img_blocks
        return w
    if idx == 5:
        n = n or 524288
        sizes = lognormal_partition(n, math.log(64.0), 1.0, 8, 1024, rng)
        return Workload("cfg5", n, heads or 4, heads or 4, 64, torch.bfloat16, 32, _cu(sizes),
                        torch.tensor([0, len(sizes)], dtype=torch.int32),
                        torch.tensor([0, n], dtype=torch.int32), seed=5,
                        lowrank={"rank": 4, "shared": 0.1})
    raise ValueError(f"unknown config {idx}")


def product_shape(n: Optional[int] = None) -> Workload:
    """Config 3's token layout with LSRM's own decoder head layout:
    num_q_heads 32, num_kv_heads 2 (main_lrm_vol_sparse.py:561-562), head dim
    32, top-16 (test_rgb.sh:97)."""
    w = config(3, n=n)
    w.name = "cfg3-product"
    w.hq, w.hkv, w.d = 32, 2, 32
    return w


def tensors(w: Workload, device, dtype: Optional[torch.dtype] = None, with_grad_out: bool = False):
    """Seeded Q, K, V (and dO) for a workload on `device`."""
    dtype = dtype or w.dtype
    gen = torch.Generator(device=device)
    gen.manual_seed(1000 + w.seed)
    shp_q = (w.n, w.hq, w.d)
    shp_k = (w.n, w.hkv, w.d)

    def randn(shape):
        return torch.randn(shape, generator=gen, device=device, dtype=torch.float32)

    if w.lowrank:
        r = w.lowrank["rank"]
        a = math.sqrt(1.0 - w.lowrank["shared"])
        b = math.sqrt(w.lowrank["shared"])
        u = randn((w.n, r))
        wq = randn((r, w.hq * w.d)) / math.sqrt(r)
        wk = randn((r, w.hkv * w.d)) / math.sqrt(r)
        q = a * randn(shp_q) + b * (u @ wq).view(shp_q)
        k = a * randn(shp_k) + b * (u @ wk).view(shp_k)
        v = randn(shp_k)
    else:
        s = w.qk_scale
        q = s * randn(shp_q)
        k = s * randn(shp_k)
        v = s * randn(shp_k)
    out = [q.to(dtype), k.to(dtype), v.to(dtype)]
    if with_grad_out:
        out.append(randn(shp_q).to(dtype))
    return out


def attended_tokens(compact: torch.Tensor, cu_block_tokens: torch.Tensor,
                    cu_seqblocks: torch.Tensor) -> int:
    """Sum over kv heads and query tokens of the attended key count, from the
    per-block selection rows [Hkv, nb, topk] (valid ids only)."""
    compact = compact.to("cpu", torch.int64)
    cu = cu_block_tokens.to("cpu", torch.int64)
    lens = cu[1:] - cu[:-1]
    cu_sb = cu_seqblocks.to("cpu", torch.int64)
    total = 0
    for e in range(cu_sb.numel() - 1):
        b0, b1 = int(cu_sb[e]), int(cu_sb[e + 1])
        rows = compact[:, b0:b1, :]
        valid = (rows >= 0) & (rows < (b1 - b0))
        gl = torch.where(valid, rows + b0, torch.zeros_like(rows))
        a = torch.where(valid, lens[gl], torch.zeros_like(gl)).sum(-1)  # [Hkv, nbb]
        total += int((a * lens[b0:b1].unsqueeze(0)).sum())
    return total
