"""Shared test utilities: tolerances, workload builders, oracle wrappers."""

from __future__ import annotations

import numpy as np
import torch

# north_star tolerances for bf16/fp16 inputs against an fp32 reference
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def assert_attn_close(out: torch.Tensor, ref: torch.Tensor, what: str,
                      max_abs: float = MAX_ABS, mean_abs: float = MEAN_ABS) -> None:
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert out.shape == ref.shape, (what, out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite values"
    err = (out - ref).abs()
    mx, mn = float(err.max()) if err.numel() else 0.0, float(err.mean()) if err.numel() else 0.0
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3e} mean-abs {mn:.3e}"


def random_topk(hkv: int, n: int, nb: int, topk: int, gen: torch.Generator,
                per_block_cu=None, pad_frac: float = 0.0) -> torch.Tensor:
    """Random selection rows; with per_block_cu the rows are shared by the
    tokens of each block, otherwise every token has its own row."""
    if per_block_cu is not None:
        cu = per_block_cu.tolist()
        nbq = len(cu) - 1
        rows = torch.stack([torch.randperm(nb, generator=gen)[:topk] for _ in range(hkv * nbq)])
        rows = rows.view(hkv, nbq, -1).to(torch.int32)
        lens = torch.tensor([cu[i + 1] - cu[i] for i in range(nbq)])
        out = rows.repeat_interleave(lens, dim=1)
    else:
        out = torch.stack([torch.randperm(nb, generator=gen)[:topk] for _ in range(hkv * n)])
        out = out.view(hkv, n, -1).to(torch.int32)
    if out.shape[-1] < topk:
        pad = torch.full((hkv, n, topk - out.shape[-1]), -1, dtype=torch.int32)
        out = torch.cat([out, pad], -1)
    if pad_frac > 0:
        # -1 suffixes keep the valid-prefix contract
        cut = (torch.rand(hkv, n, generator=gen) * topk * pad_frac).long()
        ar = torch.arange(topk).view(1, 1, -1)
        out = torch.where(ar >= topk - cut.unsqueeze(-1), torch.full_like(out, -1), out)
    return out.contiguous()
