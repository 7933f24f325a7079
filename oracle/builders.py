"""Block-metadata builder oracle (numpy, integer arithmetic).

compute_block_separation_ref restates misc/sparse_utils.py:592-641: tokens
of batch element b (coords[:, 0] == b), block id = row-major flattening of
(c[d] // block_size[d]) over resolution[d] // block_size[d] blocks per
dimension (lines 604-618), per-block token counts (torch.histc, lines
619-621) of which the non-zero ones are kept in block order, then the
prefix arrays cu_seqblocks / cu_block_include_tokens (lines 624-639).
Tokens outside the grid are not counted (histc ignores values outside its
range).

block_sort_keys_ref restates the sort keys of sort_volume_blocks
(lines 126-148) and sort_image_blocks (lines 95-115); the permutation is a
stable argsort (the reference's torch.argsort leaves the order of equal keys
unspecified).
Pins (tests/test_oracle_builders.py): a dictionary-of-counts brute force; a
full grid (every block holds block_size^dim tokens); tokens outside the grid;
the keys of known cells order blocks before in-block positions.
"""

from __future__ import annotations

import numpy as np


def compute_block_separation_ref(coords: np.ndarray, dim: int, block_size, batch: int,
                                 resolution):
    c = np.asarray(coords, dtype=np.int64)
    nbd = [int(resolution[d]) // int(block_size[d]) for d in range(dim)]
    nbins = int(np.prod(nbd))
    counts = np.zeros((batch, nbins), dtype=np.int64)
    for i in range(c.shape[0]):
        b = int(c[i, 0])
        if b < 0 or b >= batch:
            continue
        flat, ok = 0, True
        for d in range(dim):
            v = int(c[i, 1 + d])
            bd = v // int(block_size[d]) if v >= 0 else -1
            if bd < 0 or bd >= nbd[d]:
                ok = False
                break
            flat = flat * nbd[d] + bd
        if ok:
            counts[b, flat] += 1
    per_batch = [row[row > 0] for row in counts]
    seqblocks = [len(x) for x in per_batch]
    cu_sb = np.concatenate([[0], np.cumsum(seqblocks)]).astype(np.int32)
    toks = np.concatenate(per_batch) if per_batch else np.zeros(0, np.int64)
    cu_blk = np.concatenate([[0], np.cumsum(toks)]).astype(np.int32)
    return cu_sb, cu_blk


def block_sort_keys_ref(coords: np.ndarray, layout: int, block_size: int, dims) -> np.ndarray:
    c = np.asarray(coords, dtype=np.int64)
    b = int(block_size)
    if layout == 0:
        r = int(dims[0])
        blk, inb = c[:, 1:] // b, c[:, 1:] % b
        return (r ** 3 * c[:, 0] + r * r * b * blk[:, 0] + r * b * b * blk[:, 1]
                + b ** 3 * blk[:, 2] + b * b * inb[:, 0] + b * inb[:, 1] + inb[:, 2])
    im, pr = int(dims[0]), int(dims[1])
    blk, inb = c[:, 2:] // b, c[:, 2:] % b
    return (im * pr * pr * c[:, 0] + pr * pr * c[:, 1] + pr * b * blk[:, 0] + b * b * blk[:, 1]
            + b * inb[:, 0] + inb[:, 1])


def block_sort_perm_ref(coords: np.ndarray, layout: int, block_size: int, dims) -> np.ndarray:
    return np.argsort(block_sort_keys_ref(coords, layout, block_size, dims), kind="stable")
