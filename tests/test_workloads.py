"""CPU checks of the seeded benchmark workloads (lsrm_hip.workloads): block
metadata follows the reference's conventions (misc/sparse_utils.py:592-641:
int32 cumulative block sizes, block-major tokens) and each config's stated
distribution."""

import numpy as np
import pytest
import torch

from lsrm_hip import workloads as W


def _sizes(w):
    cu = w.cu_block_tokens.long()
    return (cu[1:] - cu[:-1]).numpy()


@pytest.mark.parametrize("idx", [1, 2, 3, 5])
def test_metadata_contract(idx):
    w = W.config(idx)
    cu = w.cu_block_tokens
    assert cu.dtype == torch.int32 and w.cu_seqblocks.dtype == torch.int32
    assert int(cu[0]) == 0 and int(cu[-1]) == w.n
    assert (cu[1:] >= cu[:-1]).all()
    assert w.cu_seqblocks.tolist() == [0, w.n_blocks]
    assert w.cu_seqlens.tolist() == [0, w.n]


def test_config_block_distributions():
    s1 = _sizes(W.config(1))
    assert s1.min() >= 16 and s1[:-1].max() <= 128
    s2 = _sizes(W.config(2))
    assert s2.min() >= 32 and s2[:-1].max() <= 256
    w3 = W.config(3)
    s3 = _sizes(w3)
    assert (s3[:8] == 1024).all() and w3.forced_blocks == list(range(8))
    assert s3[8:].min() >= 32 and s3[8:-1].max() <= 512
    s5 = _sizes(W.config(5))
    assert s5.min() >= 8 and s5[:-1].max() <= 1024
    assert W.config(5).topk == 32 and w3.topk == 16


def test_morton_code():
    x = np.array([1, 0, 0, 3])
    y = np.array([0, 1, 0, 3])
    z = np.array([0, 0, 1, 3])
    assert W.morton3(x, y, z, 2).tolist() == [4, 2, 1, 63]


def test_partition_merges_short_tail():
    rng = np.random.default_rng(0)
    s = W.uniform_partition(1000, 100, 200, rng)
    assert s.sum() == 1000 and s.min() >= 100


def test_tensors_seeded_and_lowrank():
    w = W.config(5, n=4096)
    a = W.tensors(w, "cpu")
    b = W.tensors(w, "cpu")
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert a[0].dtype == torch.bfloat16 and a[0].shape == (4096, 4, 64)


def test_attended_tokens_counts_valid_entries():
    cu = torch.tensor([0, 3, 5, 9], dtype=torch.int32)
    compact = torch.tensor([[[0, -1], [0, 2], [1, 7]]], dtype=torch.int32)
    # block0 (3 tok) attends 3; block1 (2 tok) attends 3+4; block2 (4 tok) attends 2
    assert W.attended_tokens(compact, cu, torch.tensor([0, 3])) == 3 * 3 + 2 * 7 + 4 * 2
