"""The sparse-attention layer forward (pool K and V, select blocks, plan and
attention) captured in one HIP graph: every step runs on the device with no
host synchronisation and no memset node, so a captured layer replays with the
same results.  The graph is replayed several times with eager work of the
program and synchronisations between the replays, and every replay is compared
bit for bit with the eager layer (the kernels are deterministic)."""

import pytest
import torch

import lsrm_hip as H
from lsrm_hip import workloads as W

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_layer_forward_replays_in_a_graph():
    w = W.config(3, n=16384, heads=2)
    q, k, v = W.tensors(w, DEV)
    cu_blk = w.cu_block_tokens.to(DEV)
    cu_sb = w.cu_seqblocks.to(DEV)
    cu_q = w.cu_seqlens.to(DEV)
    n, hkv, d = w.n, w.hkv, w.d
    k2, v2 = k.view(n, hkv * d), v.view(n, hkv * d)
    forced = torch.tensor(w.forced_blocks, dtype=torch.int32, device=DEV)

    def layer():
        pk, cv = H.block_mean_pool2(k2, v2, cu_blk, torch.float32, None)
        topk_idx, compact = H.select_blocks(q, k, cu_sb, cu_blk, w.topk, forced, True,
                                            pooled_k=pk)
        o, lse = H.sel_attn_fwd(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, w.scale)
        return pk, cv, topk_idx, compact, o, lse

    eager = [t.clone() for t in layer()]
    torch.cuda.synchronize()
    # warm up on a side stream (default priority) before capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = layer()
    torch.cuda.synchronize()

    for rep in range(3):
        # the program's own eager work between replays
        again = layer()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(again, eager)), f"eager call {rep}"
        for t in captured:
            t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(captured, eager)):
            assert torch.equal(a, b), f"replay {rep}, output {i}"
