"""The operator inside a captured HIP graph (torch.cuda.CUDAGraph).

The op makes no host synchronisation and no memset: the workspace is a
caching-allocator tensor and every counter the kernels need is zeroed by the
planning kernel itself, so the launches can be captured once and replayed
(also at a size where the attention runs as the persistent grid, whose claim
queues the plan kernel empties). Each replay gets fresh inputs copied into the captured tensors, eager
work runs between replays, and every replay is compared bit for bit with an
eager call on the same inputs (all kernels are deterministic)."""

import pytest
import torch

from flashprefill_amd import flash_prefill_varlen_func

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(seed, lens, Hq=8, Hkv=2, d=128):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = (torch.randn(T, Hq, d, generator=g) * 1.5).to(torch.bfloat16)
    k = (torch.randn(T, Hkv, d, generator=g) * 1.5).to(torch.bfloat16)
    v = torch.randn(T, Hkv, d, generator=g).to(torch.bfloat16)
    return q.to(DEV), k.to(DEV), v.to(DEV)


@pytest.mark.parametrize("lens,Hq,Hkv", [([1000, 555, 129], 8, 2),
                                         # enough attention slots for the persistent grid
                                         ([12000, 5000, 300], 32, 8)])
def test_captured_graph_replays_match_eager(lens, Hq, Hkv):
    cu_l = [0]
    for n in lens:
        cu_l.append(cu_l[-1] + n)
    cu = torch.tensor(cu_l, dtype=torch.int32, device=DEV)
    mx = max(lens)
    q, k, v = _inputs(0, lens, Hq, Hkv)
    o = torch.empty_like(q)

    # warm up on a side stream (first-call host work stays out of the capture)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        flash_prefill_varlen_func(q, k, v, o, cu, mx, 0.18)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        flash_prefill_varlen_func(q, k, v, o, cu, mx, 0.18)
    torch.cuda.synchronize()

    for seed in (1, 2, 3, 4):
        q2, k2, v2 = _inputs(seed, lens, Hq, Hkv)
        q.copy_(q2)
        k.copy_(k2)
        v.copy_(v2)
        o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        # eager work between replays, then the eager reference on the same inputs
        ref = torch.empty_like(q2)
        flash_prefill_varlen_func(q2, k2, v2, ref, cu, mx, 0.18)
        torch.cuda.synchronize()
        assert not torch.isnan(o).any(), f"replay {seed} left outputs unwritten"
        assert torch.equal(o, ref), f"replay {seed} differs from the eager call"
