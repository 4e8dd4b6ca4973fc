"""The decode operator under graph capture (torch.cuda.graph, i.e. HIP graphs).

torch.ops.sunshape.decode is captured once and the graph replayed several times, with eager work
and synchronisations between the replays; every replay must equal the eager call bit for bit.
Covered: a contiguous decode in context splits (the decode kernel and the split merge, two
kernels) and a paged decode in one kernel.  The operator allocates its outputs and split
workspace from torch's allocator, which under capture is the graph's private pool, and records
no memset."""

import pytest
import torch

from _util import log
from sunshape_amd import hip_ops, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _replays_equal_eager(fn, what):
    eager = fn().clone()
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up off the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = fn()
    for rep in range(3):
        junk = torch.randn(512, 512, device=DEV)
        (junk @ junk).sum().item()  # eager work and a synchronisation between replays
        static_out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"{what}: replay {rep} differs from the eager call"
    # eager calls after the replays still agree
    assert torch.equal(fn(), eager), f"{what}: eager call after the replays differs"


def test_contiguous_split_decode_replays_from_a_graph():
    log("graph capture: contiguous decode in splits (decode + merge)")
    p = synthetic.config3(DEV, B=4, T=4096)

    def fn():
        return hip_ops.decode(p["q"], p["codes"], p["v"], p["perm"], p["centroids"], scale=p.meta["scale"])

    _replays_equal_eager(fn, "config-3 layer B=4")


def test_paged_decode_replays_from_a_graph():
    log("graph capture: paged decode")
    p = synthetic.config4(DEV, B=8, T=2048)

    def fn():
        return hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"], scale=p.meta["scale"],
                              block_table=p["block_table"], seq_lens=p["seq_lens"])

    _replays_equal_eager(fn, "config-4 layer B=8")
