"""The decode and encode operators under graph capture (torch.cuda.graph, i.e. HIP graphs).

torch.ops.sunshape.decode (and encode_into, a decode step's append) is captured once and the
graph replayed several times, with eager work and synchronisations between the replays; every
replay must equal the eager call bit for bit.
Covered: a contiguous decode in context splits (the decode kernel and the split merge, two
kernels), a paged decode in one kernel, and a grid-search append into cache pages.  The operators
allocate outputs and split workspace from torch's allocator, which under capture is the graph's
private pool, and record no memset."""

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


def test_paged_append_replays_from_a_graph():
    """A decode step's append (encode of one token per sequence into cache pages, grid search),
    captured once: each replay writes the step's codes and passthrough values into the pages as
    the eager call does."""
    log("graph capture: paged append (encode into pages)")
    p = synthetic.config5(DEV, B=16, S=1)
    heavy = p["heavy"].tolist()
    grid = hip_ops.encode_grid(p["centroids"])
    page, Hkv, nb = 16, 2, 32
    g = torch.Generator().manual_seed(5)
    slots = (torch.randperm(64, generator=g)[:16] * page + 3).view(16, 1).to(torch.int64).to(DEV)
    cpages = torch.zeros(64, Hkv, page, nb, dtype=torch.uint8, device=DEV)
    ppages = torch.zeros(64, Hkv, page, 4, 2, dtype=torch.bfloat16, device=DEV)

    def append():
        hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy, codes_out=cpages, pt_out=ppages,
                       slot_mapping=slots, grid=grid)

    append()
    torch.cuda.synchronize()
    want_c, want_p = cpages.clone(), ppages.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        append()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        append()
    for rep in range(3):
        cpages.zero_()
        ppages.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cpages, want_c) and torch.equal(ppages, want_p), f"append replay {rep} differs"
