"""Benchmark: fused VQ-key decode attention on one MI355X.

Default workload (the north-star target): Llama-3-8B-shaped
paged decode at 2 bits/dim -- batch 64, 32 query / 8 KV heads, head_dim 128, 32 blocks
of dim 4 (256 fp32 codewords each), context 32768 in 16-token vLLM-style pages, uint8
codes, bf16 V and queries, bf16 output.  One step = one ssq_decode launch over the whole
batch with inputs resident in HBM.

Prints ONE JSON line: keys scored/s (B*Hkv*T per step / time), achieved HBM GB/s on the
algorithmic bytes and its fraction of the 8 TB/s peak, the kernel's average launch time
from HIP events on its own stream, the same launch's time with cold caches (a 1 GiB flush
before each), and a bounded CPU baseline: the reference's eager torch decode path on the
host's cores (oracle/torch_eager.py).

  python bench.py [--steps K] [--warmup W] [--workload c4|c3|c2|c5|c5enc|c4append|c5append|c4g8|c4bd2|c3p6|c4p6|c4ct|c4ctbd2|c4ctg8|c4ctmix|c4mix|c4scores|c4w|c4ctw|c4appendw|c5encpro] [--no-cpu]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "VQ-key decode attention: keys scored/sec/GPU + achieved HBM GB/s (% peak)"
HBM_PEAK_GBPS = 8000.0
MFMA_F32_PEAK_TFLOPS = 157.3


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c4", choices=["c4", "c3", "c2", "c5", "c5enc", "c4append", "c5append", "c4g8", "c4bd2", "c3p6",
                                                     "c4p6", "c4ct", "c4ctbd2", "c4ctg8", "c4ctmix", "c4mix", "c4scores", "c4w", "c4ctw", "c4appendw", "c5encpro",
                                                     "copycal"])
    ap.add_argument("--kernel", type=int, default=0, help="0 auto, 1 generic, 2 MFMA")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--settle-s", type=float, default=0.3,
                    help="untimed launches for this many seconds before the warm-up steps (clock settling)")
    ap.add_argument("--cold-steps", type=int, default=20,
                    help="extra launches timed after a cache flush each (0 skips them)")
    return ap.parse_args()


def _traffic_from_profiles(name: str):
    """HBM bytes per launch recorded from rocprofv3 --pmc runs (profiles/<name>.md), or None."""
    path = os.path.join(ROOT, "profiles", f"{name}.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


# ----------------------------------------------------------------------------- workloads
def _decode_workload(name, dev, kernel):
    import torch

    from sunshape_amd import _native as N
    from sunshape_amd import hip_ops, synthetic

    heavy, pt = None, None
    nc, code_bits = 256, 0
    if name in ("c4", "c4g8", "c4bd2", "c4p6", "c4mix", "c4scores", "c4w"):
        # c4g8 / c4bd2: the config-4 layer with 64 query heads (8 per KV head) or at 4 bits/dim
        # (64 blocks of dim 2); their LUTs exceed the LDS, so they run the MFMA-scores kernel.
        # c4p6: the layer at 3 bits/dim (64 blocks of dim 2, 64 codewords), 6-bit codes packed
        # five to an int32 word in the pages; c4w: the layer at 3 bits/dim and block_dim 4, 4,096
        # codewords per block with int16 codes (the reference fitter's codebook size for that
        # setting, sunshape/hf.py:594)
        Hq = 64 if name == "c4g8" else 32
        bd = 2 if name in ("c4bd2", "c4p6") else 4
        if name == "c4p6":
            nc, code_bits = 64, 6
        if name == "c4w":
            nc = 4096
        p = synthetic.config4(dev, Hq=Hq, bd=bd, n_centroids=nc)
        if code_bits:
            p.tensors["code_words"] = hip_ops.pack_codes(p["code_pages"], code_bits)
        B, Hkv, T, D = 64, 8, 32768, 128
        paged = True
        if name == "c4mix":
            # SunShape-Mixed on pages: the 4 blocks of dim 4 with the largest sigma mass keep their
            # bf16 key values (16 dims per token, compact [P, Hkv, 16, 4, 4]); 28 blocks are VQ-coded
            cb = synthetic.make_codebook(Hkv, D, bd, 4)
            heavy = synthetic.heavy_blocks_by_sigma(cb.sigma, cb.perm, bd, 4).tolist()
            gd = torch.Generator(device=dev).manual_seed(304)
            P = p["code_pages"].shape[0]
            pt = torch.randn(P, Hkv, 16, 4, bd, generator=gd, device=dev, dtype=torch.bfloat16)
            p.tensors["pt_pages"], p.tensors["heavy"] = pt, torch.tensor(heavy)
    elif name in ("c4ct", "c4ctbd2", "c4ctg8", "c4ctmix", "c4ctw"):
        # the config-4 layer with the reference's contiguous rows (codes [B, Hkv, T, nb], V
        # [B, Hkv, T, D]) in place of pages; c4ctbd2 at the reference's default 4 bits/dim (64 blocks
        # of dim 2), c4ctg8 with 64 query heads (8 per KV head): the 4x4-MFMA-scores kernel;
        # c4ctmix: SunShape-Mixed with 4 bf16 passthrough blocks of dim 4 (compact [B, Hkv, T, 4, 4]);
        # c4ctw: 3 bits/dim at block_dim 4, 4,096 codewords per block, int16 codes
        B, Hkv, T, D = 64, 8, 32768, 128
        Hq = 64 if name == "c4ctg8" else 32
        bd = 2 if name == "c4ctbd2" else 4
        if name == "c4ctw":
            nc = 4096
        p = synthetic.config4_contiguous(dev, Hq=Hq, bd=bd, n_centroids=nc)
        paged = False
        if name == "c4ctmix":
            cb = synthetic.make_codebook(Hkv, D, bd, 104)
            heavy = synthetic.heavy_blocks_by_sigma(cb.sigma, cb.perm, bd, 4).tolist()
            gd = torch.Generator(device=dev).manual_seed(305)
            pt = torch.randn(B, Hkv, T, 4, bd, generator=gd, device=dev, dtype=torch.bfloat16)
            p.tensors["pt"], p.tensors["heavy"] = pt, torch.tensor(heavy)  # pt: the launch's passthrough
    elif name == "c5":
        # SunShape-Mixed: the config-5 keys encoded once (28 VQ blocks + 4 bf16 passthrough blocks)
        p = synthetic.config5(dev)
        B, Hq, Hkv, T, D, bd = 16, 14, 2, 16384, 64, 2
        paged = False
        heavy = p["heavy"].tolist()
        codes5, pt = hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy)
        p.tensors["codes"], p.tensors["pt"] = codes5, pt
        p.tensors["perm"] = p["perm"][None].expand(Hkv, D)
        p.meta["T"] = T
    elif name == "c3p6":
        # the config-3 layer at 3 bits/dim: 64 codewords per block, 6-bit codes packed five to an
        # int32 word (the layout sunshape/triton_kernels.py:250-266 reads)
        B, Hq, Hkv, T, D, bd = 16, 14, 2, 8192, 64, 2
        nc, code_bits = 64, 6
        cb = synthetic.make_codebook(Hkv, D, bd, 3, n_centroids=nc)
        g = torch.Generator().manual_seed(103)
        q3 = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(dev)
        c8 = torch.randint(0, nc, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8).to(dev)
        v3 = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(dev)
        p = synthetic.Problem("C3p6", {"q": q3, "codes": hip_ops.pack_codes(c8, code_bits), "codes_u8": c8,
                                       "v": v3, "perm": cb.perm.to(dev), "centroids": cb.centroids.to(dev)},
                              {"scale": 1.0 / math.sqrt(D), "B": B, "Hq": Hq, "Hkv": Hkv, "T": T})
        paged = False
    else:
        p = synthetic.config3(dev)
        B, Hq, Hkv, T, D, bd = 16, 14, 2, 8192, 64, 2
        paged = False
    nb = D // bd
    Dv = D
    # one call through the Python surface checks shapes and builds the launch once;
    # the timed loop replays the same C-ABI call with preallocated outputs
    out = torch.empty(B, Hq, 1, Dv, device=dev, dtype=torch.bfloat16)
    perm, cent = p["perm"].contiguous(), p["centroids"].contiguous()
    q = p["q"]
    if paged:
        codes, v = p.tensors.get("code_words", p["code_pages"]), p["v_pages"]
        bt, sl = p["block_table"], p["seq_lens"]
        pt = p.tensors.get("pt_pages")
        ref = hip_ops.decode(q, codes, v, perm, cent, scale=p.meta["scale"], block_table=bt, seq_lens=sl, kernel=kernel,
                             code_bits=code_bits, heavy=heavy, pt=pt)
    else:
        codes, v = p["codes"], p["v"]
        ref = hip_ops.decode(q, codes, v, perm, cent, scale=p.meta["scale"], heavy=heavy, pt=pt, kernel=kernel,
                             code_bits=code_bits)
    scores = None
    if name == "c4scores":  # config 4 also lists the raw fp32 scores [B, Hq, 1, T] as an output
        scores = torch.empty(B, Hq, 1, T, device=dev, dtype=torch.float32)
        ref = ref if not isinstance(ref, tuple) else ref[0]
    a = N.DecodeArgs(
        q=q.data_ptr(), q_dtype=N.SSQ_BF16, q_sb=q.stride(0), q_sh=q.stride(1), q_sl=q.stride(2),
        batch=B, num_q_heads=Hq, q_len=1, head_dim=D, num_kv_heads=Hkv, has_scale=1, scale=p.meta["scale"],
        perm=perm.data_ptr(), perm_sh=D, cent=cent.data_ptr(), cent_sh=nb * nc * bd,
        block_dim=bd, n_blocks=nb, n_centroids=nc, code_bits=code_bits,
        layout=N.SSQ_PAGED if paged else N.SSQ_CONTIGUOUS, seq_len=T,
        codes=codes.data_ptr(), c_sb=codes.stride(0), c_sh=codes.stride(1), c_st=codes.stride(2),
        block_table=bt.data_ptr() if paged else None, bt_sb=bt.stride(0) if paged else 0,
        seq_lens=sl.data_ptr() if paged else None, page_size=16 if paged else 0,
        v=v.data_ptr(), v_dtype=N.SSQ_BF16, value_dim=Dv, v_sb=v.stride(0), v_sh=v.stride(1), v_st=v.stride(2),
        out=out.data_ptr(), o_sb=out.stride(0), o_sh=out.stride(1), o_sl=out.stride(2), kernel=kernel,
    )
    if scores is not None:
        a.scores, a.s_sb, a.s_sh, a.s_sl = scores.data_ptr(), scores.stride(0), scores.stride(1), scores.stride(2)
    if heavy is not None:
        a.heavy_mask[0], a.heavy_mask[1] = N.heavy_mask_words(heavy)
        a.pt, a.pt_dtype, a.pt_dense = pt.data_ptr(), N.SSQ_BF16, 0
        a.pt_sb, a.pt_sh, a.pt_st = pt.stride(0), pt.stride(1), pt.stride(2)
    L = N.lib()
    ws_bytes = L.ssq_decode_workspace_size(ctypes.byref(a))
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step():
        rc = L.ssq_decode(ctypes.byref(a), ws.data_ptr(), ws_bytes, stream)
        if rc:
            N.check(rc)

    step()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), "timed launch differs from the checked Python-surface launch"
    keys = B * Hkv * T
    code_bytes = codes.numel() * codes.element_size() if code_bits or nc > 256 else B * Hkv * T * nb
    algo_bytes = (code_bytes                       # uint8 codes (or packed words, or int16 codes)
                  + B * Hkv * T * Dv * 2           # bf16 V
                  + B * Hq * D * 2                 # bf16 q
                  + B * Hq * Dv * 2                # bf16 out
                  + Hkv * nb * nc * bd * 4         # fp32 codebooks
                  + Hkv * D * 8                    # int64 permutations
                  + (B * (T // 16) * 4 if paged else 0)  # int32 block table
                  + (pt.numel() * 2 if pt is not None else 0)  # bf16 passthrough values
                  + (scores.numel() * 4 if scores is not None else 0))  # fp32 raw scores
    cfg = {"workload": {"c4": "C4 paged fused decode (Llama-3-8B layer, 2 bits/dim)",
                        "c4g8": "C4 layer with 64 query heads (8 per KV head), paged, 2 bits/dim",
                        "c4bd2": "C4 layer at 4 bits/dim (64 blocks of dim 2), paged",
                        "c4p6": "C4 layer at 3 bits/dim: 64 codewords, 6-bit codes packed in int32 words, paged",
                        "c4ct": "C4 layer with contiguous rows (codes [B, Hkv, T, nb], V [B, Hkv, T, D]), 2 bits/dim",
                        "c4ctbd2": "C4 layer with contiguous rows at 4 bits/dim (64 blocks of dim 2)",
                        "c4ctg8": "C4 layer with contiguous rows, 64 query heads (8 per KV head), 2 bits/dim",
                        "c4ctmix": "C4 layer with contiguous rows, SunShape-Mixed: 28 VQ blocks + 4 bf16 passthrough blocks of dim 4",
                        "c4mix": "C4 paged, SunShape-Mixed: 28 VQ blocks + 4 bf16 passthrough blocks of dim 4",
                        "c4scores": "C4 paged fused decode that also writes the fp32 scores [B, Hq, 1, T]",
                        "c4w": "C4 layer at 3 bits/dim: 4,096 codewords per block of dim 4, int16 codes, paged",
                        "c4ctw": "C4 layer with contiguous rows at 3 bits/dim: 4,096 codewords per block of dim 4, int16 codes",
                        "c3": "C3 contiguous fused decode (Qwen2.5-0.5B layer, 4 bits/dim)",
                        "c5": "C5 SunShape-Mixed fused decode (config-5 keys: 28 VQ + 4 bf16 blocks of dim 2)",
                        "c3p6": "C3 layer at 3 bits/dim: 64 codewords, 6-bit codes packed in int32 words"}[name],
           "batch": B, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "context": T, "block_dim": bd,
           "bits_per_dim": (code_bits or math.log2(nc)) / bd, "n_centroids": nc,
           "layout": "paged16" if paged else "contiguous", "kernel": kernel}
    if code_bits:
        cfg["code_bits"] = code_bits
    unit_data = (p, paged)
    step.surface = _surface_call(p, paged, q, codes, v, perm, cent, heavy, pt, code_bits, kernel, ref)
    return step, keys, algo_bytes, cfg, unit_data, "ssq_decode"


def _surface_call(p, paged, q, codes, v, perm, cent, heavy, pt, code_bits, kernel, ref):
    """(name, fn): the same decode through the Python drop-in surface.  Contiguous byte codes go
    through SunShapeAttentionImpl.forward over a SunShapeQuantizedKeys payload (the reference's
    vLLM decode call, sunshape/vllm_attn_backend.py:271-305); paged and packed codes, which that
    payload does not carry, through hip_ops.decode."""
    import torch

    from sunshape_amd import hip_ops
    from sunshape_amd import vllm_attn_backend as VB
    from sunshape_amd.codec import SunShapeBlockCodec
    from sunshape_amd.hf import SunShapeBundle
    from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState

    scale = p.meta["scale"]
    if paged or code_bits or kernel:  # an explicit kernel choice: the drop-in surface has no such argument
        kw = dict(block_table=p["block_table"], seq_lens=p["seq_lens"]) if paged else {}
        return "hip_ops.decode", lambda: hip_ops.decode(q, codes, v, perm, cent, scale=scale, heavy=heavy, pt=pt,
                                                        kernel=kernel, code_bits=code_bits, **kw)
    mode = "profileperm_mixed_precision" if heavy is not None else "profileperm_baseline"
    codec = SunShapeBlockCodec.from_buffers(perm, cent, mode=mode, device=q.device,
                                            mixed_high_precision_blocks=None if heavy is None else torch.tensor(heavy))
    bundle = SunShapeBundle("bench", [0], 0.0, codec.block_dim, mode, 0, 0, 0, {0: codec})
    VB.register_runtime_state(SunShapeVLLMRuntimeState("bench", "bench", mode, 0.0, codec.block_dim, [0], bundle,
                                                       "cuda"))
    B, Hkv, T = codes.shape[0], codes.shape[1], codes.shape[2]
    qk = VB.SunShapeQuantizedKeys(quantized_heads=(), batch_size=B, num_kv_heads=Hkv, seq_len=T, codes=codes,
                                  passthrough=pt, passthrough_dense=False)
    impl = VB.get_backend_factory().make_impl(layer_idx=0)
    got = impl(q, qk, v, scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), "SunShapeAttentionImpl.forward differs from the checked launch"
    return "SunShapeAttentionImpl.forward", lambda: impl(q, qk, v, scale=scale)


def _time_surface(name, fn, n=100):
    """Host time to issue one call and wall time per call (host and kernel overlapping), over n calls."""
    import torch

    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        fn()
    host = time.perf_counter() - t0
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return {"api": name, "calls": n, "host_us_per_call": host / n * 1e6, "wall_us_per_call": wall / n * 1e6}


def _time_graph(name, fn, n=50, per_graph=10):
    """The same call captured in graphs (torch.cuda.graph: HIP graphs, as a serving loop captures
    its decode step): one call per graph replayed n times back to back, and per_graph calls per
    graph (a serving step captures every layer's call in one graph) replayed n / per_graph times.
    Per-call GPU time from events and the host's time per replay; every replay's outputs are
    checked against an eager call.  On this ROCm a graph launch costs the host 17-29 us, more than
    a small call's two direct launches (4-6 us), so one-call replays of a ~20 us call are bound by
    the host; a many-call graph amortises it."""
    import torch

    eager = fn().clone()
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    res = {"api": name}
    for calls, key in ((1, "one_call"), (per_graph, f"{per_graph}_calls")):
        graph = torch.cuda.CUDAGraph()
        outs = []
        with torch.cuda.graph(graph):
            for _ in range(calls):
                outs.append(fn())
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(o, eager) for o in outs), "graph replay differs from the eager call"
        reps = max(1, n // calls)
        t0 = time.perf_counter()
        start.record()
        for _ in range(reps):
            graph.replay()
        end.record()
        host = time.perf_counter() - t0
        torch.cuda.synchronize()
        res[key] = {"replays": reps, "us_per_call": start.elapsed_time(end) * 1e3 / (reps * calls),
                    "host_us_per_replay": host * 1e6 / reps}
    res["us_per_call"] = res["one_call"]["us_per_call"]
    return res


def _scores_workload(dev, kernel=0):
    import torch

    from sunshape_amd import _native as N
    from sunshape_amd import synthetic

    p = synthetic.config2(dev)
    B, Hq, Hkv, T, D, bd = 16, 14, 2, 8192, 64, 8
    nb = D // bd
    out = torch.empty(B, Hq, 1, T, device=dev, dtype=torch.float32)
    q, codes, perm, cent = p["q"], p["codes"], p["perm"], p["centroids"]
    a = N.DecodeArgs(
        q=q.data_ptr(), q_dtype=N.SSQ_BF16, q_sb=q.stride(0), q_sh=q.stride(1), q_sl=q.stride(2),
        batch=B, num_q_heads=Hq, q_len=1, head_dim=D, num_kv_heads=Hkv, has_scale=1, scale=p.meta["scale"],
        perm=perm.data_ptr(), perm_sh=D, cent=cent.data_ptr(), cent_sh=nb * 256 * bd,
        block_dim=bd, n_blocks=nb, n_centroids=256, layout=N.SSQ_CONTIGUOUS, seq_len=T,
        codes=codes.data_ptr(), c_sb=codes.stride(0), c_sh=codes.stride(1), c_st=codes.stride(2),
        scores=out.data_ptr(), s_sb=out.stride(0), s_sh=out.stride(1), s_sl=out.stride(2), kernel=kernel,
    )
    L = N.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step():
        rc = L.ssq_attention_scores(ctypes.byref(a), stream)
        if rc:
            N.check(rc)

    keys = B * Hkv * T
    algo = B * Hkv * T * nb + B * Hq * T * 4 + B * Hq * D * 2 + Hkv * nb * 256 * bd * 4 + Hkv * D * 8
    cfg = {"workload": "C2 GQA scores (Qwen2.5-0.5B layer, 1 bit/dim)", "batch": B, "q_heads": Hq, "kv_heads": Hkv,
           "head_dim": D, "context": T, "block_dim": bd, "bits_per_dim": 1.0, "layout": "contiguous"}
    return step, keys, algo, cfg, None, "ssq_attention_scores"


def _encode_workload(dev, kernel, pro=False):
    """c5enc: the config-5 encode (grid search by default).  c5encpro: the same keys under a
    SunShape-Pro block metric E [D, D] (sunshape/codec.py:375-376), seeded near the identity;
    the metric encode runs the MFMA screen on E x and E c."""
    import torch

    from sunshape_amd import hip_ops, synthetic

    p = synthetic.config5(dev)
    heavy = p["heavy"].tolist()
    keys_t = p["keys"]
    B, Hkv, S, D = keys_t.shape
    metric = None
    if pro:
        g = torch.Generator().manual_seed(55)
        metric = (torch.eye(D) + 0.3 * torch.randn(D, D, generator=g)).to(dev)
        ref, _ = hip_ops.encode(keys_t, p["perm"], p["centroids"], heavy=heavy, metric=metric, kernel=1)
        got, _ = hip_ops.encode(keys_t, p["perm"], p["centroids"], heavy=heavy, metric=metric, kernel=kernel)
        assert torch.equal(got, ref), "metric encode differs from the exact scan"
    # the search grid is built once per codebook (as a codec caches it); kernel 2 times the
    # exhaustive MFMA screen instead
    grid, grid_ms = None, None
    if kernel in (0, 3) and not pro:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        grid = hip_ops.encode_grid(p["centroids"])
        torch.cuda.synchronize()
        grid_ms = (time.perf_counter() - t0) * 1e3
        ref, _ = hip_ops.encode(keys_t, p["perm"], p["centroids"], heavy=heavy, kernel=2)
        got, _ = hip_ops.encode(keys_t, p["perm"], p["centroids"], heavy=heavy, kernel=kernel, grid=grid)
        assert torch.equal(got, ref), "grid encode differs from the MFMA encode"

    from sunshape_amd import _native as N

    a, codes_k, pt_k, keep = hip_ops.encode_args(keys_t, p["perm"], p["centroids"], heavy=heavy, kernel=kernel,
                                                 grid=grid, metric=metric)
    L = N.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step(_alive=(keep, codes_k, pt_k)):  # one prebuilt C-ABI call (outputs rewritten in place)
        rc = L.ssq_encode(ctypes.byref(a), stream)
        if rc:
            N.check(rc)

    n = B * Hkv * S
    algo = n * D * 2 + n * 32 + n * 4 * 2 * 2 + Hkv * 32 * 256 * 2 * 4 + (D * D * 4 if pro else 0)
    cfg = {"workload": ("C5 encode (16 x 2 x 16384 bf16 keys, 28 VQ + 4 bf16 blocks of dim 2)" +
                        (" under a SunShape-Pro block metric" if pro else "")), "keys": n,
           "head_dim": D, "block_dim": 2, "heavy_blocks": 4, "kernel": kernel,
           "search": "grid" if grid is not None else "exhaustive", "grid_build_ms": grid_ms, "metric": pro,
           "grid_bytes": None if grid is None else grid.numel(),
           "grid_budget_bytes": _grid_budget()}
    return step, n, algo, cfg, None, "ssq_encode" if grid is None else "ssq_encode_grid"


def _grid_budget():
    """The process-wide byte budget the codecs' cached encode grids share."""
    from sunshape_amd import codec as C

    return C._GRID_BUDGET[0]


def _append_workload(name, dev, kernel):
    """One serving step's append: the new key of every (sequence, KV head) encoded into its slot of
    the 16-token pages.  c4append: the config-4 codec (64 x 8 keys, 32 blocks of dim 4, per-head
    codebooks, the MFMA encode); c5append: the config-5 codec (16 x 2 keys, 28 VQ blocks of dim 2 +
    4 passthrough, the grid search with the codec's grid); c4appendw: the config-4 step with a
    4,096-codeword codec of dim 4 (3 bits/dim, int16 codes; the exhaustive scan split over lanes)."""
    import torch

    from sunshape_amd import hip_ops, synthetic

    page = 16
    g = torch.Generator(device=dev).manual_seed(44)
    heavy, grid, pt_pages = None, None, None
    nc = 256
    if name in ("c4append", "c4appendw"):
        nc = 4096 if name == "c4appendw" else 256
        p = synthetic.config4(dev, T=256, n_centroids=nc)
        B, Hkv, D, bd, T = 64, 8, 128, 4, 256
        bt = p["block_table"]
        perm, cent = p["perm"], p["centroids"]
        sigma = synthetic.make_codebook(Hkv, D, bd, 4).sigma.to(dev)  # config 4's codec (seed 4)
        keys_t = (torch.randn(B, Hkv, 1, D, generator=g, device=dev) * sigma[:, None, :]).to(torch.bfloat16)
    else:
        p = synthetic.config5(dev, B=16, S=page)
        B, Hkv, D, bd, T = 16, 2, 64, 2, 256
        keys_t = p["keys"][:, :, -1:].contiguous()  # keys drawn as the codec was fitted
        heavy = p["heavy"].tolist()
        bt = torch.randperm(B * T // page, device=dev).to(torch.int32).view(B, T // page)
        perm, cent = p["perm"], p["centroids"]
        if kernel in (0, 3):
            grid = hip_ops.encode_grid(cent)
        pt_pages = torch.zeros(B * T // page, Hkv, page, sum(heavy), bd, device=dev, dtype=torch.bfloat16)
    nb = D // bd
    code_pages = torch.zeros(B * T // page, Hkv, page, nb, device=dev, dtype=hip_ops.index_dtype(nc))
    pos = T - 1  # the step's token lands in the last slot of each sequence's last page
    slots = (bt[:, pos // page].to(torch.int64) * page + pos % page).view(B, 1).contiguous()
    ref, _ = hip_ops.encode(keys_t, perm, cent, heavy=heavy, kernel=2 if bd == 4 and nc == 256 else 1)

    # the timed loop replays one prebuilt C-ABI call: at a few microseconds per launch, the
    # Python wrapper's checks would otherwise be what the events measure
    from sunshape_amd import _native as N

    a, _, _, keep = hip_ops.encode_args(keys_t, perm, cent, heavy=heavy, codes_out=code_pages, pt_out=pt_pages,
                                        slot_mapping=slots, kernel=kernel, grid=grid)
    L = N.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step(_alive=(keep, code_pages, pt_pages)):  # the args point into these
        rc = L.ssq_encode(ctypes.byref(a), stream)
        if rc:
            N.check(rc)

    step()
    torch.cuda.synchronize()
    pages = bt[:, pos // page].long()
    got = code_pages[pages, :, pos % page]  # [B, Hkv, nb]
    assert torch.equal(got, ref[:, :, 0]), "paged append differs from the contiguous encode"
    n = B * Hkv
    nlight = nb - (sum(heavy) if heavy else 0)
    cbytes = 1 if nc <= 256 else 2
    algo = n * D * 2 + n * nb * cbytes + Hkv * nlight * nc * bd * 4 + Hkv * D * 8 + B * 8 + n * (nb - nlight) * bd * 2
    cfg = {"workload": {"c4append": "F1 paged append, one decode step at the config-4 shape "
                                    "(64 x 8 keys, 32 blocks of dim 4)",
                        "c5append": "F1 paged append, one decode step with the config-5 codec "
                                    "(16 x 2 keys, 28 VQ blocks of dim 2 + 4 bf16 passthrough)",
                        "c4appendw": "F1 paged append, one decode step at the config-4 shape with a 4,096-codeword "
                                     "codec (64 x 8 keys, 32 blocks of dim 4, int16 codes)"}[name],
           "keys": n, "head_dim": D, "block_dim": bd, "n_centroids": nc, "page_size": page, "kernel": kernel,
           "search": "grid" if grid is not None else "exhaustive"}
    return step, n, algo, cfg, None, "ssq_encode"


def _copy_workload(dev):
    """A plain 1 GiB device-to-device copy: calibrates rocprofv3's FETCH_SIZE/WRITE_SIZE counters."""
    import torch

    n = 1 << 30
    src = torch.ones(n // 2, device=dev, dtype=torch.bfloat16)
    dst = torch.empty_like(src)

    def step():
        dst.copy_(src)

    cfg = {"workload": "calibration copy, 1 GiB read + 1 GiB write", "bytes_read": n, "bytes_written": n}
    return step, n // 2, 2 * n, cfg, None, "copy"


# (workgroups per CU, loads in flight per thread, 1: a contiguous chunk per workgroup / 0: grid-stride)
READ_PROBE_SHAPES = ((16, 4, 0), (8, 8, 0), (2, 8, 1), (4, 8, 1), (8, 4, 1), (2, 16, 1))


def _stream_probe(dev, launches=10):
    """Achievable HBM rates on this box, reference points for the roofline fraction: a 2 GiB
    read-only stream (sunshape_amd/csrc/probe: 16-byte non-temporal loads, grid-stride) and a
    1 GiB device-to-device copy (1 GiB read + 1 GiB written), each timed with events per launch,
    median of `launches`.  Both buffers exceed the 256 MB Infinity Cache."""
    import torch

    from sunshape_amd import _native as N
    from sunshape_amd.build import PROBE_PATH

    def timed(fn):
        for _ in range(3):
            fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(launches)]
        for s0, e0 in ev:
            s0.record()
            fn()
            e0.record()
        torch.cuda.synchronize()
        return sorted(s0.elapsed_time(e0) for s0, e0 in ev)[launches // 2]

    out = {"launches": launches}
    n = 2 << 30
    if os.path.exists(PROBE_PATH):
        probe = ctypes.CDLL(PROBE_PATH)
        probe.ssq_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int,
                                                ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        buf = torch.ones(n // 2, device=dev, dtype=torch.bfloat16)
        sink = torch.zeros(1, device=dev, dtype=torch.int32)
        stream = N.stream_of(dev)
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        best = None
        for per_cu, unroll, chunked in READ_PROBE_SHAPES:  # the best of a small sweep of launch shapes
            def read():
                rc = probe.ssq_probe_stream_read(buf.data_ptr(), n, sink.data_ptr(), per_cu * cus, unroll, chunked,
                                                 stream)
                if rc:
                    raise RuntimeError(f"stream probe launch failed: HIP error {rc}")

            gbps = n / (timed(read) * 1e-3) / 1e9
            out.setdefault("read_sweep", []).append([per_cu, unroll, chunked, round(gbps, 1)])
            if best is None or gbps > best[0]:
                best = (gbps, per_cu, unroll, chunked)
        out["read"] = ("2 GiB read, 16-byte non-temporal loads (csrc/probe/ssq_probe_stream.hip), best of %d launch "
                       "shapes: %d workgroups of 256 per CU, %d loads in flight per thread, %s"
                       % (len(READ_PROBE_SHAPES), best[1], best[2], "a chunk per workgroup" if best[3] else "grid-stride"))
        out["read_GBps"] = best[0]
        del buf
    src = torch.ones(1 << 29, device=dev, dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    out["copy"] = "1 GiB read + 1 GiB written (torch copy_)"
    out["copy_GBps"] = 2 * (1 << 30) / (timed(lambda: dst.copy_(src)) * 1e-3) / 1e9
    del src, dst
    return out


# ----------------------------------------------------------------------------- CPU baseline
def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_baseline(unit_data, seconds):
    """The reference's eager PyTorch decode path on the host's cores (oracle/torch_eager.py).

    One (batch, KV head) unit at a time, as sunshape/vllm_attn_backend.py:228-252 loops: per-block
    dequantize, fp32 q . k_hat^T, softmax, cast to the value dtype, P.V.  Units are drawn at random
    from the workload until about ``seconds`` of CPU work is timed; only the torch calls are timed
    (the unit's codes and values are copied to the host outside the timed region).  keys/s is the
    sample's rate, i.e. the whole batch's rate extrapolated from the sampled units.
    """
    import numpy as np
    import torch

    from oracle import torch_eager as TE

    p, paged = unit_data
    G = p.meta["Hq"] // p.meta["Hkv"] if "Hq" in p.meta else 7
    T = p.meta["T"]
    perm, cent = p["perm"].cpu(), p["centroids"].cpu()
    inv = torch.argsort(perm, dim=-1)
    q = p["q"].cpu()
    threads = torch.get_num_threads()
    rng = np.random.default_rng(0)
    units, elapsed = 0, 0.0
    n_units = p.meta["B"] * p.meta["Hkv"]
    wall0 = time.perf_counter()
    while elapsed < seconds and units < 4096 and time.perf_counter() - wall0 < 4 * seconds:
        b = int(rng.integers(p.meta["B"]))
        kv = int(rng.integers(p.meta["Hkv"]))
        if paged:
            pages = p["block_table"][b].long()
            codes = p["code_pages"][pages][:, kv].reshape(-1, p["code_pages"].shape[-1]).cpu()
            v = p["v_pages"][pages][:, kv].permute(0, 2, 1).reshape(-1, p["v_pages"].shape[2]).cpu()
        else:
            codes = p.tensors.get("codes_u8", p["codes"])[b, kv].cpu()  # byte codes (unpacked)
            v = p["v"][b, kv].cpu()
        heavy, ptv = None, None
        if "pt" in p.tensors or "pt_pages" in p.tensors:  # SunShape-Mixed: the reference's dense fp32 layout
            heavy = [bool(x) for x in p["heavy"].tolist()]
            ptv = torch.zeros(codes.shape + (cent.shape[-1],), dtype=torch.float32)
            if paged:
                ptu = p["pt_pages"][pages][:, kv].reshape(-1, *p["pt_pages"].shape[-2:])
            else:
                ptu = p["pt"][b, kv]
            ptv[:, torch.tensor(heavy)] = ptu.float().cpu()
        qu = q[b, kv * G:(kv + 1) * G]
        t0 = time.perf_counter()
        TE.decode_unit(qu, codes, v, cent[kv], inv[kv], p.meta["scale"], heavy, ptv)
        elapsed += time.perf_counter() - t0
        units += 1
    return {"value": units * T / elapsed, "unit": "keys/s", "cores": threads, "kind": "port",
            "host_cpus": os.cpu_count(), "cpu_model": _cpu_model(),
            "sample": f"{units} (batch, KV head) units drawn with replacement from the workload's {n_units}, x {T} keys each, eager torch restatement of the "
                      f"reference decode path (per-block dequantize, fp32 q.k_hat^T, softmax, bf16 cast, P.V; "
                      f"sunshape/vllm_attn_backend.py:228-252) on {threads} torch threads, {elapsed:.1f} s timed; "
                      f"keys/s extrapolates the sampled units' rate to the batch"}


def _cold_launches(step, n, algo_bytes, dev):
    """The same launch with cold caches: before each event-timed launch, a 1 GiB read-modify-write
    pass (stream-ordered before it) evicts the inputs from L2 and the 256 MB Infinity Cache, so every
    input byte comes from HBM.  The main timed loop is warm: a workload smaller than the Infinity
    Cache (configs 2, 3, 5) can be served from it on repeated launches."""
    import torch

    flush = torch.zeros(1 << 28, device=dev, dtype=torch.int32)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for i in range(n):
        flush.add_(1)
        starts[i].record()
        step()
        ends[i].record()
    torch.cuda.synchronize()
    ms = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    med = ms[len(ms) // 2]
    del flush
    return {"launches": n, "kernel_median_ms": med, "kernel_min_ms": ms[0],
            "hbm_GBps": algo_bytes / (med * 1e-3) / 1e9, "flush_bytes": 1 << 30}


# ----------------------------------------------------------------------------- main
def main():
    args = _args()
    if args.gpus != 1:
        sys.exit(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}")
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload in ("c4", "c3", "c5", "c4g8", "c4bd2", "c3p6", "c4p6", "c4ct", "c4ctbd2", "c4ctg8", "c4ctmix",
                         "c4mix", "c4scores", "c4w", "c4ctw"):
        step, keys, algo_bytes, cfg, unit_data, kname = _decode_workload(args.workload, dev, args.kernel)
    elif args.workload == "c2":
        step, keys, algo_bytes, cfg, unit_data, kname = _scores_workload(dev, args.kernel)
    elif args.workload in ("c4append", "c5append", "c4appendw"):
        step, keys, algo_bytes, cfg, unit_data, kname = _append_workload(args.workload, dev, args.kernel)
    elif args.workload == "copycal":
        step, keys, algo_bytes, cfg, unit_data, kname = _copy_workload(dev)
    else:
        step, keys, algo_bytes, cfg, unit_data, kname = _encode_workload(dev, args.kernel, args.workload == "c5encpro")

    # Clock settling, before the warm-up steps: on a box that was idle, the first ~100 launches of
    # a sustained HBM-bound decode run up to 35 % slower than the steady state (per-dispatch kernel
    # traces: 0.745 ms, then 1.06 ms falling back to 0.76 ms over ~100 back-to-back launches of
    # c4g8) while the GPU's power management settles.  Untimed; the line reports how many ran.
    settle_n, t_settle = 0, time.perf_counter()
    while time.perf_counter() - t_settle < args.settle_s:
        for _ in range(8):
            step()
        settle_n += 8
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_settle
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # per-launch HIP events on the launch stream (torch's current stream, which the C ABI is given)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record()
        step()
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    avg_ms = sum(launch_ms) / len(launch_ms)
    ms_per_step = wall * 1e3 / args.steps
    achieved_gbps = algo_bytes / (avg_ms * 1e-3) / 1e9
    traffic = _traffic_from_profiles(f"{kname}_{args.workload}_pmc")
    line = {
        "metric": METRIC,
        "value": keys / (ms_per_step * 1e-3),
        "unit": "keys/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": cfg,
        "settle": {"launches": settle_n, "seconds": settle_s},
        "hbm_GBps": achieved_gbps,
        "pct_hbm_peak": 100.0 * achieved_gbps / HBM_PEAK_GBPS,
        "kernel_avg_ms": avg_ms,
        "kernel_min_ms": min(launch_ms),
        "kernel_median_ms": sorted(launch_ms)[len(launch_ms) // 2],
        "roofline": {"bound": "hbm", "achieved": achieved_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved_gbps / HBM_PEAK_GBPS, "traffic": traffic,
                     "kernel": kname, "algorithmic_bytes_per_launch": algo_bytes},
    }
    if "q_heads" in cfg:  # every query head scores every key: q.k scores/s = keys/s x G
        line["qk_scores_per_s"] = line["value"] * (cfg["q_heads"] // cfg["kv_heads"])
    if args.workload in ("c5enc", "c5encpro"):
        # the exhaustive search's distance work (28 light blocks x 256 codewords x the 4-term
        # augmented dot product [-2x, |x|^2, 1] . [c, 1, |c|^2], a multiply-add per term); the grid
        # search evaluates a few codewords per block instead, so its roofline is HBM on the
        # algorithmic bytes and this figure is only a comparison
        flop = keys * 28 * 256 * 2 * 4 + (keys * 28 * 2 * 2 * 2 if cfg["metric"] else 0)  # + E_b x (2x2) per block
        tf = flop / (avg_ms * 1e-3) / 1e12
        line["unit"] = "keys/s"
        line["metric"] = "VQ encode: keys encoded/sec/GPU"
        line["exhaustive_equiv_tflops"] = tf
        if cfg["search"] == "exhaustive":
            line["roofline"] = {"bound": "mfma", "achieved": tf, "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                                "frac": tf / MFMA_F32_PEAK_TFLOPS, "traffic": traffic, "kernel": kname,
                                "algorithmic_flop_per_launch": flop}
    if args.workload != "copycal":
        line["hbm_stream"] = _stream_probe(dev)
        if "read_GBps" in line["hbm_stream"]:
            line["hbm_stream"]["frac_of_read"] = achieved_gbps / line["hbm_stream"]["read_GBps"]
    if args.workload != "copycal" and args.cold_steps > 0:
        line["cold"] = _cold_launches(step, args.cold_steps, algo_bytes, dev)
    if getattr(step, "surface", None) is not None:
        # the same decode through the Python drop-in, beside the prebuilt C-ABI replay timed above
        line["python_surface"] = _time_surface(*step.surface)
        line["python_surface"]["c_abi_kernel_avg_us"] = avg_ms * 1e3
        try:  # a measurement beside the contract's figures: never the reason the line is missing
            line["graph_replay"] = _time_graph(*step.surface)
        except Exception as exc:  # noqa: BLE001
            line["graph_replay"] = {"error": f"{type(exc).__name__}: {exc}"}
    if not args.no_cpu and unit_data is not None:
        line["cpu_baseline"] = _cpu_baseline(unit_data, args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
