"""ssq_decode_noalloc (split workspace in the library's per-device scratch) against ssq_decode
(workspace from the caller): same kernels, so outputs must agree bit for bit.  Two calls in a
row, the second with a smaller input; a problem whose workspace exceeds the scratch is refused
before any launch."""

import ctypes

import pytest
import torch

from _util import log
from sunshape_amd import _native as N
from sunshape_amd import hip_ops, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _decode_args(q, codes, v, perm, cent, scale, out, lse, *, block_table=None, seq_lens=None, num_splits=0,
                 kernel=0):
    """ssq_decode_args for a contiguous (or paged, with block_table) problem, through the C ABI."""
    B, Hq, Lq, D = q.shape
    Hkv = codes.shape[1]
    nb = codes.shape[-1]
    bd = D // nb
    paged = block_table is not None
    T = block_table.shape[1] * codes.shape[2] if paged else codes.shape[2]
    Dv = v.shape[2] if paged else v.shape[3]
    a = N.DecodeArgs(
        q=N.ptr(q), q_dtype=N.dtype_code(q.dtype), q_sb=q.stride(0), q_sh=q.stride(1), q_sl=q.stride(2),
        batch=B, num_q_heads=Hq, q_len=Lq, head_dim=D, num_kv_heads=Hkv, has_scale=1, scale=float(scale),
        perm=N.ptr(perm), perm_sh=D if perm.ndim == 2 else 0, cent=N.ptr(cent),
        cent_sh=cent[0].numel() if cent.ndim == 4 else 0,
        block_dim=bd, n_blocks=nb, n_centroids=cent.shape[-2],
        layout=N.SSQ_PAGED if paged else N.SSQ_CONTIGUOUS, seq_len=T,
        codes=N.ptr(codes), c_sb=codes.stride(0), c_sh=codes.stride(1), c_st=codes.stride(2),
        block_table=N.ptr(block_table), bt_sb=block_table.stride(0) if paged else 0, seq_lens=N.ptr(seq_lens),
        page_size=codes.shape[2] if paged else 0,
        v=N.ptr(v), v_dtype=N.dtype_code(v.dtype), value_dim=Dv, v_sb=v.stride(0), v_sh=v.stride(1),
        v_st=v.stride(2),
        out=N.ptr(out), o_sb=out.stride(0), o_sh=out.stride(1), o_sl=out.stride(2), lse=N.ptr(lse),
        num_splits=num_splits, kernel=kernel,
    )
    return a


def _both(p, paged=False, **kw):
    """(out, lse) from ssq_decode with a torch workspace and from ssq_decode_noalloc."""
    lib = N.lib()
    q = p["q"]
    if paged:
        codes, v = p["code_pages"], p["v_pages"]
        Dv = v.shape[2]
        extra = dict(block_table=p["block_table"], seq_lens=p["seq_lens"])
    else:
        codes, v = p["codes"], p["v"]
        Dv = v.shape[3]
        extra = {}
    B, Hq, Lq, _ = q.shape
    res = []
    for no_alloc in (False, True):
        out = torch.full((B, Hq, Lq, Dv), float("nan"), device=DEV, dtype=v.dtype)
        lse = torch.full((B, Hq, Lq), float("nan"), device=DEV, dtype=torch.float32)
        a = _decode_args(q, codes, v, p["perm"], p["centroids"], p.meta["scale"], out, lse, **extra, **kw)
        ws_bytes = lib.ssq_decode_workspace_size(ctypes.byref(a))
        assert 0 < ws_bytes <= N.NOALLOC_SCRATCH_BYTES, ws_bytes  # the case exercises the workspace
        st = N.stream_of(DEV)
        if no_alloc:
            N.check(lib.ssq_decode_noalloc(ctypes.byref(a), st))
        else:
            ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
            N.check(lib.ssq_decode(ctypes.byref(a), N.ptr(ws), ws_bytes, st))
        torch.cuda.synchronize()
        res.append((out, lse))
    return res


def _same(res, what):
    (o1, l1), (o2, l2) = res
    assert not torch.isnan(o1.float()).any() and not torch.isnan(l1).any(), what
    assert torch.equal(o1, o2), f"{what}: outputs differ"
    assert torch.equal(l1, l2), f"{what}: lse differ"


def test_noalloc_matches_decode_contiguous_two_calls():
    log("no-alloc decode: contiguous, B=8 T=8192 then B=2 T=1500")
    _same(_both(synthetic.config3(DEV, B=8, T=8192)), "config-3 layer, B=8")
    _same(_both(synthetic.config3(DEV, seed=7, B=2, T=1500)), "config-3 layer, B=2 (smaller)")


def test_noalloc_matches_decode_paged_and_generic():
    log("no-alloc decode: paged MFMA kernel (B=2 T=4096), then generic kernel (B=1 T=2048)")
    p = synthetic.config4(DEV, B=2, T=4096)
    _same(_both(p, paged=True), "paged, B=2")
    _same(_both(synthetic.config3(DEV, seed=9, B=1, T=2048), kernel=1), "generic kernel, B=1 (smaller)")


def test_noalloc_refuses_workspace_beyond_scratch():
    log("no-alloc decode: workspace above the scratch is refused before launch")
    lib = N.lib()
    p = synthetic.config3(DEV, B=4, T=8192)
    q = torch.zeros(4, 14, 80, 64, device=DEV, dtype=torch.bfloat16)  # 80 query rows per head
    out = torch.empty(4, 14, 80, 64, device=DEV, dtype=torch.bfloat16)
    lse = torch.empty(4, 14, 80, device=DEV, dtype=torch.float32)
    a = _decode_args(q, p["codes"], p["v"], p["perm"], p["centroids"], p.meta["scale"], out, lse,
                     num_splits=32, kernel=1)
    need = lib.ssq_decode_workspace_size(ctypes.byref(a))
    assert need > N.NOALLOC_SCRATCH_BYTES, need
    rc = lib.ssq_decode_noalloc(ctypes.byref(a), N.stream_of(DEV))
    assert rc == N.SSQ_ERR_UNSUPPORTED
    assert b"scratch" in lib.ssq_last_error()
    with pytest.raises(N.SunShapeKernelError, match="scratch"):
        hip_ops.decode(q, p["codes"], p["v"], p["perm"], p["centroids"], scale=p.meta["scale"], num_splits=32,
                       kernel=1, no_alloc=True)
