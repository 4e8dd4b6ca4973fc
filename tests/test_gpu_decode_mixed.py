"""SunShape-Mixed passthrough blocks and additive masks on the 4x4-MFMA-scores decode kernel, over
vLLM-style pages and over contiguous rows at head_dim 128, against the oracle.

The reference scores passthrough blocks from the stored key values instead of codes
(sunshape/codec.py:387-398, dense fp32 [T, nb, bd] with zeros on light blocks) and adds the
mask slice before the softmax (sunshape/vllm_attn_backend.py:241-249).  Here the kernel zeroes the
query on passthrough dims in its codeword pass and adds one 4x4 MFMA per passthrough dim with the
stored value as the B operand, so scores agree within fp32 rounding (SCORE_TOL)."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PAGE = 16


def _problem(B, Hq, Hkv, Lq, D, bd, T, n_heavy, pdt, dense, seed, vdt=torch.bfloat16):
    """Contiguous inputs (CPU): q, codes, v, the dense fp32 passthrough the oracle reads, the stored
    passthrough the kernel reads (compact [.., n_heavy, bd] in pdt, or the dense layout), heavy mask."""
    nb = D // bd
    cb = synthetic.make_codebook(Hkv, D, bd, seed)
    g = torch.Generator().manual_seed(seed + 1)
    hidx = sorted(torch.randperm(nb, generator=g)[:n_heavy].tolist())
    heavy = [i in hidx for i in range(nb)]
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, nb), generator=g, dtype=torch.uint8)
    v = torch.randn(B, Hkv, T, D, generator=g).to(vdt)
    ptd = torch.zeros(B, Hkv, T, nb, bd)
    if n_heavy:
        ptd[:, :, :, hidx] = torch.randn(B, Hkv, T, n_heavy, bd, generator=g).to(pdt).float()
    stored = ptd.to(pdt) if dense else ptd[:, :, :, hidx].to(pdt).contiguous()
    return cb, q, codes, v, ptd, stored, heavy


def _paginate(codes, v, stored, seq_lens, seed):
    """Scatter contiguous rows into shuffled 16-token pages: code pages [P, Hkv, 16, nb], value pages
    [P, Hkv, Dv, 16] (vLLM's layout), passthrough pages [P, Hkv, 16, slots, bd], block table [B, T/16].
    Slots past a sequence's length hold NaN values and passthrough (never read)."""
    B, Hkv, T, nb = codes.shape
    n = (T + PAGE - 1) // PAGE
    g = torch.Generator().manual_seed(seed)
    table = torch.randperm(B * n, generator=g).view(B, n).to(torch.int32)
    cp = torch.randint(0, 256, (B * n, Hkv, PAGE, nb), generator=g, dtype=torch.uint8)
    vp = torch.full((B * n, Hkv, v.shape[-1], PAGE), float("nan"), dtype=v.dtype)
    pp = None if stored is None else torch.full((B * n,) + (Hkv, PAGE) + tuple(stored.shape[-2:]), float("nan"),
                                                dtype=stored.dtype)
    for b in range(B):
        L = int(seq_lens[b])
        for j in range(n):
            pg = int(table[b, j])
            t0, t1 = j * PAGE, min((j + 1) * PAGE, L)
            if t1 <= t0:
                continue
            cp[pg, :, :t1 - t0] = codes[b, :, t0:t1]
            vp[pg, :, :, :t1 - t0] = v[b, :, t0:t1].transpose(-1, -2)
            if pp is not None:
                pp[pg, :, :t1 - t0] = stored[b, :, t0:t1]
    return cp, vp, pp, table


def _check(out, lse, scores, q, codes, v, cb, scale, heavy, ptd, mask, seq_lens, vdt="bf16"):
    """Oracle per sequence over its own length (the mask sliced to it)."""
    o, l, sc = np_of(out), np_of(lse), np_of(scores)
    hv = np.array(heavy) if any(heavy) else None
    for b in range(q.shape[0]):
        L = int(seq_lens[b])
        m = None if mask is None else mask[b:b + 1, ..., :L].numpy()
        ro, rs, rl = O.decode_attention(q[b:b + 1].float().numpy(), codes[b:b + 1, :, :L].numpy(),
                                        v[b:b + 1, :, :L].float().numpy(), cb.centroids.numpy(), cb.perm.numpy(), scale,
                                        "bf16", vdt, mask=m, heavy=hv,
                                        pt_values=None if hv is None else ptd[b:b + 1, :, :L].numpy(),
                                        return_scores=True)
        assert_rel(o[b:b + 1], ro, BF16_TOL, f"out b={b}")
        fin = np.isfinite(rs)
        assert np.array_equal(np.isfinite(sc[b:b + 1, ..., :L]), fin), f"finite scores b={b}"
        assert_rel(sc[b:b + 1, ..., :L][fin], rs[fin], SCORE_TOL, f"scores b={b}")
        assert_rel(l[b:b + 1], rl, SCORE_TOL, f"lse b={b}")


def _mask(kind, B, Hq, Lq, T, seed):
    if kind is None:
        return None
    g = torch.Generator().manual_seed(seed)
    if kind == "causal":
        pos = torch.arange(T)
        last = T - Lq + torch.arange(Lq)
        return torch.zeros(1, 1, Lq, T).masked_fill(pos[None, :] > last[:, None], float("-inf")).expand(B, Hq, Lq, T)
    m = torch.where(torch.rand(B, Hq, Lq, T, generator=g) < 0.2, float("-inf"), 0.0)
    m[..., 0] = 0.0
    m[0, :2] += -1.5  # a finite bias too
    return m


@pytest.mark.parametrize("B,Hq,Hkv,Lq,D,bd,T,n_heavy,pdt,dense,mask,splits", [
    (2, 32, 8, 1, 128, 4, 1024, 4, torch.bfloat16, False, None, 0),     # config-4 shape, 16 bf16 dims: vector loads
    (2, 32, 8, 1, 128, 4, 512, 4, torch.float32, True, None, 2),        # the reference's dense fp32 layout
    (2, 64, 8, 1, 128, 2, 640, 3, torch.float16, False, None, 0),       # 8 rows over 64 blocks, 6 f16 dims
    (2, 14, 2, 1, 64, 2, 800, 4, torch.bfloat16, False, None, 0),       # Qwen shape at head_dim 64, 8 dims
    (2, 32, 8, 1, 128, 4, 700, 0, torch.bfloat16, False, "random", 0),  # mask only (with a finite bias)
    (1, 16, 4, 3, 128, 4, 400, 0, torch.bfloat16, False, "causal", 1),  # three new tokens, causal
    (2, 32, 8, 1, 128, 4, 600, 2, torch.bfloat16, False, "random", 3),  # mask and passthrough
    (1, 64, 4, 1, 128, 8, 320, 2, torch.float32, True, "random", 0),    # 16 rows, mask and dense fp32 passthrough
])
def test_paged_q4_passthrough_and_masks(B, Hq, Hkv, Lq, D, bd, T, n_heavy, pdt, dense, mask, splits):
    log(f"paged q4 mixed B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} D={D} bd={bd} T={T} heavy={n_heavy} {pdt} dense={dense} "
        f"mask={mask} splits={splits}")
    seed = 400 + T + n_heavy
    cb, q, codes, v, ptd, stored, heavy = _problem(B, Hq, Hkv, Lq, D, bd, T, n_heavy, pdt, dense, seed)
    seq_lens = torch.tensor([T] + [T - 37 * (i + 1) for i in range(B - 1)], dtype=torch.int32)
    cp, vp, pp, table = _paginate(codes, v, stored if n_heavy else None, seq_lens, seed + 2)
    m = _mask(mask, B, Hq, Lq, table.shape[1] * PAGE, seed + 3)  # over the table's whole span
    scale = 1 / math.sqrt(D)
    kw = dict(scale=scale, block_table=table.to(DEV), seq_lens=seq_lens.to(DEV), num_splits=splits,
              heavy=heavy if n_heavy else None, pt=None if pp is None else pp.to(DEV), pt_dense=dense,
              mask=None if m is None else m.to(DEV))
    args = (q.to(DEV), cp.to(DEV), vp.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    out, lse, scores = hip_ops.decode(*args, return_lse=True, return_scores=True, **kw)
    _check(out, lse, scores, q, codes, v, cb, scale, heavy, ptd, m, seq_lens)
    # the automatic choice is the 4x4-MFMA kernel (kernel 4), bit for bit
    assert torch.equal(hip_ops.decode(*args, kernel=4, **kw), out)


@pytest.mark.parametrize("B,Hq,Hkv,Lq,bd,T,n_heavy,pdt,dense,mask,splits", [
    (2, 32, 8, 1, 2, 700, 4, torch.bfloat16, False, None, 0),     # 4 bits/dim, 8 bf16 dims: vector loads
    (2, 32, 8, 1, 4, 555, 1, torch.bfloat16, False, None, 2),     # 4 dims (one heavy block of 4)
    (2, 32, 8, 1, 4, 500, 4, torch.float32, True, None, 0),       # the reference's dense fp32 layout
    (2, 64, 8, 1, 4, 333, 2, torch.float16, False, None, 1),      # 8 rows, 8 f16 dims
    (1, 32, 8, 4, 2, 300, 0, torch.bfloat16, False, "causal", 0),  # a causal chunk of 4 at 4 bits/dim
    (2, 32, 8, 1, 4, 400, 3, torch.bfloat16, False, "random", 2),  # mask and passthrough
])
def test_contiguous_q4_passthrough_and_masks(B, Hq, Hkv, Lq, bd, T, n_heavy, pdt, dense, mask, splits):
    """Contiguous rows at head_dim 128: passthrough layouts the LUT kernel does not take (other than 8
    or 16 consecutive 16-bit values), passthrough at 4 bits/dim, and masks whose LUT would need row
    groups run on the 4x4-MFMA kernel."""
    log(f"contig q4 mixed B={B} Hq={Hq} Lq={Lq} bd={bd} T={T} heavy={n_heavy} {pdt} dense={dense} mask={mask}")
    D = 128
    seed = 500 + T + n_heavy
    cb, q, codes, v, ptd, stored, heavy = _problem(B, Hq, Hkv, Lq, D, bd, T, n_heavy, pdt, dense, seed)
    m = _mask(mask, B, Hq, Lq, T, seed + 3)
    scale = 1 / math.sqrt(D)
    kw = dict(scale=scale, num_splits=splits, heavy=heavy if n_heavy else None,
              pt=stored.to(DEV) if n_heavy else None, pt_dense=dense, mask=None if m is None else m.to(DEV))
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    out, lse, scores = hip_ops.decode(*args, return_lse=True, return_scores=True, kernel=4, **kw)
    _check(out, lse, scores, q, codes, v, cb, scale, heavy, ptd, m, [T] * B)
    assert torch.equal(hip_ops.decode(*args, **kw), out)  # the automatic choice
    # the generic kernel agrees with the oracle too
    og, gl, gs = hip_ops.decode(*args, kernel=1, return_lse=True, return_scores=True, **kw)
    _check(og, gl, gs, q, codes, v, cb, scale, heavy, ptd, m, [T] * B)
