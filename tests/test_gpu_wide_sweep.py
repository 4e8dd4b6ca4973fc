"""A seeded sweep of k_decode_wide, the staged-codebook decode for 16-bit codes over long contexts
(splits of at least 2,048 tokens): random head_dim / block_dim (16 to 64 blocks of dim 2 or 4),
512 to 4,096 codewords per block (per KV head), contiguous rows or pages, value dims 64 or 128 in
bf16 or f16, query heads per KV head (row groups past 4), one or two query tokens, an additive mask,
one or two splits, and the scale.  Output and lse against the oracle's restatement of the
reference's decode (sunshape/vllm_attn_backend.py:216-253); the raw scores against the oracle and,
bit for bit, against the same call split into 256-token pieces, which takes the per-token gathers
of k_decode_generic (same arithmetic, sunshape/triton_kernels.py:174-196)."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
VDT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _draw(seed):
    rng = np.random.default_rng(seed)
    D, bd = [(64, 2), (64, 4), (128, 4), (128, 2)][int(rng.integers(0, 4))]
    nc = int(rng.choice([512, 1024, 4096] if bd == 4 else [512, 1024, 4096, 8192]))
    T = int(rng.integers(2048, 6000))
    return dict(seed=seed, D=D, bd=bd, nc=nc, T=T, B=int(rng.integers(1, 3)), Hkv=int(rng.integers(1, 3)),
                G=int(rng.choice([1, 2, 4, 5, 8])), Lq=int(rng.choice([1, 1, 2])), Dv=int(rng.choice([64, 128])),
                vdt=str(rng.choice(["bf16", "f16"])), paged=bool(rng.integers(0, 2)), mask=bool(rng.integers(0, 2)),
                splits=2 if T >= 4096 and rng.integers(0, 2) else 1,
                scale=str(rng.choice(["inv_sqrt", "other"])))


@pytest.mark.parametrize("seed", list(range(700, 712)))
def test_wide_decode_sweep_vs_oracle(seed):
    c = _draw(seed)
    log(f"wide decode sweep {c}")
    D, bd, nc, T, B, Hkv, G, Lq, Dv = (c[k] for k in ("D", "bd", "nc", "T", "B", "Hkv", "G", "Lq", "Dv"))
    nb, Hq = D // bd, Hkv * G
    rng = np.random.default_rng(seed + 1)
    cb = synthetic.make_codebook(Hkv, D, bd, seed, n_centroids=nc)
    g = torch.Generator().manual_seed(seed + 2)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    idx = torch.from_numpy(rng.integers(0, nc, (B, Hkv, T, nb)))
    v = torch.randn(B, Hkv, T, Dv, generator=g).to(VDT[c["vdt"]])
    m = None
    if c["mask"]:
        m = torch.from_numpy(np.where(rng.random((B, Hq, Lq, T)) < 0.15, -np.inf,
                                      rng.uniform(-1.0, 0.0, (B, Hq, Lq, T))).astype(np.float32))
        m[..., 0] = 0.0
    scale = 1 / math.sqrt(D) if c["scale"] == "inv_sqrt" else 0.3
    codes = idx.to(hip_ops.index_dtype(nc))
    if c["paged"]:
        page = 16
        n = (T + page - 1) // page
        table = torch.randperm(B * n, generator=g).view(B, n).to(torch.int32)
        cp = torch.zeros(B * n, Hkv, page, nb, dtype=codes.dtype)
        vp = torch.zeros(B * n, Hkv, Dv, page, dtype=v.dtype)
        for b in range(B):
            for j in range(n):
                t0, t1 = j * page, min((j + 1) * page, T)
                cp[table[b, j], :, :t1 - t0] = codes[b, :, t0:t1]
                vp[table[b, j], :, :, :t1 - t0] = v[b, :, t0:t1].transpose(-1, -2)
        args = (q.to(DEV), cp.to(DEV), vp.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
        kw = dict(block_table=table.to(DEV), seq_lens=torch.full((B,), T, dtype=torch.int32, device=DEV))
        md = None if m is None else torch.nn.functional.pad(m, (0, n * page - T))  # over the table's capacity
    else:
        args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
        kw = {}
        md = m
    kw.update(scale=scale, mask=None if md is None else md.to(DEV), return_lse=True, return_scores=True)
    out, lse, sc = hip_ops.decode(*args, num_splits=c["splits"], **kw)
    _, _, sc_g = hip_ops.decode(*args, num_splits=(T + 255) // 256, **kw)
    assert torch.equal(sc[..., :T], sc_g[..., :T]), "staged and gathered scores differ"
    ro, rs, rl = O.decode_attention(q.float().numpy(), idx.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                    cb.perm.numpy(), scale, "bf16", c["vdt"], mask=None if m is None else m.numpy(),
                                    return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    got = np_of(sc[..., :T])
    fin = np.isfinite(rs)
    assert np.array_equal(np.isfinite(got), fin)
    assert_rel(got[fin], rs[fin], SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")
