"""Contiguous rows at head_dim 128 (the reference's own layout, codes [B, Hkv, T, nb] and V
[B, Hkv, T, 128]) on the 4x4-MFMA-scores kernel with contiguous tiles: the shapes whose LUT would
need row groups (the reference's default 4 bits/dim at block_dim 2, 8 or more query heads per KV
head), packed codes, and the full-size config-4 layer in contiguous rows, all against the oracle.

The kernel's scores sum in MFMA order, so they agree with the LUT kernels within fp32 rounding
(SCORE_TOL), not bit for bit."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _oracle_units(q, codes, v, cent, perm, scale, units, G, vdt="bf16"):
    """Oracle (out, scores, lse) per (batch, KV head) unit of contiguous rows (numpy inputs)."""
    res = {}
    for b, kv in units:
        ro, rs, rl = O.decode_attention(q[b, kv * G:(kv + 1) * G][None], codes[b, kv][None, None],
                                        v[b, kv][None, None], cent[kv][None], perm[kv][None], scale, "bf16", vdt,
                                        return_scores=True)
        res[(b, kv)] = (ro[0], rs[0], rl[0])
    return res


@pytest.mark.parametrize("B,Hq,Hkv,Lq,bd,T,vdt,splits,strided,nc", [
    (2, 32, 8, 1, 2, 1000, torch.bfloat16, 0, False, 256),   # reference default: 4 bits/dim, 4 rows, 64 blocks
    (2, 64, 8, 1, 4, 777, torch.bfloat16, 2, False, 256),    # 8 query heads per KV head
    (1, 16, 2, 1, 2, 333, torch.float16, 3, False, 256),     # 8 rows over 64 blocks, f16 values
    (2, 128, 8, 1, 4, 300, torch.bfloat16, 0, False, 256),   # 16 rows: four row quads
    (1, 24, 2, 1, 4, 129, torch.bfloat16, 1, False, 256),    # 12 rows: three row quads, a tile + 1
    (2, 32, 8, 1, 2, 700, torch.bfloat16, 2, True, 256),     # [B, T, Hkv, *] buffers viewed as [B, Hkv, T, *]
    (2, 16, 4, 2, 4, 65, torch.bfloat16, 1, False, 256),     # two query tokens: 8 rows
    (1, 8, 2, 1, 2, 1, torch.bfloat16, 0, False, 256),       # one token
    (2, 8, 2, 1, 8, 64, torch.bfloat16, 0, False, 256),      # exactly one tile, 16 blocks of 8
    (1, 64, 2, 3, 4, 515, torch.bfloat16, 0, False, 256),    # 96 rows: six row groups of 16
    (2, 32, 8, 1, 2, 400, torch.bfloat16, 0, False, 100),    # a 100-codeword codebook
])
def test_contiguous_q4_kernel_128_dim(B, Hq, Hkv, Lq, bd, T, vdt, splits, strided, nc):
    log(f"contig q4 D128 B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} bd={bd} T={T} vdt={vdt} splits={splits} "
        f"strided={strided} nc={nc}")
    D = 128
    cb = synthetic.make_codebook(Hkv, D, bd, 300 + bd + T, n_centroids=nc)
    g = torch.Generator().manual_seed(301 + T)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    if strided:
        codes = torch.randint(0, nc, (B, T, Hkv, D // bd), generator=g, dtype=torch.uint8).transpose(1, 2)
        v = torch.randn(B, T, Hkv, D, generator=g).to(vdt).transpose(1, 2)
    else:
        codes = torch.randint(0, nc, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
        v = torch.randn(B, Hkv, T, D, generator=g).to(vdt)
    scale = 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    out, lse, scores = hip_ops.decode(*args, scale=scale, return_lse=True, return_scores=True, kernel=4,
                                      num_splits=splits)
    vname = "bf16" if vdt == torch.bfloat16 else "f16"
    ro, rs, rl = O.decode_attention(q.float().numpy(), codes.contiguous().numpy(), v.float().contiguous().numpy(),
                                    cb.centroids.numpy(), cb.perm.numpy(), scale, "bf16", vname, return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    assert_rel(np_of(scores), rs, SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")
    # asking for the scores changes nothing else
    o2 = hip_ops.decode(*args, scale=scale, kernel=4, num_splits=splits)
    assert torch.equal(o2, out)
    # the generic kernel agrees with the oracle on the same inputs
    og = np_of(hip_ops.decode(*args, scale=scale, kernel=1))
    assert_rel(og, ro, BF16_TOL, "generic kernel")


def _lut_rows(Hq, Hkv, Lq, bd, D=128):
    """Rows per LUT of the contiguous LUT kernel (a 128 KiB LUT, at most 8 rows)."""
    return min(32768 // ((D // bd) * 256), 8, (Hq // Hkv) * Lq)


@pytest.mark.parametrize("Hq,bd,want_q4", [(32, 2, True), (64, 4, True), (32, 4, False), (16, 8, False)])
def test_contiguous_128_dim_routing(Hq, bd, want_q4):
    """The automatic choice: the 4x4-MFMA kernel where the LUT would need row groups, the LUT kernel
    otherwise.  Each choice equals the launch that forces it, bit for bit."""
    log(f"contig D128 routing Hq={Hq} bd={bd}")
    B, Hkv, T, D = 2, 8, 300, 128
    p = synthetic.config4_contiguous(DEV, B=B, T=T, Hq=Hq, Hkv=Hkv, bd=bd)
    args = (p["q"], p["codes"], p["v"], p["perm"], p["centroids"])
    rows = Hq // Hkv
    assert (rows > _lut_rows(Hq, Hkv, 1, bd)) == want_q4
    auto = hip_ops.decode(*args, scale=p.meta["scale"])
    forced = hip_ops.decode(*args, scale=p.meta["scale"], kernel=4)
    lut = hip_ops.decode(*args, scale=p.meta["scale"], kernel=2)
    assert torch.equal(auto, forced if want_q4 else lut)


@pytest.mark.parametrize("bits,nc,bd", [(4, 16, 2), (6, 64, 2), (4, 16, 4)])
def test_contiguous_q4_kernel_packed_codes(bits, nc, bd):
    """4- and 6-bit codes packed in int32 words on contiguous rows: bit-equal to the byte-code launch
    of the same kernel, and within tolerance of the oracle."""
    log(f"contig q4 D128 packed bits={bits} nc={nc} bd={bd}")
    B, Hq, Hkv, T, D = 2, 32, 8, 500, 128
    p = synthetic.config4_contiguous(DEV, B=B, T=T, Hq=Hq, Hkv=Hkv, bd=bd, n_centroids=nc, seed=320 + bits)
    words = hip_ops.pack_codes(p["codes"], bits)
    kw = dict(scale=p.meta["scale"], return_lse=True)
    o8, l8 = hip_ops.decode(p["q"], p["codes"], p["v"], p["perm"], p["centroids"], kernel=4, **kw)
    ow, lw = hip_ops.decode(p["q"], words, p["v"], p["perm"], p["centroids"], code_bits=bits, kernel=4, **kw)
    assert torch.equal(o8, ow) and torch.equal(l8, lw)
    oa = hip_ops.decode(p["q"], words, p["v"], p["perm"], p["centroids"], code_bits=bits, scale=p.meta["scale"])
    assert torch.equal(oa, ow)  # the automatic choice for packed contiguous rows at head_dim 128
    G = Hq // Hkv
    q, c, v = np_of(p["q"]), np_of(p["codes"]), np_of(p["v"])
    ref = _oracle_units(q, c, v, np_of(p["centroids"]), np_of(p["perm"]), p.meta["scale"],
                        [(b, kv) for b in range(B) for kv in range(Hkv)], G)
    o, l = np_of(ow), np_of(lw)
    for (b, kv), (ro, _, rl) in ref.items():
        assert_rel(o[b, kv * G:(kv + 1) * G], ro, BF16_TOL, f"out b={b} kv={kv}")
        assert_rel(l[b, kv * G:(kv + 1) * G], rl, SCORE_TOL, f"lse b={b} kv={kv}")


def _full_size_units_vs_oracle(p, out, lse, scores, units):
    G = p.meta["Hq"] // p.meta["Hkv"]
    q, perm, cent = np_of(p["q"]), np_of(p["perm"]), np_of(p["centroids"])
    by_b = {}
    for b, kv in units:
        by_b.setdefault(b, []).append(kv)
    for b, kvs in sorted(by_b.items()):
        codes_b = np_of(p["codes"][b])  # [Hkv, T, nb]
        v_b = np_of(p["v"][b])          # [Hkv, T, D] fp32
        for kv in kvs:
            ro, rs, rl = O.decode_attention(q[b, kv * G:(kv + 1) * G][None], codes_b[kv][None, None],
                                            v_b[kv][None, None], cent[kv][None], perm[kv][None], p.meta["scale"],
                                            "bf16", "bf16", return_scores=True)
            sl = slice(kv * G, (kv + 1) * G)
            assert_rel(out[b, sl], ro[0], BF16_TOL, f"out b={b} kv={kv}")
            assert_rel(lse[b, sl], rl[0], SCORE_TOL, f"lse b={b} kv={kv}")
            if scores is not None:
                assert_rel(scores[b, sl], rs[0], SCORE_TOL, f"scores b={b} kv={kv}")


@pytest.mark.parametrize("Hq,bd", [(32, 4), (32, 2), (64, 4)])
def test_contiguous_config4_full_size(Hq, bd):
    """The config-4 layer in contiguous rows at full size (64 x 8 x 32768; V spans 2^32 bytes):
    c4ct (4 query heads per KV head, block_dim 4: the LUT kernel), c4ctbd2 (the reference's default
    4 bits/dim) and c4ctg8 (8 query heads per KV head), both on the 4x4-MFMA kernel.  Outputs and
    lse of 64 units (the corners (0, 0) and (63, 7) among them) against the oracle; then the launch
    that also returns the fp32 scores gives the same outputs, and 8 units' scores match."""
    log(f"contiguous config4 full size Hq={Hq} bd={bd}")
    p = synthetic.config4_contiguous(DEV, Hq=Hq, bd=bd)
    assert p["v"].numel() * 2 == 1 << 32
    # one split per (batch, KV head) -- what the planner picks at this size (512 units on 256 CUs) --
    # stated, so that the sub-batch launch below runs the same schedule
    kw = dict(scale=p.meta["scale"], return_lse=True, num_splits=1)
    out, lse = hip_ops.decode(p["q"], p["codes"], p["v"], p["perm"], p["centroids"], **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, hip_ops.decode(p["q"], p["codes"], p["v"], p["perm"], p["centroids"],
                                           scale=p.meta["scale"]))
    o, l = np_of(out), np_of(lse)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    assert (l > math.log(32768) - 5).all()
    rng = np.random.default_rng(40 + bd + Hq)
    units = sorted({(int(rng.integers(64)), int(rng.integers(8))) for _ in range(80)} | {(0, 0), (63, 7)})[:64]
    if (0, 0) not in units:
        units[0] = (0, 0)
    if (63, 7) not in units:
        units[-1] = (63, 7)
    _full_size_units_vs_oracle(p, o, l, None, units)
    log(f"contiguous config4 full size with scores Hq={Hq} bd={bd}")
    # the scores of 8 units, from a launch over those sequences only (the full [64, Hq, 1, 32768]
    # fp32 scores would take 8-16 GiB)
    bs = sorted({b for b, _ in units[:8]} | {0, 63})
    sub = torch.tensor(bs, device=DEV)
    out2, lse2, sc2 = hip_ops.decode(p["q"][sub], p["codes"][sub], p["v"][sub], p["perm"], p["centroids"],
                                     return_scores=True, **kw)
    assert torch.equal(out2, out[sub]) and torch.equal(lse2, lse[sub])
    ps = synthetic.Problem("sub", {k: (p[k][sub] if k in ("q", "codes", "v") else p[k]) for k in p.tensors}, p.meta)
    _full_size_units_vs_oracle(ps, np_of(out2), np_of(lse2), np_of(sc2),
                               [(i, kv) for i, b in enumerate(bs) for kv in (0, 7)])
