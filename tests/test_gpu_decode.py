"""Fused HIP decode vs the oracle: golden fixture, config 3 (contiguous), config 4
(paged, reduced and full size), masks, q_len > 1, value dtypes, split counts,
SunShape-Mixed passthrough, ragged paged sequences."""

import math
import os

import numpy as np
import pytest
import torch

from _util import BF16_TOL, SCORE_TOL, assert_rel, bf16_from_bits, log, np_of, torch_bf16_from_bits
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _oracle_unit(q, codes, v, cent, perm, scale, qdt="bf16", vdt="bf16", mask=None, heavy=None, pt=None):
    """Oracle for one (batch, KV head): q [G, Lq, D], codes [T, nb], v [T, Dv]."""
    out, scores, lse = O.decode_attention(q[None], codes[None, None], v[None, None], cent[None], perm[None], scale,
                                          qdt, vdt, mask=mask, heavy=heavy,
                                          pt_values=None if pt is None else pt[None, None], return_scores=True)
    return out[0], scores[0], lse[0]


def test_decode_golden_fixture():
    log("decode golden fixture")
    f = np.load(os.path.join(GOLD, "decode_small.npz"))
    q = torch_bf16_from_bits(f["q_bf16_bits"], DEV)
    v = torch_bf16_from_bits(f["v_bf16_bits"], DEV)
    codes = torch.from_numpy(f["codes"]).to(DEV)
    out, lse, scores = hip_ops.decode(q, codes, v, torch.from_numpy(f["perm"]).to(DEV),
                                      torch.from_numpy(f["centroids"]).to(DEV), scale=float(f["scale"]),
                                      return_lse=True, return_scores=True)
    assert_rel(np_of(out), bf16_from_bits(f["out_bf16_bits"]), BF16_TOL, "out vs golden")
    assert_rel(np_of(scores), f["scores"], SCORE_TOL, "scores vs golden")


@pytest.mark.parametrize("B,T", [(2, 1500), (16, 8192)])
def test_config3_decode_vs_oracle(B, T):
    log(f"config3 decode B={B} T={T}")
    p = synthetic.config3(DEV, B=B, T=T)
    out, lse, scores = hip_ops.decode(p["q"], p["codes"], p["v"], p["perm"], p["centroids"], scale=p.meta["scale"],
                                      return_lse=True, return_scores=True)
    out, lse, scores = np_of(out), np_of(lse), np_of(scores)
    q, codes, v, perm, cent = (np_of(p[k]) for k in ("q", "codes", "v", "perm", "centroids"))
    G = 7
    units = [(b, kv) for b in range(B) for kv in range(2)]  # every unit, also at full size
    for b, kv in units:
        ro, rs, rl = _oracle_unit(q[b, kv * G:(kv + 1) * G], codes[b, kv], v[b, kv], cent[kv], perm[kv], p.meta["scale"])
        sl = slice(kv * G, (kv + 1) * G)
        assert_rel(out[b, sl], ro, BF16_TOL, f"out b={b} kv={kv}")
        assert_rel(scores[b, sl], rs, SCORE_TOL, f"scores b={b} kv={kv}")
        assert_rel(lse[b, sl], rl, SCORE_TOL, f"lse b={b} kv={kv}")


def test_decode_split_counts_agree():
    log("decode split counts")
    p = synthetic.config3(DEV, B=2, T=4096)
    v32 = p["v"].float()
    outs = [np_of(hip_ops.decode(p["q"], p["codes"], v32, p["perm"], p["centroids"], scale=p.meta["scale"], num_splits=s))
            for s in (1, 3, 16, 40)]
    assert_rel(outs[1], outs[0], 1e-5, "3 vs 1 splits")
    assert_rel(outs[2], outs[0], 1e-5, "16 vs 1 splits")
    assert_rel(outs[3], outs[0], 1e-5, "40 vs 1 splits")  # the merge takes several passes


@pytest.mark.parametrize("vdt", [torch.float16, torch.float32])
def test_decode_value_dtypes_and_fp32_query(vdt):
    log(f"decode v dtype {vdt}")
    p = synthetic.config3(DEV, B=2, T=700)
    q = p["q"].float() if vdt == torch.float32 else p["q"].to(torch.float16)
    v = p["v"].to(vdt)
    out = np_of(hip_ops.decode(q, p["codes"], v, p["perm"], p["centroids"], scale=p.meta["scale"]))
    qn, codes, vn, perm, cent = np_of(q), np_of(p["codes"]), np_of(v), np_of(p["perm"]), np_of(p["centroids"])
    qdt = "f32" if vdt == torch.float32 else "f16"
    vd = "f32" if vdt == torch.float32 else "f16"
    tol = 1e-4 if vdt == torch.float32 else BF16_TOL
    for b in range(2):
        for kv in range(2):
            ro, _, _ = _oracle_unit(qn[b, kv * 7:(kv + 1) * 7], codes[b, kv], vn[b, kv], cent[kv], perm[kv],
                                    p.meta["scale"], qdt, vd)
            assert_rel(out[b, kv * 7:(kv + 1) * 7], ro, tol, f"b={b} kv={kv}")


def test_decode_q_len_2_and_masks_through_backend():
    """SunShapeAttentionImpl.forward with 2-D/3-D/4-D masks and q_len 2 (sunshape/vllm_attn_backend.py:216-253)."""
    from sunshape_amd import vllm_attn_backend as VB
    from sunshape_amd.codec import SunShapeBlockCodec
    from sunshape_amd.hf import SunShapeBundle
    from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState

    log("backend masks q_len 2")
    B, Hq, Hkv, T, Lq, D = 2, 8, 2, 600, 2, 64
    cb = synthetic.make_codebook(1, D, 2, seed=21)
    codec = SunShapeBlockCodec.from_buffers(cb.perm[0], cb.centroids[0], device=DEV)
    bundle = SunShapeBundle("m", [3], 4.0, 2, "profileperm_baseline", 0, 0, 0, {3: codec})
    rs = SunShapeVLLMRuntimeState("p", "m", "sunshape_base", 4.0, 2, [3], bundle, "cuda")
    g = torch.Generator().manual_seed(22)
    keys = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    VB.register_runtime_state(rs)
    try:
        qk = VB.quantize_key_states(3, keys)
    finally:
        VB.clear_registered_runtime()
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    full = torch.where(torch.rand(B, Hq, Lq, T, generator=g) < 0.25, float("-inf"), 0.0)
    full[..., :3] = 0.0
    masks = {"none": None, "2d": full[0, 0], "3d_batch": full[:, 0], "3d_heads": full[0], "4d": full}
    impl = VB.SunShapeAttentionImpl(layer_idx=3, runtime_state=rs)
    codes = np_of(qk.codes)
    qn, vn = np_of(q), np_of(v)
    for name, m in masks.items():
        log(f"backend mask {name}")
        out = np_of(impl.forward(q, qk, v, attn_mask=None if m is None else m.to(DEV), scale=1 / math.sqrt(D)))
        mn = None if m is None else m.numpy()
        ref = O.decode_attention(qn, codes, vn, np_of(codec.centroids), np_of(codec.permutation), 1 / math.sqrt(D),
                                 "bf16", "bf16", mask=mn)
        assert_rel(out, ref, BF16_TOL, f"mask {name}")


def _paged_oracle_check(p, out, lse, scores, units, seq_lens=None):
    """Gather each checked sequence's pages on the device, then run the oracle on the host."""
    q = np_of(p["q"])
    perm, cent = np_of(p["perm"]), np_of(p["centroids"])
    G = p.meta["Hq"] // p.meta["Hkv"]
    T = p.meta["T"]
    for b, kv in units:
        L = T if seq_lens is None else int(seq_lens[b])
        pages = p["block_table"][b].long()
        cp = p["code_pages"][pages][:, kv]                      # [n_pages, page, nb]
        vp = p["v_pages"][pages][:, kv]                         # [n_pages, Dv, page]
        codes = np_of(cp.reshape(-1, cp.shape[-1]))[:L]
        v = np_of(vp.permute(0, 2, 1).reshape(-1, vp.shape[1]))[:L]
        ro, rs, rl = _oracle_unit(q[b, kv * G:(kv + 1) * G], codes, v, cent[kv], perm[kv], p.meta["scale"])
        sl = slice(kv * G, (kv + 1) * G)
        assert_rel(out[b, sl], ro, BF16_TOL, f"paged out b={b} kv={kv}")
        if lse is not None:
            assert_rel(lse[b, sl], rl, SCORE_TOL, f"paged lse b={b} kv={kv}")
        if scores is not None:
            assert_rel(scores[b, sl, :, :L], rs, SCORE_TOL, f"paged scores b={b} kv={kv}")


@pytest.mark.parametrize("kernel", [1, 0])
def test_config4_paged_small_vs_oracle(kernel):
    log(f"config4 paged small kernel={kernel}")
    p = synthetic.config4(DEV, B=3, T=2048)
    out, lse, scores = hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"],
                                      scale=p.meta["scale"], block_table=p["block_table"], seq_lens=p["seq_lens"],
                                      return_lse=True, return_scores=True, kernel=kernel)
    _paged_oracle_check(p, np_of(out), np_of(lse), np_of(scores), [(b, kv) for b in range(3) for kv in range(8)])


@pytest.mark.parametrize("Hq,bd,lq,D", [(64, 4, 1, 128), (128, 4, 1, 128), (32, 2, 1, 128), (64, 8, 2, 128),
                                        (32, 2, 2, 128), (128, 4, 2, 128), (64, 2, 1, 64), (64, 8, 1, 256)])
def test_paged_mfma_row_groups_vs_oracle(Hq, bd, lq, D):
    """More query rows per KV head than one LUT holds (8 or 16 heads at 32 blocks, 64 blocks of
    dim 2 at head_dim 128, two query tokens): head_dim 64 and 128 take the 4x4-MFMA-scores kernel
    (16 rows per pass, row groups beyond), head_dim 256 the LUT kernel in row groups.  Outputs, lse
    and raw scores against the oracle, per (sequence, KV head)."""
    log(f"paged MFMA row groups Hq={Hq} bd={bd} q_len={lq} D={D}")
    p = synthetic.config4(DEV, B=2, T=1024 if D <= 128 else 256, Hq=Hq, bd=bd, D=D)
    if lq > 1:
        g = torch.Generator().manual_seed(9)
        p.tensors["q"] = torch.randn(2, Hq, lq, D, generator=g).to(torch.bfloat16).to(DEV)
    out, lse, scores = hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"],
                                      scale=p.meta["scale"], block_table=p["block_table"], seq_lens=p["seq_lens"],
                                      return_lse=True, return_scores=True, kernel=2)
    o, l, sc = np_of(out), np_of(lse), np_of(scores)
    if lq == 1:
        _paged_oracle_check(p, o, l, sc, [(b, kv) for b in range(2) for kv in (0, 3, 7)])
        return
    # two query tokens: each is its own row of the kernel's group; check token by token
    for qi in range(lq):
        pq = synthetic.Problem(p.name, dict(p.tensors), dict(p.meta))
        pq.tensors["q"] = p["q"][:, :, qi:qi + 1]
        _paged_oracle_check(pq, o[:, :, qi:qi + 1], l[:, :, qi:qi + 1], sc[:, :, qi:qi + 1],
                            [(b, kv) for b in range(2) for kv in (1, 6)])


def test_paged_lut_256_dim_values_several_tiles_per_wave():
    """head_dim-256 values on the paged LUT kernel keep one register set per wave (two would not fit
    the registers); a context of 2,000 tokens gives each wave several tiles in one split."""
    log("paged LUT D256 several tiles per wave")
    p = synthetic.config4(DEV, B=2, T=2048, Hq=8, bd=8, D=256)
    lens = torch.tensor([2000, 1333], dtype=torch.int32, device=DEV)
    out, lse, scores = hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"],
                                      scale=p.meta["scale"], block_table=p["block_table"], seq_lens=lens,
                                      return_lse=True, return_scores=True, kernel=2, num_splits=1)
    _paged_oracle_check(p, np_of(out), np_of(lse), np_of(scores), [(0, 0), (1, 5), (0, 7)], seq_lens=np_of(lens))


def test_paged_ragged_sequence_lengths():
    log("paged ragged seq_lens")
    p = synthetic.config4(DEV, B=4, T=1024)
    lens = torch.tensor([1024, 1, 517, 16 * 7 + 3], dtype=torch.int32, device=DEV)
    out, lse = hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"], scale=p.meta["scale"],
                              block_table=p["block_table"], seq_lens=lens, return_lse=True)
    _paged_oracle_check(p, np_of(out), np_of(lse), None, [(b, kv) for b in range(4) for kv in (0, 5)],
                        seq_lens=np_of(lens))


def _paged_units_vs_oracle(p, out, lse, scores, units):
    """Oracle check of paged-decode units, gathering each sequence's pages once for all its KV heads."""
    bt = np_of(p["block_table"])
    cp, vp = p["code_pages"], p["v_pages"]
    G = p.meta["Hq"] // p.meta["Hkv"]
    q, perm, cent = np_of(p["q"]), np_of(p["perm"]), np_of(p["centroids"])
    T = p.meta["T"]
    by_b = {}
    for b, kv in units:
        by_b.setdefault(b, []).append(kv)
    for b, kvs in sorted(by_b.items()):
        pages = torch.from_numpy(bt[b].astype(np.int64)).to(DEV)
        codes = np_of(cp[pages].transpose(0, 1).reshape(cp.shape[1], -1, cp.shape[3]))      # [Hkv, T, nb]
        vals = np_of(vp[pages].permute(1, 0, 3, 2).reshape(vp.shape[1], -1, vp.shape[2]))   # [Hkv, T, Dv]
        for kv in kvs:
            ro, rs, rl = _oracle_unit(q[b, kv * G:(kv + 1) * G], codes[kv, :T], vals[kv, :T], cent[kv], perm[kv],
                                      p.meta["scale"])
            sl = slice(kv * G, (kv + 1) * G)
            assert_rel(out[b, sl], ro, BF16_TOL, f"c4 out b={b} kv={kv}")
            assert_rel(lse[b, sl], rl, SCORE_TOL, f"c4 lse b={b} kv={kv}")
            if scores is not None:
                assert_rel(scores[b, sl], rs, SCORE_TOL, f"c4 scores b={b} kv={kv}")


def test_config4_full_size_units():
    """Config 4 at full size (64 x 8 x 32768, paged): every one of the 512 (batch, KV head) units'
    output and lse against the oracle, then the launch that also returns the fp32 scores (config 4
    lists them as an output), with 128 units' scores, outputs and lse against the oracle."""
    log("config4 full size")
    p = synthetic.config4(DEV)
    kw = dict(scale=p.meta["scale"], block_table=p["block_table"], seq_lens=p["seq_lens"], return_lse=True)
    out, lse = hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"], **kw)
    torch.cuda.synchronize()
    o, l = np_of(out), np_of(lse)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    # softmax over 32768 N(0,1)-valued keys: lse >= max score >= log-uniform floor
    assert (l > math.log(32768) - 5).all()
    rng = np.random.default_rng(0)
    _paged_units_vs_oracle(p, o, l, None, [(b, kv) for b in range(64) for kv in range(8)])
    log("config4 full size with scores")
    out2, lse2, sc2 = hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"],
                                     return_scores=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out2, out) and torch.equal(lse2, lse)  # asking for scores changes nothing else
    units = sorted({(int(rng.integers(64)), int(rng.integers(8))) for _ in range(200)} | {(0, 0), (63, 7)})[:128]
    _paged_units_vs_oracle(p, o, l, np_of(sc2), units)

def test_config4_layer_3bit_packed_full_size():
    """The config-4 layer at 3 bits/dim (64 codewords, bd 2) at full size: 6-bit words and byte
    codes give the same output bit for bit (64-codeword LUT kernel), and sampled units match the
    oracle."""
    log("config4 3-bit packed full size")
    p = synthetic.config4(DEV, bd=2, n_centroids=64)
    kw = dict(scale=p.meta["scale"], block_table=p["block_table"], seq_lens=p["seq_lens"], return_lse=True)
    out8, lse8 = hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"], **kw)
    words = hip_ops.pack_codes(p["code_pages"], 6)
    out6, lse6 = hip_ops.decode(p["q"], words, p["v_pages"], p["perm"], p["centroids"], code_bits=6, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out8, out6) and torch.equal(lse8, lse6)
    del words
    rng = np.random.default_rng(3)
    units = [(int(rng.integers(64)), int(rng.integers(8))) for _ in range(3)] + [(63, 7)]
    _paged_oracle_check(p, np_of(out6), np_of(lse6), None, units)


@pytest.mark.parametrize("B,S", [(2, 1200), (16, 16384)])
def test_mixed_passthrough_decode_config5_shape(B, S):
    """SunShape-Mixed: encode the config-5 keys (28 VQ blocks + 4 bf16 passthrough), then decode
    over the mixed cache; every (batch, KV head) unit's outputs and scores against the oracle, at a
    small size and at config 5's full 16 x 2 x 16384.  Codes: every row against the oracle at the
    small size; at full size 2000 sampled rows per unit (test_config5_full_encode checks every row
    of the same keys across the three encode kernels), and the oracle decodes the cache the GPU
    wrote (dense passthrough rebuilt from the compact one)."""
    log(f"mixed passthrough decode B={B} S={S}")
    p = synthetic.config5(DEV, B=B, S=S)
    heavy = p["heavy"].tolist()
    keys = p["keys"]
    codes, pt = hip_ops.encode(keys, p["perm"], p["centroids"], heavy=heavy)  # compact bf16 passthrough
    out, scores = hip_ops.decode(p["q"], codes, p["v"], p["perm"], p["centroids"], scale=p.meta["scale"],
                                 heavy=heavy, pt=pt, pt_dense=False, return_scores=True)
    qn, vn, kn = np_of(p["q"]), np_of(p["v"]), np_of(keys)
    perm, cent, hv = np_of(p["perm"]), np_of(p["centroids"]), np.array(heavy)
    o, s = np_of(out), np_of(scores)
    cn, ptn = np_of(codes), np_of(pt)
    rng = np.random.default_rng(5)
    for b in range(B):
        for kv in range(2):
            if S <= 4096:
                rc, rpt = O.encode(kn[b, kv], perm, cent[kv], hv)
                assert np.array_equal(cn[b, kv], rc)
            else:
                rows = rng.choice(S, 2000, replace=False)
                rc_s, rpt_s = O.encode(kn[b, kv, rows], perm, cent[kv], hv)
                assert np.array_equal(cn[b, kv, rows], rc_s)
                assert np.array_equal(ptn[b, kv, rows], rpt_s[:, hv])
                rc = cn[b, kv]
                rpt = np.zeros((S, len(heavy), 2), np.float32)
                rpt[:, hv] = ptn[b, kv]
            ro, rs, _ = _oracle_unit(qn[b, kv * 7:(kv + 1) * 7], rc, vn[b, kv], cent[kv], perm, p.meta["scale"],
                                     heavy=hv, pt=rpt)
            assert_rel(o[b, kv * 7:(kv + 1) * 7], ro, BF16_TOL, f"mixed out b={b} kv={kv}")
            assert_rel(s[b, kv * 7:(kv + 1) * 7], rs, SCORE_TOL, f"mixed scores b={b} kv={kv}")


# ---------------------------------------------------------------------------
# contiguous-layout MFMA kernel (kernel 3): every block_dim, value width and dtype, with mask,
# lse, raw scores and split counts; its scores sum in MFMA order, so they agree with the LUT
# kernels within fp32 rounding (SCORE_TOL), not bit for bit
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("bd,Dv,vdt", [(1, 64, torch.bfloat16), (2, 64, torch.bfloat16), (4, 128, torch.bfloat16),
                                       (8, 64, torch.float16), (2, 128, torch.float16)])
def test_contiguous_mfma_kernel_vs_oracle(bd, Dv, vdt):
    log(f"contig mfma bd={bd} Dv={Dv} vdt={vdt}")
    B, Hkv, Hq, T, D = 2, 2, 14, 777, 64
    cb = synthetic.make_codebook(Hkv, D, bd, 70 + bd)
    g = torch.Generator().manual_seed(71 + bd)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    v = torch.randn(B, Hkv, T, Dv, generator=g).to(vdt)
    mask = torch.zeros(B, Hq, 1, T)
    mask[0, :, :, :37] = float("-inf")
    mask[1, 3:9, :, 500:] = -2.5
    scale = 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    out, lse, scores = hip_ops.decode(*args, scale=scale, mask=mask.to(DEV), return_lse=True, return_scores=True,
                                      kernel=3)
    vname = "bf16" if vdt == torch.bfloat16 else "f16"
    ro, rs, rl = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                    cb.perm.numpy(), scale, "bf16", vname, mask=mask.numpy(), return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    fin = np.isfinite(rs)
    assert np.array_equal(np.isfinite(np_of(scores)), fin)
    assert_rel(np_of(scores)[fin], rs[fin], SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")
    # split counts agree, and the LUT kernel agrees within rounding
    o1 = np_of(hip_ops.decode(*args, scale=scale, mask=mask.to(DEV), kernel=3, num_splits=1))
    o5 = np_of(hip_ops.decode(*args, scale=scale, mask=mask.to(DEV), kernel=3, num_splits=5))
    assert_rel(o5, o1, 1e-2, "5 vs 1 splits")
    og = np_of(hip_ops.decode(*args, scale=scale, mask=mask.to(DEV), kernel=1))
    assert_rel(np_of(out), og, BF16_TOL, "vs LUT kernel")


@pytest.mark.parametrize("bd,n_heavy,dense,pdt", [(1, 13, False, torch.bfloat16), (2, 4, False, torch.bfloat16),
                                                  (4, 3, True, torch.float32), (8, 2, False, torch.float16)])
def test_contiguous_mfma_kernel_mixed_passthrough(bd, n_heavy, dense, pdt):
    """Passthrough (SunShape-Mixed) blocks on kernel 3: their score terms come from the stored
    values (dense or compact slots, any pt dtype), the codebook supplies the rest."""
    log(f"contig mfma mixed bd={bd} n_heavy={n_heavy} dense={dense} pdt={pdt}")
    B, Hkv, Hq, T, D = 2, 2, 14, 555, 64
    nb = D // bd
    cb = synthetic.make_codebook(Hkv, D, bd, 90 + bd)
    g = torch.Generator().manual_seed(91 + bd)
    hidx = sorted(torch.randperm(nb, generator=g)[:n_heavy].tolist())
    heavy = [i in hidx for i in range(nb)]
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, nb), generator=g, dtype=torch.uint8)
    v = torch.randn(B, Hkv, T, 64, generator=g).to(torch.bfloat16)
    ptd = torch.zeros(B, Hkv, T, nb, bd)
    ptd[:, :, :, hidx] = torch.randn(B, Hkv, T, n_heavy, bd, generator=g)
    ptd = ptd.to(pdt)
    pt = ptd if dense else ptd[:, :, :, hidx].contiguous()
    mask = torch.zeros(B, Hq, 1, T)
    mask[1, :, :, 400:] = float("-inf")
    scale = 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    kw = dict(scale=scale, mask=mask.to(DEV), heavy=heavy, pt=pt.to(DEV), pt_dense=dense)
    out, lse, scores = hip_ops.decode(*args, **kw, return_lse=True, return_scores=True, kernel=3)
    ro, rs, rl = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                    cb.perm.numpy(), scale, "bf16", "bf16", mask=mask.numpy(), heavy=np.array(heavy),
                                    pt_values=ptd.float().numpy(), return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    fin = np.isfinite(rs)
    assert np.array_equal(np.isfinite(np_of(scores)), fin)
    assert_rel(np_of(scores)[fin], rs[fin], SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")
    og = np_of(hip_ops.decode(*args, **kw, kernel=1))
    assert_rel(np_of(out), og, BF16_TOL, "vs LUT kernel")


@pytest.mark.parametrize("T,splits", [(1, 0), (37, 0), (64, 1), (65, 1), (300, 1), (300, 3), (511, 7), (1333, 2)])
def test_contiguous_mfma_kernel_edge_lengths(T, splits):
    """Contexts shorter than a tile, tile boundaries, and split counts that leave each wave an
    odd number of tiles (the kernel's loop then runs one step past the last tile), with q_len 2
    and a mask; the LUT kernel on the same inputs (masked) must agree too."""
    log(f"contig edge T={T} splits={splits}")
    B, Hkv, Hq, Lq, D, bd = 2, 2, 14, 2, 64, 2
    cb = synthetic.make_codebook(Hkv, D, bd, 100 + T)
    g = torch.Generator().manual_seed(101 + T)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    v = torch.randn(B, Hkv, T, 64, generator=g).to(torch.bfloat16)
    mask = torch.where(torch.rand(B, Hq, Lq, T, generator=g) < 0.2, float("-inf"), 0.0)
    mask[..., 0] = 0.0  # every row keeps a key
    scale = 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    for m in (None, mask):
        md = None if m is None else m.to(DEV)
        out, lse = hip_ops.decode(*args, scale=scale, mask=md, return_lse=True, kernel=3, num_splits=splits)
        ro, _, rl = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                       cb.perm.numpy(), scale, "bf16", "bf16", mask=None if m is None else m.numpy(),
                                       return_scores=True)
        assert_rel(np_of(out), ro, BF16_TOL, f"out mask={m is not None}")
        assert_rel(np_of(lse), rl, SCORE_TOL, f"lse mask={m is not None}")
        og = np_of(hip_ops.decode(*args, scale=scale, mask=md, kernel=1))
        assert_rel(og, ro, BF16_TOL, f"LUT kernel mask={m is not None}")


@pytest.mark.parametrize("pattern,splits", [("rising", 1), ("falling", 1), ("step", 1), ("step", 3), ("wide", 1),
                                            ("wide", 0)])
def test_contiguous_running_max_patterns(pattern, splits):
    """The contiguous kernel's running maximum may lag the true one by a slack and is raised only
    when a score exceeds it by more.  Scores that rise across the context (raised again and
    again), fall (set by the first tiles), jump by 40 halfway, or spread wide (scale 3, no mask)
    must all match the oracle."""
    log(f"contig running max {pattern} splits={splits}")
    B, Hkv, Hq, Lq, D, bd, T = 2, 2, 8, 1, 64, 2, 3000
    cb = synthetic.make_codebook(Hkv, D, bd, 131)
    g = torch.Generator().manual_seed(132)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    v = torch.randn(B, Hkv, T, 64, generator=g).to(torch.bfloat16)
    t = torch.arange(T, dtype=torch.float32)
    bias = {"rising": 0.03 * t, "falling": -0.03 * t, "step": torch.where(t >= T // 2, 40.0, 0.0),
            "wide": None}[pattern]
    mask = None if bias is None else bias.expand(B, Hq, Lq, T).contiguous()
    scale = 3.0 if pattern == "wide" else 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    out, lse = hip_ops.decode(*args, scale=scale, mask=None if mask is None else mask.to(DEV), return_lse=True,
                              kernel=3, num_splits=splits)
    ro, _, rl = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                   cb.perm.numpy(), scale, "bf16", "bf16", mask=None if mask is None else mask.numpy(),
                                   return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, f"out {pattern}")
    assert_rel(np_of(lse), rl, SCORE_TOL, f"lse {pattern}")


# contiguous rows past head_dim 64 (128-dim values) on the LUT kernel, kernel 2: V tiles pass
# through a per-wave LDS buffer 16 tokens at a time and come back transposed for the matrix cores
@pytest.mark.parametrize("B,Hq,Hkv,Lq,bd,T,vdt,splits,strided", [
    (2, 32, 8, 1, 4, 777, torch.bfloat16, 0, False),   # Llama-shaped: 4 rows, 32 blocks
    (2, 32, 8, 1, 4, 700, torch.bfloat16, 2, True),    # [B, T, Hkv, *] buffers viewed as [B, Hkv, T, *]
    (2, 32, 8, 1, 2, 1000, torch.bfloat16, 3, False),  # 64 blocks: two row groups of 2
    (1, 16, 2, 1, 8, 333, torch.float16, 0, False),    # 8 rows, 16 blocks
    (2, 8, 8, 1, 4, 64, torch.bfloat16, 1, False),     # one row, exactly one tile
    (2, 16, 4, 2, 4, 65, torch.bfloat16, 1, False),    # two query tokens: two row groups of 4; a tile + 1
    (1, 12, 4, 1, 16, 1, torch.bfloat16, 0, False),    # 8 blocks of 16 dims (3 rows), one token
])
def test_contiguous_lut_kernel_128_dim(B, Hq, Hkv, Lq, bd, T, vdt, splits, strided):
    log(f"contig LUT D128 B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} bd={bd} T={T} vdt={vdt} splits={splits} strided={strided}")
    D = 128
    cb = synthetic.make_codebook(Hkv, D, bd, 150 + bd + T)
    g = torch.Generator().manual_seed(151 + T)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    if strided:
        codes = torch.randint(0, 256, (B, T, Hkv, D // bd), generator=g, dtype=torch.uint8).transpose(1, 2)
        v = torch.randn(B, T, Hkv, D, generator=g).to(vdt).transpose(1, 2)
    else:
        codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
        v = torch.randn(B, Hkv, T, D, generator=g).to(vdt)
    scale = 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    if strided:
        assert args[1].stride(2) == Hkv * (D // bd) and args[2].stride(2) == Hkv * D
    out, lse, scores = hip_ops.decode(*args, scale=scale, return_lse=True, return_scores=True, kernel=2,
                                      num_splits=splits)
    vname = "bf16" if vdt == torch.bfloat16 else "f16"
    ro, rs, rl = O.decode_attention(q.float().numpy(), codes.contiguous().numpy(), v.float().contiguous().numpy(),
                                    cb.centroids.numpy(), cb.perm.numpy(), scale, "bf16", vname, return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    assert_rel(np_of(scores), rs, SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")
    # the automatic choice is this kernel (bit-identical), and the generic kernel agrees
    oa = np_of(hip_ops.decode(*args, scale=scale, num_splits=splits))
    assert np.array_equal(oa, np_of(out))
    if not strided:  # codes as 8-bit int32 words: the byte rows, the same result bit for bit
        w8 = hip_ops.pack_codes(args[1], 8)
        o8 = np_of(hip_ops.decode(args[0], w8, *args[2:], scale=scale, code_bits=8, kernel=2, num_splits=splits))
        assert np.array_equal(o8, np_of(out))
    og = np_of(hip_ops.decode(*args, scale=scale, kernel=1))
    assert_rel(og, ro, BF16_TOL, "generic kernel")


@pytest.mark.parametrize("B,Hq,Hkv,Lq,bd,T,kind,splits", [
    (2, 32, 8, 1, 4, 777, "rows", 0),      # per-(batch, head) padding and a finite bias
    (2, 16, 4, 3, 4, 500, "causal", 1),    # three new tokens, HF's causal mask broadcast over batch and heads
    (1, 32, 8, 2, 2, 300, "causal", 2),    # 64 blocks: row groups of 2, causal over two tokens
    (2, 8, 8, 1, 8, 129, "random-f16", 0),  # one row, 16 blocks, a fifth of the keys masked, f16 values
    (1, 8, 2, 64, 4, 300, "causal", 0),    # a 64-token causal chunk: 256 rows, 64 row groups of 4
])
def test_contiguous_lut_kernel_128_dim_masks(B, Hq, Hkv, Lq, bd, T, kind, splits):
    """Additive masks on the contiguous 128-dim LUT kernel: read with each tile's codes, added to
    the scores before the softmax (and in the returned scores)."""
    log(f"contig LUT D128 mask B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} bd={bd} T={T} kind={kind} splits={splits}")
    D = 128
    cb = synthetic.make_codebook(Hkv, D, bd, 170 + T)
    g = torch.Generator().manual_seed(171 + T)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    vdt = torch.float16 if kind.endswith("f16") else torch.bfloat16
    v = torch.randn(B, Hkv, T, D, generator=g).to(vdt)
    if kind == "rows":
        mask = torch.zeros(B, Hq, Lq, T)
        mask[0, :, :, :37] = float("-inf")
        mask[1, 3:9, :, 500:] = -2.5
    elif kind == "causal":
        pos = torch.arange(T)
        last = T - Lq + torch.arange(Lq)
        mask = torch.zeros(1, 1, Lq, T).masked_fill(pos[None, :] > last[:, None], float("-inf"))
    else:
        mask = torch.where(torch.rand(B, Hq, Lq, T, generator=g) < 0.2, float("-inf"), 0.0)
        mask[..., 0] = 0.0  # every row keeps a key
    full = mask.expand(B, Hq, Lq, T).contiguous()
    scale = 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    md = mask.to(DEV)
    out, lse, scores = hip_ops.decode(*args, scale=scale, mask=md, return_lse=True, return_scores=True, kernel=2,
                                      num_splits=splits)
    ro, rs, rl = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                    cb.perm.numpy(), scale, "bf16", "f16" if vdt == torch.float16 else "bf16",
                                    mask=full.numpy(), return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    fin = np.isfinite(rs)
    assert np.array_equal(np.isfinite(np_of(scores)), fin)
    assert_rel(np_of(scores)[fin], rs[fin], SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")
    oa = np_of(hip_ops.decode(*args, scale=scale, mask=md, num_splits=splits))
    assert np.array_equal(oa, np_of(out))


@pytest.mark.parametrize("B,Hq,Hkv,Lq,bd,T,splits", [
    (2, 32, 8, 1, 4, 1000, 0),  # 4 rows, 32 blocks
    (1, 16, 2, 2, 2, 333, 3),   # 16 rows over 64 blocks: 8 row groups of 2
    (2, 12, 4, 1, 8, 64, 1),    # 3 rows, 16 blocks, one tile
    (1, 8, 8, 1, 16, 1, 0),     # one row, 8 blocks of 16 dims, one token
])
def test_contiguous_lut_kernel_128_dim_scores_only(B, Hq, Hkv, Lq, bd, T, splits):
    """Scores only (gqa_scores) on contiguous rows at head_dim 128: the LUT kernel without values
    stores every tile's scores; the automatic choice is this kernel."""
    log(f"contig LUT D128 scores B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} bd={bd} T={T} splits={splits}")
    D, scale = 128, 0.088
    cb = synthetic.make_codebook(Hkv, D, bd, 190 + T)
    g = torch.Generator().manual_seed(191 + T)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    args = (q.to(DEV), codes.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    s2 = np_of(hip_ops.gqa_scores(*args, scale=scale, kernel=2, num_splits=splits))
    s0 = np_of(hip_ops.gqa_scores(*args, scale=scale, num_splits=splits))
    assert np.array_equal(s0, s2)
    G = Hq // Hkv
    for b in range(B):
        for kv in range(Hkv):
            qs = O.query_scale(q[b, kv * G:(kv + 1) * G].reshape(-1, D).float().numpy(), scale, "bf16")
            ref = O.attention_scores(qs, codes[b, kv].numpy(), cb.centroids[kv].numpy(), cb.perm[kv].numpy())
            assert_rel(s2[b, kv * G:(kv + 1) * G].reshape(-1, T), ref, SCORE_TOL, f"b={b} kv={kv}")


@pytest.mark.parametrize("bd,n_heavy,dense,pdt,vdt,ct", [(4, 4, False, torch.bfloat16, torch.bfloat16, True),
                                                         (4, 2, False, torch.bfloat16, torch.bfloat16, True),
                                                         (8, 2, False, torch.float16, torch.float16, True),
                                                         (2, 8, True, torch.float32, torch.bfloat16, False),
                                                         (4, 1, True, torch.bfloat16, torch.bfloat16, False)])
def test_contiguous_lut_kernel_128_dim_passthrough(bd, n_heavy, dense, pdt, vdt, ct):
    """SunShape-Mixed passthrough blocks on the contiguous 128-dim LUT kernel (ct, kernel 2): 8 or 16
    consecutive 16-bit stored values per token; the heavy blocks' LUT rows are zero and their
    scores come from the stored values.  Other passthrough layouts (fp32, dense slots of blocks that
    are not adjacent, 4 dims) take the 4x4-MFMA kernel, as does the automatic choice; all match the
    oracle."""
    log(f"contig LUT D128 passthrough bd={bd} n_heavy={n_heavy} dense={dense} pdt={pdt} vdt={vdt}")
    B, Hkv, Hq, T, D = 2, 8, 32, 555, 128
    nb = D // bd
    cb = synthetic.make_codebook(Hkv, D, bd, 210 + bd + n_heavy)
    g = torch.Generator().manual_seed(211 + bd)
    hidx = sorted(torch.randperm(nb, generator=g)[:n_heavy].tolist())
    heavy = [i in hidx for i in range(nb)]
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, nb), generator=g, dtype=torch.uint8)
    v = torch.randn(B, Hkv, T, D, generator=g).to(vdt)
    ptd = torch.zeros(B, Hkv, T, nb, bd)
    ptd[:, :, :, hidx] = torch.randn(B, Hkv, T, n_heavy, bd, generator=g)
    ptd = ptd.to(pdt)
    pt = ptd if dense else ptd[:, :, :, hidx].contiguous()
    scale = 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    kw = dict(scale=scale, heavy=heavy, pt=pt.to(DEV), pt_dense=dense)
    out, lse, scores = hip_ops.decode(*args, **kw, return_lse=True, return_scores=True, kernel=2 if ct else 0)
    ro, rs, rl = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                    cb.perm.numpy(), scale, "bf16", "f16" if vdt == torch.float16 else "bf16",
                                    heavy=np.array(heavy), pt_values=ptd.float().numpy(), return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    assert_rel(np_of(scores), rs, SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")
    # the automatic choice: the 4x4-MFMA kernel, which takes contiguous passthrough at head_dim 128
    oa = hip_ops.decode(*args, **kw)
    assert torch.equal(oa, hip_ops.decode(*args, **kw, kernel=4))
    assert_rel(np_of(oa), ro, BF16_TOL, "out, automatic choice")


def test_contiguous_mfma_kernel_rejects_wide_passthrough():
    """More than 16 passthrough dims do not fit the kernel's passthrough pass: an explicit
    kernel 3 request is refused, and auto dispatch serves the call on the LUT kernel."""
    log("contig mfma wide passthrough")
    B, Hkv, Hq, T, D, bd = 1, 2, 8, 130, 64, 4
    cb = synthetic.make_codebook(Hkv, D, bd, 95)
    g = torch.Generator().manual_seed(96)
    heavy = [i in (0, 3, 5, 9, 12) for i in range(D // bd)]  # 20 passthrough dims
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8).to(DEV)
    v = torch.randn(B, Hkv, T, 64, generator=g).to(torch.bfloat16).to(DEV)
    pt = torch.randn(B, Hkv, T, sum(heavy), bd, generator=g).to(torch.bfloat16).to(DEV)
    args = (q, codes, v, cb.perm.to(DEV), cb.centroids.to(DEV))
    with pytest.raises(RuntimeError):
        hip_ops.decode(*args, scale=0.125, heavy=heavy, pt=pt, kernel=3)
    oa = hip_ops.decode(*args, scale=0.125, heavy=heavy, pt=pt)
    o1 = hip_ops.decode(*args, scale=0.125, heavy=heavy, pt=pt, kernel=1)
    assert torch.equal(oa, o1)


@pytest.mark.parametrize("bd", [2, 8])
def test_contiguous_mfma_scores_only_vs_oracle(bd):
    log(f"contig mfma scores bd={bd}")
    B, Hkv, Hq, T, D = 2, 2, 14, 1000, 64
    cb = synthetic.make_codebook(Hkv, D, bd, 80 + bd)
    g = torch.Generator().manual_seed(81 + bd)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    s3 = np_of(hip_ops.gqa_scores(q.to(DEV), codes.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV), scale=0.125,
                                  kernel=3))
    s1 = np_of(hip_ops.gqa_scores(q.to(DEV), codes.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV), scale=0.125,
                                  kernel=1))
    assert_rel(s3, s1, SCORE_TOL, "MFMA vs LUT scores")
    G = Hq // Hkv
    for b in range(B):
        for kv in range(Hkv):
            qs = O.query_scale(q[b, kv * G:(kv + 1) * G, 0].float().numpy(), 0.125, "bf16")
            ref = O.attention_scores(qs, codes[b, kv].numpy(), cb.centroids[kv].numpy(), cb.perm[kv].numpy())
            assert_rel(s3[b, kv * G:(kv + 1) * G, 0], ref, SCORE_TOL, f"b={b} kv={kv}")


@pytest.mark.parametrize("G,bd,D,Dv,nc,vdt,splits", [
    (1, 4, 128, 128, 256, torch.bfloat16, 0), (3, 2, 128, 128, 256, torch.bfloat16, 0),
    (4, 2, 128, 128, 256, torch.float16, 3), (5, 1, 64, 64, 256, torch.bfloat16, 0),
    (8, 4, 128, 128, 16, torch.bfloat16, 0), (13, 8, 64, 64, 64, torch.bfloat16, 2),
    (16, 2, 64, 64, 256, torch.float16, 0), (4, 8, 128, 64, 256, torch.bfloat16, 0)])
def test_paged_q4_kernel_vs_oracle(G, bd, D, Dv, nc, vdt, splits):
    """The 4x4-MFMA-scores paged kernel (kernel 4) over its shape range: 1 to 16 query rows per KV
    head (1 to 4 row quads), block_dim 1/2/4/8, head_dim 64/128, value_dim 64/128, 16/64/256
    codewords, fp16 values, forced splits, ragged sequence lengths; outputs, lse and raw scores
    against the oracle."""
    log(f"paged q4 G={G} bd={bd} D={D} Dv={Dv} nc={nc} vdt={vdt} splits={splits}")
    B, Hkv, T, page = 3, 2, 1024, 16
    cb = synthetic.make_codebook(Hkv, D, bd, 70 + G + bd, n_centroids=nc)
    g = torch.Generator().manual_seed(71 + G)
    q = torch.randn(B, G * Hkv, 1, D, generator=g).to(torch.bfloat16)
    P = B * T // page
    table = torch.randperm(P, generator=g).to(torch.int32).view(B, T // page)
    code_pages = torch.randint(0, nc, (P, Hkv, page, D // bd), generator=g, dtype=torch.uint8)
    v_pages = torch.randn(P, Hkv, Dv, page, generator=g).to(vdt)
    lens = torch.tensor([T, 517, 16 * 9 + 5], dtype=torch.int32)
    out, lse, scores = hip_ops.decode(q.to(DEV), code_pages.to(DEV), v_pages.to(DEV), cb.perm.to(DEV),
                                      cb.centroids.to(DEV), scale=1 / math.sqrt(D), block_table=table.to(DEV),
                                      seq_lens=lens.to(DEV), return_lse=True, return_scores=True, kernel=4,
                                      num_splits=splits)
    o, l, sc = np_of(out), np_of(lse), np_of(scores)
    vn = "f16" if vdt == torch.float16 else "bf16"
    for b in range(B):
        L = int(lens[b])
        codes = O.gather_pages_codes(code_pages.numpy(), table[b].numpy(), L)
        vals = O.gather_pages_values(v_pages.float().numpy(), table[b].numpy(), L)
        for kv in range(Hkv):
            ro, rs, rl = _oracle_unit(np_of(q)[b, kv * G:(kv + 1) * G], codes[kv], vals[kv], cb.centroids[kv].numpy(),
                                      cb.perm[kv].numpy(), 1 / math.sqrt(D), vdt=vn)
            sl = slice(kv * G, (kv + 1) * G)
            assert_rel(o[b, sl], ro, BF16_TOL, f"q4 out b={b} kv={kv}")
            assert_rel(l[b, sl], rl, SCORE_TOL, f"q4 lse b={b} kv={kv}")
            assert_rel(sc[b, sl, :, :L], rs, SCORE_TOL, f"q4 scores b={b} kv={kv}")
            assert np.all(sc[b, sl, :, L:] == -np.inf)


@pytest.mark.parametrize("Hq,Hkv,Lq,bd,hidx,dense,splits", [
    (8, 8, 1, 4, [5, 20], False, 0),         # one row per KV head (RP 1), 8 passthrough dims
    (16, 8, 1, 4, [3, 9, 11, 30], False, 2),  # two rows (RP 2), 16 dims, two splits
    (16, 2, 1, 8, [1, 6], False, 0),         # eight rows (RP 8) over 16 blocks of dim 8, 16 dims
    (4, 2, 3, 8, [4, 12], False, 3),         # three query tokens: 6 rows in an 8-row LUT, three splits
    (8, 8, 1, 4, [2, 3], True, 0),           # dense slots of adjacent heavy blocks: values 8..15 of each row
    (32, 8, 1, 4, [2, 3, 4, 5], True, 1),    # dense slots, four adjacent blocks: values 8..23
])
def test_contiguous_lut_kernel_128_dim_passthrough_rows(Hq, Hkv, Lq, bd, hidx, dense, splits):
    """The contiguous 128-dim LUT kernel's passthrough variant (8 or 16 consecutive 16-bit values per
    token in 16-byte aligned rows) at 1, 2 and 8 rows per LUT, with several query tokens and splits,
    and with the reference's dense slots where the heavy blocks are adjacent (so their values are
    consecutive from a 16-byte aligned slot); against the oracle."""
    log(f"contig LUT D128 passthrough rows Hq={Hq} Hkv={Hkv} Lq={Lq} bd={bd} heavy={hidx} dense={dense}")
    B, T, D = 2, 431, 128
    nb = D // bd
    cb = synthetic.make_codebook(Hkv, D, bd, 230 + Hq + bd)
    g = torch.Generator().manual_seed(231 + Hq + bd)
    heavy = [i in hidx for i in range(nb)]
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, nb), generator=g, dtype=torch.uint8)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    ptd = torch.zeros(B, Hkv, T, nb, bd)
    ptd[:, :, :, hidx] = torch.randn(B, Hkv, T, len(hidx), bd, generator=g)
    ptd = ptd.to(torch.bfloat16)
    pt = ptd if dense else ptd[:, :, :, hidx].contiguous()
    scale = 1 / math.sqrt(D)
    args = (q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    kw = dict(scale=scale, heavy=heavy, pt=pt.to(DEV), pt_dense=dense, num_splits=splits)
    out, lse, scores = hip_ops.decode(*args, **kw, return_lse=True, return_scores=True, kernel=2)
    ro, rs, rl = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                    cb.perm.numpy(), scale, "bf16", "bf16", heavy=np.array(heavy),
                                    pt_values=ptd.float().numpy(), return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    assert_rel(np_of(scores), rs, SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")
    # the automatic choice: the 4x4-MFMA kernel, which takes contiguous passthrough at head_dim 128
    oa = hip_ops.decode(*args, **kw)
    assert torch.equal(oa, hip_ops.decode(*args, **kw, kernel=4))
    assert_rel(np_of(oa), ro, BF16_TOL, "out, automatic choice")
