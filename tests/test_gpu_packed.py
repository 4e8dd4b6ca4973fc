"""Sub-byte packed codes on the GPU: pack/unpack kernels against the oracle, and scores /
decode over packed words equal to the same kernel over uint8 codes, bit for bit."""

import math

import numpy as np
import pytest
import torch

from _util import SCORE_TOL, BF16_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("bits,nb", [(1, 33), (3, 11), (4, 32), (6, 32), (6, 8), (7, 9), (8, 16)])
def test_pack_unpack_kernels_vs_oracle(bits, nb):
    log(f"pack bits={bits} nb={nb}")
    rng = np.random.default_rng(bits * 10 + nb)
    c = rng.integers(0, 1 << bits, size=(3, 101, nb), dtype=np.uint8)
    ct = torch.from_numpy(c).to(DEV)
    w = hip_ops.pack_codes(ct, bits)
    assert np.array_equal(np_of(w), O.pack_codes(c, bits))
    assert torch.equal(hip_ops.unpack_codes(w, nb, bits), ct)
    if bits < 8:
        with pytest.raises(RuntimeError, match="fit"):
            hip_ops.pack_codes(torch.full((2, nb), 1 << bits, dtype=torch.uint8, device=DEV), bits)


def _case(nc=64, bd=2, D=64, B=2, Hkv=2, Hq=8, T=700, seed=21):
    cb = synthetic.make_codebook(Hkv, D, bd, seed, n_centroids=nc)
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, nc, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    return cb, codes, q, v


def test_scores_over_packed_codes_equal_uint8():
    log("packed scores")
    cb, codes, q, _ = _case()
    perm, cent = cb.perm[0].to(DEV), cb.centroids[0].to(DEV)
    c2 = codes[0, 0].to(DEV)
    w = hip_ops.pack_codes(c2, 6)
    qq = q[0, :, 0].float().to(DEV)
    # the same (generic LUT) kernel reads both forms
    s8 = hip_ops.attention_scores(qq, c2, perm, cent, kernel=1)
    s6 = hip_ops.attention_scores(qq, w, perm, cent, code_bits=6, kernel=1)
    assert torch.equal(s8, s6)
    ref = O.attention_scores(np_of(qq), np_of(c2), cb.centroids[0].numpy(), cb.perm[0].numpy())
    assert_rel(np_of(s6), ref, SCORE_TOL, "packed scores vs oracle")
    with pytest.raises(RuntimeError, match="n_centroids"):
        hip_ops.attention_scores(qq, hip_ops.pack_codes(c2 & 31, 5), perm, cent, code_bits=5)


@pytest.mark.parametrize("paged", [False, True])
def test_decode_over_packed_codes_equals_uint8(paged):
    log(f"packed decode paged={paged}")
    cb, codes, q, v = _case(T=640)
    B, Hkv, T, nb = codes.shape
    perm, cent = cb.perm.to(DEV), cb.centroids.to(DEV)
    scale = 1 / math.sqrt(64)
    if not paged:
        c8 = codes.to(DEV)
        w = hip_ops.pack_codes(c8, 6)
        o8, l8 = hip_ops.decode(q.to(DEV), c8, v.to(DEV), perm, cent, scale=scale, return_lse=True, kernel=1)
        o6, l6 = hip_ops.decode(q.to(DEV), w, v.to(DEV), perm, cent, scale=scale, return_lse=True, code_bits=6,
                                kernel=1)
    else:
        page = 16
        n = T // page
        P = B * n + 5
        table = torch.randperm(P, generator=torch.Generator().manual_seed(2))[: B * n].view(B, n).to(torch.int32)
        cp = torch.zeros(P, Hkv, page, nb, dtype=torch.uint8)
        vp = torch.zeros(P, Hkv, 64, page, dtype=torch.bfloat16)
        for b in range(B):
            cp[table[b].long()] = codes[b].view(Hkv, n, page, nb).permute(1, 0, 2, 3)
            vp[table[b].long()] = v[b].view(Hkv, n, page, 64).permute(1, 0, 3, 2)
        lens = torch.full((B,), T, dtype=torch.int32).to(DEV)
        cpd, vpd, tbl = cp.to(DEV), vp.to(DEV), table.to(DEV)
        w = hip_ops.pack_codes(cpd, 6)
        o8, l8 = hip_ops.decode(q.to(DEV), cpd, vpd, perm, cent, scale=scale, block_table=tbl, seq_lens=lens,
                                return_lse=True, kernel=1)
        o6, l6 = hip_ops.decode(q.to(DEV), w, vpd, perm, cent, scale=scale, block_table=tbl, seq_lens=lens,
                                return_lse=True, code_bits=6, kernel=1)
    assert torch.equal(o8, o6) and torch.equal(l8, l6)
    ref = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                             cb.perm.numpy(), scale, "bf16", "bf16")
    assert_rel(np_of(o6), ref, BF16_TOL, "packed decode vs oracle")


@pytest.mark.parametrize("bits,bd,nc,Hq,T", [(6, 2, 64, 14, 700), (4, 2, 16, 8, 640), (6, 1, 64, 4, 333),
                                             (4, 4, 16, 16, 1000), (6, 8, 64, 2, 129), (8, 2, 256, 14, 700),
                                             (1, 1, 2, 8, 300), (2, 2, 4, 14, 640), (3, 4, 8, 4, 517),
                                             (5, 2, 32, 16, 700), (7, 8, 128, 6, 1000), (7, 1, 128, 14, 257),
                                             (3, 1, 8, 2, 129), (5, 2, 32, 8, 1), (1, 2, 2, 14, 63)])
def test_contig_mfma_decode_over_packed_codes_equals_uint8(bits, bd, nc, Hq, T):
    """The contiguous MFMA kernel unpacks packed words in registers (4 and 6 bits with the width
    fixed at compile time, 1-3, 5 and 7 bits at run time; 8-bit words are read as byte rows):
    output, LSE and raw scores equal its own uint8-code launch bit for bit."""
    log(f"packed contig decode bits={bits} bd={bd} nc={nc} Hq={Hq} T={T}")
    cb, codes, q, v = _case(nc=nc, bd=bd, Hq=Hq, T=T, seed=40 + bits + bd)
    perm, cent = cb.perm.to(DEV), cb.centroids.to(DEV)
    scale = 1 / math.sqrt(64)
    c8 = codes.to(DEV)
    w = hip_ops.pack_codes(c8, bits)
    qd, vd = q.to(DEV), v.to(DEV)
    o8, l8, s8 = hip_ops.decode(qd, c8, vd, perm, cent, scale=scale, return_lse=True, return_scores=True, kernel=3)
    o6, l6, s6 = hip_ops.decode(qd, w, vd, perm, cent, scale=scale, return_lse=True, return_scores=True,
                                code_bits=bits, kernel=3)
    assert torch.equal(o8, o6) and torch.equal(l8, l6) and torch.equal(s8, s6)
    # the default choice takes the same kernel; the scores-only launch reads packed words too
    assert torch.equal(hip_ops.decode(qd, w, vd, perm, cent, scale=scale, code_bits=bits), o6)
    g8 = hip_ops.gqa_scores(qd, c8, perm, cent, scale=scale, kernel=3)
    assert torch.equal(hip_ops.gqa_scores(qd, w, perm, cent, scale=scale, code_bits=bits, kernel=3), g8)
    assert torch.equal(g8, s8)
    ref, ref_s, _ = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                       cb.perm.numpy(), scale, "bf16", "bf16", return_scores=True)
    assert_rel(np_of(o6), ref, BF16_TOL, "packed contig decode vs oracle")
    assert_rel(np_of(s6), ref_s, SCORE_TOL, "packed contig scores vs oracle")


def _pages(codes, v, seed):
    """Scatter [B, Hkv, T, nb] codes and [B, Hkv, T, Dv] values into shuffled 16-token pages
    (the last page of each sequence zero-padded): codes [P, Hkv, 16, nb], values [P, Hkv, Dv, 16]."""
    B, Hkv, T, nb = codes.shape
    Dv = v.shape[-1]
    page = 16
    n = (T + page - 1) // page
    P = B * n + 3
    table = torch.randperm(P, generator=torch.Generator().manual_seed(seed))[: B * n].view(B, n).to(torch.int32)
    cp = torch.zeros(P, Hkv, page, nb, dtype=torch.uint8)
    vp = torch.zeros(P, Hkv, Dv, page, dtype=v.dtype)
    pad = n * page - T
    for b in range(B):
        cb_ = torch.cat([codes[b], torch.zeros(Hkv, pad, nb, dtype=codes.dtype)], 1)
        vb_ = torch.cat([v[b], torch.zeros(Hkv, pad, Dv, dtype=v.dtype)], 1)
        cp[table[b].long()] = cb_.view(Hkv, n, page, nb).permute(1, 0, 2, 3)
        vp[table[b].long()] = vb_.view(Hkv, n, page, Dv).permute(1, 0, 3, 2)
    return cp.to(DEV), vp.to(DEV), table.to(DEV), torch.full((B,), T, dtype=torch.int32, device=DEV)


@pytest.mark.parametrize("bits,bd,nc,Hq,D,T", [(6, 2, 64, 8, 64, 640), (4, 2, 16, 32, 64, 300), (6, 4, 64, 4, 128, 1000),
                                               (6, 1, 64, 2, 64, 77), (8, 2, 256, 8, 64, 500), (0, 2, 64, 8, 64, 640)])
def test_paged_mfma_decode_over_packed_codes(bits, bd, nc, Hq, D, T):
    """Paged decode of 4- / 6-bit packed codes and of codebooks under 256 codewords: 64-codeword
    codebooks with 2-8 rows run the LUT kernel (a 64-entry table per block, codes unpacked from
    the words in registers), the others the 4x4-MFMA-scores kernel (codes taken from the words in
    registers).  Equal to the same kernel's uint8-code launch bit for bit (8-bit words are read as the
    byte rows), and to the oracle."""
    log(f"packed paged decode bits={bits} bd={bd} nc={nc} Hq={Hq} D={D} T={T}")
    cb, codes, q, v = _case(nc=nc, bd=bd, D=D, Hq=Hq, T=T, seed=60 + bits + bd)
    perm, cent = cb.perm.to(DEV), cb.centroids.to(DEV)
    scale = 1 / math.sqrt(D)
    cpd, vpd, tbl, lens = _pages(codes, v, seed=bits + 7)
    qd = q.to(DEV)
    kw = dict(scale=scale, block_table=tbl, seq_lens=lens, return_lse=True, return_scores=True, kernel=2)
    o8, l8, s8 = hip_ops.decode(qd, cpd, vpd, perm, cent, **kw)
    if bits:
        w = hip_ops.pack_codes(cpd, bits)
        o6, l6, s6 = hip_ops.decode(qd, w, vpd, perm, cent, code_bits=bits, **kw)
        assert torch.equal(o8, o6) and torch.equal(l8, l6) and torch.equal(s8, s6)
        kw.pop("kernel")
        assert torch.equal(hip_ops.decode(qd, w, vpd, perm, cent, code_bits=bits, **kw)[0], o6)
    assert s8.shape[-1] == (T + 15) // 16 * 16 and bool((s8[..., T:] == float("-inf")).all())
    ref, ref_s, _ = O.decode_attention(q.float().numpy(), codes.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                       cb.perm.numpy(), scale, "bf16", "bf16", return_scores=True)
    assert_rel(np_of(o8), ref, BF16_TOL, "paged packed decode vs oracle")
    assert_rel(np_of(s8[..., :T]), ref_s, SCORE_TOL, "paged packed scores vs oracle")


@pytest.mark.parametrize("Hq", [8, 2])
def test_codes_past_the_codebook_read_its_last_codeword(Hq):
    """Byte codes >= n_centroids (invalid input) read the last codeword in every decode kernel:
    generic and contiguous MFMA over the contiguous layout, generic and paged (64-codeword LUT at
    4 rows per KV head, MFMA scores at 1) over pages.  Checked against the oracle on clamped codes."""
    log(f"codes past the codebook Hq={Hq}")
    nc = 64
    cb, codes, q, v = _case(nc=nc, bd=2, Hq=Hq, T=320, seed=77)
    codes = torch.randint(0, 256, codes.shape, generator=torch.Generator().manual_seed(78), dtype=torch.uint8)
    perm, cent = cb.perm.to(DEV), cb.centroids.to(DEV)
    scale = 1 / math.sqrt(64)
    ref = O.decode_attention(q.float().numpy(), np.minimum(codes.numpy(), nc - 1), v.float().numpy(),
                             cb.centroids.numpy(), cb.perm.numpy(), scale, "bf16", "bf16")
    qd = q.to(DEV)
    for kernel in (1, 3):
        o = hip_ops.decode(qd, codes.to(DEV), v.to(DEV), perm, cent, scale=scale, kernel=kernel)
        assert_rel(np_of(o), ref, BF16_TOL, f"contiguous kernel {kernel}")
    cpd, vpd, tbl, lens = _pages(codes, v, seed=79)
    for kernel in (1, 2):
        o = hip_ops.decode(qd, cpd, vpd, perm, cent, scale=scale, block_table=tbl, seq_lens=lens, kernel=kernel)
        assert_rel(np_of(o), ref, BF16_TOL, f"paged kernel {kernel}")
