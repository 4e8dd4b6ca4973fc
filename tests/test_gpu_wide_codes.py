"""Codebooks of more than 256 codewords (the reference's int16 / int32 indices, sunshape/codec.py:78-83;
its default fitter's n_centroids = 2^round(bits_per_dim * block_dim), sunshape/hf.py:594, gives 4,096
codewords at 3 bits/dim and block_dim 4): encode bit-exact against the oracle, dequantize, scores and
the fused decode (contiguous and paged, masks, passthrough) against the oracle, and the codec, backend
and cache surfaces end to end.

16-bit codes are int16 tensors read as unsigned by the kernels; the oracle returns uint16 (the same
bits), and int32 past 65,535 codewords."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic
from sunshape_amd.codec import SunShapeBlockCodec

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _idx(t: torch.Tensor) -> np.ndarray:
    """Device codes as unsigned indices (int16 bits read as uint16)."""
    a = t.cpu().numpy()
    return a.view(np.uint16).astype(np.int64) if a.dtype == np.int16 else a.astype(np.int64)


def _keys(B, Hkv, S, D, sigma, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, Hkv, S, D, generator=g) * sigma).to(torch.bfloat16)


@pytest.mark.parametrize("D,bd,nc,heavy_n,metric,paged", [
    (128, 4, 4096, 0, False, False),    # the reference default at 3 bits/dim: 4,096 codewords, int16
    (64, 2, 512, 3, False, False),      # 512 codewords with three passthrough blocks
    (16, 1, 65536, 0, False, False),    # 65,536 codewords: int32 indices
    (32, 4, 4096, 0, True, False),      # SunShape-Pro block metric
    (64, 4, 1024, 0, False, True),      # written into pages through a slot mapping
])
def test_wide_encode_bit_exact(D, bd, nc, heavy_n, metric, paged):
    log(f"wide encode D={D} bd={bd} nc={nc} heavy={heavy_n} metric={metric} paged={paged}")
    B, Hkv, S = 2, 2, 300
    cb = synthetic.make_codebook(Hkv, D, bd, 600 + nc + D, n_centroids=nc)
    keys = _keys(B, Hkv, S, D, cb.sigma[:, None, :], 601 + nc)
    nb = D // bd
    heavy = [i < heavy_n for i in range(nb)] if heavy_n else None
    E = None
    if metric:
        g = torch.Generator().manual_seed(602)
        E = (torch.eye(D) + 0.1 * torch.randn(D, D, generator=g)).float()
    kw = dict(heavy=heavy, metric=None if E is None else E.to(DEV))
    if paged:
        page, P = 16, 64
        slots = torch.randperm(P * page, generator=torch.Generator().manual_seed(603))[:B * S].view(B, S)
        pages = torch.zeros(P, Hkv, page, nb, dtype=hip_ops.index_dtype(nc), device=DEV)
        hip_ops.encode(keys.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV), codes_out=pages,
                       slot_mapping=slots.to(DEV), **kw)
        flat = pages.permute(0, 2, 1, 3).reshape(P * page, Hkv, nb)
        codes = flat[slots.reshape(-1).to(DEV)].view(B, S, Hkv, nb).permute(0, 2, 1, 3)
        pt = None
    else:
        codes, pt = hip_ops.encode(keys.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV), **kw)
    assert codes.dtype == hip_ops.index_dtype(nc)
    got = _idx(codes)
    for b in range(B):
        for kv in range(Hkv):
            rc, rpt = O.encode(keys[b, kv].float().numpy(), cb.perm[kv].numpy(), cb.centroids[kv].numpy(),
                               None if heavy is None else np.array(heavy), metric=None if E is None else E.numpy(),
                               threads=8)
            assert np.array_equal(got[b, kv], rc.astype(np.int64)), f"b={b} kv={kv}"
            if heavy is not None:
                assert np.array_equal(np_of(pt[b, kv]), rpt[:, np.array(heavy)])
    # kernels 2 (MFMA screen) and 3 (grid search) serve at most 256 codewords: refused, not mis-served
    with pytest.raises(RuntimeError, match="exact scan"):
        hip_ops.encode(keys.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV), kernel=2)


def _merge_codebook(seed, nb, nc, bd, n):
    """Codewords in pairs one to three ulps apart in one coordinate (shuffled), and keys far from the
    codebook's cloud: nearest distances then often differ by less than a sqrt rounding, so the
    first argmin of the distance often is not the first argmin of the pre-sqrt value, and successive
    pre-sqrt minima fall within 2^-20 of each other."""
    rng = np.random.default_rng(seed)
    cent = np.empty((nb, nc, bd), np.float32)
    for b in range(nb):
        base = (rng.standard_normal((nc // 2, bd)) * 0.05).astype(np.float32)
        part = base.copy()
        bits = part.view(np.int32)
        steps = rng.integers(1, 4, nc // 2) * rng.choice([-1, 1], nc // 2)
        bits[np.arange(nc // 2), rng.integers(0, bd, nc // 2)] += steps.astype(np.int32)
        cent[b] = np.concatenate([base, part])[rng.permutation(nc)]
    x = (rng.standard_normal((n, nb * bd)) * 0.6).astype(np.float32)
    return cent, x


@pytest.mark.parametrize("n,direct", [(66000, False), (2000, False), (20, True)])
def test_wide_encode_sqrt_merges(n, direct):
    """4,096 codewords of dim 4 built so that sqrt merges are common (the first argmin of the
    distance has a larger pre-sqrt value than another codeword in hundreds of (key, block) pairs):
    bit-exact with the oracle with one lane per scan (66,000 keys), split scans (2,000 keys) and
    torch.cdist's direct distance (20 keys)."""
    log(f"wide encode sqrt merges n={n} direct={direct}")
    nb, nc, bd = 4, 4096, 4
    cent, x = _merge_codebook(11 + n, nb, nc, bd, n)
    perm = np.arange(nb * bd)
    keep = 0
    for b in range(nb):
        e2, d = O.block_distances(x[:, b * bd:(b + 1) * bd], cent[b], direct=direct)
        jd = d.argmin(1)
        keep += int((np.maximum(e2[np.arange(n), jd], 0) > np.maximum(e2, 0).min(1)).sum())
    if n >= 2000:
        assert keep > 50, keep  # the construction reaches the tie cases it is for
    ref, _ = O.encode(x, perm, cent, direct=direct, threads=8)
    codes, _ = hip_ops.encode(torch.from_numpy(x)[None, None].to(DEV), torch.from_numpy(perm)[None].to(DEV),
                              torch.from_numpy(cent)[None].to(DEV), direct=direct)
    got = _idx(codes)[0, 0]
    assert np.array_equal(got, ref.astype(np.int64)), int((got != ref.astype(np.int64)).sum())


@pytest.mark.parametrize("nc,bd", [(4096, 4), (65536, 2)])
def test_wide_dequantize_and_scores(nc, bd):
    log(f"wide dequantize/scores nc={nc} bd={bd}")
    D, T = 32, 700
    cb = synthetic.make_codebook(1, D, bd, 610 + nc, n_centroids=nc)
    perm, cent = cb.perm[0], cb.centroids[0]
    g = torch.Generator().manual_seed(611)
    idx = torch.randint(0, nc, (T, D // bd), generator=g)
    codes = idx.to(hip_ops.index_dtype(nc))  # 16-bit: the int16 bits of each index
    k_hat = hip_ops.dequantize(codes.to(DEV), perm.to(DEV), cent.to(DEV))
    ref = O.dequantize(idx.numpy(), cent.numpy(), perm.numpy())
    assert np.array_equal(np_of(k_hat), ref)
    q = torch.randn(5, D, generator=g)
    s = hip_ops.attention_scores(q.to(DEV), codes.to(DEV), perm.to(DEV), cent.to(DEV))
    assert_rel(np_of(s), O.attention_scores(q.numpy(), idx.numpy(), cent.numpy(), perm.numpy()), SCORE_TOL, "scores")


@pytest.mark.parametrize("B,Hq,Hkv,Lq,D,bd,nc,T,paged,mask,heavy_n,splits,Dv", [
    (2, 32, 8, 1, 128, 4, 4096, 600, False, False, 0, 0, 128),   # Llama-shaped layer at 3 bits/dim
    (2, 14, 2, 1, 64, 2, 512, 777, False, True, 0, 3, 64),       # Qwen-shaped, 512 codewords, a mask, 3 splits
    (2, 16, 4, 2, 64, 4, 4096, 500, True, False, 2, 0, 64),      # paged, two query tokens, passthrough blocks
    (1, 8, 2, 1, 32, 2, 65536, 300, False, False, 0, 2, 32),     # int32 indices
    # 16-bit codes read 16 blocks per batch: 24 blocks end in a half batch, 8 blocks fill half of one
    (2, 8, 2, 1, 96, 4, 4096, 333, False, True, 2, 3, 64),       # 24 blocks, mask, passthrough, 3 splits
    (2, 8, 2, 2, 32, 4, 1024, 250, True, False, 0, 0, 32),       # 8 blocks, pages, two query tokens
    (1, 4, 1, 1, 48, 2, 2048, 400, True, False, 2, 2, 64),       # 24 blocks of dim 2, pages, passthrough
])
def test_wide_decode_vs_oracle(B, Hq, Hkv, Lq, D, bd, nc, T, paged, mask, heavy_n, splits, Dv):
    log(f"wide decode B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} D={D} bd={bd} nc={nc} T={T} paged={paged} mask={mask} "
        f"heavy={heavy_n} Dv={Dv}")
    nb = D // bd
    cb = synthetic.make_codebook(Hkv, D, bd, 620 + nc + T, n_centroids=nc)
    g = torch.Generator().manual_seed(621 + T)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, nc, (B, Hkv, T, nb), generator=g)
    v = torch.randn(B, Hkv, T, Dv, generator=g).to(torch.bfloat16)
    heavy = [i in (1, 3) for i in range(nb)] if heavy_n else None
    ptd = torch.zeros(B, Hkv, T, nb, bd)
    if heavy_n:
        ptd[:, :, :, [1, 3]] = torch.randn(B, Hkv, T, 2, bd, generator=g).to(torch.bfloat16).float()
    m = None
    if mask:
        m = torch.where(torch.rand(B, Hq, Lq, T, generator=g) < 0.2, float("-inf"), 0.0)
        m[..., 0] = 0.0
    scale = 1 / math.sqrt(D)
    codes = idx.to(hip_ops.index_dtype(nc))
    kw = dict(scale=scale, num_splits=splits, mask=None if m is None else m.to(DEV), heavy=heavy)
    if paged:
        page = 16
        n = (T + page - 1) // page
        table = torch.randperm(B * n, generator=g).view(B, n).to(torch.int32)
        cp = torch.zeros(B * n, Hkv, page, nb, dtype=codes.dtype)
        vp = torch.zeros(B * n, Hkv, Dv, page, dtype=v.dtype)
        pp = torch.zeros(B * n, Hkv, page, 2, bd, dtype=torch.bfloat16)
        for b in range(B):
            for j in range(n):
                t0, t1 = j * page, min((j + 1) * page, T)
                pg = int(table[b, j])
                cp[pg, :, :t1 - t0] = codes[b, :, t0:t1]
                vp[pg, :, :, :t1 - t0] = v[b, :, t0:t1].transpose(-1, -2)
                pp[pg, :, :t1 - t0] = ptd[b, :, t0:t1, [1, 3]].to(torch.bfloat16)
        out, lse, sc = hip_ops.decode(q.to(DEV), cp.to(DEV), vp.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV),
                                      block_table=table.to(DEV), seq_lens=torch.full((B,), T, dtype=torch.int32,
                                                                                     device=DEV),
                                      pt=pp.to(DEV) if heavy_n else None, return_lse=True, return_scores=True, **kw)
        sc = sc[..., :T]
    else:
        out, lse, sc = hip_ops.decode(q.to(DEV), codes.to(DEV), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV),
                                      pt=ptd[:, :, :, [1, 3]].to(torch.bfloat16).contiguous().to(DEV) if heavy_n else None,
                                      return_lse=True, return_scores=True, **kw)
    ro, rs, rl = O.decode_attention(q.float().numpy(), idx.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                    cb.perm.numpy(), scale, "bf16", "bf16", mask=None if m is None else m.numpy(),
                                    heavy=None if heavy is None else np.array(heavy),
                                    pt_values=ptd.numpy() if heavy_n else None, return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    fin = np.isfinite(rs)
    assert np.array_equal(np.isfinite(np_of(sc)), fin)
    assert_rel(np_of(sc)[fin], rs[fin], SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")


@pytest.mark.parametrize("B,Hq,Hkv,Lq,D,bd,nc,T,paged,mask,splits", [
    (2, 32, 8, 1, 128, 4, 4096, 4500, False, False, 1),  # 3 bits/dim, Llama-shaped: two super-tiles, the last partial
    (2, 32, 8, 1, 128, 4, 4096, 5000, False, True, 2),   # two splits of 2,560 tokens, a mask
    (1, 16, 4, 2, 128, 4, 4096, 2300, True, False, 1),   # pages, two query tokens (8 rows: 4-tile super-tiles)
    (2, 14, 2, 1, 64, 2, 1024, 3000, False, True, 1),    # 5 bits/dim at block_dim 2, 7 query heads per KV head
    (1, 8, 2, 1, 64, 2, 2048, 2100, True, True, 1),      # pages, a mask, 52 tokens past the first super-tile
])
def test_wide_decode_staged_codebook(B, Hq, Hkv, Lq, D, bd, nc, T, paged, mask, splits):
    """Long contexts (at least 2,048 tokens per split) take k_decode_wide, which stages each block's
    codebook in LDS for a super-tile of tokens instead of gathering codewords per token.  Output,
    lse and raw scores against the oracle; the raw scores also equal bit for bit those of the same
    call split finely enough (256 tokens per split) to take the per-token gathers of
    k_decode_generic."""
    log(f"wide staged decode B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} D={D} bd={bd} nc={nc} T={T} paged={paged} "
        f"mask={mask} splits={splits}")
    nb = D // bd
    cb = synthetic.make_codebook(Hkv, D, bd, 640 + nc + T, n_centroids=nc)
    g = torch.Generator().manual_seed(641 + T)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, nc, (B, Hkv, T, nb), generator=g)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    m = None
    if mask:
        m = torch.where(torch.rand(B, Hq, Lq, T, generator=g) < 0.2, float("-inf"), 0.0)
        m[..., 0] = 0.0
    scale = 1 / math.sqrt(D)
    codes = idx.to(hip_ops.index_dtype(nc))
    if paged:
        page = 16
        n = (T + page - 1) // page
        table = torch.randperm(B * n, generator=g).view(B, n).to(torch.int32)
        cp = torch.zeros(B * n, Hkv, page, nb, dtype=codes.dtype)
        vp = torch.zeros(B * n, Hkv, D, page, dtype=v.dtype)
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
    out, lse, sc = hip_ops.decode(*args, num_splits=splits, **kw)
    _, _, sc_g = hip_ops.decode(*args, num_splits=(T + 255) // 256, **kw)
    assert torch.equal(sc[..., :T], sc_g[..., :T]), "staged and gathered scores differ"
    ro, rs, rl = O.decode_attention(q.float().numpy(), idx.numpy(), v.float().numpy(), cb.centroids.numpy(),
                                    cb.perm.numpy(), scale, "bf16", "bf16", mask=None if m is None else m.numpy(),
                                    return_scores=True)
    assert_rel(np_of(out), ro, BF16_TOL, "out")
    got = np_of(sc[..., :T])
    fin = np.isfinite(rs)
    assert np.array_equal(np.isfinite(got), fin)
    assert_rel(got[fin], rs[fin], SCORE_TOL, "scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "lse")


def test_wide_codec_backend_and_caches_end_to_end():
    """A 4,096-codeword codec (3 bits/dim at block_dim 4) through the reference's surfaces: codec
    quantize (int16 indices, bit-exact) / dequantize / attention_scores, quantize_key_states +
    SunShapeAttentionImpl.forward, the HF code cache's decode step and the paged cache."""
    from sunshape_amd import vllm_attn_backend as VB
    from sunshape_amd.cache import SunShapeCodeLayer, sunshape_attention_forward
    from sunshape_amd.hf import SunShapeBundle
    from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState
    from sunshape_amd.paged import PagedSunShapeCache

    log("wide codec end to end")
    B, Hq, Hkv, S, D, bd, nc = 2, 8, 2, 300, 64, 4, 4096
    cb = synthetic.make_codebook(1, D, bd, 630, n_centroids=nc)
    codec = SunShapeBlockCodec.from_buffers(cb.perm[0], cb.centroids[0], device=DEV)
    keys = _keys(B, Hkv, S, D, cb.sigma[0], 631)
    perm, cent = cb.perm[0].numpy(), cb.centroids[0].numpy()
    qz = codec.quantize(keys[0, 0].to(DEV))
    assert qz.indices.dtype == torch.int16
    rc, _ = O.encode(keys[0, 0].float().numpy(), perm, cent)
    assert np.array_equal(_idx(qz.indices), rc.astype(np.int64))
    assert np.array_equal(np_of(codec.dequantize(qz)), O.dequantize(rc, cent, perm))
    g = torch.Generator().manual_seed(632)
    q1 = torch.randn(3, D, generator=g)
    assert_rel(np_of(codec.attention_scores(q1.to(DEV), qz)), O.attention_scores(q1.numpy(), rc, cent, perm),
               SCORE_TOL, "codec.attention_scores")
    # the vLLM drop-in: quantize_key_states + forward
    bundle = SunShapeBundle("m", [0], 3.0, bd, "profileperm_baseline", 0, 0, 0, {0: codec})
    rs = SunShapeVLLMRuntimeState("p", "m", "sunshape_base", 3.0, bd, [0], bundle, "cuda")
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    VB.register_runtime_state(rs)
    try:
        qk = VB.quantize_key_states(0, keys.to(DEV))
        codes = np.stack([np.stack([O.encode(keys[b, h].float().numpy(), perm, cent)[0] for h in range(Hkv)])
                          for b in range(B)]).astype(np.int64)
        assert qk.codes.dtype == torch.int16 and np.array_equal(_idx(qk.codes), codes)
        out = VB.get_backend_factory().make_impl(layer_idx=0)(q.to(DEV), qk, v.to(DEV), scale=1 / math.sqrt(D))
    finally:
        VB.clear_registered_runtime()
    ref = O.decode_attention(q.float().numpy(), codes, v.float().numpy(), cent, perm, 1 / math.sqrt(D), "bf16", "bf16")
    assert_rel(np_of(out), ref, BF16_TOL, "impl.forward")
    # HF code cache: one decode step
    layer = SunShapeCodeLayer(codec)
    ck, cv = layer.update(keys.to(DEV), v.to(DEV))
    assert ck.codes.dtype == torch.int16 and np.array_equal(_idx(ck.codes), codes)
    mod = torch.nn.Module()
    mod.num_key_value_groups = Hq // Hkv
    o2, _ = sunshape_attention_forward(mod, q.to(DEV), ck, cv, None, scaling=1 / math.sqrt(D))
    assert_rel(np_of(o2.transpose(1, 2)), ref, BF16_TOL, "code cache decode")
    # paged cache: append the keys, decode
    pc = PagedSunShapeCache(codec, num_pages=64, num_kv_heads=Hkv, value_dim=D)
    pc.append([0, 1], keys.to(DEV), v.to(DEV))
    o3 = pc.decode([0, 1], q.to(DEV), scale=1 / math.sqrt(D))
    assert_rel(np_of(o3), ref, BF16_TOL, "paged cache decode")
