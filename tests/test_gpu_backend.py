"""Drop-in surfaces on the GPU: codec quantize/dequantize/forward/attention_scores,
quantize_key_states + SunShapeAttentionImpl.forward, bundle round trip, per-KV-head codecs."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import synthetic
from sunshape_amd import vllm_attn_backend as VB
from sunshape_amd.codec import SunShapeBlockCodec
from sunshape_amd.hf import SunShapeBundle
from sunshape_amd.integration.vllm import load_runtime_state

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _mixed_codec(seed=31, D=64, bd=2):
    cb = synthetic.make_codebook(1, D, bd, seed, shared_sigma=True)
    heavy = synthetic.heavy_blocks_by_sigma(cb.sigma[0], cb.perm[0], bd, 4)
    cent = cb.centroids[0].clone()
    cent[heavy] = 0
    codec = SunShapeBlockCodec.from_buffers(cb.perm[0], cent, mode="profileperm_mixed_precision",
                                            mixed_high_precision_blocks=heavy, device=DEV)
    return codec, cb.sigma[0]


def test_codec_quantize_dequantize_forward_mixed():
    log("codec mixed quantize/dequantize")
    codec, sigma = _mixed_codec()
    keys = (torch.randn(2000, 64) * sigma).to(torch.bfloat16)
    qz = codec.quantize(keys.to(DEV))
    assert qz.indices.dtype == torch.uint8 and qz.indices.shape == (2000, 32)
    assert qz.passthrough_values.shape == (2000, 32, 2) and qz.passthrough_values.dtype == torch.float32
    heavy = codec.mixed_high_precision_blocks.cpu().numpy()
    rc, rpt = O.encode(keys.float().numpy(), codec.permutation.cpu().numpy(), codec.centroids.cpu().numpy(), heavy)
    assert np.array_equal(np_of(qz.indices), rc)
    assert np.array_equal(np_of(qz.passthrough_values), rpt)
    k_hat = np_of(codec.dequantize(qz))
    ref = O.dequantize(rc, codec.centroids.cpu().numpy(), codec.permutation.cpu().numpy(), heavy, rpt)
    assert np.array_equal(k_hat, ref)
    assert np.array_equal(np_of(codec(keys.to(DEV))), ref)
    q = torch.randn(5, 64, device=DEV)
    s = np_of(codec.attention_scores(q, qz))
    assert_rel(s, np_of(q).astype(np.float64) @ ref.astype(np.float64).T, SCORE_TOL, "mixed scores")


def test_codec_encode_grid_cached_and_rebuilt_on_codebook_change():
    """codec.quantize runs the grid search for block_dim 2 (the codec builds and caches the
    grid); the codes equal the exhaustive encode's, and an in-place codebook write rebuilds it."""
    log("codec encode grid cache")
    codec, sigma = _mixed_codec(seed=41)
    keys = (torch.randn(3000, 64) * sigma).to(torch.bfloat16).to(DEV)
    qz = codec.quantize(keys)
    assert len(codec._grid_cache) == 1
    grid = next(iter(codec._grid_cache.values()))[1]
    codec.use_encode_grid = False
    assert np.array_equal(np_of(codec.quantize(keys).indices), np_of(qz.indices))
    codec.use_encode_grid = True
    assert codec.quantize(keys).indices.equal(qz.indices)
    assert next(iter(codec._grid_cache.values()))[1] is grid  # reused
    with torch.no_grad():
        codec.centroids.mul_(1.5)
    qz2 = codec.quantize(keys)
    assert next(iter(codec._grid_cache.values()))[1] is not grid  # rebuilt
    heavy = codec.mixed_high_precision_blocks.cpu().numpy()
    rc, _ = O.encode(keys.float().cpu().numpy(), codec.permutation.cpu().numpy(), codec.centroids.cpu().numpy(), heavy)
    assert np.array_equal(np_of(qz2.indices), rc)


def test_codec_identity_mode_ignores_permutation_buffer():
    log("codec identity mode")
    cb = synthetic.make_codebook(1, 64, 8, 5)
    codec = SunShapeBlockCodec.from_buffers(cb.perm[0], cb.centroids[0], mode="identity_baseline", device=DEV)
    keys = torch.randn(300, 64)
    rc, _ = O.encode(keys.numpy(), np.arange(64), cb.centroids[0].numpy())
    assert np.array_equal(np_of(codec.quantize(keys.to(DEV)).indices), rc)


def test_quantize_key_states_and_impl_forward_per_kv_head_codec():
    log("backend per-kv-head end to end")
    B, Hq, Hkv, S, D, bd = 2, 8, 2, 900, 128, 4
    cb = synthetic.make_codebook(Hkv, D, bd, 41)
    codec = SunShapeBlockCodec.from_buffers(cb.perm, cb.centroids, device=DEV)
    bundle = SunShapeBundle("m", [0], 2.0, bd, "profileperm_baseline", 0, 0, 0, {0: codec})
    from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState

    rs = SunShapeVLLMRuntimeState("p", "m", "sunshape_base", 2.0, bd, [0], bundle, "cuda")
    VB.register_runtime_state(rs)
    try:
        g = torch.Generator().manual_seed(42)
        keys = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
        qk = VB.quantize_key_states(0, keys.to(DEV))
        assert qk.batch_size == B and qk.num_kv_heads == Hkv and qk.seq_len == S
        codes = np_of(qk.codes)
        for b in range(B):
            for h in range(Hkv):
                rc, _ = O.encode(keys[b, h].float().numpy(), cb.perm[h].numpy(), cb.centroids[h].numpy())
                assert np.array_equal(codes[b, h], rc)
                assert torch.equal(qk.head(b, h).indices, qk.codes[b, h])
        q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
        impl = VB.get_backend_factory().make_impl(layer_idx=0)
        out = np_of(impl(q, qk, v, scale=1 / math.sqrt(D), is_causal=True))
        ref = O.decode_attention(np_of(q), codes, np_of(v), cb.centroids.numpy(), cb.perm.numpy(), 1 / math.sqrt(D),
                                 "bf16", "bf16")
        assert_rel(out, ref, BF16_TOL, "impl.forward")
        # payload rebuilt from the per-head tuple only (no batched backing store)
        qk2 = VB.SunShapeQuantizedKeys(quantized_heads=qk.quantized_heads, batch_size=B, num_kv_heads=Hkv, seq_len=S)
        assert np.array_equal(np_of(impl(q, qk2, v, scale=1 / math.sqrt(D))), out)
    finally:
        VB.clear_registered_runtime()


def _per_head_runtime(Hkv, D, bd, seed):
    from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState

    cb = synthetic.make_codebook(Hkv, D, bd, seed)
    codec = SunShapeBlockCodec.from_buffers(cb.perm, cb.centroids, device=DEV)
    bundle = SunShapeBundle("m", [0], 2.0, bd, "profileperm_baseline", 0, 0, 0, {0: codec})
    return cb, codec, SunShapeVLLMRuntimeState("p", "m", "sunshape_base", 2.0, bd, [0], bundle, "cuda")


@pytest.mark.parametrize("scale", [None, 0.5])
def test_impl_forward_causal_rows_over_quantized_payload(scale):
    """Causal attention with several query rows over a quantized payload (chunked prefill).  The
    reference dequantizes the payload and runs scaled_dot_product_attention(query * scale, key,
    value, is_causal=True) (sunshape/vllm_attn_backend.py:306-345): scores scaled by
    scale / sqrt(D) (1 / sqrt(D) without a scale) under torch's top-left causal mask.  The fused
    kernel computes that from the codes: checked against the oracle with the same mask and scale,
    and against torch's fp32 scaled_dot_product_attention over the oracle's dequantized keys."""
    import torch.nn.functional as F

    log(f"backend causal rows over a quantized payload scale={scale}")
    B, Hq, Hkv, S, D, bd, Lq = 2, 8, 2, 300, 64, 2, 3
    cb, codec, rs = _per_head_runtime(Hkv, D, bd, 71)
    VB.register_runtime_state(rs)
    try:
        g = torch.Generator().manual_seed(72)
        keys = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
        qk = VB.quantize_key_states(0, keys.to(DEV))
        q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
        v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
        impl = VB.get_backend_factory().make_impl(layer_idx=0)
        out = np_of(impl(q.to(DEV), qk, v.to(DEV), scale=scale, is_causal=True))
        eff = (1.0 if scale is None else scale) / math.sqrt(D)
        mask = np.triu(np.full((Lq, S), -np.inf, dtype=np.float32), 1)
        codes = np_of(qk.codes)
        ref = O.decode_attention(np_of(q), codes, np_of(v), cb.centroids.numpy(), cb.perm.numpy(), eff, "bf16", "bf16",
                                 mask=mask)
        assert_rel(out, ref, BF16_TOL, "causal rows vs oracle")
        k_hat = np.stack([np.stack([O.dequantize(codes[b, h], cb.centroids[h].numpy(), cb.perm[h].numpy())
                                    for h in range(Hkv)]) for b in range(B)])
        qs = q.float() * (1.0 if scale is None else scale)
        kk = torch.from_numpy(k_hat).repeat_interleave(Hq // Hkv, dim=1)
        vv = v.float().repeat_interleave(Hq // Hkv, dim=1)
        sdpa = F.scaled_dot_product_attention(qs, kk, vv, is_causal=True)
        assert_rel(out, sdpa.numpy(), BF16_TOL, "causal rows vs fp32 SDPA on the dequantized keys")
    finally:
        VB.clear_registered_runtime()


def test_impl_forward_quantized_payload_to_delegate_is_dequantized():
    """Off the fused path with a delegate, the reference hands the delegate the dequantized keys
    (sunshape/vllm_attn_backend.py:306-323): one codec.dequantize per (batch, KV head)."""
    log("backend quantized payload to a delegate")
    B, Hq, Hkv, S, D, bd = 2, 4, 2, 100, 64, 2
    cb, codec, rs = _per_head_runtime(Hkv, D, bd, 81)
    VB.register_runtime_state(rs)
    seen = {}

    def delegate(query, key, value, **kw):
        seen["key"], seen["kw"] = key, kw
        return torch.zeros_like(query)

    try:
        g = torch.Generator().manual_seed(82)
        qk = VB.quantize_key_states(0, torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV))
        q = torch.randn(B, Hq, 2, D, generator=g).to(torch.bfloat16).to(DEV)
        v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
        impl = VB.get_backend_factory().make_impl(layer_idx=0, delegate=delegate)
        impl(q, qk, v, is_causal=True, scale=0.25)
        codes = np_of(qk.codes)
        want = np.stack([np.stack([O.dequantize(codes[b, h], cb.centroids[h].numpy(), cb.perm[h].numpy())
                                   for h in range(Hkv)]) for b in range(B)])
        assert seen["key"].shape == (B, Hkv, S, D)
        assert_rel(np_of(seen["key"]), want, SCORE_TOL, "delegate keys")
        assert seen["kw"]["is_causal"] is True and seen["kw"]["scale"] == 0.25
    finally:
        VB.clear_registered_runtime()


def test_bundle_roundtrip_on_gpu_and_runtime_state(tmp_path):
    log("bundle round trip")
    codec, _ = _mixed_codec(seed=51)
    b = SunShapeBundle("m", [2], 4.0, 2, "profileperm_mixed_precision", 0, 0, 0, {2: codec})
    path = b.save(tmp_path / "b.pt")
    rs = load_runtime_state(bundle_path=path, model_name="m", mode="sunshape_mixed", bits_per_dim=4.0, block_dim=2,
                            layers=[2], device="cuda")
    c2 = rs.codec_for_layer(2)
    keys = torch.randn(100, 64, device=DEV)
    assert torch.equal(c2.quantize(keys).indices, codec.quantize(keys).indices)


@pytest.mark.parametrize("mixed", [False, True])
def test_paged_cache_append_and_decode(mixed):
    """Prefill + two single-token appends into pages for 3 sequences, then decode (F1)."""
    from sunshape_amd.paged import PagedSunShapeCache

    log(f"paged cache mixed={mixed}")
    Hkv, Hq, D, bd = 2, 8, 64, 2
    if mixed:
        codec, sigma = _mixed_codec(seed=61)
    else:
        cb = synthetic.make_codebook(1, D, bd, 62)
        codec, sigma = SunShapeBlockCodec.from_buffers(cb.perm[0], cb.centroids[0], device=DEV), cb.sigma[0]
    cache = PagedSunShapeCache(codec, num_pages=64, num_kv_heads=Hkv, value_dim=D, device=DEV)
    g = torch.Generator().manual_seed(63)
    seqs = [5, 9, 2]
    hist_k = {s: [] for s in seqs}
    hist_v = {s: [] for s in seqs}
    for S in (100, 1, 1):
        k = (torch.randn(3, Hkv, S, D, generator=g) * sigma).to(torch.bfloat16)
        v = torch.randn(3, Hkv, S, D, generator=g).to(torch.bfloat16)
        cache.append(seqs, k.to(DEV), v.to(DEV))
        for i, s in enumerate(seqs):
            hist_k[s].append(k[i])
            hist_v[s].append(v[i])
    q = torch.randn(3, Hq, 1, D, generator=g).to(torch.bfloat16)
    out = np_of(cache.decode(seqs, q.to(DEV), scale=1 / math.sqrt(D)))
    heavy = None if codec.heavy_blocks() is None else np.array(codec.heavy_blocks())
    perm, cent = codec.permutation.cpu().numpy(), codec.centroids.cpu().numpy()
    for i, s in enumerate(seqs):
        keys = torch.cat(hist_k[s], dim=1).float().numpy()   # [Hkv, 102, D]
        vals = torch.cat(hist_v[s], dim=1).float().numpy()
        codes, pts = [], []
        for h in range(Hkv):
            c, pt = O.encode(keys[h], perm, cent, heavy)
            codes.append(c)
            pts.append(pt)
        pt_all = None if heavy is None else O.bf16_round(np.stack(pts))[None]
        ref = O.decode_attention(q[i:i + 1].float().numpy(), np.stack(codes)[None], vals[None], cent, perm,
                                 1 / math.sqrt(D), "bf16", "bf16", heavy=heavy, pt_values=pt_all)
        assert_rel(out[i:i + 1], ref, BF16_TOL, f"seq {s}")
    cache.free(9)
    assert 9 not in cache.block_tables
