"""HF cache layers on the GPU: the reference-mirroring quantise-dequantise layer bit-exact
against the oracle, the code-storing layer's encode/growth/decode against the oracle, and a
tiny random Llama stepping through both caches."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import synthetic
from sunshape_amd.cache import (SunShapeCache, SunShapeCodedKeys, SunShapeCodeLayer, SunShapeLayer,
                                register_sunshape_attention, sunshape_attention_forward)
from sunshape_amd.codec import SunShapeBlockCodec

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _codec(D=64, bd=4, seed=3, mixed=False, per_head=0):
    cb = synthetic.make_codebook(max(per_head, 1), D, bd, seed, shared_sigma=mixed)
    if mixed:
        heavy = synthetic.heavy_blocks_by_sigma(cb.sigma[0], cb.perm[0], bd, 3)
        cent = cb.centroids[0].clone()
        cent[heavy] = 0
        return SunShapeBlockCodec.from_buffers(cb.perm[0], cent, mode="profileperm_mixed_precision",
                                               mixed_high_precision_blocks=heavy, device=DEV), cb.sigma[0]
    if per_head:
        return SunShapeBlockCodec.from_buffers(cb.perm, cb.centroids, device=DEV), cb.sigma[0]
    return SunShapeBlockCodec.from_buffers(cb.perm[0], cb.centroids[0], device=DEV), cb.sigma[0]


def _oracle_codes(codec, keys_f32, h=None):
    """Oracle encode of keys [N, D] with the codec (head h for per-head codecs)."""
    perm = codec.effective_permutation(h).cpu().numpy()
    cent = codec.codebook(h).cpu().numpy()
    heavy = codec.heavy_blocks()
    return O.encode(keys_f32, perm, cent, None if heavy is None else np.array(heavy))


@pytest.mark.parametrize("kind", ["shared", "mixed", "per_head"])
def test_sunshape_layer_is_quantize_dequantize(kind):
    """sunshape/cache.py:35-46: stored keys = codec(keys.float()).to(dtype), bit-exact."""
    log(f"SunShapeLayer {kind}")
    codec, sigma = _codec(mixed=kind == "mixed", per_head=2 if kind == "per_head" else 0)
    B, Hkv, S, D = 2, 2, 70, 64
    keys = (torch.randn(B, Hkv, S, D, generator=torch.Generator().manual_seed(1)) * sigma).to(torch.bfloat16)
    vals = torch.randn(B, Hkv, S, D).to(torch.bfloat16)
    layer = SunShapeLayer(codec)
    k_out, v_out = layer.update(keys.to(DEV), vals.to(DEV))
    assert torch.equal(v_out.cpu(), vals)
    for h in range(Hkv):
        hh = h if kind == "per_head" else None
        flat = keys[:, h].reshape(-1, D).float().numpy()
        codes, pt = _oracle_codes(codec, flat, hh)
        heavy = codec.heavy_blocks()
        ref = O.dequantize(codes, codec.codebook(hh).cpu().numpy(), codec.effective_permutation(hh).cpu().numpy(),
                           None if heavy is None else np.array(heavy), pt)
        got = k_out[:, h].reshape(-1, D).float().cpu().numpy()
        assert np.array_equal(got, O.bf16_round(ref))


def test_code_layer_append_growth_and_decode():
    """Prefill 300 tokens then single-token appends across the 256 -> 512 capacity step."""
    log("SunShapeCodeLayer growth")
    codec, sigma = _codec(mixed=True, bd=2)
    B, Hkv, Hq, D = 2, 2, 8, 64
    layer = SunShapeCodeLayer(codec, block_tokens=256)
    g = torch.Generator().manual_seed(5)
    hist_k, hist_v = [], []
    for S in [300] + [1] * 3:
        k = (torch.randn(B, Hkv, S, D, generator=g) * sigma).to(torch.bfloat16)
        v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
        keys, values = layer.update(k.to(DEV), v.to(DEV))
        hist_k.append(k)
        hist_v.append(v)
    assert isinstance(keys, SunShapeCodedKeys) and keys.shape == (B, Hkv, 303, D)
    assert layer.get_seq_length() == 303 and layer._codes.shape[2] == 512
    allk = torch.cat(hist_k, 2).float().numpy()
    allv = torch.cat(hist_v, 2)
    assert torch.equal(values.cpu(), allv)
    heavy = np.array(codec.heavy_blocks())
    enc = [[_oracle_codes(codec, allk[b, h]) for h in range(Hkv)] for b in range(B)]
    codes_ref = np.stack([np.stack([e[0] for e in row]) for row in enc])
    assert np.array_equal(np_of(keys.codes), codes_ref)
    # the layer keeps passthrough values compact ([.., n_heavy, bd]) in the key dtype
    pt_ref = O.bf16_round(np.stack([np.stack([e[1] for e in row]) for row in enc]))   # dense [B, Hkv, T, nb, bd]
    assert np.array_equal(np_of(keys.passthrough).astype(np.float32), pt_ref[:, :, :, heavy])
    # decode step through the registered attention function vs the oracle's decode
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    mod = torch.nn.Module()
    mod.num_key_value_groups = Hq // Hkv
    out, w = sunshape_attention_forward(mod, q.to(DEV), keys, values, None, scaling=1 / math.sqrt(D))
    assert w is None and out.shape == (B, 1, Hq, D)
    ref = O.decode_attention(q.float().numpy(), codes_ref, allv.float().numpy(), codec.centroids.cpu().numpy(),
                             codec.permutation.cpu().numpy(), 1 / math.sqrt(D), "bf16", "bf16", heavy=heavy,
                             pt_values=pt_ref)
    assert_rel(np_of(out.transpose(1, 2)), ref, BF16_TOL, "code-layer decode")
    # a boolean padding mask (first 5 keys of batch 1 masked) as HF's SDPA mask builder makes it
    keep = torch.ones(B, 1, 1, 303, dtype=torch.bool)
    keep[1, :, :, :5] = False
    out_m, _ = sunshape_attention_forward(mod, q.to(DEV), keys, values, keep.to(DEV), scaling=1 / math.sqrt(D))
    add = np.broadcast_to(np.where(keep.numpy(), 0.0, -np.inf).astype(np.float32), (B, Hq, 1, 303))
    ref_m = O.decode_attention(q.float().numpy(), codes_ref, allv.float().numpy(), codec.centroids.cpu().numpy(),
                               codec.permutation.cpu().numpy(), 1 / math.sqrt(D), "bf16", "bf16", heavy=heavy,
                               pt_values=pt_ref, mask=add)
    assert_rel(np_of(out_m.transpose(1, 2)), ref_m, BF16_TOL, "code-layer decode masked")
    # a 3-token step (speculative verification) without a mask: the fused decode, the new tokens
    # being the last 3 positions (token i sees keys up to 300 + i)
    q3 = torch.randn(B, Hq, 3, D, generator=g).to(torch.bfloat16)
    out3, _ = sunshape_attention_forward(mod, q3.to(DEV), keys, values, None, scaling=1 / math.sqrt(D))
    causal = np.where(np.arange(303)[None, :] > (300 + np.arange(3))[:, None], -np.inf, 0.0).astype(np.float32)
    ref3 = O.decode_attention(q3.float().numpy(), codes_ref, allv.float().numpy(), codec.centroids.cpu().numpy(),
                              codec.permutation.cpu().numpy(), 1 / math.sqrt(D), "bf16", "bf16", heavy=heavy,
                              pt_values=pt_ref, mask=np.broadcast_to(causal, (B, Hq, 3, 303)))
    assert_rel(np_of(out3.transpose(1, 2)), ref3, BF16_TOL, "code-layer 3-token step")
    layer.crop(-3)
    assert layer.get_seq_length() == 300
    layer.reorder_cache(torch.tensor([1, 0], device=DEV))
    assert torch.equal(layer.keys[0], keys.codes[1, :, :300])


def test_code_layer_head_dim_128_multi_token_step():
    """At head_dim 128 (128-dim values, no passthrough blocks) a multi-token step of 8 new tokens
    at 4 query heads per KV head (32 rows per KV head, past the head_dim-64 limit of 16) takes the
    fused decode with a causal mask; it matches the oracle."""
    log("SunShapeCodeLayer head_dim 128, 8-token step")
    codec, sigma = _codec(D=128, bd=4, seed=11)
    B, Hkv, Hq, D, S, L = 2, 2, 8, 128, 200, 8
    layer = SunShapeCodeLayer(codec, block_tokens=256)
    g = torch.Generator().manual_seed(12)
    k = (torch.randn(B, Hkv, S, D, generator=g) * sigma).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    keys, values = layer.update(k.to(DEV), v.to(DEV))
    kf = k.float().numpy()
    codes_ref = np.stack([np.stack([_oracle_codes(codec, kf[b, h])[0] for h in range(Hkv)]) for b in range(B)])
    assert np.array_equal(np_of(keys.codes), codes_ref)
    q = torch.randn(B, Hq, L, D, generator=g).to(torch.bfloat16)
    mod = torch.nn.Module()
    mod.num_key_value_groups = Hq // Hkv
    out, _ = sunshape_attention_forward(mod, q.to(DEV), keys, values, None, scaling=1 / math.sqrt(D))
    causal = np.where(np.arange(S)[None, :] > (S - L + np.arange(L))[:, None], -np.inf, 0.0).astype(np.float32)
    ref = O.decode_attention(q.float().numpy(), codes_ref, v.float().numpy(), codec.centroids.cpu().numpy(),
                             codec.permutation.cpu().numpy(), 1 / math.sqrt(D), "bf16", "bf16",
                             mask=np.broadcast_to(causal, (B, Hq, L, S)))
    assert_rel(np_of(out.transpose(1, 2)), ref, BF16_TOL, "head_dim-128 8-token step")


def test_tiny_llama_code_cache_tracks_dequant_cache():
    """Prefill through the code cache is bit-identical to the reference-mirroring cache (both attend
    bf16 k_hat); decode steps and a 3-token step use the fused decode and stay within bf16
    tolerance of it."""
    from transformers import LlamaConfig, LlamaForCausalLM

    log("tiny llama code cache")
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=32, max_position_embeddings=256)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to(DEV, torch.bfloat16).eval()
    codecs = {0: _codec(D=32, bd=4, seed=8)[0], 1: _codec(D=32, bd=2, seed=9)[0]}
    ids = torch.randint(0, 512, (2, 40), generator=torch.Generator().manual_seed(2)).to(DEV)
    steps = torch.randint(0, 512, (2, 4), generator=torch.Generator().manual_seed(3)).to(DEV)
    multi = torch.randint(0, 512, (2, 3), generator=torch.Generator().manual_seed(4)).to(DEV)
    with torch.no_grad():
        model.set_attn_implementation("sdpa")
        ref_cache = SunShapeCache.from_codecs(codecs, config=cfg)
        ref_logits = [model(ids, past_key_values=ref_cache).logits]
        for i in range(steps.shape[1]):
            ref_logits.append(model(steps[:, i:i + 1], past_key_values=ref_cache).logits)
        ref_logits.append(model(multi, past_key_values=ref_cache).logits)  # a 3-token step
        model.set_attn_implementation(register_sunshape_attention())
        cache = SunShapeCache.from_codecs(codecs, config=cfg, store_codes=True)
        logits = [model(ids, past_key_values=cache).logits]
        for i in range(steps.shape[1]):
            logits.append(model(steps[:, i:i + 1], past_key_values=cache).logits)
        logits.append(model(multi, past_key_values=cache).logits)  # fused decode, 12 rows per KV head
    assert isinstance(cache.layers[0], SunShapeCodeLayer) and cache.get_seq_length() == 47
    assert torch.equal(logits[0], ref_logits[0])
    for a, r in zip(logits[1:], ref_logits[1:]):
        assert_rel(a.float().cpu().numpy(), r.float().cpu().numpy(), 3e-2, "decode logits")


def test_code_layer_multi_token_step_not_causal_and_default_scale():
    """A multi-token step with no mask attends causally only when the call is causal (is_causal, else the
    module's is_causal), as HF's SDPA function decides; scaling=None is SDPA's 1/sqrt(head_dim)."""
    log("SunShapeCodeLayer is_causal=False, scaling=None")
    codec, sigma = _codec(D=64, bd=4, seed=13)
    B, Hkv, Hq, D, S, L = 2, 2, 8, 64, 120, 3
    layer = SunShapeCodeLayer(codec, block_tokens=256)
    g = torch.Generator().manual_seed(14)
    k = (torch.randn(B, Hkv, S, D, generator=g) * sigma).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    keys, values = layer.update(k.to(DEV), v.to(DEV))
    kf = k.float().numpy()
    codes_ref = np.stack([np.stack([_oracle_codes(codec, kf[b, h])[0] for h in range(Hkv)]) for b in range(B)])
    q = torch.randn(B, Hq, L, D, generator=g).to(torch.bfloat16)
    args = (q.float().numpy(), codes_ref, v.float().numpy(), codec.centroids.cpu().numpy(),
            codec.permutation.cpu().numpy(), 1 / math.sqrt(D), "bf16", "bf16")
    full = O.decode_attention(*args)
    causal = np.where(np.arange(S)[None, :] > (S - L + np.arange(L))[:, None], -np.inf, 0.0).astype(np.float32)
    ref_causal = O.decode_attention(*args, mask=np.broadcast_to(causal, (B, Hq, L, S)))
    mod = torch.nn.Module()
    mod.num_key_value_groups = Hq // Hkv
    out, _ = sunshape_attention_forward(mod, q.to(DEV), keys, values, None, scaling=None, is_causal=False)
    assert_rel(np_of(out.transpose(1, 2)), full, BF16_TOL, "is_causal=False")
    mod.is_causal = False
    out, _ = sunshape_attention_forward(mod, q.to(DEV), keys, values, None)
    assert_rel(np_of(out.transpose(1, 2)), full, BF16_TOL, "module.is_causal=False")
    mod.is_causal = True
    out, _ = sunshape_attention_forward(mod, q.to(DEV), keys, values, None)
    assert_rel(np_of(out.transpose(1, 2)), ref_causal, BF16_TOL, "module.is_causal=True")


def test_tiny_sliding_window_code_cache_tracks_dequant_cache():
    """Sliding-window layers (a tiny Mistral, window 16): both SunShape caches keep every token, as the
    reference's layer does (sunshape/cache.py:86-104), and HF's sliding mask limits attention.  The code
    cache's prefill equals the dequantising cache's bit for bit, and its decode steps (47 tokens, past the
    window: the mask is what keeps them equal) track it within bf16 tolerance."""
    from transformers import MistralConfig, MistralForCausalLM

    from sunshape_amd.hf import SunShapeBundle

    log("tiny mistral sliding-window code cache")
    cfg = MistralConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                        num_attention_heads=8, num_key_value_heads=2, head_dim=32, max_position_embeddings=256,
                        sliding_window=16)
    torch.manual_seed(0)
    model = MistralForCausalLM(cfg).to(DEV, torch.bfloat16).eval()
    codecs = {0: _codec(D=32, bd=4, seed=18)[0], 1: _codec(D=32, bd=2, seed=19)[0]}
    bundle = SunShapeBundle("tiny-mistral", [0, 1], 2.0, 4, "profileperm_baseline", 0, 0, 0, codecs)
    ids = torch.randint(0, 512, (2, 40), generator=torch.Generator().manual_seed(6)).to(DEV)
    steps = torch.randint(0, 512, (2, 5), generator=torch.Generator().manual_seed(7)).to(DEV)
    with torch.no_grad():
        model.set_attn_implementation("sdpa")
        ref_cache = bundle.make_cache(config=cfg)
        ref_logits = [model(ids, past_key_values=ref_cache).logits]
        for i in range(steps.shape[1]):
            ref_logits.append(model(steps[:, i:i + 1], past_key_values=ref_cache).logits)
        model.set_attn_implementation(register_sunshape_attention())
        cache = bundle.make_cache(config=cfg, store_codes=True)
        logits = [model(ids, past_key_values=cache).logits]
        for i in range(steps.shape[1]):
            logits.append(model(steps[:, i:i + 1], past_key_values=cache).logits)
    assert isinstance(cache.layers[0], SunShapeCodeLayer) and cache.layers[0].sliding_window == 16
    assert cache.layers[0].get_seq_length() == 45 and cache.layers[1].get_seq_length() == 45
    assert torch.equal(logits[0], ref_logits[0])
    for a, r in zip(logits[1:], ref_logits[1:]):
        assert_rel(a.float().cpu().numpy(), r.float().cpu().numpy(), 3e-2, "decode logits")
