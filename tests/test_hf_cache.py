"""HF cache surface on the CPU (sunshape/cache.py:24-190): layer selection, constructors,
and the "sunshape" attention implementation delegating dense layers to SDPA unchanged."""

import pytest
import torch

from sunshape_amd import synthetic
from sunshape_amd.cache import (IdentityLayer, SunShapeCache, SunShapeCodeLayer, SunShapeLayer,
                                register_sunshape_attention)
from sunshape_amd.codec import SunShapeBlockCodec

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig, LlamaForCausalLM  # noqa: E402
from transformers.cache_utils import DynamicLayer  # noqa: E402


def _cfg(layers=3):
    return LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=32, max_position_embeddings=128)


def _codec():
    cb = synthetic.make_codebook(1, 32, 4, 5)
    return SunShapeBlockCodec.from_buffers(cb.perm[0], cb.centroids[0], device="cpu")


def test_layer_selection_mirrors_reference():
    c = _codec()
    cache = SunShapeCache(num_layers=4, layer_codecs={1: c, 3: c}, identity_layers={2})
    kinds = [type(l) for l in cache.layers]
    assert kinds == [DynamicLayer, SunShapeLayer, IdentityLayer, SunShapeLayer]
    assert cache.layers[1].codec is c
    coded = SunShapeCache.from_codecs({0: c}, num_layers=2, store_codes=True)
    assert isinstance(coded.layers[0], SunShapeCodeLayer) and type(coded.layers[1]) is DynamicLayer
    ident = SunShapeCache.identity([0], num_layers=2)
    assert isinstance(ident.layers[0], IdentityLayer)
    with_cfg = SunShapeCache(config=_cfg(3), layer_codecs={2: c})
    assert len(with_cfg.layers) == 3 and isinstance(with_cfg.layers[2], SunShapeLayer)
    with pytest.raises(ValueError, match="num_layers"):
        SunShapeCache()
    with pytest.raises(NotImplementedError):
        SunShapeCache.from_traces({}, [0])
    assert not cache.has_previous_state()
    assert coded.layers[0].get_seq_length() == 0


def test_code_layer_rejects_codecs_the_kernels_cannot_serve():
    wide = SunShapeBlockCodec(head_dim=32, block_dim=4, n_centroids=4096, device="cpu")
    assert SunShapeCodeLayer(wide).codec is wide  # 16-bit codes (the reference's int16 indices)
    huge = SunShapeBlockCodec(head_dim=4, block_dim=4, n_centroids=(1 << 20) + 1, device="cpu")
    with pytest.raises(RuntimeError, match="2\\^20"):
        SunShapeCodeLayer(huge)
    rot = SunShapeBlockCodec(head_dim=32, block_dim=4, use_rotation=True, device="cpu")
    assert SunShapeCodeLayer(rot).codec is rot  # rotated codecs run on the kernels


def test_sunshape_attention_delegates_dense_layers_exactly():
    cfg = _cfg(2)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    ids = torch.randint(0, 256, (2, 10))
    with torch.no_grad():
        model.set_attn_implementation("sdpa")
        ref_cache = SunShapeCache(config=cfg)
        ref = model(ids, past_key_values=ref_cache).logits
        nxt = ref[:, -1:].argmax(-1)
        ref2 = model(nxt, past_key_values=ref_cache).logits
        model.set_attn_implementation(register_sunshape_attention())
        cache = SunShapeCache(config=cfg)
        out = model(ids, past_key_values=cache).logits
        out2 = model(nxt, past_key_values=cache).logits
    assert torch.equal(out, ref) and torch.equal(out2, ref2)
    assert cache.has_previous_state() and cache.get_seq_length() == 11


def test_bundle_make_cache():
    """SunShapeBundle.make_cache (sunshape/hf.py:267-268): the bundle's codecs on their layers, in the
    reference's dequantising cache or, with store_codes, the code-storing one."""
    from sunshape_amd.hf import SunShapeBundle

    c = _codec()
    bundle = SunShapeBundle("m", [1], 2.0, 4, "profileperm_baseline", 0, 0, 0, {1: c})
    cache = bundle.make_cache(config=_cfg(3))
    assert [type(l) for l in cache.layers] == [DynamicLayer, SunShapeLayer, DynamicLayer]
    assert cache.layers[1].codec is c
    coded = bundle.make_cache(num_layers=2, store_codes=True)
    assert isinstance(coded.layers[1], SunShapeCodeLayer) and coded.layers[1].codec is c


def test_sliding_window_layers_keep_their_window():
    """Sliding-window layers become SunShape layers with the window copied (sunshape/cache.py:86-104),
    for the code-storing cache too: every token is kept and HF's sliding mask limits attention."""
    from transformers import MistralConfig

    cfg = MistralConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                        num_attention_heads=4, num_key_value_heads=2, head_dim=32, max_position_embeddings=128,
                        sliding_window=16)
    c = _codec()
    for store in (False, True):
        cache = SunShapeCache(config=cfg, layer_codecs={0: c}, store_codes=store)
        assert isinstance(cache.layers[0], SunShapeCodeLayer if store else SunShapeLayer)
        assert cache.layers[0].sliding_window == 16 and cache.layers[1].sliding_window == 16
