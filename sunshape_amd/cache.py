"""HuggingFace cache layers for SunShape-compressed keys.

Two layer kinds, selected per layer by ``SunShapeCache``:

* ``SunShapeLayer`` -- the reference's behaviour (sunshape/cache.py:24-46): keys are
  quantised and immediately dequantised through the codec (HIP encode + dequantize
  kernels, bit-exact with the reference's arithmetic) and stored dense, so the
  model's own attention runs unchanged.  A fidelity path: it saves no memory.
* ``SunShapeCodeLayer`` -- stores the codes (uint8, or int16 / int32 past 256 codewords; plus
  compact passthrough values for SunShape-Mixed heavy blocks) and dense values in preallocated, geometrically grown
  buffers, and hands attention a ``SunShapeCodedKeys`` payload instead of a key
  tensor.  The ``"sunshape"`` attention implementation (``register_sunshape_attention``)
  runs single-token decode steps through the fused decode kernel on the codes (fp32
  LUT scores, the vLLM backend's arithmetic, sunshape/vllm_attn_backend.py:216-253) and
  prefill through dequantize + SDPA, which is what the reference's layer computes.
  Keys take nb bytes per token instead of 2*D.

Dense (non-SunShape) layers keep HF's DynamicLayer and are attended by SDPA.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional

import torch
from transformers.cache_utils import DynamicCache, DynamicLayer

from . import hip_ops


def _per_head_arrays(codec):
    return codec.effective_permutation(), codec.centroids


class SunShapeLayer(DynamicLayer):
    """Quantise-dequantise keys through the codec before storing them (sunshape/cache.py:24-46)."""

    def __init__(self, codec=None):
        super().__init__()
        self.codec = codec

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        if self.codec is not None:
            shape, dtype = key_states.shape, key_states.dtype
            n_kv = getattr(self.codec, "num_kv_heads", None)
            if n_kv:  # per-KV-head codecs (extension): one codebook per head
                heads = [self.codec(key_states[:, h].reshape(-1, shape[-1]).float(), kv_head=h).to(dtype)
                         .view(shape[0], shape[2], shape[3]) for h in range(shape[1])]
                key_states = torch.stack(heads, dim=1)
            else:
                flat = key_states.reshape(-1, shape[-1])
                key_states = self.codec(flat.float()).to(dtype).view(shape)
        return super().update(key_states, value_states, *args, **kwargs)


class IdentityLayer(DynamicLayer):
    """Control layer: the SunShapeLayer path with no quantisation (sunshape/cache.py:49-52)."""


@dataclass(frozen=True)
class SunShapeCodedKeys:
    """Keys of one SunShapeCodeLayer as attention sees them: codes [B, Hkv, T, nb] (the codec's index dtype) and
    optional compact passthrough [B, Hkv, T, n_heavy, bd], views of the layer's buffers."""

    codes: torch.Tensor
    passthrough: Optional[torch.Tensor]
    codec: Any
    head_dim: int
    dtype: torch.dtype

    @property
    def shape(self) -> torch.Size:
        b, h, t, _ = self.codes.shape
        return torch.Size((b, h, t, self.head_dim))

    @property
    def device(self) -> torch.device:
        return self.codes.device

    def dequantize(self) -> torch.Tensor:
        """Dense k_hat [B, Hkv, T, D] in the key dtype (what SunShapeLayer stores)."""
        B, Hkv, T, nb = self.codes.shape
        heavy = self.codec.heavy_blocks()
        n_kv = getattr(self.codec, "num_kv_heads", None)
        out = torch.empty((B, Hkv, T, self.head_dim), device=self.codes.device, dtype=self.dtype)
        for h in range(Hkv):
            kv = h if n_kv else None
            perm = self.codec.effective_permutation(kv)
            cent = self.codec.codebook(kv)
            codes = self.codes[:, h].reshape(B * T, nb)
            pt = None
            if heavy is not None:
                pt = self.passthrough[:, h].reshape(B * T, -1, self.passthrough.shape[-1])
            k_hat = hip_ops.dequantize(codes, perm, cent, heavy=heavy, pt=pt, pt_dense=False,
                                       rotation=self.codec.rotation_matrix())
            out[:, h] = k_hat.view(B, T, self.head_dim).to(self.dtype)
        return out


class SunShapeCodeLayer(DynamicLayer):
    """Cache layer that keeps SunShape codes instead of dense keys.

    Buffers grow geometrically (capacity doubles, in multiples of ``block_tokens``), so
    appending a decode token costs one encode launch and one value copy, never a
    re-concatenation of the whole history.
    """

    def __init__(self, codec, *, block_tokens: int = 256, passthrough_dtype: Optional[torch.dtype] = None):
        super().__init__()
        reason = codec.unsupported_reason()
        if reason is not None:
            raise RuntimeError(reason)
        self.codec = codec
        self.block_tokens = int(block_tokens)
        self.passthrough_dtype = passthrough_dtype
        self.heavy = codec.heavy_blocks()
        self._codes = self._pt = self._vals = None
        self._len = 0

    # ----------------------------------------------------------------- storage
    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.dtype, self.device = key_states.dtype, key_states.device
        self.head_dim = key_states.shape[-1]
        self._len = 0
        self.is_initialized = True

    def _reserve(self, B: int, Hkv: int, Dv: int, need: int, vdtype: torch.dtype) -> None:
        cap = 0 if self._codes is None else self._codes.shape[2]
        if self._codes is not None and need <= cap:
            return
        step = self.block_tokens
        new_cap = max(need, 2 * cap)
        new_cap = (new_cap + step - 1) // step * step
        nb, bd = self.codec.n_blocks, self.codec.block_dim
        codes = torch.empty((B, Hkv, new_cap, nb), device=self.device, dtype=hip_ops.index_dtype(self.codec.n_centroids))
        vals = torch.empty((B, Hkv, new_cap, Dv), device=self.device, dtype=vdtype)
        pt = None
        if self.heavy is not None:
            pt = torch.empty((B, Hkv, new_cap, sum(self.heavy), bd), device=self.device,
                             dtype=self.passthrough_dtype or self.dtype)
        if self._len:
            codes[:, :, :self._len] = self._codes[:, :, :self._len]
            vals[:, :, :self._len] = self._vals[:, :, :self._len]
            if pt is not None:
                pt[:, :, :self._len] = self._pt[:, :, :self._len]
        self._codes, self._vals, self._pt = codes, vals, pt

    def _views(self):
        n = self._len
        keys = SunShapeCodedKeys(self._codes[:, :, :n], None if self._pt is None else self._pt[:, :, :n],
                                 self.codec, self.head_dim, self.dtype)
        # HF utilities read .keys/.values shapes (dim -2 = sequence length)
        self.keys = self._codes[:, :, :n]
        self.values = self._vals[:, :, :n]
        return keys, self.values

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        B, Hkv, S, _ = key_states.shape
        if self._codes is not None and (self._codes.shape[0] != B or self._codes.shape[1] != Hkv):
            raise RuntimeError("SunShapeCodeLayer: batch or kv-head count changed between updates")
        self._reserve(B, Hkv, value_states.shape[-1], self._len + S, value_states.dtype)
        lo, hi = self._len, self._len + S
        perm, cent = _per_head_arrays(self.codec)
        # SunShapeLayer quantizes the flattened [B * Hkv * S, D] keys in one cdist (per KV head for
        # per-head codecs), which fixes torch's distance formulation
        rows = B * S if getattr(self.codec, "num_kv_heads", None) else B * Hkv * S
        hip_ops.encode(key_states, perm, cent, heavy=self.heavy, codes_out=self._codes[:, :, lo:hi],
                       pt_out=None if self._pt is None else self._pt[:, :, lo:hi], metric=self.codec.encode_metric(),
                       grid=self.codec.encode_search_grid(cent),
                       direct=hip_ops.cdist_direct(rows, self.codec.n_centroids),
                       rotation=self.codec.rotation_matrix())
        self._vals[:, :, lo:hi] = value_states
        self._len = hi
        return self._views()

    def get_seq_length(self) -> int:
        return self._len if self.is_initialized else 0

    def crop(self, tokens_to_remove: int) -> None:
        if tokens_to_remove > 0:  # legacy form: the absolute length to keep
            tokens_to_remove = max(self._len - tokens_to_remove, 0)
        self._len = max(self._len - abs(tokens_to_remove), 0)
        if self._codes is not None:
            self._views()

    def reset(self) -> None:
        self._len = 0
        if self._codes is not None:
            self._views()

    def _reindex(self, fn) -> None:
        if self._codes is None:
            return
        self._codes, self._vals = fn(self._codes), fn(self._vals)
        if self._pt is not None:
            self._pt = fn(self._pt)
        self._views()

    def batch_repeat_interleave(self, repeats: int) -> None:
        self._reindex(lambda t: t.repeat_interleave(repeats, dim=0))

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        self._reindex(lambda t: t[indices].contiguous())

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        self._reindex(lambda t: t.index_select(0, beam_idx.to(t.device)))

    def offload(self):
        raise NotImplementedError("SunShapeCodeLayer keeps its codes on the GPU")

    def prefetch(self):
        pass


class SunShapeCache(DynamicCache):
    """DynamicCache whose selected layers quantise keys via SunShape codecs (sunshape/cache.py:55-106).

    ``store_codes=False`` (default) mirrors the reference: selected layers become
    ``SunShapeLayer`` (quantise-dequantise, dense storage).  ``store_codes=True`` makes them
    ``SunShapeCodeLayer``; the model must then use the ``"sunshape"`` attention
    implementation (``register_sunshape_attention``).
    """

    def __init__(self, config=None, num_layers: int | None = None, layer_codecs: dict[int, Any] | None = None,
                 identity_layers: set[int] | None = None, *, store_codes: bool = False, **kwargs):
        if config is not None:
            kwargs["config"] = config
        super().__init__(**kwargs)
        layer_codecs = layer_codecs or {}
        identity_layers = identity_layers or set()
        if len(self.layers) == 0:
            if num_layers is None:
                raise ValueError("Must provide either config or num_layers")
            for _ in range(num_layers):
                self.layers.append(DynamicLayer())
        self.store_codes = bool(store_codes)
        for i in range(len(self.layers)):
            sliding = getattr(self.layers[i], "sliding_window", None)
            if i in layer_codecs:
                codec = layer_codecs[i]
                new_layer = SunShapeCodeLayer(codec) if self.store_codes else SunShapeLayer(codec=codec)
            elif i in identity_layers:
                new_layer = IdentityLayer()
            else:
                continue
            if sliding is not None:
                # As the reference's layer (sunshape/cache.py:86-104): every token is kept and HF's
                # sliding-window mask limits attention (the code layer's attention takes that mask).
                new_layer.sliding_window = sliding
            self.layers[i] = new_layer

    @classmethod
    def from_codecs(cls, codecs_dict: dict[int, Any], config=None, num_layers: int | None = None, *,
                    store_codes: bool = False) -> "SunShapeCache":
        """Cache with pre-fitted codecs for specific layers (sunshape/cache.py:110-118)."""
        return cls(config=config, num_layers=num_layers, layer_codecs=codecs_dict, store_codes=store_codes)

    @classmethod
    def identity(cls, patched_layers: list[int], config=None, num_layers: int | None = None) -> "SunShapeCache":
        """Identity-only control cache (sunshape/cache.py:120-134)."""
        return cls(config=config, num_layers=num_layers, identity_layers=set(patched_layers))

    @classmethod
    def from_traces(cls, *args, **kwargs) -> "SunShapeCache":
        """Fitting codecs from traces is offline calibration (sunshape/cache.py:136-186), not in this package."""
        raise NotImplementedError(
            "SunShapeCache.from_traces fits codecs (offline calibration); fit them with the reference "
            "package and load them with sunshape_amd.hf.SunShapeBundle, then use SunShapeCache.from_codecs")

    def has_previous_state(self, layer_idx: int | None = None) -> bool:
        """Required by hybrid models in newer transformers versions (sunshape/cache.py:188-190)."""
        return self.get_seq_length() > 0


# ---------------------------------------------------------------------------- attention
# multi-token steps take the fused decode up to this many query rows per KV head; longer ones attend
# dequantized keys.  16 is the row count the head_dim-64 contiguous MFMA kernel holds in one pass.
# At head_dim 128 with 128-dim values the step runs on the contiguous LUT kernel or, with more rows
# than its LUT holds, with passthrough blocks (at most 16 dims) or both, on the 4x4-MFMA kernel (16
# rows per pass); the fused decode measured faster than dequantize + SDPA up to 256 rows per KV
# head there (B4 · 32/8 heads · T16384: 1.07 against 2.09 ms at 64 new tokens, LUT kernel).
_FUSED_MAX_ROWS = 16
_FUSED_MAX_ROWS_128 = 256


def _additive_mask(mask: Optional[torch.Tensor], dtype=torch.float32) -> Optional[torch.Tensor]:
    if mask is None:
        return None
    if mask.dtype == torch.bool:
        zero = torch.zeros((), device=mask.device, dtype=dtype)
        return torch.where(mask, zero, torch.full((), float("-inf"), device=mask.device, dtype=dtype))
    return mask.to(dtype)


def sunshape_attention_forward(module: torch.nn.Module, query: torch.Tensor, key, value: torch.Tensor,
                               attention_mask: Optional[torch.Tensor], dropout: float = 0.0,
                               scaling: Optional[float] = None, is_causal: Optional[bool] = None, **kwargs):
    """HF attention implementation for caches holding SunShapeCodedKeys.

    query [B, Hq, Lq, D]; key a SunShapeCodedKeys (codes) or a dense tensor; value
    [B, Hkv, T, Dv].  Returns (attn_output [B, Lq, Hq, Dv], None) like HF's SDPA function.
    """
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    if not isinstance(key, SunShapeCodedKeys):
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                      scaling=scaling, is_causal=is_causal, **kwargs)
    if dropout:
        raise RuntimeError("SunShape attention over coded keys does not implement dropout")
    if kwargs.get("output_attentions", False):
        raise RuntimeError("SunShape attention over coded keys does not return attention weights")
    B, Hq, Lq, D = query.shape
    T = key.codes.shape[2]
    rows = (Hq // value.shape[1]) * Lq  # query rows per KV head
    heavy = key.codec.heavy_blocks()
    pt_dims = 0 if heavy is None else sum(heavy) * key.codec.block_dim
    fused128 = D == 128 and value.shape[-1] == 128 and pt_dims <= 16
    if Lq == 1 or (T > Lq and rows <= (_FUSED_MAX_ROWS_128 if fused128 else _FUSED_MAX_ROWS)):
        # a decode step, or a short multi-token step over a filled cache (speculative verification,
        # small chunks): the fused decode over the codes, masked as HF's mask builder says, or without
        # a mask causally (the new tokens being the last Lq positions) when the call is causal, as
        # HF's SDPA function decides it (is_causal, else the module's is_causal, else causal)
        mask = _additive_mask(attention_mask)
        causal = is_causal if is_causal is not None else getattr(module, "is_causal", True)
        if mask is not None:
            mask = mask[..., -T:]
        elif Lq > 1 and causal:
            pos = torch.arange(T, device=query.device)
            last = T - Lq + torch.arange(Lq, device=query.device)
            mask = torch.zeros(1, 1, Lq, T, device=query.device).masked_fill(pos[None, :] > last[:, None],
                                                                              float("-inf"))
        if scaling is None:  # SDPA's default scale
            scaling = 1.0 / D ** 0.5
        perm, cent = _per_head_arrays(key.codec)
        out = hip_ops.decode(query, key.codes, value, perm, cent, scale=scaling, mask=mask,
                             heavy=key.codec.heavy_blocks(), pt=key.passthrough, pt_dense=False,
                             rotation=key.codec.rotation_matrix())
        return out.transpose(1, 2).contiguous(), None
    # prefill / long multi-token step: dense k_hat in the key dtype, as the reference's cache layer stores
    return sdpa_attention_forward(module, query, key.dequantize(), value, attention_mask, dropout=0.0,
                                  scaling=scaling, is_causal=is_causal, **kwargs)


def register_sunshape_attention(name: str = "sunshape") -> str:
    """Register ``name`` as a transformers attention implementation (with SDPA's mask builder).

    Use ``model.set_attn_implementation(name)`` (or ``attn_implementation=name`` at load).
    """
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

    AttentionInterface.register(name, sunshape_attention_forward)
    AttentionMaskInterface.register(name, sdpa_mask)
    return name


__all__ = ["SunShapeCache", "SunShapeLayer", "IdentityLayer", "SunShapeCodeLayer", "SunShapeCodedKeys",
           "sunshape_attention_forward", "register_sunshape_attention"]
