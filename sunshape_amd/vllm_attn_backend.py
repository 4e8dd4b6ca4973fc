"""SunShape attention backend shim (drop-in for ``sunshape.vllm_attn_backend``).

Same surface as sunshape/vllm_attn_backend.py: mode toggles, handle/runtime
registration globals, ``SunShapeQuantizedKeys``, ``quantize_key_states``,
``SunShapeAttentionImpl.forward`` and the backend factory.  The quantized fast
path is one fused HIP launch over every (batch, KV head) instead of the
reference's Python loop (:230-252).

Differences by design:
* ``SunShapeQuantizedKeys`` may carry the batched code tensor it was built from
  (``codes`` [B, Hkv, S, nb]) and the passthrough values of SunShape-Mixed codecs
  in the compact layout (``passthrough`` [B, Hkv, S, n_heavy, bd] in the key dtype:
  the reference's dense fp32 [S, nb, bd] holds ``keys.float()`` on heavy blocks and
  zeros elsewhere, so the compact values are the same numbers in 1/8-1/32 of the
  bytes).  The per-head view ``quantized_heads`` still yields the reference's
  ``SunShapeQuantized`` payloads, each built (with its dense fp32 passthrough) when
  it is read.
* A causal call with several query rows over a quantized payload runs the fused
  kernel from the codes with the mask and scale the reference's SDPA route applies
  (:306-345); any other payload that fails the fast-path gate is dequantized in
  one batched launch and handed to the delegate or SDPA as in the reference.
"""

from __future__ import annotations

import math

import os
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn.functional as F

from . import hip_ops
from .codec import SunShapeQuantized
from .integration.vllm import SunShapeVLLMConfig, SunShapeVLLMHandle, SunShapeVLLMRuntimeState, install_hooks

MODE_ACTIVE = "active"
MODE_CAPTURE = "capture"
MODE_OFF = "off"

_MODE = MODE_OFF
_ACTIVE_HANDLE: SunShapeVLLMHandle | None = None
_RUNTIME_STATE: SunShapeVLLMRuntimeState | None = None


class _HeadPayloads(Sequence):
    """The per-(batch, KV head) ``SunShapeQuantized`` payloads of one batched encode, index
    ``b * Hkv + h`` (the reference's tuple order, sunshape/vllm_attn_backend.py:112-123).  Each is
    built when read: indices are a view of the batched codes, and a SunShape-Mixed payload's
    passthrough_values the reference's dense fp32 [S, nb, bd] (zeros on light blocks) expanded from
    the compact values."""

    def __init__(self, codes: torch.Tensor, passthrough: torch.Tensor | None, passthrough_blocks: torch.Tensor | None,
                 head_dim: int, block_dim: int, n_blocks: int):
        self._codes = codes
        self._pt = passthrough
        self._pblocks = passthrough_blocks
        self._dims = (int(head_dim), int(block_dim), int(n_blocks))
        self._hkv = int(codes.shape[1])

    def __len__(self) -> int:
        return int(self._codes.shape[0]) * self._hkv

    def __getitem__(self, i):
        if isinstance(i, slice):
            return tuple(self[j] for j in range(*i.indices(len(self))))
        n = len(self)
        if not -n <= i < n:
            raise IndexError("quantized head index out of range")
        b, h = divmod(i % n, self._hkv)
        head_dim, block_dim, n_blocks = self._dims
        dense = None
        if self._pt is not None:
            heavy = self._pblocks.to(self._pt.device, torch.bool)
            dense = torch.zeros(self._codes.shape[2], n_blocks, block_dim, device=self._pt.device, dtype=torch.float32)
            dense[:, heavy] = self._pt[b, h].float()
        return SunShapeQuantized(indices=self._codes[b, h], head_dim=head_dim, block_dim=block_dim, n_blocks=n_blocks,
                                 passthrough_blocks=None if self._pblocks is None else self._pblocks.clone(),
                                 passthrough_values=dense)


@dataclass(frozen=True)
class SunShapeQuantizedKeys:
    """Per-head quantized key cache payload (sunshape/vllm_attn_backend.py:38-53)."""

    quantized_heads: tuple[Any, ...]
    batch_size: int
    num_kv_heads: int
    seq_len: int
    codes: torch.Tensor | None = None          # [B, Hkv, S, nb] backing store (the codec's index dtype)
    passthrough: torch.Tensor | None = None    # [B, Hkv, S, slots, bd]
    passthrough_dense: bool = False

    def head(self, batch_idx: int, kv_head_idx: int) -> Any:
        return self.quantized_heads[batch_idx * self.num_kv_heads + kv_head_idx]

    def batched(self) -> tuple[torch.Tensor, torch.Tensor | None, bool]:
        """(codes [B, Hkv, S, nb], passthrough or None, dense flag), stacking the heads if needed."""
        if self.codes is not None:
            return self.codes, self.passthrough, self.passthrough_dense
        heads = self.quantized_heads
        codes = torch.stack([h.indices for h in heads]).reshape(self.batch_size, self.num_kv_heads, self.seq_len, -1)
        if codes.dtype not in (torch.uint8, torch.int16, torch.int32):  # the reference's compact index dtypes
            codes = codes.to(torch.uint8)
        pt = None
        if heads and getattr(heads[0], "passthrough_values", None) is not None:
            pt = torch.stack([h.passthrough_values for h in heads])
            pt = pt.reshape(self.batch_size, self.num_kv_heads, self.seq_len, *pt.shape[-2:])
        return codes, pt, True


def set_mode(mode: str):
    global _MODE
    _MODE = mode


def get_mode() -> str:
    return _MODE


def register_handle(handle: SunShapeVLLMHandle) -> SunShapeVLLMHandle:
    global _ACTIVE_HANDLE
    _ACTIVE_HANDLE = handle
    set_mode(MODE_ACTIVE)
    return handle


def register_runtime_state(state: SunShapeVLLMRuntimeState) -> SunShapeVLLMRuntimeState:
    global _RUNTIME_STATE
    _RUNTIME_STATE = state
    set_mode(MODE_ACTIVE)
    return state


def clear_registered_handle() -> None:
    global _ACTIVE_HANDLE
    _ACTIVE_HANDLE = None
    if _RUNTIME_STATE is None:
        set_mode(MODE_OFF)


def clear_registered_runtime() -> None:
    global _RUNTIME_STATE
    _RUNTIME_STATE = None
    if _ACTIVE_HANDLE is None:
        set_mode(MODE_OFF)


def get_registered_handle() -> SunShapeVLLMHandle | None:
    return _ACTIVE_HANDLE


def get_registered_runtime() -> SunShapeVLLMRuntimeState | None:
    return _RUNTIME_STATE


def _codec_head_arrays(codec, num_kv_heads: int):
    """(perm, centroids) for hip_ops: shared [D]/[nb,nc,bd] or per-KV-head [Hkv, ...]."""
    perm = codec.effective_permutation() if hasattr(codec, "effective_permutation") else codec.permutation
    cent = codec.centroids
    if cent.ndim == 4 and cent.shape[0] != num_kv_heads:
        raise RuntimeError(f"codec holds {cent.shape[0]} KV-head codebooks, keys have {num_kv_heads} KV heads")
    return perm, cent


def quantize_key_states(layer_idx: int, key_states: torch.Tensor) -> SunShapeQuantizedKeys:
    """Encode [B, Hkv, S, D] keys in one HIP launch (sunshape/vllm_attn_backend.py:101-123)."""
    runtime = get_registered_runtime()
    if runtime is None:
        raise RuntimeError("SunShape runtime state is not registered.")
    codec = runtime.codec_for_layer(int(layer_idx))
    if codec is None:
        raise RuntimeError(f"No SunShape codec is registered for layer {layer_idx}.")
    if key_states.ndim != 4:
        raise RuntimeError(
            "quantize_key_states expects key_states with shape [batch, kv_heads, seq_len, head_dim]."
        )
    reason = codec.unsupported_reason()
    if reason is not None:
        raise RuntimeError(reason)
    batch_size, num_kv_heads, seq_len, _ = key_states.shape
    perm, cent = _codec_head_arrays(codec, num_kv_heads)
    heavy = codec.heavy_blocks()
    keys = key_states.to(codec.device)
    if keys.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        keys = keys.float()
    metric = codec.encode_metric() if hasattr(codec, "encode_metric") else None
    grid = codec.encode_search_grid(cent) if hasattr(codec, "encode_search_grid") else None
    rot = codec.rotation_matrix() if hasattr(codec, "rotation_matrix") else None
    # Passthrough values compact [B, Hkv, S, n_heavy, bd] in the key dtype: the reference stores
    # keys.float() there (sunshape/codec.py:368-372), which the key dtype holds exactly.  Under a
    # rotation they are transformed values, kept in fp32.
    pt_dtype = torch.float32 if rot is not None else keys.dtype
    # the reference quantizes one (batch, KV head) per call: seq_len keys per cdist
    codes, pt = hip_ops.encode(keys, perm, cent, heavy=heavy, pt_dtype=pt_dtype, pt_dense=False, metric=metric,
                               grid=grid, direct=hip_ops.cdist_direct(seq_len, cent.shape[-2]), rotation=rot)
    mixed = codec.mode == "profileperm_mixed_precision"
    pblocks = codec.mixed_high_precision_blocks.detach().clone() if mixed else None
    return SunShapeQuantizedKeys(
        quantized_heads=_HeadPayloads(codes, pt, pblocks, codec.head_dim, codec.block_dim, codec.n_blocks),
        batch_size=int(batch_size),
        num_kv_heads=int(num_kv_heads),
        seq_len=int(seq_len),
        codes=codes,
        passthrough=pt,
        passthrough_dense=False,
    )


def _dequantize_key_payload_if_needed(layer_idx: int | None, key_states: Any) -> Any:
    """Dense fp32 keys [B, Hkv, S, D] from a quantized payload (what the reference's per-head
    ``codec.dequantize`` loop gives, sunshape/vllm_attn_backend.py:140-156): one ssq_dequantize
    launch over every (batch, KV head) of a per-layer codec, one per KV head of a per-KV-head
    codec.  Other key states pass through."""
    if not isinstance(key_states, SunShapeQuantizedKeys):
        return key_states
    runtime = get_registered_runtime()
    if runtime is None or layer_idx is None:
        raise RuntimeError("SunShape runtime state is required to dequantize quantized key payloads.")
    codec = runtime.codec_for_layer(int(layer_idx))
    if codec is None:
        raise RuntimeError(f"No codec is registered for layer {layer_idx}.")
    B, Hkv, S = key_states.batch_size, key_states.num_kv_heads, key_states.seq_len
    codes, pt, dense = key_states.batched()
    heavy = codec.heavy_blocks() if hasattr(codec, "heavy_blocks") else None
    if heavy is not None and pt is None:
        raise ValueError("Mixed-precision quantized keys are missing passthrough values.")
    rot = codec.rotation_matrix() if hasattr(codec, "rotation_matrix") else None
    nb = codes.shape[-1]
    out = torch.empty(B, Hkv, S, codec.head_dim, device=codes.device, dtype=torch.float32)
    heads = range(Hkv) if getattr(codec, "num_kv_heads", None) is not None else [None]
    for h in heads:
        sel = slice(None) if h is None else h
        c = codes[:, sel].reshape(-1, nb)
        p = None if heavy is None else pt[:, sel].reshape(-1, *pt.shape[-2:])
        k = hip_ops.dequantize(c, codec.effective_permutation(h), codec.codebook(h), heavy=heavy, pt=p,
                               pt_dense=dense, rotation=rot)
        out[:, sel] = k.view(B, -1, S, codec.head_dim) if h is None else k.view(B, S, codec.head_dim)
    return out


def _causal_mask(query_len: int, seq_len: int, device) -> torch.Tensor:
    """Additive fp32 [query_len, seq_len] mask of scaled_dot_product_attention(is_causal=True):
    query row i sees tokens 0..i (torch aligns a non-square causal mask to the top left)."""
    return torch.full((query_len, seq_len), float("-inf"), device=device, dtype=torch.float32).triu_(1)


def _decode_keys_if_needed(layer_idx: int | None, key_states: torch.Tensor) -> torch.Tensor:
    """Dense keys through the codec round trip (sunshape/vllm_attn_backend.py:126-137)."""
    runtime = get_registered_runtime()
    if runtime is None or layer_idx is None:
        return key_states
    codec = runtime.codec_for_layer(int(layer_idx))
    if codec is None or key_states.ndim < 2:
        return key_states
    orig_shape = key_states.shape
    orig_dtype = key_states.dtype
    if codec.num_kv_heads is not None and key_states.ndim == 4:
        heads = [codec(key_states[:, h].reshape(-1, orig_shape[-1]).float(), kv_head=h).reshape(orig_shape[0], 1, orig_shape[2], orig_shape[3])
                 for h in range(orig_shape[1])]
        return torch.cat(heads, dim=1).to(orig_dtype)
    flat = key_states.reshape(-1, orig_shape[-1])
    decoded = codec(flat.float())
    return decoded.to(orig_dtype).reshape(orig_shape)


def _quantized_fast_path_unavailable_reason(
    *,
    runtime_state: SunShapeVLLMRuntimeState | None,
    layer_idx: int | None,
    query: torch.Tensor,
    key: Any,
    value: torch.Tensor,
    attn_mask: torch.Tensor | None,
    is_causal: bool,
) -> str | None:
    """Same checks and messages as sunshape/vllm_attn_backend.py:159-194."""
    if runtime_state is None or layer_idx is None:
        return "No registered runtime state for quantized attention."
    if not isinstance(key, SunShapeQuantizedKeys):
        return "Key payload is not SunShapeQuantizedKeys."
    codec = runtime_state.codec_for_layer(int(layer_idx))
    if codec is None:
        return f"No codec for layer {layer_idx}."
    if query.ndim != 4 or value.ndim != 4:
        return "Quantized attention expects query/value tensors with shape [batch, heads, seq, dim]."
    if key.batch_size != int(query.shape[0]):
        return "Quantized key batch size does not match query batch size."
    if key.batch_size != int(value.shape[0]):
        return "Quantized key batch size does not match value batch size."
    if key.num_kv_heads != int(value.shape[1]):
        return "Quantized key kv-head count does not match value kv-head count."
    if key.seq_len != int(value.shape[2]):
        return "Quantized key sequence length does not match value sequence length."
    if int(query.shape[-1]) != int(codec.head_dim):
        return "Query head_dim does not match codec head_dim."
    if int(query.shape[1]) % int(key.num_kv_heads) != 0:
        return "Query head count must be divisible by kv-head count."
    if is_causal and int(query.shape[2]) != 1:
        return "Causal quantized fast path currently targets decode (query_len == 1)."
    if attn_mask is not None and attn_mask.ndim not in {2, 3, 4}:
        return "Unsupported attention-mask rank for quantized fast path."
    reason = codec.unsupported_reason() if hasattr(codec, "unsupported_reason") else None
    if reason is not None:
        return reason
    return None


def _mask_view(attn_mask: torch.Tensor | None, batch: int, hq: int, lq: int, seq: int) -> torch.Tensor | None:
    """4-D view of the mask with the reference's per-(batch, head) slicing (vllm_attn_backend.py:197-213)."""
    if attn_mask is None:
        return None
    m = attn_mask
    if m.ndim == 2:                       # [Lq, S] for every batch and head
        return m[None, None]
    if m.ndim == 3:
        if m.shape[0] == batch:           # [B, Lq, S]: same for every head of a batch
            return m[:, None]
        return m[None]                    # [Hq, Lq, S]: same for every batch
    return m


def _apply_quantized_attention(
    *,
    codec,
    query: torch.Tensor,
    key: SunShapeQuantizedKeys,
    value: torch.Tensor,
    attn_mask: torch.Tensor | None,
    scale: float | None,
) -> torch.Tensor:
    """One fused HIP launch for sunshape/vllm_attn_backend.py:216-253."""
    batch_size, num_query_heads, query_len, _ = query.shape
    _, num_kv_heads, seq_len, _ = value.shape
    codes, pt, dense = key.batched()
    perm, cent = _codec_head_arrays(codec, num_kv_heads)
    heavy = codec.heavy_blocks() if hasattr(codec, "heavy_blocks") else None
    mask = _mask_view(attn_mask, batch_size, num_query_heads, query_len, seq_len)
    q = query if query.stride(-1) == 1 else query.contiguous()
    v = value if value.stride(-1) == 1 else value.contiguous()
    rot = codec.rotation_matrix() if hasattr(codec, "rotation_matrix") else None
    return hip_ops.decode(q, codes, v, perm, cent, scale=scale, mask=mask, heavy=heavy, pt=pt, pt_dense=dense,
                          rotation=rot)


class SunShapeAttentionImpl:
    """Attention shim for vLLM integration (sunshape/vllm_attn_backend.py:256-347)."""

    def __init__(self, *, delegate: Any = None, layer_idx: int | None = None, runtime_state: SunShapeVLLMRuntimeState | None = None):
        self.delegate = delegate
        self.layer_idx = layer_idx
        self.runtime_state = runtime_state or get_registered_runtime()

    def forward(
        self,
        query: torch.Tensor,
        key: Any,
        value: torch.Tensor,
        *,
        attn_mask: torch.Tensor | None = None,
        is_causal: bool = False,
        scale: float | None = None,
        layer_idx: int | None = None,
        **kwargs: Any,
    ) -> torch.Tensor:
        layer = self.layer_idx if layer_idx is None else layer_idx
        runtime_state = self.runtime_state or get_registered_runtime()
        reason = _quantized_fast_path_unavailable_reason(
            runtime_state=runtime_state,
            layer_idx=layer,
            query=query,
            key=key,
            value=value,
            attn_mask=attn_mask,
            is_causal=is_causal,
        )
        if reason is None:
            codec = runtime_state.codec_for_layer(int(layer)) if runtime_state is not None else None
            if codec is None:
                raise RuntimeError(f"No codec is registered for layer {layer}.")
            return _apply_quantized_attention(
                codec=codec, query=query, key=key, value=value, attn_mask=attn_mask, scale=scale,
            )
        delegate = self.delegate
        if (isinstance(key, SunShapeQuantizedKeys) and delegate is None and is_causal and attn_mask is None
                and _quantized_fast_path_unavailable_reason(runtime_state=runtime_state, layer_idx=layer, query=query,
                                                            key=key, value=value, attn_mask=None,
                                                            is_causal=False) is None):
            # Causal attention over more than one query row (chunked prefill): the reference
            # dequantizes the payload and runs scaled_dot_product_attention(query * scale, key,
            # value, is_causal=True) (:306-345), i.e. scores scaled by scale / sqrt(head_dim) (1 /
            # sqrt(head_dim) without a scale) under a top-left causal mask.  The fused kernel
            # computes the same attention from the codes.
            codec = runtime_state.codec_for_layer(int(layer))
            head_dim = int(query.shape[-1])
            eff = (1.0 if scale is None else float(scale)) / math.sqrt(head_dim)
            mask = _causal_mask(int(query.shape[2]), int(value.shape[2]), query.device)
            return _apply_quantized_attention(codec=codec, query=query, key=key, value=value, attn_mask=mask,
                                              scale=eff)
        key = _dequantize_key_payload_if_needed(layer, key)
        key = _decode_keys_if_needed(layer, key)
        if delegate is not None:
            if hasattr(delegate, "forward"):
                return delegate.forward(query, key, value, attn_mask=attn_mask, is_causal=is_causal,
                                        scale=scale, layer_idx=layer, **kwargs)
            if callable(delegate):
                return delegate(query, key, value, attn_mask=attn_mask, is_causal=is_causal,
                                scale=scale, layer_idx=layer, **kwargs)
        if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
            raise RuntimeError(
                "SunShapeAttentionImpl fallback expects 4D [batch, heads, seq, dim] tensors "
                "when no delegate backend is provided."
            )
        if scale is not None:
            query = query * float(scale)
        return F.scaled_dot_product_attention(query, key, value, attn_mask=attn_mask, is_causal=is_causal)

    __call__ = forward


class SunShapeAttentionBackend:
    """Backend/factory surface (sunshape/vllm_attn_backend.py:350-366)."""

    backend_name = "sunshape"

    def __init__(self, *, delegate_backend: Any = None):
        self.delegate_backend = delegate_backend

    def make_impl(self, *, layer_idx: int | None = None, delegate: Any = None) -> SunShapeAttentionImpl:
        return SunShapeAttentionImpl(
            delegate=delegate if delegate is not None else self.delegate_backend,
            layer_idx=layer_idx,
            runtime_state=get_registered_runtime(),
        )

    def describe(self) -> dict[str, Any]:
        return describe_backend()


def get_backend_factory(*, delegate_backend: Any = None) -> SunShapeAttentionBackend:
    return SunShapeAttentionBackend(delegate_backend=delegate_backend)


def ensure_backend_registered() -> dict[str, Any]:
    runtime = get_registered_runtime()
    handle = get_registered_handle()
    return {
        "backend": "sunshape",
        "mode": get_mode(),
        "registered": handle is not None,
        "runtime_loaded": runtime is not None,
        "install_entrypoint": "sunshape_amd.vllm_attn_backend:install_sunshape_hooks",
        "env_backend": os.environ.get("VLLM_ATTENTION_BACKEND"),
    }


def describe_backend() -> dict[str, Any]:
    handle = get_registered_handle()
    if handle is None:
        return {"mode": get_mode(), "registered": False, "config": None, "runtime": None}
    return {
        "mode": get_mode(),
        "registered": True,
        "config": handle.config.to_dict(),
        "hooks_installed": handle.hooks_installed,
        "connector_registered": handle.connector_registered,
        "runtime_patch_available": handle.runtime_patch_available,
        "notes": list(handle.notes),
        "runtime": _RUNTIME_STATE.to_dict() if _RUNTIME_STATE is not None else None,
    }


def install_sunshape_hooks(*args, **kwargs) -> SunShapeVLLMHandle:
    return register_handle(install_hooks(*args, **kwargs))


__all__ = [
    "MODE_ACTIVE", "MODE_CAPTURE", "MODE_OFF",
    "SunShapeVLLMConfig", "SunShapeVLLMHandle", "SunShapeVLLMRuntimeState",
    "SunShapeAttentionBackend", "SunShapeAttentionImpl", "SunShapeQuantizedKeys",
    "clear_registered_handle", "clear_registered_runtime", "describe_backend", "ensure_backend_registered",
    "get_mode", "get_registered_handle", "get_registered_runtime", "get_backend_factory",
    "install_sunshape_hooks", "quantize_key_states", "register_handle", "register_runtime_state", "set_mode",
]
