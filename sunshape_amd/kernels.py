"""Attention scores against SunShape block-VQ keys, on HIP kernels.

Drop-in for the public functions of ``sunshape.triton_kernels``
(sunshape/triton_kernels.py:319-373, :549-609):

* ``sunshape_attention_scores(codec, query, quantized_key)`` -> fp32 [n_qh, T]
* ``sunshape_attention_scores_strict`` (same; kept for the reference's name)
* ``require_triton_fast_path`` / ``_triton_fast_path_unavailable_reason``

Behavioural difference, by design: the reference silently falls back to an
eager dequantize + matmul when its Triton gate rejects an input
(triton_kernels.py:598-609).  Here every supported input runs the HIP kernel
(including SunShape-Mixed passthrough blocks, which the reference's Triton gate
rejects) and every unsupported input raises ``RuntimeError(reason)`` -- there
is no second code path.
"""

from __future__ import annotations

import torch

from . import _native, hip_ops


def _triton_fast_path_unavailable_reason(codec, query: torch.Tensor, quantized_key, kv_head: int | None = None) -> str | None:
    """Host-side gate, same checks and messages as sunshape/triton_kernels.py:327-363 where they apply."""
    if not hasattr(quantized_key, "indices"):
        return "Quantized key must expose an .indices tensor."
    reason = codec.unsupported_reason() if hasattr(codec, "unsupported_reason") else None
    if reason is not None:
        return reason
    if not query.is_cuda:
        return "Query tensor must be on a HIP device for the HIP fast path."
    if not quantized_key.indices.is_cuda:
        return "Quantized key indices must be on a HIP device for the HIP fast path."
    if query.ndim != 2:
        return f"Expected query.ndim == 2, got {query.ndim}."
    if quantized_key.indices.ndim != 2:
        return f"Expected quantized_key.indices.ndim == 2, got {quantized_key.indices.ndim}."
    if quantized_key.indices.shape[1] != codec.n_blocks:
        return (
            "Quantized key block count does not match codec: "
            f"indices.shape[1]={quantized_key.indices.shape[1]}, codec.n_blocks={codec.n_blocks}."
        )
    if query.shape[1] != codec.head_dim:
        return f"Query head dim {query.shape[1]} does not match codec.head_dim {codec.head_dim}."
    if codec.centroids.ndim not in (3, 4):
        return f"Expected codec.centroids.ndim == 3, got {codec.centroids.ndim}."
    if codec.centroids.ndim == 4 and kv_head is None:
        return "Per-KV-head codec: pass kv_head= to select the codebook."
    pb = getattr(quantized_key, "passthrough_blocks", None)
    if pb is not None and bool(pb.any()) and getattr(quantized_key, "passthrough_values", None) is None:
        return "Mixed-precision quantized keys are missing passthrough values."
    if query.dtype not in _native.DTYPE_CODE:
        return f"Unsupported query dtype {query.dtype}."
    return None


def _supports_triton_fast_path(codec, query: torch.Tensor, quantized_key, kv_head: int | None = None) -> bool:
    return _triton_fast_path_unavailable_reason(codec, query, quantized_key, kv_head) is None


def require_triton_fast_path(codec, query: torch.Tensor, quantized_key, kv_head: int | None = None) -> None:
    """sunshape/triton_kernels.py:366-373."""
    reason = _triton_fast_path_unavailable_reason(codec, query, quantized_key, kv_head)
    if reason is not None:
        raise RuntimeError(reason)


def _codec_arrays(codec, kv_head):
    if hasattr(codec, "effective_permutation"):
        return codec.effective_permutation(kv_head), codec.codebook(kv_head)
    perm = codec.permutation if kv_head is None else codec.permutation[kv_head]
    cent = codec.centroids if kv_head is None else codec.centroids[kv_head]
    return perm, cent


def sunshape_attention_scores_strict(codec, query: torch.Tensor, quantized_key, kv_head: int | None = None) -> torch.Tensor:
    """Scores on the HIP kernel, or RuntimeError(reason).  sunshape/triton_kernels.py:549-562."""
    require_triton_fast_path(codec, query, quantized_key, kv_head)
    perm, cent = _codec_arrays(codec, kv_head)
    idx = quantized_key.indices
    want = hip_ops.index_dtype(int(cent.shape[-2]))
    if idx.dtype != want:  # e.g. int64 indices: the stored dtype's bits (16-bit codes read unsigned)
        idx = idx.to(want)
    heavy = None
    pb = getattr(quantized_key, "passthrough_blocks", None)
    if pb is not None:
        heavy = codec.heavy_blocks() if hasattr(codec, "heavy_blocks") else None
        if heavy is None or len(heavy) != pb.numel():
            heavy = tuple(bool(x) for x in pb.tolist())
        if not any(heavy):
            heavy = None
    pt = getattr(quantized_key, "passthrough_values", None)
    dense = pt is not None and pt.ndim == 3 and pt.shape[1] == codec.n_blocks
    rot = codec.rotation_matrix() if hasattr(codec, "rotation_matrix") else None
    return hip_ops.attention_scores(query, idx, perm, cent, heavy=heavy, pt=pt, pt_dense=dense, rotation=rot)


def sunshape_attention_scores(codec, query: torch.Tensor, quantized_key, kv_head: int | None = None) -> torch.Tensor:
    """``<query, k_hat>`` fp32 [n_qh, T] against block-quantized keys (sunshape/triton_kernels.py:570-609).

    query is [n_qh, D] in the original model basis; it is permuted into the
    codec basis inside the kernel (rotated codecs: q @ R^T first, on the GPU).  Raises
    RuntimeError for unsupported inputs.
    """
    return sunshape_attention_scores_strict(codec, query, quantized_key, kv_head=kv_head)


def _precompute_query_centroid_dots(query: torch.Tensor, centroids: torch.Tensor, n_blocks: int, block_dim: int) -> torch.Tensor:
    """LUT [n_qh, nb, nc] for a query already in the codec basis (sunshape/triton_kernels.py:381-408)."""
    ident = torch.arange(query.shape[1], device=query.device, dtype=torch.long)
    return hip_ops.lut_build(query, ident, centroids.float())


__all__ = [
    "require_triton_fast_path",
    "sunshape_attention_scores",
    "sunshape_attention_scores_strict",
]
