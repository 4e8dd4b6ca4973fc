"""sunshape_amd: MI355X-native SunShape VQ-key decode attention.

Hand-written gfx950 HIP kernels behind a C ABI (include/sunshape_amd.h), with
the reference's Python surface on top:

* ``sunshape_amd.codec``            SunShapeBlockCodec / SunShapeQuantized
* ``sunshape_amd.kernels``          sunshape_attention_scores[_strict]
  (also importable as ``sunshape_amd.triton_kernels``)
* ``sunshape_amd.vllm_attn_backend`` SunShapeAttentionImpl, quantize_key_states
* ``sunshape_amd.hf``               SunShapeBundle on-disk format
* ``sunshape_amd.paged``            vLLM-style paged cache (append + decode)
* ``sunshape_amd.hip_ops``          tensor-level wrappers of the C ABI
"""

from .codec import SunShapeBlockCodec, SunShapeQuantized
from .kernels import require_triton_fast_path, sunshape_attention_scores, sunshape_attention_scores_strict

__all__ = [
    "SunShapeBlockCodec",
    "SunShapeQuantized",
    "require_triton_fast_path",
    "sunshape_attention_scores",
    "sunshape_attention_scores_strict",
]
