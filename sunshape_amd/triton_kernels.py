"""Import-compatible name for ``sunshape.triton_kernels``.

The reference's public score entry points live in a module called
``triton_kernels``; code written against it keeps working with
``from sunshape_amd.triton_kernels import sunshape_attention_scores``.  There
is no Triton here: these are the HIP entry points of ``sunshape_amd.kernels``.
"""

from .kernels import (  # noqa: F401
    _precompute_query_centroid_dots,
    _supports_triton_fast_path,
    _triton_fast_path_unavailable_reason,
    require_triton_fast_path,
    sunshape_attention_scores,
    sunshape_attention_scores_strict,
)

__all__ = ["require_triton_fast_path", "sunshape_attention_scores", "sunshape_attention_scores_strict"]
