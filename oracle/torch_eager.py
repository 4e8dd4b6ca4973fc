"""The reference's eager PyTorch decode path, restated on the CPU -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg may import this module: it is the CPU
path a host without the GPU kernels runs, timed beside the GPU as a baseline.  The product
package ``sunshape_amd`` never imports it.

It follows the reference's own call sequence with the same torch calls, one (batch, KV head)
at a time (paths relative to the gauravsaini/sunshape tree):
  query_slice * float(scale) in the query dtype          sunshape/vllm_attn_backend.py:232-236
  sunshape_attention_scores -> _torch_attention_scores   sunshape/triton_kernels.py:300-311
    (a CPU tensor fails the Triton gate, :346-347, so the public entry takes this path)
    k_hat = codec.dequantize(quantized)                  sunshape/codec.py:387-398
      per block: k_hat[:, sl] = centroids[b][indices[:, b]]; then x[..., inv_permutation]
    scores = query.float() @ k_hat.float().T
  scores.view(G, Lq, T); softmax(-1).to(value.dtype)     sunshape/vllm_attn_backend.py:239-251
  torch.matmul(probs, value[b, kv])                      sunshape/vllm_attn_backend.py:252
Pinned in tests/test_oracle_numerics.py against the numpy oracle's decode_attention.
"""

from __future__ import annotations

import torch


def dequantize(indices: torch.Tensor, centroids: torch.Tensor, inv_perm: torch.Tensor,
               heavy: list[bool] | None = None, passthrough_values: torch.Tensor | None = None) -> torch.Tensor:
    """sunshape/codec.py:387-398 for the permutation modes (heavy blocks read the dense
    passthrough values [T, nb, bd], as SunShape-Mixed stores them)."""
    nb, _, bd = centroids.shape
    k_hat = torch.zeros(indices.shape[0], nb * bd, dtype=centroids.dtype)
    idx = indices.long()
    for b in range(nb):
        sl = slice(b * bd, (b + 1) * bd)
        if heavy is not None and heavy[b]:
            k_hat[:, sl] = passthrough_values[:, b, :]
        else:
            k_hat[:, sl] = centroids[b][idx[:, b]]
    return k_hat[..., inv_perm]


def decode_unit(query: torch.Tensor, indices: torch.Tensor, value: torch.Tensor, centroids: torch.Tensor,
                inv_perm: torch.Tensor, scale: float | None, heavy: list[bool] | None = None,
                passthrough_values: torch.Tensor | None = None) -> torch.Tensor:
    """One (batch, KV head) of sunshape/vllm_attn_backend.py:228-252 (no mask).

    query [G, Lq, D] (bf16/f16/fp32), indices [T, nb] uint8, value [T, Dv], centroids
    [nb, nc, bd] fp32, inv_perm [D] int64.  Returns [G, Lq, Dv] in value's dtype.
    """
    G, Lq, D = query.shape
    q = query * float(scale) if scale is not None else query
    q = q.reshape(-1, D)
    k_hat = dequantize(indices, centroids, inv_perm, heavy, passthrough_values)
    scores = torch.matmul(q.float(), k_hat.float().transpose(-2, -1))
    scores = scores.view(G, Lq, indices.shape[0])
    probs = torch.softmax(scores, dim=-1).to(value.dtype)
    return torch.matmul(probs, value)
