"""Writes the golden fixtures under tests/golden/ (run in this repo; CPU only).

The reference (gauravsaini/sunshape) ships no tests or fixtures.  These vectors
replay the reference's eager path with the same torch library calls, in the
same order, that its source makes -- an implementation independent of the
numpy/C oracle under oracle/:

  c1_scores.npz   sunshape/triton_kernels.py:300-311 (_torch_attention_scores:
                  codec.dequantize + torch.matmul) and :381-408 + :176-196
                  (einsum LUT, block-ordered gather-sum) on config 1.
  encode_mixed.npz sunshape/codec.py:362-385 (quantize: keys.float(), x[..., perm],
                  torch.cdist(...).argmin(-1) per light block, passthrough copy)
                  on a 4096-key slice of the config-5 distribution.
  decode_small.npz sunshape/vllm_attn_backend.py:216-253 (_apply_quantized_attention:
                  q * scale in bf16, scores, softmax fp32, .to(bf16), matmul with V)
                  on a 2 x 512 slice of the config-3 shape, one codec per KV head.

Inputs are stored next to the expected outputs, so the fixtures are
self-contained; the GPU box only reads the .npz files.
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from sunshape_amd.synthetic import config1, heavy_blocks_by_sigma, make_codebook  # noqa: E402


def dequant_torch(codes: torch.Tensor, cent: torch.Tensor, perm: torch.Tensor, heavy=None, pt=None) -> torch.Tensor:
    """codec.dequantize, sunshape/codec.py:387-398."""
    nb, _, bd = cent.shape
    k_hat = torch.zeros(codes.shape[0], nb * bd, dtype=torch.float32)
    idx = codes.long()
    for b in range(nb):
        sl = slice(b * bd, (b + 1) * bd)
        if heavy is not None and bool(heavy[b]):
            k_hat[:, sl] = pt[:, b, :]
        else:
            k_hat[:, sl] = cent[b][idx[:, b]]
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(len(perm))
    return k_hat[..., inv]


def make_c1():
    p = config1("cpu")
    q, codes, perm, cent = p["q"], p["codes"], p["perm"], p["centroids"]
    k_hat = dequant_torch(codes, cent, perm)
    scores_dq = torch.matmul(q.float(), k_hat.float().transpose(-2, -1))
    qp = q[..., perm].float()
    lut = torch.einsum("qbd,bcd->qbc", qp.view(1, 8, 8), cent).contiguous()
    acc = torch.zeros(1, codes.shape[0])
    for b in range(8):
        acc = acc + lut[:, b, codes[:, b].long()]
    np.savez_compressed(os.path.join(HERE, "c1_scores.npz"), q=q.numpy(), codes=codes.numpy(), perm=perm.numpy(),
                        centroids=cent.numpy(), scores_dequant=scores_dq.numpy(), scores_lut=acc.numpy(),
                        lut=lut.numpy(), scale=np.float32(1.0 / math.sqrt(64)))


def make_encode():
    D, bd, n = 64, 2, 4096
    cb = make_codebook(1, D, bd, seed=55, shared_sigma=True)
    heavy = heavy_blocks_by_sigma(cb.sigma[0], cb.perm[0], bd, 4)
    cent = cb.centroids[0].clone()
    cent[heavy] = 0.0
    g = torch.Generator().manual_seed(56)
    keys = (torch.randn(n, D, generator=g) * cb.sigma[0]).to(torch.bfloat16)
    perm = cb.perm[0]
    x = keys.float()[..., perm]
    nb = D // bd
    idx = torch.zeros(n, nb, dtype=torch.long)
    pt = torch.zeros(n, nb, bd)
    for b in range(nb):
        sl = slice(b * bd, (b + 1) * bd)
        if bool(heavy[b]):
            pt[:, b, :] = x[:, sl]
            continue
        e = torch.eye(bd)
        dists = torch.cdist(x[:, sl] @ e.T, cent[b] @ e.T)
        idx[:, b] = dists.argmin(dim=-1)
    np.savez_compressed(os.path.join(HERE, "encode_mixed.npz"),
                        keys_bf16_bits=keys.view(torch.int16).numpy(), perm=perm.numpy(), centroids=cent.numpy(),
                        heavy=heavy.numpy(), codes=idx.to(torch.uint8).numpy(), passthrough=pt.numpy())


def make_decode():
    B, Hq, Hkv, D, bd, T = 2, 14, 2, 64, 2, 512
    G = Hq // Hkv
    cb = make_codebook(Hkv, D, bd, seed=77)
    g = torch.Generator().manual_seed(78)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    out = torch.empty(B, Hq, 1, D, dtype=torch.bfloat16)
    scores_all = torch.empty(B, Hq, 1, T)
    for b in range(B):
        for h in range(Hkv):
            qs = q[b, h * G:(h + 1) * G] * float(scale)
            qf = qs.reshape(-1, D)
            k_hat = dequant_torch(codes[b, h], cb.centroids[h], cb.perm[h])
            s = torch.matmul(qf.float(), k_hat.float().transpose(-2, -1)).view(G, 1, T)
            scores_all[b, h * G:(h + 1) * G] = s
            probs = torch.softmax(s, dim=-1).to(v.dtype)
            out[b, h * G:(h + 1) * G] = torch.matmul(probs, v[b, h])
    np.savez_compressed(os.path.join(HERE, "decode_small.npz"),
                        q_bf16_bits=q.view(torch.int16).numpy(), codes=codes.numpy(),
                        v_bf16_bits=v.view(torch.int16).numpy(), perm=cb.perm.numpy(), centroids=cb.centroids.numpy(),
                        scale=np.float32(scale), out_bf16_bits=out.view(torch.int16).numpy(),
                        scores=scores_all.numpy())


if __name__ == "__main__":
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    make_c1()
    make_encode()
    make_decode()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
