"""Seeded synthetic inputs for the five benchmark configurations.

No datasets or checkpoints are involved: codebooks, permutations, codes,
queries and values are drawn from the distributions the configurations name.

* per-dim sigma_d ~ logU[0.1, 3] over the original dims;
* permutation = seeded randperm(D) (per KV head unless stated);
* codebook C[h, b, c, j] ~ N(0, sigma_{perm[b*bd+j]}^2), fp32, in the permuted basis;
* codes ~ U{0..255} uint8; q ~ N(0, 1); V ~ N(0, 1) bf16; scale = 1/sqrt(D).

Small tensors come from a CPU generator (identical on every machine); the
multi-GiB config-4 tensors are drawn on the device.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch

N_CENTROIDS = 256


@dataclass
class Codebook:
    perm: torch.Tensor        # [Hkv, D] int64 (or [D] when shared)
    centroids: torch.Tensor   # [Hkv, nb, nc, bd] fp32
    sigma: torch.Tensor       # [Hkv, D] or [D] fp32, per original dim

    def to(self, device) -> "Codebook":
        return Codebook(self.perm.to(device), self.centroids.to(device), self.sigma.to(device))


def make_codebook(n_kv: int, head_dim: int, block_dim: int, seed: int, *, shared_perm: bool = False,
                  shared_sigma: bool = False, n_centroids: int = N_CENTROIDS) -> Codebook:
    g = torch.Generator().manual_seed(seed)
    nb = head_dim // block_dim
    rows = 1 if shared_sigma else n_kv
    sigma = torch.exp(torch.empty(rows, head_dim).uniform_(math.log(0.1), math.log(3.0), generator=g))
    sigma = sigma.expand(n_kv, head_dim).contiguous()
    if shared_perm:
        perm = torch.randperm(head_dim, generator=g).expand(n_kv, head_dim).contiguous()
    else:
        perm = torch.stack([torch.randperm(head_dim, generator=g) for _ in range(n_kv)])
    sig_perm = torch.gather(sigma, 1, perm).view(n_kv, nb, 1, block_dim)
    cent = torch.randn(n_kv, nb, n_centroids, block_dim, generator=g) * sig_perm
    return Codebook(perm.to(torch.int64), cent.float().contiguous(), sigma.float())


@dataclass
class Problem:
    name: str
    tensors: dict = field(default_factory=dict)
    meta: dict = field(default_factory=dict)

    def __getitem__(self, k):
        return self.tensors[k]


def config1(device="cpu", seed: int = 1) -> Problem:
    """One KV head, one fp32 query, D 64, 8 blocks of 8, 4096 keys at 1 bit/dim."""
    cb = make_codebook(1, 64, 8, seed)
    g = torch.Generator().manual_seed(seed + 100)
    q = torch.randn(1, 64, generator=g)
    codes = torch.randint(0, 256, (4096, 8), generator=g, dtype=torch.uint8)
    return Problem("C1", {"q": q.to(device), "codes": codes.to(device), "perm": cb.perm[0].to(device),
                          "centroids": cb.centroids[0].to(device)},
                   {"scale": 1.0 / math.sqrt(64), "keys": 4096, "head_dim": 64, "block_dim": 8})


def _gqa(name: str, device, seed: int, *, B: int, Hq: int, Hkv: int, D: int, bd: int, T: int,
         with_v: bool, Dv: Optional[int] = None) -> Problem:
    cb = make_codebook(Hkv, D, bd, seed)
    g = torch.Generator().manual_seed(seed + 100)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 256, (B, Hkv, T, D // bd), generator=g, dtype=torch.uint8)
    t = {"q": q.to(device), "codes": codes.to(device), "perm": cb.perm.to(device), "centroids": cb.centroids.to(device)}
    if with_v:
        t["v"] = torch.randn(B, Hkv, T, Dv or D, generator=g).to(torch.bfloat16).to(device)
    return Problem(name, t, {"scale": 1.0 / math.sqrt(D), "keys": B * Hkv * T, "head_dim": D, "block_dim": bd,
                             "B": B, "Hq": Hq, "Hkv": Hkv, "T": T})


def config2(device="cpu", seed: int = 2, *, B: int = 16, T: int = 8192) -> Problem:
    """Qwen2.5-0.5B-shaped GQA scores at 1 bit/dim: 14 q heads / 2 KV heads, D 64, bd 8."""
    return _gqa("C2", device, seed, B=B, Hq=14, Hkv=2, D=64, bd=8, T=T, with_v=False)


def config3(device="cpu", seed: int = 3, *, B: int = 16, T: int = 8192) -> Problem:
    """Same layer at 4 bits/dim (bd 2, 32 blocks) with bf16 V: fused decode."""
    return _gqa("C3", device, seed, B=B, Hq=14, Hkv=2, D=64, bd=2, T=T, with_v=True)


def _codes(n_centroids: int, shape, gen: torch.Generator, dev) -> torch.Tensor:
    """Uniform codes: uint8 up to 256 codewords, else int16 holding each index's 16 bits (the
    reference's compact index dtype, sunshape/codec.py:78-83)."""
    if n_centroids <= 256:
        return torch.randint(0, n_centroids, shape, generator=gen, device=dev, dtype=torch.uint8)
    if n_centroids > 65536:
        raise ValueError("synthetic codes take at most 65,536 codewords")
    idx = torch.randint(0, n_centroids, shape, generator=gen, device=dev, dtype=torch.int32)
    return torch.where(idx >= 32768, idx - 65536, idx).to(torch.int16)


def config4(device="cpu", seed: int = 4, *, B: int = 64, T: int = 32768, page: int = 16,
            Hq: int = 32, Hkv: int = 8, D: int = 128, bd: int = 4, n_centroids: int = N_CENTROIDS) -> Problem:
    """Llama-3-8B-shaped paged decode at 2 bits/dim.

    Pages hold every KV head (vLLM-style): code pages [P, Hkv, page, nb] uint8,
    value pages [P, Hkv, D, page] bf16 (vLLM's dim-major value layout); the block
    table [B, T/page] int32 is a seeded permutation of all P = B*T/page pages.
    """
    dev = torch.device(device)
    cb = make_codebook(Hkv, D, bd, seed, n_centroids=n_centroids)
    g = torch.Generator().manual_seed(seed + 100)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    P = B * T // page
    table = torch.randperm(P, generator=g).to(torch.int32).view(B, T // page)
    gd = torch.Generator(device=dev).manual_seed(seed + 200)
    code_pages = _codes(n_centroids, (P, Hkv, page, D // bd), gd, dev)
    v_pages = torch.randn(P, Hkv, D, page, generator=gd, device=dev, dtype=torch.bfloat16)
    t = {"q": q.to(dev), "code_pages": code_pages, "v_pages": v_pages, "block_table": table.to(dev),
         "seq_lens": torch.full((B,), T, dtype=torch.int32, device=dev),
         "perm": cb.perm.to(dev), "centroids": cb.centroids.to(dev)}
    return Problem("C4", t, {"scale": 1.0 / math.sqrt(D), "keys": B * Hkv * T, "head_dim": D, "block_dim": bd,
                             "B": B, "Hq": Hq, "Hkv": Hkv, "T": T, "page": page})


def config4_contiguous(device="cpu", seed: int = 104, *, B: int = 64, T: int = 32768, Hq: int = 32, Hkv: int = 8,
                       D: int = 128, bd: int = 4, n_centroids: int = N_CENTROIDS) -> Problem:
    """The config-4 layer with the reference's contiguous rows in place of pages: codes
    [B, Hkv, T, nb] uint8 and V [B, Hkv, T, D] bf16 (token-major), the layout
    sunshape/vllm_attn_backend.py:216-253 hands its kernel.  Codes and V are drawn on the device."""
    dev = torch.device(device)
    cb = make_codebook(Hkv, D, bd, seed, n_centroids=n_centroids)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    gd = torch.Generator(device=dev).manual_seed(seed + 100)
    codes = _codes(n_centroids, (B, Hkv, T, D // bd), gd, dev)
    v = torch.randn(B, Hkv, T, D, generator=gd, device=dev, dtype=torch.bfloat16)
    t = {"q": q.to(dev), "codes": codes, "v": v, "perm": cb.perm.to(dev), "centroids": cb.centroids.to(dev)}
    return Problem("C4ct", t, {"scale": 1.0 / math.sqrt(D), "keys": B * Hkv * T, "head_dim": D, "block_dim": bd,
                               "B": B, "Hq": Hq, "Hkv": Hkv, "T": T})


def heavy_blocks_by_sigma(sigma: torch.Tensor, perm: torch.Tensor, block_dim: int, n_heavy: int) -> torch.Tensor:
    """bool [nb]: the n_heavy blocks with the largest sum of sigma^2 in the permuted basis."""
    mass = (torch.gather(sigma, -1, perm) ** 2).reshape(*perm.shape[:-1], -1, block_dim).sum(-1)
    while mass.ndim > 1:
        mass = mass.sum(0)
    top = torch.topk(mass, n_heavy).indices
    mask = torch.zeros(mass.shape[0], dtype=torch.bool)
    mask[top] = True
    return mask


def config5(device="cpu", seed: int = 5, *, B: int = 16, S: int = 16384, n_heavy: int = 4) -> Problem:
    """Encode/append + SunShape-Mixed on the config-3 layer shape.

    keys bf16 [B, 2, S, 64] ~ N(0, sigma_d^2) with one per-dim sigma for the layer and one
    ProfilePerm permutation for the layer (the reference's codec granularity), per-KV-head
    codebooks; the n_heavy blocks with the largest sigma mass stay in bf16 (passthrough).
    The decode step then attends over those S keys with bf16 V and 14 bf16 query heads.
    """
    Hkv, Hq, D, bd = 2, 14, 64, 2
    cb = make_codebook(Hkv, D, bd, seed, shared_perm=True, shared_sigma=True)
    heavy = heavy_blocks_by_sigma(cb.sigma[0], cb.perm[0], bd, n_heavy)
    # heavy blocks carry no codebook in a fitted mixed codec (sunshape/codec.py:335-337)
    cent = cb.centroids.clone()
    cent[:, heavy] = 0.0
    g = torch.Generator().manual_seed(seed + 100)
    keys = (torch.randn(B, Hkv, S, D, generator=g) * cb.sigma[:, None, :]).to(torch.bfloat16)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    t = {"keys": keys.to(device), "q": q.to(device), "v": v.to(device), "perm": cb.perm[0].to(device),
         "centroids": cent.to(device), "heavy": heavy}
    return Problem("C5", t, {"scale": 1.0 / math.sqrt(D), "keys": B * Hkv * S, "head_dim": D, "block_dim": bd,
                             "B": B, "Hq": Hq, "Hkv": Hkv, "S": S, "n_heavy": n_heavy})
