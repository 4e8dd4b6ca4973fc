"""A seeded sweep of SunShapeAttentionImpl.forward over quantize_key_states payloads, the
reference's vLLM decode call (sunshape/vllm_attn_backend.py:271-345).  Each case draws a
per-layer or per-KV-head codec, baseline or SunShape-Mixed, 256 or 1,024 codewords; the batch,
KV heads, query heads per KV head, context and new tokens; the value dtype; the scale (none,
1/sqrt(D) or another); an attention mask of rank 2, 3 (per sequence or per query head) or 4,
sliced as the reference slices it (:197-213); and causal steps: one token (the fast path) or
several without a mask, which the reference sends to scaled_dot_product_attention over the
dequantized keys and the fused kernel computes from the codes.  The payload's codes are checked
bit for bit against the oracle's encode, and every output against the oracle's restatement of
the reference's arithmetic."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import synthetic
from sunshape_amd import vllm_attn_backend as VB
from sunshape_amd.codec import SunShapeBlockCodec
from sunshape_amd.hf import SunShapeBundle
from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
VDT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _draw(seed):
    rng = np.random.default_rng(seed)
    D = int(rng.choice([64, 128]))
    bd = int(rng.choice([2, 4, 8]))
    c = dict(seed=seed, D=D, bd=bd, nb=D // bd, nc=int(rng.choice([256, 256, 1024])),
             per_head=bool(rng.integers(0, 2)), mixed=bool(rng.integers(0, 3) == 0), B=int(rng.integers(1, 4)),
             Hkv=int(rng.choice([1, 2, 4])), G=int(rng.choice([1, 2, 4, 7])), S=int(rng.integers(1, 600)),
             Lq=int(rng.choice([1, 1, 2, 3])), vdt=str(rng.choice(["bf16", "bf16", "f16"])),
             scale=str(rng.choice(["none", "inv_sqrt", "other"])),
             mask=str(rng.choice(["none", "2d", "3d_batch", "3d_head", "4d"])), causal=bool(rng.integers(0, 2)))
    if c["Lq"] > 1 and c["causal"]:
        c["mask"] = "none"  # several causal rows: the reference's SDPA route, taken here without a mask
    return c


def _mask(kind, B, Hq, Lq, S, rng):
    shape = {"2d": (Lq, S), "3d_batch": (B, Lq, S), "3d_head": (Hq, Lq, S), "4d": (B, Hq, Lq, S)}[kind]
    m = rng.uniform(-2.0, 0.0, shape).astype(np.float32) * (rng.random(shape) < 0.3)
    m[rng.random(shape) < 0.2] = -np.inf
    m[..., 0] = np.where(np.isinf(m[..., 0]), 0.0, m[..., 0])  # every row keeps a finite score
    return m


@pytest.mark.parametrize("seed", list(range(500, 540)))
def test_backend_forward_sweep_vs_oracle(seed):
    c = _draw(seed)
    log(f"backend sweep {c}")
    D, bd, nb, nc, B, Hkv, G, S, Lq = (c[k] for k in ("D", "bd", "nb", "nc", "B", "Hkv", "G", "S", "Lq"))
    Hq = Hkv * G
    rng = np.random.default_rng(seed + 1)
    cb = synthetic.make_codebook(Hkv if c["per_head"] else 1, D, bd, seed, n_centroids=nc, shared_sigma=True)
    heavy = None
    if c["mixed"]:
        heavy = synthetic.heavy_blocks_by_sigma(cb.sigma, cb.perm, bd, min(4, nb - 1))
    perm, cent = (cb.perm, cb.centroids) if c["per_head"] else (cb.perm[0], cb.centroids[0])
    mode = "profileperm_mixed_precision" if c["mixed"] else "profileperm_baseline"
    codec = SunShapeBlockCodec.from_buffers(perm, cent, mode=mode, mixed_high_precision_blocks=heavy, device=DEV)
    bundle = SunShapeBundle("m", [0], math.log2(nc) / bd, bd, mode, 0, 0, 0, {0: codec})
    VB.register_runtime_state(SunShapeVLLMRuntimeState("p", "m", mode, 0.0, bd, [0], bundle, "cuda"))
    try:
        g = torch.Generator().manual_seed(seed + 2)
        keys = (torch.randn(B, Hkv, S, D, generator=g) * cb.sigma[0]).to(torch.bfloat16)
        qk = VB.quantize_key_states(0, keys.to(DEV))
        codes = np_of(qk.codes)
        codes = codes.view(np.uint16).astype(np.int64) if codes.dtype == np.int16 else codes.astype(np.int64)
        hv = None if heavy is None else heavy.numpy()
        pt = None if hv is None else np.zeros((B, Hkv, S, nb, bd), np.float32)
        for b in range(B):
            for h in range(Hkv):
                ph = (cb.perm[h] if c["per_head"] else cb.perm[0]).numpy()
                ch = (cb.centroids[h] if c["per_head"] else cb.centroids[0]).numpy()
                rc, rpt = O.encode(keys[b, h].float().numpy(), ph, ch, hv)
                assert np.array_equal(codes[b, h], rc.astype(np.int64)), f"codes b={b} h={h}"
                if pt is not None:
                    pt[b, h][:, hv] = rpt[:, hv]
        q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16)
        v = torch.randn(B, Hkv, S, D, generator=g).to(VDT[c["vdt"]])
        scale = {"none": None, "inv_sqrt": 1 / math.sqrt(D), "other": 0.37}[c["scale"]]
        m = None if c["mask"] == "none" else _mask(c["mask"], B, Hq, Lq, S, rng)
        impl = VB.get_backend_factory().make_impl(layer_idx=0)
        out = np_of(impl(q.to(DEV), qk, v.to(DEV), attn_mask=None if m is None else torch.from_numpy(m).to(DEV),
                         is_causal=c["causal"], scale=scale))
        if Lq > 1 and c["causal"]:
            # the reference's route: SDPA over the dequantized keys with query * scale, its own
            # 1/sqrt(D) and the top-left causal mask
            eff = (1.0 if scale is None else scale) / math.sqrt(D)
            ref = O.decode_attention(np_of(q), codes, np_of(v), cb.centroids.numpy() if c["per_head"] else
                                     cb.centroids[0].numpy(), cb.perm.numpy() if c["per_head"] else cb.perm[0].numpy(),
                                     eff, "bf16", c["vdt"], mask=np.triu(np.full((Lq, S), -np.inf, np.float32), 1),
                                     heavy=hv, pt_values=pt)
        else:
            ref = O.decode_attention(np_of(q), codes, np_of(v), cb.centroids.numpy() if c["per_head"] else
                                     cb.centroids[0].numpy(), cb.perm.numpy() if c["per_head"] else cb.perm[0].numpy(),
                                     scale, "bf16", c["vdt"], mask=m, heavy=hv, pt_values=pt)
        assert_rel(out, ref, BF16_TOL, "forward")
    finally:
        VB.clear_registered_runtime()
