"""A seeded sweep of the code-storing HF cache layer (SunShapeCodeLayer with the registered
attention function), driven the way HF drives it: a prefill (no mask, causal: HF's mask builder
leaves the mask out when query and key lengths are equal), then decode steps (with or without a
boolean padding mask), multi-token steps over the filled cache (HF's boolean mask: causal over
the last positions plus left padding; or a non-causal step without a mask), crops and beam
reorders.  Steps within the fused kernel's row limits run on the codes; the prefill and longer
steps attend the dequantized keys through SDPA.  Per case one codec (per layer or per KV head,
baseline or SunShape-Mixed, 256 or 1,024 codewords), head_dim 32, 64 or 128.  The stored codes
are checked bit for bit against the oracle's encode of the kept history, and every attention
output against the oracle's decode over it (sunshape/cache.py:24-46 for the keys the reference
cache attends, sunshape/vllm_attn_backend.py:216-253 for the arithmetic)."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import synthetic
from sunshape_amd.cache import SunShapeCodeLayer, sunshape_attention_forward
from sunshape_amd.codec import SunShapeBlockCodec

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _draw(seed):
    rng = np.random.default_rng(seed)
    return dict(seed=seed, D=int(rng.choice([32, 64, 128])), bd=int(rng.choice([2, 4])),
                nc=int(rng.choice([256, 256, 1024])), per_head=bool(rng.integers(0, 2)),
                mixed=bool(rng.integers(0, 3) == 0), B=int(rng.integers(1, 3)), Hkv=int(rng.choice([1, 2])),
                G=int(rng.choice([1, 2, 4, 8])), ops=int(rng.integers(6, 11)),
                scaling=str(rng.choice(["none", "inv_sqrt", "other"])))


@pytest.mark.parametrize("seed", list(range(400, 424)))
def test_code_layer_sweep_vs_oracle(seed):
    c = _draw(seed)
    log(f"code layer sweep {c}")
    D, bd, nc, B, Hkv, G = c["D"], c["bd"], c["nc"], c["B"], c["Hkv"], c["G"]
    nb, Hq = D // bd, Hkv * G
    rng = np.random.default_rng(seed + 1)
    g = torch.Generator().manual_seed(seed + 2)
    cb = synthetic.make_codebook(Hkv if c["per_head"] else 1, D, bd, seed, n_centroids=nc, shared_sigma=True)
    heavy = synthetic.heavy_blocks_by_sigma(cb.sigma, cb.perm, bd, 3) if c["mixed"] else None
    perm, cent = (cb.perm, cb.centroids) if c["per_head"] else (cb.perm[0], cb.centroids[0])
    mode = "profileperm_mixed_precision" if c["mixed"] else "profileperm_baseline"
    codec = SunShapeBlockCodec.from_buffers(perm, cent, mode=mode, mixed_high_precision_blocks=heavy, device=DEV)
    layer = SunShapeCodeLayer(codec, block_tokens=64)
    hv = None if heavy is None else heavy.numpy()
    scaling = {"none": None, "inv_sqrt": 1 / math.sqrt(D), "other": 0.2}[c["scaling"]]
    mod = torch.nn.Module()
    mod.num_key_value_groups = G
    hk = torch.zeros(B, Hkv, 0, D)
    hvals = torch.zeros(B, Hkv, 0, D)

    def oracle_codes():
        T = hk.shape[2]
        codes = np.zeros((B, Hkv, T, nb), np.int64)
        pt = None if hv is None else np.zeros((B, Hkv, T, nb, bd), np.float32)
        for b in range(B):
            for h in range(Hkv):
                ph = (cb.perm[h] if c["per_head"] else cb.perm[0]).numpy()
                ch = (cb.centroids[h] if c["per_head"] else cb.centroids[0]).numpy()
                rc, rpt = O.encode(hk[b, h].numpy(), ph, ch, hv)
                codes[b, h] = rc.astype(np.int64)
                if pt is not None:
                    pt[b, h][:, hv] = rpt[:, hv]
        return codes, pt

    def step(S, kind):
        nonlocal hk, hvals
        k = (torch.randn(B, Hkv, S, D, generator=g) * cb.sigma[0]).to(torch.bfloat16)
        v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
        keys, values = layer.update(k.to(DEV), v.to(DEV))
        hk = torch.cat([hk, k.float()], 2)
        hvals = torch.cat([hvals, v.float()], 2)
        T = hk.shape[2]
        codes, pt = oracle_codes()
        got = np_of(keys.codes)
        got = got.view(np.uint16).astype(np.int64) if got.dtype == np.int16 else got.astype(np.int64)
        assert np.array_equal(got, codes), "stored codes"
        q = torch.randn(B, Hq, S, D, generator=g).to(torch.bfloat16)
        last = T - S + np.arange(S)
        causal = np.arange(T)[None, :] <= last[:, None]                        # [S, T]
        keep = np.broadcast_to(causal, (B, 1, S, T)).copy()
        if kind == "masked":  # left padding of each sequence, as HF's mask builder adds it
            for b in range(B):
                keep[b, :, :, :int(rng.integers(0, max(1, T - S)))] = False
        if kind == "full":  # a non-causal step without a mask
            mask_t, causal_arg, keep = None, False, np.ones((B, 1, S, T), bool)
        elif kind == "prefill" or (kind == "decode" and S == 1):
            mask_t, causal_arg = None, True
        else:
            mask_t, causal_arg = torch.from_numpy(keep).to(DEV), None
        out, _ = sunshape_attention_forward(mod, q.to(DEV), keys, values, mask_t, scaling=scaling, is_causal=causal_arg)
        add = np.broadcast_to(np.where(keep, 0.0, -np.inf).astype(np.float32), (B, Hq, S, T))
        ref = O.decode_attention(q.float().numpy(), codes, hvals.numpy(),
                                 cb.centroids.numpy() if c["per_head"] else cb.centroids[0].numpy(),
                                 cb.perm.numpy() if c["per_head"] else cb.perm[0].numpy(),
                                 1 / math.sqrt(D) if scaling is None else scaling, "bf16", "bf16", mask=add,
                                 heavy=hv, pt_values=pt)
        assert_rel(np_of(out.transpose(1, 2)), ref, BF16_TOL, f"{kind} step of {S} at length {T}")

    step(int(rng.integers(1, 200)), "prefill")
    for i in range(c["ops"]):
        op = str(rng.choice(["decode", "decode", "decode_masked", "multi", "multi_full", "crop", "reorder"]))
        log(f"op {i}: {op} at length {hk.shape[2]}")
        if op == "decode":
            step(1, "decode")
        elif op == "decode_masked":
            step(1, "masked")
        elif op == "multi":
            step(int(rng.integers(2, 25)), "masked")
        elif op == "multi_full":
            step(int(rng.integers(2, 25)), "full")
        elif op == "crop":
            if hk.shape[2] < 2:
                continue
            n = int(rng.integers(1, min(6, hk.shape[2])))
            layer.crop(-n)
            hk, hvals = hk[:, :, :-n], hvals[:, :, :-n]
            assert layer.get_seq_length() == hk.shape[2]
        else:
            beam = torch.from_numpy(rng.permutation(B)).long()
            layer.reorder_cache(beam.to(DEV))
            hk, hvals = hk[beam], hvals[beam]
