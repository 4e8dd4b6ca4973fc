"""A seeded serving loop over PagedSunShapeCache: prefills of random lengths, single-token
appends to random subsets of sequences, decodes of random subsets (one or two new tokens), and
sequences freed and started again, so that recycled pages hold stale codes and values past
every live sequence's length.  Per case one codec (per layer or per KV head, baseline or
SunShape-Mixed, 256 or 1,024 codewords, block_dim 2 (grid-search encode) or 4).  Every decode is
compared with the oracle over the sequence's whole key and value history
(sunshape/codec.py:362-385 for the codes, sunshape/vllm_attn_backend.py:216-253 for the
attention); the pages' codes are checked bit for bit against the oracle's encode."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import synthetic
from sunshape_amd.codec import SunShapeBlockCodec
from sunshape_amd.paged import PagedSunShapeCache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _draw(seed):
    rng = np.random.default_rng(seed)
    return dict(seed=seed, D=int(rng.choice([64, 128])), bd=int(rng.choice([2, 4])),
                nc=int(rng.choice([256, 256, 1024])), per_head=bool(rng.integers(0, 2)),
                mixed=bool(rng.integers(0, 3) == 0), Hkv=int(rng.choice([1, 2])), G=int(rng.choice([1, 4, 7])),
                steps=int(rng.integers(6, 12)))


@pytest.mark.parametrize("seed", list(range(300, 320)))
def test_paged_serving_loop_vs_oracle(seed):
    c = _draw(seed)
    log(f"paged serving loop {c}")
    D, bd, nc, Hkv, G = c["D"], c["bd"], c["nc"], c["Hkv"], c["G"]
    nb, Hq = D // bd, Hkv * c["G"]
    rng = np.random.default_rng(seed + 1)
    g = torch.Generator().manual_seed(seed + 2)
    cb = synthetic.make_codebook(Hkv if c["per_head"] else 1, D, bd, seed, n_centroids=nc, shared_sigma=True)
    heavy = synthetic.heavy_blocks_by_sigma(cb.sigma, cb.perm, bd, 4) if c["mixed"] else None
    perm, cent = (cb.perm, cb.centroids) if c["per_head"] else (cb.perm[0], cb.centroids[0])
    mode = "profileperm_mixed_precision" if c["mixed"] else "profileperm_baseline"
    codec = SunShapeBlockCodec.from_buffers(perm, cent, mode=mode, mixed_high_precision_blocks=heavy, device=DEV)
    cache = PagedSunShapeCache(codec, num_pages=256, num_kv_heads=Hkv, value_dim=D, device=DEV)
    hv = None if heavy is None else heavy.numpy()
    hist = {}  # seq id -> (keys [Hkv, S, D] fp32 list, values list)
    next_id = 0
    sigma = cb.sigma[0]

    def append(ids, S):
        k = (torch.randn(len(ids), Hkv, S, D, generator=g) * sigma).to(torch.bfloat16)
        v = torch.randn(len(ids), Hkv, S, D, generator=g).to(torch.bfloat16)
        cache.append(ids, k.to(DEV), v.to(DEV))
        for i, s in enumerate(ids):
            hist.setdefault(s, ([], []))
            hist[s][0].append(k[i].float())
            hist[s][1].append(v[i].float())

    def check(ids, Lq):
        q = torch.randn(len(ids), Hq, Lq, D, generator=g).to(torch.bfloat16)
        out = np_of(cache.decode(ids, q.to(DEV), scale=1 / math.sqrt(D)))
        pages = np_of(cache.code_pages)
        pages = pages.view(np.uint16).astype(np.int64) if pages.dtype == np.int16 else pages.astype(np.int64)
        for i, s in enumerate(ids):
            keys = torch.cat(hist[s][0], dim=1).numpy()
            vals = torch.cat(hist[s][1], dim=1).numpy()
            T = keys.shape[1]
            table = cache.block_tables[s]
            got = np.concatenate([pages[pg] for pg in table], axis=1)[:, :T]  # [Hkv, T, nb]
            codes = np.zeros((Hkv, T, nb), np.int64)
            pt = None if hv is None else np.zeros((Hkv, T, nb, bd), np.float32)
            for h in range(Hkv):
                ph = (cb.perm[h] if c["per_head"] else cb.perm[0]).numpy()
                ch = (cb.centroids[h] if c["per_head"] else cb.centroids[0]).numpy()
                rc, rpt = O.encode(keys[h], ph, ch, hv)
                codes[h] = rc.astype(np.int64)
                if pt is not None:
                    pt[h][:, hv] = rpt[:, hv]
            assert np.array_equal(got, codes), f"seq {s}: page codes"
            ref = O.decode_attention(q[i:i + 1].float().numpy(), codes[None], vals[None],
                                     cb.centroids.numpy() if c["per_head"] else cb.centroids[0].numpy(),
                                     cb.perm.numpy() if c["per_head"] else cb.perm[0].numpy(), 1 / math.sqrt(D),
                                     "bf16", "bf16", heavy=hv, pt_values=None if pt is None else pt[None])
            assert_rel(out[i:i + 1], ref, BF16_TOL, f"seq {s}")

    # prefills: two sequences of one length, one of another
    ids = [next_id, next_id + 1]
    next_id += 2
    append(ids, int(rng.integers(1, 300)))
    append([next_id], int(rng.integers(1, 300)))
    next_id += 1
    for step in range(c["steps"]):
        live = sorted(hist)
        act = int(rng.integers(0, 4))
        if act == 0 and len(live) > 1:  # a sequence ends; its pages go back to the pool
            s = int(rng.choice(live))
            cache.free(s)
            del hist[s]
        elif act == 1:  # a new sequence's prefill (recycled pages)
            append([next_id], int(rng.integers(1, 200)))
            next_id += 1
        else:  # a decode step's append for a subset of the live sequences
            sub = sorted(rng.choice(live, size=int(rng.integers(1, len(live) + 1)), replace=False).tolist())
            append(sub, 1)
        live = sorted(hist)
        sub = sorted(rng.choice(live, size=int(rng.integers(1, len(live) + 1)), replace=False).tolist())
        log(f"step {step}: action {act}, decode {sub} of lengths {[cache.seq_lens[s] for s in sub]}")
        check(sub, int(rng.choice([1, 1, 2])))
