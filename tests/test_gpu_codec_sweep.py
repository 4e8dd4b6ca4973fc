"""A seeded sweep of the codec surface the reference's callers use (sunshape/codec.py:362-422,
sunshape/triton_kernels.py:549-609): codec.quantize, codec.dequantize, codec(keys) and the two
score entry points, codec.attention_scores and sunshape_attention_scores, over every mode the
kernels serve -- identity, ProfilePerm, SunShape-Mixed, SunShape-Pro's block metric
(profileperm_localmetric_dsq), legacy_strict (identity permutation under a metric) and
rotated -- with per-layer or per-KV-head codebooks (kv_head=), 16 to 1,024 codewords, block
dims 1 to 8 and key and query dtypes.  Codes, passthrough values and dequantized keys are
bit-exact with the oracle; the two score entry points agree bit for bit and with the oracle
within the scores tolerance."""

import numpy as np
import pytest
import torch

from _util import SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import kernels, synthetic
from sunshape_amd.codec import SunShapeBlockCodec

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
MODES = ["identity_baseline", "profileperm_baseline", "profileperm_mixed_precision", "profileperm_localmetric_dsq",
         "legacy_strict", "rotated"]


def _draw(seed):
    rng = np.random.default_rng(seed)
    D = int(rng.choice([32, 64, 128]))
    bd = int(rng.choice([b for b in (1, 2, 4, 8) if D // b <= 128]))
    return dict(seed=seed, D=D, bd=bd, nc=int(rng.choice([16, 256, 256, 1024])), mode=str(rng.choice(MODES)),
                nkv=int(rng.choice([0, 0, 2])), N=int(rng.integers(1, 800)), R=int(rng.integers(1, 40)),
                kdt=str(rng.choice(["bf16", "f32"])), qdt=str(rng.choice(["f32", "bf16", "f16"])))


@pytest.mark.parametrize("seed", list(range(600, 636)))
def test_codec_surface_sweep_vs_oracle(seed):
    c = _draw(seed)
    log(f"codec sweep {c}")
    D, bd, nc, mode, nkv = c["D"], c["bd"], c["nc"], c["mode"], c["nkv"]
    nb = D // bd
    rng = np.random.default_rng(seed + 1)
    cb = synthetic.make_codebook(max(nkv, 1), D, bd, seed, n_centroids=nc, shared_sigma=True)
    codec = SunShapeBlockCodec(head_dim=D, block_dim=bd, n_centroids=nc, mode=mode if mode != "rotated" else
                               "profileperm_baseline", use_rotation=mode == "rotated", device=DEV,
                               num_kv_heads=nkv or None)
    codec.centroids.copy_((cb.centroids if nkv else cb.centroids[0]).to(DEV))
    codec.permutation.copy_((cb.perm if nkv else cb.perm[0]).to(DEV))
    codec.inv_permutation.copy_(torch.argsort(codec.permutation, dim=-1))
    heavy = None
    if mode == "profileperm_mixed_precision":
        heavy = synthetic.heavy_blocks_by_sigma(cb.sigma, cb.perm, bd, min(3, nb - 1) or 1)
        codec.mixed_high_precision_blocks.copy_(heavy.to(DEV))
    E = R = None
    if mode in ("profileperm_localmetric_dsq", "legacy_strict"):
        E = (np.eye(D) + 0.2 * rng.standard_normal((D, D)) / np.sqrt(D)).astype(np.float32)
        codec.E = torch.from_numpy(E).to(DEV)
    if mode == "rotated":
        R = np.linalg.qr(rng.standard_normal((D, D)))[0].astype(np.float32)
        codec.rotation.copy_(torch.from_numpy(R).to(DEV))
    assert codec.unsupported_reason() is None
    hv = None if heavy is None else heavy.numpy()
    g = torch.Generator().manual_seed(seed + 2)
    for h in (range(nkv) if nkv else [None]):
        hh = 0 if h is None else h
        keys = (torch.randn(c["N"], D, generator=g) * cb.sigma[0]).to(DT[c["kdt"]])
        q = torch.randn(c["R"], D, generator=g).to(DT[c["qdt"]])
        perm = codec.effective_permutation(h).cpu().numpy()
        cent = cb.centroids[hh].numpy()
        qz = codec.quantize(keys.to(DEV), kv_head=h)
        direct = c["N"] <= 25 and nc <= 25  # torch.cdist evaluates such a call directly
        rc, rpt = O.encode(keys.float().numpy(), perm, cent, hv, metric=E, direct=direct, rotation=R)
        got = np_of(qz.indices)
        got = got.view(np.uint16).astype(np.int64) if got.dtype == np.int16 else got.astype(np.int64)
        assert np.array_equal(got, rc.astype(np.int64)), f"codes head {h}"
        pt = None
        if hv is not None:
            pt = np.zeros_like(rpt)
            pt[:, hv] = rpt[:, hv]
            assert np.array_equal(np_of(qz.passthrough_values), pt), f"passthrough head {h}"
        k_hat = np_of(codec.dequantize(qz, kv_head=h))
        ref_k = O.dequantize(rc, cent, perm, hv, pt, rotation=R)
        assert np.array_equal(k_hat, ref_k), f"dequantize head {h}"
        assert np.array_equal(np_of(codec(keys.to(DEV), kv_head=h)), ref_k), f"codec(keys) head {h}"
        s1 = np_of(codec.attention_scores(q.to(DEV), qz, kv_head=h))
        s2 = np_of(kernels.sunshape_attention_scores(codec, q.to(DEV), qz, kv_head=h))
        assert np.array_equal(s1, s2), "the two score entry points differ"
        ref_s = O.attention_scores(q.float().numpy(), rc, cent, perm, hv, pt, rotation=R)
        assert_rel(s1, ref_s, SCORE_TOL, f"scores head {h}")
