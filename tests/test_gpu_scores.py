"""HIP score path vs the oracle: LUT build, single-head scores (config 1),
batched GQA scores (config 2), passthrough blocks, error paths."""

import math
import os

import numpy as np
import pytest
import torch

from _util import SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic
from sunshape_amd.codec import SunShapeBlockCodec, SunShapeQuantized
from sunshape_amd.kernels import sunshape_attention_scores, sunshape_attention_scores_strict

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_native_library_is_the_one_loaded():
    from sunshape_amd import _native as N

    N.lib()
    maps = open("/proc/self/maps").read()
    assert N.LIB_PATH in maps
    hip = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
    assert len(hip) == 1, hip


@pytest.mark.parametrize("D,bd,R", [(64, 8, 1), (64, 2, 7), (128, 4, 4), (64, 1, 3)])
def test_lut_build_vs_oracle(D, bd, R):
    log(f"lut_build D={D} bd={bd} R={R}")
    rng = np.random.default_rng(D + bd + R)
    perm = rng.permutation(D)
    cent = rng.standard_normal((D // bd, 256, bd)).astype(np.float32)
    q = rng.standard_normal((R, D)).astype(np.float32)
    got = hip_ops.lut_build(torch.from_numpy(q).to(DEV), torch.from_numpy(perm).to(DEV), torch.from_numpy(cent).to(DEV))
    ref = O.lut_build(O.forward_transform(q, perm), cent)
    assert_rel(np_of(got), ref, 1e-6, "lut")


def test_config1_scores_vs_golden_and_oracle():
    log("config1 scores")
    f = np.load(os.path.join(GOLD, "c1_scores.npz"))
    codec = SunShapeBlockCodec.from_buffers(torch.from_numpy(f["perm"]), torch.from_numpy(f["centroids"]), device=DEV)
    qk = SunShapeQuantized(torch.from_numpy(f["codes"]).to(DEV), 64, 8, 8)
    q = torch.from_numpy(f["q"]).to(DEV)
    got = np_of(sunshape_attention_scores(codec, q, qk))
    assert_rel(got, f["scores_lut"], SCORE_TOL, "c1 vs golden LUT path")
    assert_rel(got, f["scores_dequant"], SCORE_TOL, "c1 vs golden dequant path")
    assert_rel(got, O.attention_scores(f["q"], f["codes"], f["centroids"], f["perm"]), SCORE_TOL, "c1 vs oracle")
    # the configuration's output: scores scaled by 1/sqrt(64), exact for a power of two
    scaled = np_of(sunshape_attention_scores(codec, q * float(f["scale"]), qk))
    assert np.array_equal(scaled, got * np.float32(f["scale"]))
    # codec-level entry point (sunshape/codec.py:403-422)
    assert np.array_equal(np_of(codec.attention_scores(q, qk)), got)


@pytest.mark.parametrize("B,T", [(2, 1000), (16, 8192)])
@pytest.mark.parametrize("kernel", [0, 1])  # auto (the contiguous 4x4-MFMA kernel), the LUT kernel
def test_config2_gqa_scores_vs_oracle(B, T, kernel):
    log(f"config2 gqa scores B={B} T={T} kernel={kernel}")
    p = synthetic.config2(DEV, B=B, T=T)
    scale = p.meta["scale"]
    got = np_of(hip_ops.gqa_scores(p["q"], p["codes"], p["perm"], p["centroids"], scale=scale, kernel=kernel))
    q = np_of(p["q"])
    codes = np_of(p["codes"])
    perm = np_of(p["perm"])
    cent = np_of(p["centroids"])
    G = 7
    for b in range(B):
        for kv in range(2):
            qs = O.query_scale(q[b, kv * G:(kv + 1) * G, 0], scale, "bf16")
            ref = O.attention_scores(qs, codes[b, kv], cent[kv], perm[kv])
            assert_rel(got[b, kv * G:(kv + 1) * G, 0], ref, SCORE_TOL, f"c2 b={b} kv={kv}")


@pytest.mark.parametrize("kernel", [0, 1])
def test_scores_single_head_shapes_and_ragged_T(kernel):
    log(f"scores ragged T kernel={kernel}")
    rng = np.random.default_rng(3)
    perm = rng.permutation(64)
    cent = rng.standard_normal((8, 256, 8)).astype(np.float32)
    for T in (1, 7, 255, 256, 257, 3001):
        for R in (1, 9, 16):
            codes = rng.integers(0, 256, (T, 8)).astype(np.uint8)
            q = rng.standard_normal((R, 64)).astype(np.float32)
            got = hip_ops.attention_scores(torch.from_numpy(q).to(DEV), torch.from_numpy(codes).to(DEV),
                                           torch.from_numpy(perm).to(DEV), torch.from_numpy(cent).to(DEV),
                                           kernel=kernel)
            assert_rel(np_of(got), O.attention_scores(q, codes, cent, perm), SCORE_TOL, f"T={T} R={R}")


def test_scores_fewer_centroids_and_bf16_query():
    log("scores nc=16 bf16 q")
    rng = np.random.default_rng(4)
    perm = rng.permutation(64)
    cent = rng.standard_normal((16, 16, 4)).astype(np.float32)
    codes = rng.integers(0, 16, (500, 16)).astype(np.uint8)
    q = torch.randn(5, 64).to(torch.bfloat16)
    got = hip_ops.attention_scores(q.to(DEV), torch.from_numpy(codes).to(DEV), torch.from_numpy(perm).to(DEV),
                                   torch.from_numpy(cent).to(DEV))
    assert_rel(np_of(got), O.attention_scores(q.float().numpy(), codes, cent, perm), SCORE_TOL, "nc=16")


def test_scores_with_passthrough_dense_and_compact():
    log("scores passthrough")
    rng = np.random.default_rng(5)
    D, bd, T = 64, 2, 777
    perm = rng.permutation(D)
    cent = rng.standard_normal((32, 256, bd)).astype(np.float32)
    heavy = np.zeros(32, bool)
    heavy[[1, 7, 8, 30]] = True
    codes = rng.integers(0, 256, (T, 32)).astype(np.uint8)
    codes[:, heavy] = 0
    pt = np.zeros((T, 32, bd), np.float32)
    pt[:, heavy] = rng.standard_normal((T, 4, bd)).astype(np.float32)
    q = rng.standard_normal((6, D)).astype(np.float32)
    ref = O.attention_scores(q, codes, cent, perm, heavy, pt)
    args = [torch.from_numpy(x).to(DEV) for x in (q, codes, perm, cent)]
    dense = hip_ops.attention_scores(*args, heavy=heavy.tolist(), pt=torch.from_numpy(pt).to(DEV), pt_dense=True)
    assert_rel(np_of(dense), ref, SCORE_TOL, "dense pt")
    compact = torch.from_numpy(np.ascontiguousarray(pt[:, heavy])).to(DEV).to(torch.bfloat16)
    ref_c = O.attention_scores(q, codes, cent, perm, heavy, O.bf16_round(pt))
    got_c = hip_ops.attention_scores(*args, heavy=heavy.tolist(), pt=compact, pt_dense=False)
    assert_rel(np_of(got_c), ref_c, SCORE_TOL, "compact bf16 pt")


def test_scores_error_paths_raise():
    log("scores errors")
    codec = SunShapeBlockCodec(head_dim=64, block_dim=8, device=DEV)
    q = torch.randn(2, 64, device=DEV)
    with pytest.raises(RuntimeError, match="block count"):
        sunshape_attention_scores_strict(codec, q, SunShapeQuantized(torch.zeros(4, 7, dtype=torch.uint8, device=DEV), 64, 8, 7))
    with pytest.raises(RuntimeError, match="head dim"):
        sunshape_attention_scores(codec, torch.randn(2, 32, device=DEV), SunShapeQuantized(torch.zeros(4, 8, dtype=torch.uint8, device=DEV), 64, 8, 8))
    with pytest.raises(RuntimeError, match="ndim"):
        sunshape_attention_scores(codec, torch.randn(2, 1, 64, device=DEV), SunShapeQuantized(torch.zeros(4, 8, dtype=torch.uint8, device=DEV), 64, 8, 8))
