"""Rotated-mode codecs (dense rotation R, sunshape/codec.py:241-259) and torch.cdist's direct
distance (<= 25 keys per reference call with <= 25 codewords) on the HIP path, against the oracle.

Rotated mode: the row transform is bit-exact with the oracle's; encode indices and dequantized
keys are bit-exact; scores within 1e-4 and bf16 outputs within 2e-2 (norm-relative).
Direct distance: encode indices bit-exact with the oracle's direct mode, and equal to this host's
torch.cdist except on near-ties."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic
from sunshape_amd import vllm_attn_backend as VB
from sunshape_amd.codec import SunShapeBlockCodec, SunShapeQuantized

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _rotation(D, seed):
    g = torch.Generator().manual_seed(seed)
    qm, _ = torch.linalg.qr(torch.randn(D, D, generator=g, dtype=torch.float64))
    return qm.float()


def _rotated_codec(D, bd, seed, nkv=None, nc=256):
    """A rotated-mode codec with a random orthogonal R and codebooks in the rotated basis."""
    cb = synthetic.make_codebook(nkv or 1, D, bd, seed, n_centroids=nc)
    cent = cb.centroids if nkv else cb.centroids[0]
    codec = SunShapeBlockCodec(head_dim=D, block_dim=bd, n_centroids=nc, use_rotation=True, device=DEV,
                               num_kv_heads=nkv)
    codec.centroids.copy_(cent.to(DEV))
    codec.rotation.copy_(_rotation(D, seed + 1).to(DEV))
    assert codec.mode == "rotated" and codec.unsupported_reason() is None
    return codec


@pytest.mark.parametrize("D,rows,dtype,scale", [(64, 1000, torch.float32, None), (128, 77, torch.bfloat16, 0.125),
                                                (256, 33, torch.float16, 0.0625), (300, 5, torch.float32, None)])
def test_transform_rows_bit_exact_vs_oracle(D, rows, dtype, scale):
    log(f"transform rows D={D} rows={rows} {dtype} scale={scale}")
    g = torch.Generator().manual_seed(D + rows)
    x = (torch.randn(rows, D, generator=g) * 3).to(dtype)
    R = torch.randn(D, D, generator=g)
    xs = O.query_scale(x.float().numpy(), scale, {torch.float32: "f32", torch.bfloat16: "bf16",
                                                 torch.float16: "f16"}[dtype])
    for transpose in (False, True):
        got = np_of(hip_ops.transform_rows(x.to(DEV), R.to(DEV), transpose=transpose, scale=scale))
        ref = O.transform_rows(xs, R.numpy(), transpose=transpose)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (transpose, np.abs(got - ref).max())


@pytest.mark.parametrize("D,bd", [(64, 2), (128, 4), (64, 8)])
def test_rotated_codec_quantize_dequantize_bit_exact(D, bd):
    log(f"rotated codec quantize/dequantize D={D} bd={bd}")
    codec = _rotated_codec(D, bd, 61 + D + bd)
    R = codec.rotation.cpu().numpy()
    g = torch.Generator().manual_seed(7)
    keys = torch.randn(2500, D, generator=g).to(torch.bfloat16)
    qz = codec.quantize(keys.to(DEV))
    ref_codes, _ = O.encode(keys.float().numpy(), np.arange(D), codec.centroids.cpu().numpy(), rotation=R)
    assert np.array_equal(np_of(qz.indices), ref_codes), int((np_of(qz.indices) != ref_codes).sum())
    k_hat = np_of(codec.dequantize(qz))
    ref_hat = O.dequantize(ref_codes, codec.centroids.cpu().numpy(), np.arange(D), rotation=R)
    assert np.array_equal(k_hat.view(np.uint32), ref_hat.view(np.uint32))
    # the inverse transform really is x @ R (an orthogonal R brings the codewords back near the keys)
    err = np.abs(k_hat - keys.float().numpy()).mean()
    assert err < np.abs(keys.float().numpy()).mean()


def test_rotated_scores_vs_oracle_and_dequantize_matmul():
    log("rotated attention_scores")
    D, bd = 64, 8
    codec = _rotated_codec(D, bd, 71)
    R = codec.rotation.cpu().numpy()
    g = torch.Generator().manual_seed(8)
    codes = torch.randint(0, 256, (3000, D // bd), generator=g, dtype=torch.uint8)
    q = torch.randn(5, D, generator=g)
    qz = SunShapeQuantized(indices=codes.to(DEV), head_dim=D, block_dim=bd, n_blocks=D // bd)
    got = np_of(codec.attention_scores(q.to(DEV), qz))
    ref = O.attention_scores(q.numpy(), codes.numpy(), codec.centroids.cpu().numpy(), np.arange(D), rotation=R)
    assert_rel(got, ref, SCORE_TOL, "rotated scores vs oracle")
    # the reference's fallback: dequantize to the original basis, then q @ k_hat^T
    k_hat = O.dequantize(codes.numpy(), codec.centroids.cpu().numpy(), np.arange(D), rotation=R)
    assert_rel(got, q.numpy().astype(np.float64) @ k_hat.astype(np.float64).T, SCORE_TOL, "vs dequantize+matmul")


@pytest.mark.parametrize("paged", [False, True])
def test_rotated_decode_vs_oracle(paged):
    log(f"rotated decode paged={paged}")
    if paged:
        B, Hq, Hkv, T, D, bd = 2, 32, 8, 2048, 128, 4
        p = synthetic.config4(DEV, B=B, T=T)
        R = _rotation(D, 81).to(DEV)
        out, lse, scores = hip_ops.decode(p["q"], p["code_pages"], p["v_pages"], p["perm"], p["centroids"],
                                          scale=p.meta["scale"], block_table=p["block_table"],
                                          seq_lens=p["seq_lens"], return_lse=True, return_scores=True, rotation=R)
        bt = p["block_table"].cpu().numpy()
        codes = np.stack([O.gather_pages_codes(np_of(p["code_pages"]), bt[b], T) for b in range(B)])
        v = np.stack([O.gather_pages_values(np_of(p["v_pages"]), bt[b], T) for b in range(B)])
    else:
        B, Hq, Hkv, T, D, bd = 4, 14, 2, 3000, 64, 2
        p = synthetic.config3(DEV, B=B, T=T)
        R = _rotation(D, 82).to(DEV)
        out, lse, scores = hip_ops.decode(p["q"], p["codes"], p["v"], p["perm"], p["centroids"],
                                          scale=p.meta["scale"], return_lse=True, return_scores=True, rotation=R)
        codes, v = np_of(p["codes"]), np_of(p["v"])
    ro, rs, rl = O.decode_attention(np_of(p["q"]), codes, v, np_of(p["centroids"]), np_of(p["perm"]),
                                    p.meta["scale"], "bf16", "bf16", return_scores=True, rotation=np_of(R))
    assert_rel(np_of(out), ro, BF16_TOL, "rotated decode out")
    assert_rel(np_of(scores), rs, SCORE_TOL, "rotated decode scores")
    assert_rel(np_of(lse), rl, SCORE_TOL, "rotated decode lse")


def test_rotated_backend_end_to_end():
    """quantize_key_states + SunShapeAttentionImpl.forward on a rotated per-layer codec."""
    log("rotated backend end to end")
    from sunshape_amd.hf import SunShapeBundle
    from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState

    B, Hq, Hkv, S, D, bd = 2, 8, 2, 700, 64, 2
    codec = _rotated_codec(D, bd, 91)
    bundle = SunShapeBundle("m", [0], 4.0, bd, "rotated", 0, 0, 0, {0: codec})
    VB.register_runtime_state(SunShapeVLLMRuntimeState("p", "m", "rotated", 4.0, bd, [0], bundle, "cuda"))
    try:
        g = torch.Generator().manual_seed(92)
        keys = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
        qk = VB.quantize_key_states(0, keys.to(DEV))
        R = codec.rotation.cpu().numpy()
        cent = codec.centroids.cpu().numpy()
        for b in range(B):
            for h in range(Hkv):
                rc, _ = O.encode(keys[b, h].float().numpy(), np.arange(D), cent, rotation=R)
                assert np.array_equal(np_of(qk.codes[b, h]), rc)
        q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
        impl = VB.get_backend_factory().make_impl(layer_idx=0)
        out = np_of(impl(q, qk, v, scale=1 / math.sqrt(D)))
        ref = O.decode_attention(np_of(q), np_of(qk.codes), np_of(v), cent, np.arange(D), 1 / math.sqrt(D),
                                 "bf16", "bf16", rotation=R)
        assert_rel(out, ref, BF16_TOL, "rotated impl.forward")
    finally:
        VB.clear_registered_runtime()


# ----------------------------------------------------------------------------- direct distance
def _midpoint_problem(seed, n, D=64, bd=2, nc=16):
    """Keys near midpoints of codeword pairs (where the formulation decides the winner) plus
    random keys, for a 16-codeword codec (2 bits/dim at block_dim 2)."""
    rng = np.random.default_rng(seed)
    nb = D // bd
    perm = rng.permutation(D)
    cent = (rng.standard_normal((nb, nc, bd)) * 2).astype(np.float32)
    i, j = rng.integers(0, nc, (n, nb)), rng.integers(0, nc, (n, nb))
    xp = 0.5 * (cent[np.arange(nb), i] + cent[np.arange(nb), j]) + rng.standard_normal((n, nb, bd)) * 1e-6
    xp = xp.reshape(n, D).astype(np.float32)
    xp[n // 2:] = (rng.standard_normal((n - n // 2, D)) * 2).astype(np.float32)
    keys = np.empty_like(xp)
    keys[:, perm] = xp          # x[..., perm] == xp
    return keys, perm, cent


def test_direct_distance_encode_bit_exact_vs_oracle():
    log("direct-distance encode vs oracle (nc=16, <= 25 keys per call)")
    keys, perm, cent = _midpoint_problem(101, 4000)
    t = lambda a: torch.from_numpy(a).to(DEV)
    got, _ = hip_ops.encode(t(keys)[None, None], t(perm), t(cent), direct=True)
    ref, _ = O.encode(keys, perm, cent, direct=True)
    assert np.array_equal(np_of(got[0, 0]), ref), int((np_of(got[0, 0]) != ref).sum())
    mm, _ = O.encode(keys, perm, cent, direct=False)
    assert (mm != ref).any(), "the midpoint keys should separate the two formulations"
    with pytest.raises(RuntimeError, match="direct_dist"):
        hip_ops.encode(t(keys)[None, None], t(perm), t(cent), direct=True, kernel=2)


def test_direct_distance_through_codec_and_quantize_key_states():
    """The host picks the formulation from the reference call's row count: codec.quantize with
    <= 25 keys and quantize_key_states with seq_len <= 25 take the direct distance, larger calls
    the mm formulation; each against the oracle, and against this host's torch.cdist up to
    near-ties."""
    log("direct-distance encode through the codec and quantize_key_states")
    from sunshape_amd.hf import SunShapeBundle
    from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState

    keys, perm, cent = _midpoint_problem(102, 3 * 64)
    codec = SunShapeBlockCodec.from_buffers(torch.from_numpy(perm), torch.from_numpy(cent), device=DEV)
    for n in (1, 25, 26, 64):
        got = np_of(codec.quantize(torch.from_numpy(keys[:n]).to(DEV)).indices)
        ref, _ = O.encode(keys[:n], perm, cent, direct=n <= 25)
        assert np.array_equal(got, ref), n
        xp = keys[:n][:, perm]
        for b in range(cent.shape[0]):
            tc = torch.cdist(torch.from_numpy(xp[:, 2 * b:2 * b + 2].copy()), torch.from_numpy(cent[b]))
            want = tc.argmin(-1).numpy()
            d = tc.numpy()
            for r in np.nonzero(got[:, b] != want)[0]:
                a, c2 = d[r, got[r, b]], d[r, want[r]]
                assert abs(a - c2) <= 4 * np.spacing(np.float32(max(min(a, c2), 1e-30))), (n, b, r, a, c2)
    bundle = SunShapeBundle("m", [0], 2.0, 2, "profileperm_baseline", 0, 0, 0, {0: codec})
    VB.register_runtime_state(SunShapeVLLMRuntimeState("p", "m", "sunshape_base", 2.0, 2, [0], bundle, "cuda"))
    try:
        for S in (1, 25, 30):
            B, Hkv = 64 // S if S < 64 else 1, 2
            k4 = keys[:B * Hkv * S].reshape(B, Hkv, S, -1)
            qk = VB.quantize_key_states(0, torch.from_numpy(k4).to(DEV))
            for b in range(B):
                for h in range(Hkv):
                    ref, _ = O.encode(k4[b, h], perm, cent, direct=S <= 25)
                    assert np.array_equal(np_of(qk.codes[b, h]), ref), (S, b, h)
    finally:
        VB.clear_registered_runtime()
