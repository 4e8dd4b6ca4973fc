"""Oracle vs the committed golden fixtures (tests/golden/make_golden.py).  CPU only."""

import os

import numpy as np

from oracle import vq_oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _bf16(bits):
    return (np.asarray(bits).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)


def test_c1_scores_fixture():
    f = np.load(os.path.join(G, "c1_scores.npz"))
    got = O.attention_scores(f["q"], f["codes"], f["centroids"], f["perm"])
    ref = f["scores_lut"]
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    ref_dq = f["scores_dequant"]
    assert np.abs(got - ref_dq).max() <= 1e-5 * np.abs(ref_dq).max()
    lut = O.lut_build(O.forward_transform(f["q"], f["perm"]), f["centroids"])
    np.testing.assert_allclose(lut, f["lut"], rtol=1e-6, atol=1e-6 * np.abs(f["lut"]).max())


def test_encode_fixture_bit_exact():
    f = np.load(os.path.join(G, "encode_mixed.npz"))
    keys = _bf16(f["keys_bf16_bits"])
    codes, pt = O.encode(keys, f["perm"], f["centroids"], f["heavy"])
    assert np.array_equal(codes, f["codes"])
    assert np.array_equal(pt, f["passthrough"])


def test_decode_fixture():
    f = np.load(os.path.join(G, "decode_small.npz"))
    q = _bf16(f["q_bf16_bits"])
    v = _bf16(f["v_bf16_bits"])
    out, scores, _ = O.decode_attention(q, f["codes"], v, f["centroids"], f["perm"], float(f["scale"]), "bf16", "bf16",
                                        return_scores=True)
    ref = _bf16(f["out_bf16_bits"])
    assert np.abs(out - ref).max() <= 2e-2 * np.abs(ref).max()
    assert np.abs(scores - f["scores"]).max() <= 1e-5 * np.abs(f["scores"]).max()
