"""Pins the numpy oracle (oracle/vq_oracle.py) against closed forms, invariants,
brute force and the torch library calls the reference makes.  CPU only."""

import math

import numpy as np
import pytest
import torch

from oracle import vq_oracle as O


def _rng(seed=0):
    return np.random.default_rng(seed)


def _codec(rng, D, bd, nc=256):
    perm = rng.permutation(D)
    sig = np.exp(rng.uniform(math.log(0.1), math.log(3), D)).astype(np.float32)
    cent = (rng.standard_normal((D // bd, nc, bd)) * sig[perm].reshape(D // bd, 1, bd)).astype(np.float32)
    return perm, cent


# ----------------------------------------------------------------------------- dtype rounding
def test_bf16_round_bit_exact_vs_torch():
    rng = _rng(1)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-20, 20, 200000))).astype(np.float32)
    # exact ties (low half == 0x8000) with even and odd upper halves
    ties = (rng.integers(0x3F00, 0x4100, 5000).astype(np.uint32) << 16) | 0x8000
    x = np.concatenate([x, ties.view(np.float32), np.float32([0.0, -0.0, 1.0, -1.5, 3.0e38])])
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.bf16_round(x).view(np.uint32), ref.view(np.uint32))


def test_f16_round_bit_exact_vs_torch():
    x = (_rng(2).standard_normal(100000) * 10).astype(np.float32)
    ref = torch.from_numpy(x.copy()).to(torch.float16).float().numpy()
    assert np.array_equal(O.f16_round(x), ref)


def test_query_scale_matches_torch_bf16_multiply():
    q = torch.randn(64, 128).to(torch.bfloat16)
    for scale in (1 / math.sqrt(128), 1 / math.sqrt(64), 0.3):
        ref = (q * float(scale)).float().numpy()
        got = O.query_scale(q.float().numpy(), scale, "bf16")
        assert np.array_equal(got, ref)


# ----------------------------------------------------------------------------- transforms
def test_permutation_adjointness_exact():
    """q . inv(k) == fwd(q) . k for integer vectors (exact); fails for a swapped direction."""
    rng = _rng(3)
    D = 64
    perm = rng.permutation(D)
    while np.array_equal(perm[perm], np.arange(D)):  # need a non-involution
        perm = rng.permutation(D)
    q = rng.integers(-50, 50, D).astype(np.float64)
    k = rng.integers(-50, 50, D).astype(np.float64)
    assert q @ O.inverse_transform(k, perm) == O.forward_transform(q, perm) @ k
    assert np.array_equal(O.inverse_transform(O.forward_transform(q, perm), perm), q)
    # the mistake of using perm in both directions is detected by the same identity
    wrong = k[..., perm]
    assert q @ wrong != O.forward_transform(q, perm) @ k


def test_invert_permutation_matches_torch_scatter():
    perm = _rng(4).permutation(128)
    inv = torch.empty(128, dtype=torch.long)
    inv[torch.from_numpy(perm)] = torch.arange(128)
    assert np.array_equal(O.invert_permutation(perm), inv.numpy())


# ----------------------------------------------------------------------------- LUT
def test_lut_brute_force_tiny():
    rng = _rng(5)
    D, bd, nc, R = 8, 2, 5, 3
    cent = rng.standard_normal((D // bd, nc, bd)).astype(np.float32)
    qp = rng.standard_normal((R, D)).astype(np.float32)
    lut = O.lut_build(qp, cent)
    for r in range(R):
        for b in range(D // bd):
            for c in range(nc):
                ref = sum(float(qp[r, b * bd + d]) * float(cent[b, c, d]) for d in range(bd))
                assert abs(lut[r, b, c] - ref) <= 1e-6 * (abs(ref) + 1e-6)


def test_lut_one_hot_query_reads_codebook_coordinate():
    rng = _rng(6)
    D, bd = 64, 4
    perm, cent = _codec(rng, D, bd)
    inv = O.invert_permutation(perm)
    for j in (0, 17, 63):
        q = np.zeros((1, D), np.float32)
        q[0, j] = 1.0
        lut = O.lut_build(O.forward_transform(q, perm), cent)
        p = inv[j]
        b, d = divmod(int(p), bd)
        assert np.array_equal(lut[0, b], cent[b, :, d])
        others = np.delete(lut[0], b, axis=0)
        assert not others.any()


def test_lut_matches_torch_einsum():
    rng = _rng(7)
    perm, cent = _codec(rng, 128, 4)
    qp = rng.standard_normal((4, 128)).astype(np.float32)
    ref = torch.einsum("qbd,bcd->qbc", torch.from_numpy(qp).view(4, 32, 4), torch.from_numpy(cent)).numpy()
    np.testing.assert_allclose(O.lut_build(qp, cent), ref, rtol=2e-6, atol=2e-6 * np.abs(ref).max())


# ----------------------------------------------------------------------------- scores
@pytest.mark.parametrize("D,bd", [(64, 8), (64, 2), (128, 4)])
def test_scores_gather_sum_equals_dequantize_matmul(D, bd):
    rng = _rng(8 + D + bd)
    perm, cent = _codec(rng, D, bd)
    T, R = 3000, 5
    codes = rng.integers(0, 256, (T, D // bd)).astype(np.uint8)
    q = rng.standard_normal((R, D)).astype(np.float32)
    got = O.attention_scores(q, codes, cent, perm)
    k_hat = O.dequantize(codes, cent, perm)
    ref = q.astype(np.float64) @ k_hat.astype(np.float64).T
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    # and against torch's fp32 matmul of the dequantized keys (the reference's eager oracle)
    ref32 = torch.matmul(torch.from_numpy(q), torch.from_numpy(k_hat).T).numpy()
    assert np.abs(got - ref32).max() <= 1e-5 * np.abs(ref32).max()


def test_scores_with_passthrough_blocks():
    rng = _rng(9)
    D, bd = 64, 2
    perm, cent = _codec(rng, D, bd)
    nb = D // bd
    heavy = np.zeros(nb, bool)
    heavy[[3, 10, 11, 30]] = True
    T = 500
    codes = rng.integers(0, 256, (T, nb)).astype(np.uint8)
    codes[:, heavy] = 0
    pt = np.zeros((T, nb, bd), np.float32)
    pt[:, heavy] = rng.standard_normal((T, heavy.sum(), bd)).astype(np.float32)
    q = rng.standard_normal((3, D)).astype(np.float32)
    got = O.attention_scores(q, codes, cent, perm, heavy, pt)
    k_hat = O.dequantize(codes, cent, perm, heavy, pt)
    ref = q.astype(np.float64) @ k_hat.astype(np.float64).T
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_scores_power_of_two_scale_is_exact():
    rng = _rng(10)
    perm, cent = _codec(rng, 64, 8)
    codes = rng.integers(0, 256, (4096, 8)).astype(np.uint8)
    q = rng.standard_normal((1, 64)).astype(np.float32)
    a = O.attention_scores(q * np.float32(0.125), codes, cent, perm)
    b = O.attention_scores(q, codes, cent, perm) * np.float32(0.125)
    assert np.array_equal(a, b)


def test_scores_brute_force_tiny():
    rng = _rng(11)
    D, bd, nc = 6, 3, 4
    perm = rng.permutation(D)
    cent = rng.standard_normal((2, nc, bd)).astype(np.float32)
    codes = rng.integers(0, nc, (5, 2)).astype(np.uint8)
    q = rng.standard_normal((2, D)).astype(np.float32)
    got = O.attention_scores(q, codes, cent, perm)
    for r in range(2):
        for t in range(5):
            k = np.zeros(D)
            for b in range(2):
                for d in range(bd):
                    k[perm[b * bd + d]] = cent[b, codes[t, b], d]
            assert abs(got[r, t] - q[r].astype(np.float64) @ k) <= 1e-6 * (np.abs(q[r]) @ np.abs(k) + 1e-9)


# ----------------------------------------------------------------------------- decode
def _decode_problem(rng, B=2, Hq=8, Hkv=2, D=64, bd=2, T=300, Dv=64, Lq=1):
    cents, perms = [], []
    for _ in range(Hkv):
        p, c = _codec(rng, D, bd)
        perms.append(p)
        cents.append(c)
    q = O.bf16_round(rng.standard_normal((B, Hq, Lq, D)).astype(np.float32))
    codes = rng.integers(0, 256, (B, Hkv, T, D // bd)).astype(np.uint8)
    v = O.bf16_round(rng.standard_normal((B, Hkv, T, Dv)).astype(np.float32))
    return q, codes, v, np.stack(cents), np.stack(perms)


def _textbook(q, codes, v, cents, perms, scale, qdtype, mask=None):
    B, Hq, Lq, D = q.shape
    Hkv = codes.shape[1]
    G = Hq // Hkv
    out = np.zeros((B, Hq, Lq, v.shape[-1]))
    for b in range(B):
        for kv in range(Hkv):
            k_hat = O.dequantize(codes[b, kv], cents[kv], perms[kv]).astype(np.float64)
            for g in range(G):
                h = kv * G + g
                qs = O.query_scale(q[b, h], scale, qdtype).astype(np.float64)
                s = qs @ k_hat.T
                if mask is not None:
                    s = s + mask[b, h]
                p = np.exp(s - s.max(-1, keepdims=True))
                p /= p.sum(-1, keepdims=True)
                out[b, h] = p @ v[b, kv].astype(np.float64)
    return out


def test_decode_f32_values_match_fp64_textbook():
    rng = _rng(12)
    q, codes, v, cents, perms = _decode_problem(rng)
    got = O.decode_attention(q, codes, v, cents, perms, 0.125, "bf16", "f32")
    ref = _textbook(q, codes, v, cents, perms, 0.125, "bf16")
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_decode_bf16_within_tolerance_and_lse():
    rng = _rng(13)
    q, codes, v, cents, perms = _decode_problem(rng, Lq=2)
    out, scores, lse = O.decode_attention(q, codes, v, cents, perms, 1 / 8, "bf16", "bf16", return_scores=True)
    ref = _textbook(q, codes, v, cents, perms, 1 / 8, "bf16")
    assert np.abs(out - ref).max() <= 2e-2 * np.abs(ref).max()
    s64 = scores.astype(np.float64)
    ref_lse = s64.max(-1) + np.log(np.exp(s64 - s64.max(-1, keepdims=True)).sum(-1))
    np.testing.assert_allclose(lse, ref_lse, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("kind", ["2d", "3d_batch", "3d_heads", "4d"])
def test_decode_mask_slices_follow_reference(kind):
    rng = _rng(14)
    B, Hq, Hkv, T, Lq = 3, 6, 2, 200, 1
    q, codes, v, cents, perms = _decode_problem(rng, B=B, Hq=Hq, Hkv=Hkv, T=T)
    full = np.where(rng.random((B, Hq, Lq, T)) < 0.3, -np.inf, 0.0).astype(np.float32)
    full[..., 0] = 0.0
    if kind == "2d":
        mask = full[0, 0]
        exp = np.broadcast_to(mask, full.shape)
    elif kind == "3d_batch":
        mask = full[:, 0]
        exp = np.broadcast_to(mask[:, None], full.shape)
    elif kind == "3d_heads":
        mask = full[0, :Hq] if B != Hq else full[0]
        exp = np.broadcast_to(mask[None], full.shape)
    else:
        mask = full
        exp = full
    got = O.decode_attention(q, codes, v, cents, perms, 0.125, "bf16", "f32", mask=mask)
    ref = _textbook(q, codes, v, cents, perms, 0.125, "bf16", mask=exp[:, :, 0])
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_decode_matches_torch_call_sequence():
    """The reference's exact torch calls (bf16 q*scale, fp32 softmax, .to(bf16), matmul)."""
    rng = _rng(15)
    q, codes, v, cents, perms = _decode_problem(rng, B=1, Hq=4, Hkv=1, T=700)
    got = O.decode_attention(q, codes, v, cents, perms, 1 / math.sqrt(64), "bf16", "bf16")
    qt = torch.from_numpy(q).to(torch.bfloat16)
    k_hat = torch.from_numpy(O.dequantize(codes[0, 0], cents[0], perms[0]))
    qs = qt[0] * float(1 / math.sqrt(64))
    s = torch.matmul(qs.reshape(-1, 64).float(), k_hat.T).view(4, 1, -1)
    probs = torch.softmax(s, dim=-1).to(torch.bfloat16)
    ref = torch.matmul(probs, torch.from_numpy(v[0, 0]).to(torch.bfloat16)).float().numpy()
    assert np.abs(got[0] - ref).max() <= 2e-2 * np.abs(ref).max()
    assert np.mean(got[0] == ref) > 0.9


def test_torch_eager_baseline_matches_oracle():
    """oracle/torch_eager.py (bench.py's CPU baseline) computes what the oracle computes."""
    from oracle import torch_eager as TE

    rng = _rng(16)
    q, codes, v, cents, perms = _decode_problem(rng, B=1, Hq=6, Hkv=2, T=900)
    ref = O.decode_attention(q, codes, v, cents, perms, 1 / math.sqrt(64), "bf16", "bf16")
    for kv in range(2):
        inv = torch.from_numpy(O.invert_permutation(perms[kv]))
        k_hat = TE.dequantize(torch.from_numpy(codes[0, kv]), torch.from_numpy(cents[kv]), inv)
        assert np.array_equal(k_hat.numpy(), O.dequantize(codes[0, kv], cents[kv], perms[kv]))
        got = TE.decode_unit(torch.from_numpy(q[0, 3 * kv:3 * kv + 3]).to(torch.bfloat16),
                             torch.from_numpy(codes[0, kv]), torch.from_numpy(v[0, kv]).to(torch.bfloat16),
                             torch.from_numpy(cents[kv]), inv, 1 / math.sqrt(64)).float().numpy()
        r = ref[0, 3 * kv:3 * kv + 3]
        assert np.abs(got - r).max() <= 2e-2 * np.abs(r).max()
        assert np.mean(got == r) > 0.9


# ----------------------------------------------------------------------------- paging, merging
def test_page_gather_inverts_page_scatter():
    rng = _rng(16)
    B, Hkv, T, nb, Dv, page = 3, 2, 80, 8, 16, 16
    codes = rng.integers(0, 256, (B, Hkv, T, nb)).astype(np.uint8)
    v = rng.standard_normal((B, Hkv, T, Dv)).astype(np.float32)
    npg = T // page
    P = B * npg + 5
    table = rng.permutation(P)[: B * npg].reshape(B, npg)
    cp = np.zeros((P, Hkv, page, nb), np.uint8)
    vp = np.zeros((P, Hkv, Dv, page), np.float32)
    for b in range(B):
        for i in range(npg):
            cp[table[b, i]] = codes[b, :, i * page:(i + 1) * page]
            vp[table[b, i]] = v[b, :, i * page:(i + 1) * page].transpose(0, 2, 1)
    for b in range(B):
        for L in (T, T - 7):
            assert np.array_equal(O.gather_pages_codes(cp, table[b], L), codes[b, :, :L])
            assert np.array_equal(O.gather_pages_values(vp, table[b], L), v[b, :, :L])


def test_lse_merge_equals_full_softmax():
    rng = _rng(17)
    s = rng.standard_normal((4, 1000)) * 3
    vv = rng.standard_normal((1000, 8))
    full = np.exp(s - s.max(-1, keepdims=True))
    ref = (full @ vv) / full.sum(-1, keepdims=True)
    ms, ls, os_ = [], [], []
    for lo, hi in ((0, 300), (300, 301), (301, 1000)):
        part = s[:, lo:hi]
        m = part.max(-1)
        e = np.exp(part - m[:, None])
        ms.append(m)
        ls.append(e.sum(-1))
        os_.append(e @ vv[lo:hi])
    out, lse = O.lse_merge(np.stack(ms), np.stack(ls), np.stack(os_))
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, np.log(np.exp(s).sum(-1)), rtol=1e-6)


# ---------------------------------------------------------------------------
# packed codes (sunshape/triton_kernels.py:250-266)
# ---------------------------------------------------------------------------

def test_pack_codes_hand_example():
    """6-bit codes, 5 per word: word0 = 1 | 2<<6 | 3<<12 | 4<<18 | 5<<24, word1 = 6 (order within a word pinned)."""
    w = O.pack_codes(np.array([[1, 2, 3, 4, 5, 6]], dtype=np.uint8), 6)
    assert w.shape == (1, 2)
    assert int(w[0, 0]) == 1 | 2 << 6 | 3 << 12 | 4 << 18 | 5 << 24 and int(w[0, 1]) == 6


def test_pack_codes_8bit_is_little_endian_byte_view():
    rng = np.random.default_rng(0)
    c = rng.integers(0, 256, size=(7, 32), dtype=np.uint8)
    assert np.array_equal(O.pack_codes(c, 8), c.view("<i4"))


@pytest.mark.parametrize("bits,nb", [(1, 33), (2, 16), (3, 11), (4, 32), (5, 7), (6, 32), (7, 9), (8, 3)])
def test_pack_unpack_round_trip(bits, nb):
    rng = np.random.default_rng(bits * 100 + nb)
    c = rng.integers(0, 1 << bits, size=(2, 5, nb), dtype=np.uint8)
    w = O.pack_codes(c, bits)
    vpe = 32 // bits
    assert w.shape == (2, 5, (nb + vpe - 1) // vpe) and w.dtype == np.int32
    assert np.array_equal(O.unpack_codes(w, nb, bits), c)
    # unused high bits of each word are zero
    used = vpe * bits
    if used < 32:
        assert not (w.view(np.uint32) >> np.uint32(used)).any()
