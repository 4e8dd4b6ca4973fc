"""Pins the oracle's encode (oracle/vq_encode.c) against torch.cdist, the library
call the reference's quantize makes (sunshape/codec.py:376-377).  CPU only.

torch.cdist on these sizes computes sqrt(clamp_min([-2x, |x|^2, 1] @ [c, 1, |c|^2]^T, 0)).
The pre-sqrt GEMM is reproduced bit-for-bit.  torch's CPU sqrt is not correctly
rounded (its last bit depends on the host CPU: about 0.6% of inputs differ on this
container's Xeon and ~17% on an EPYC host), so the oracle uses the IEEE sqrt, and
the two argmins can differ only where two codewords' distances are within a few ulps
(a sqrt-rounding tie).  The tests below check the GEMM bitwise, and check that every
argmin difference against torch.cdist is such a tie.
"""

import math

import numpy as np
import pytest
import torch

from oracle import vq_oracle as O


def _torch_mm_dist2(x: np.ndarray, c: np.ndarray) -> np.ndarray:
    """ATen's _euclidean_dist before clamp/sqrt, via the same torch calls."""
    x1 = torch.from_numpy(x)
    x2 = torch.from_numpy(c)
    x1n = x1.pow(2).sum(-1, keepdim=True)
    x2n = x2.pow(2).sum(-1, keepdim=True)
    x1_ = torch.cat([x1.mul(-2), x1n, torch.ones_like(x1n)], -1)
    x2_ = torch.cat([x2, torch.ones_like(x2n), x2n], -1)
    return x1_.matmul(x2_.mT).numpy()


def _data(seed, n, bd, nc=256, bf16=True):
    rng = np.random.default_rng(seed)
    sig = np.exp(rng.uniform(math.log(0.1), math.log(3), bd)).astype(np.float32)
    x = (rng.standard_normal((n, bd)) * sig).astype(np.float32)
    if bf16:
        x = O.bf16_round(x)
    c = (rng.standard_normal((nc, bd)) * sig).astype(np.float32)
    return x, c


@pytest.mark.parametrize("bd", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("n", [30, 1000, 6000])
def test_presqrt_gemm_bit_exact_vs_torch(bd, n):
    x, c = _data(100 + bd * 7 + n, n, bd)
    e2, _ = O.block_distances(x, c)
    ref = _torch_mm_dist2(x, c)
    assert np.array_equal(e2.view(np.uint32), ref.view(np.uint32))


def test_check_detects_unfused_accumulation():
    """A plausible mistake (separately rounded products) is caught by the bitwise check."""
    x, c = _data(7, 2000, 4)
    ref = _torch_mm_dist2(x, c)
    xn = (x * x).astype(np.float32)
    xn = (((xn[:, 0] + xn[:, 1]).astype(np.float32) + xn[:, 2]).astype(np.float32) + xn[:, 3]).astype(np.float32)
    cn = (c * c).astype(np.float32)
    cn = (((cn[:, 0] + cn[:, 1]).astype(np.float32) + cn[:, 2]).astype(np.float32) + cn[:, 3]).astype(np.float32)
    acc = ((-2 * x[:, None, 0]) * c[None, :, 0]).astype(np.float32)
    for d in range(1, 4):
        acc = (acc + ((-2 * x[:, None, d]) * c[None, :, d]).astype(np.float32)).astype(np.float32)
    acc = ((acc + xn[:, None]).astype(np.float32) + cn[None, :]).astype(np.float32)
    assert not np.array_equal(acc, ref)


def test_post_sqrt_is_ieee_sqrt_of_clamped_gemm():
    x, c = _data(8, 3000, 2)
    e2, d = O.block_distances(x, c)
    assert np.array_equal(d, np.sqrt(np.maximum(e2, np.float32(0))))


def _assert_only_sqrt_ties(x, c, got, ref):
    """Rows where two argmins differ must hold a tie of the pre-sqrt values within 4 ulps."""
    e2 = _torch_mm_dist2(x, c)
    bad = np.nonzero(got != ref)[0]
    for i in bad:
        a, b = e2[i, got[i]], e2[i, ref[i]]
        lo = min(a, b)
        assert abs(a - b) <= 4 * np.spacing(np.float32(max(abs(lo), 1e-30))), (i, a, b)
    return len(bad)


@pytest.mark.parametrize("bd", [2, 4, 8])
def test_encode_argmin_matches_torch_cdist(bd):
    n = 20000
    x, c = _data(200 + bd, n, bd)
    got, _ = O.encode(x, np.arange(bd), c[None])
    ref = torch.cdist(torch.from_numpy(x), torch.from_numpy(c)).argmin(-1).numpy()
    n_ties = _assert_only_sqrt_ties(x, c, got[:, 0], ref)
    assert n_ties <= max(2, n // 10000)


def test_encode_near_ties_constructed():
    """Codewords duplicated or nudged by one ulp: first index on exact ties, smaller d otherwise."""
    rng = np.random.default_rng(9)
    bd = 2
    c = rng.standard_normal((256, bd)).astype(np.float32)
    c[200] = c[17]                      # exact duplicate: lower index must win
    c[201] = np.nextafter(c[40], np.float32(np.inf))
    x = np.concatenate([c[[17, 40, 201, 5]], rng.standard_normal((500, bd)).astype(np.float32)])
    got, _ = O.encode(x, np.arange(bd), c[None])
    ref = torch.cdist(torch.from_numpy(x), torch.from_numpy(c)).argmin(-1).numpy()
    assert got[0, 0] == 17
    _assert_only_sqrt_ties(x, c, got[:, 0], ref)


def test_encode_exact_centroid_rows():
    rng = np.random.default_rng(10)
    D, bd = 16, 2
    perm = rng.permutation(D)
    cent = rng.standard_normal((D // bd, 256, bd)).astype(np.float32) * 3
    pick = rng.integers(0, 256, (50, D // bd))
    xp = np.stack([np.concatenate([cent[b, pick[i, b]] for b in range(D // bd)]) for i in range(50)])
    keys = O.inverse_transform(xp, perm).astype(np.float32)
    codes, _ = O.encode(keys, perm, cent)
    assert np.array_equal(codes, pick.astype(np.uint8))


def test_encode_heavy_blocks_passthrough():
    rng = np.random.default_rng(11)
    D, bd = 64, 2
    perm = rng.permutation(D)
    cent = rng.standard_normal((32, 256, bd)).astype(np.float32)
    heavy = np.zeros(32, bool)
    heavy[[0, 9, 20, 31]] = True
    keys = O.bf16_round(rng.standard_normal((300, D)).astype(np.float32))
    codes, pt = O.encode(keys, perm, cent, heavy)
    xp = O.forward_transform(keys, perm).reshape(300, 32, bd)
    assert not codes[:, heavy].any()
    assert np.array_equal(pt[:, heavy], xp[:, heavy])
    assert not pt[:, ~heavy].any()
    # light blocks agree with per-block cdist argmin
    for b in np.nonzero(~heavy)[0][:5]:
        ref = torch.cdist(torch.from_numpy(xp[:, b].copy()), torch.from_numpy(cent[b])).argmin(-1).numpy()
        _assert_only_sqrt_ties(xp[:, b].copy(), cent[b], codes[:, b], ref)


# ---------------------------------------------------------------------------
# SunShape-Pro block metric: argmin_c cdist(x_b @ E_b^T, C_b @ E_b^T) (sunshape/codec.py:375-376)
# ---------------------------------------------------------------------------

def _metric_case(seed, n=800, D=32, bd=4, nc=64):
    rng = np.random.default_rng(seed)
    keys = O.bf16_round(rng.standard_normal((n, D)).astype(np.float32))
    perm = rng.permutation(D)
    cent = rng.standard_normal((D // bd, nc, bd)).astype(np.float32)
    E = rng.standard_normal((D, D)).astype(np.float32)  # not symmetric: a transpose would show
    return keys, perm, cent, E


def _gap_ok(dist, chosen, other, rel=1e-5):
    """Two indices may differ only where their exact distances are within rounding of each other."""
    a = dist[np.arange(len(chosen)), chosen]
    b = dist[np.arange(len(other)), other]
    return np.abs(a - b) <= rel * np.maximum(np.abs(a), np.abs(b)) + 1e-30


def test_metric_identity_reproduces_plain_encode():
    keys, perm, cent, _ = _metric_case(11)
    c0, _ = O.encode(keys, perm, cent)
    c1, _ = O.encode(keys, perm, cent, metric=np.eye(keys.shape[1], dtype=np.float32))
    assert np.array_equal(c0, c1)


def test_metric_vs_fp64_brute_force_and_torch_restatement():
    keys, perm, cent, E = _metric_case(12)
    D, bd = keys.shape[1], cent.shape[2]
    codes, _ = O.encode(keys, perm, cent, metric=E)
    xp = torch.from_numpy(keys[:, perm])
    diffs = 0
    for b in range(D // bd):
        sl = slice(b * bd, (b + 1) * bd)
        Eb = torch.from_numpy(E[sl, sl])
        y64 = xp[:, sl].double() @ Eb.double().T
        c64 = torch.from_numpy(cent[b]).double() @ Eb.double().T
        dist = torch.cdist(y64, c64).pow(2).numpy()
        brute = dist.argmin(1)
        ref = torch.cdist(xp[:, sl] @ Eb.T, torch.from_numpy(cent[b]) @ Eb.T).argmin(-1).numpy()
        for other in (brute, ref):
            neq = codes[:, b] != other
            diffs += int(neq.sum())
            assert _gap_ok(dist, codes[:, b], other)[neq].all()
    assert diffs <= 0.01 * keys.shape[0] * (D // bd)


def test_metric_transposed_is_detected():
    """Applying E_b instead of E_b^T (a plausible slip) changes many codes."""
    keys, perm, cent, E = _metric_case(13)
    good, _ = O.encode(keys, perm, cent, metric=E)
    bad, _ = O.encode(keys, perm, cent, metric=np.ascontiguousarray(E.T))
    assert (good != bad).mean() > 0.2


def test_metric_power_of_two_scale_and_off_block_entries_invariant():
    """2E scales every fp32 step exactly (same codes); entries outside the diagonal blocks are never read."""
    keys, perm, cent, E = _metric_case(14)
    bd = cent.shape[2]
    base, _ = O.encode(keys, perm, cent, metric=E)
    scaled, _ = O.encode(keys, perm, cent, metric=2.0 * E)
    assert np.array_equal(base, scaled)
    E2 = E.copy()
    mask = np.kron(np.eye(E.shape[0] // bd), np.ones((bd, bd))).astype(bool)
    E2[~mask] = 123.0
    off, _ = O.encode(keys, perm, cent, metric=E2)
    assert np.array_equal(base, off)


def test_metric_keys_on_codewords():
    """x = a codeword: that codeword's index (well-separated codebook, any invertible E_b)."""
    rng = np.random.default_rng(15)
    D, bd, nc = 16, 2, 32
    grid = np.stack(np.meshgrid(np.arange(8), np.arange(4)), -1).reshape(-1, 2).astype(np.float32) * 4.0
    cent = np.stack([grid[rng.permutation(nc)] for _ in range(D // bd)])
    idx = rng.integers(0, nc, size=(50, D // bd))
    xp = np.concatenate([cent[b][idx[:, b]] for b in range(D // bd)], axis=1)
    perm = np.arange(D)
    E = (np.eye(D) + 0.1 * rng.standard_normal((D, D))).astype(np.float32)
    codes, _ = O.encode(xp.astype(np.float32), perm, cent, metric=E)
    assert np.array_equal(codes, idx.astype(np.uint8))


# ----------------------------------------------------------------------------- direct distance
# torch.cdist evaluates sqrt(sum_k (x_k - c_k)^2) directly when both inputs have at most 25 rows.
# Its scalar CPU kernel (ATEN_CPU_CAPABILITY=default) sums the rounded squares in k order, which
# the oracle's direct mode restates bit for bit.  Vectorised builds (AVX2 / AVX-512) reorder that
# sum for some block sizes, so against them only near-ties may differ.
_DIRECT_SCRIPT = r"""
import sys, numpy as np, torch
d = np.load(sys.argv[1])
out = {}
for k in d.files:
    if k.startswith("x"):
        i = k[1:]
        out["d" + i] = torch.cdist(torch.from_numpy(d["x" + i]), torch.from_numpy(d["c" + i])).numpy()
np.savez(sys.argv[2], **out)
"""


def _direct_cases():
    cases = []
    for bd in (1, 2, 3, 4, 8):
        for seed in range(6):
            x, c = _data(900 + 10 * bd + seed, 25 - seed, bd, nc=16)
            cases.append((x, c))
    return cases


def _torch_cdist_subprocess(cases, tmp_path, capability):
    import os
    import subprocess
    import sys

    src = tmp_path / "in.npz"
    dst = tmp_path / "out.npz"
    np.savez(src, **{f"x{i}": x for i, (x, _) in enumerate(cases)}, **{f"c{i}": c for i, (_, c) in enumerate(cases)})
    env = dict(os.environ, ATEN_CPU_CAPABILITY=capability)
    subprocess.run([sys.executable, "-c", _DIRECT_SCRIPT, str(src), str(dst)], check=True, env=env)
    d = np.load(dst)
    return [d[f"d{i}"] for i in range(len(cases))]


def test_direct_distance_bit_exact_vs_torch_scalar_cdist(tmp_path):
    cases = _direct_cases()
    ref = _torch_cdist_subprocess(cases, tmp_path, "default")
    for (x, c), r in zip(cases, ref):
        _, d = O.block_distances(x, c, direct=True)
        assert np.array_equal(d.view(np.uint32), r.view(np.uint32)), (x.shape, c.shape)
        codes, _ = O.encode(x, np.arange(x.shape[1]), c[None], direct=True)
        assert np.array_equal(codes[:, 0], np.argmin(r, axis=1))


def test_direct_distance_vs_vectorised_torch_only_near_ties():
    for x, c in _direct_cases():
        r = torch.cdist(torch.from_numpy(x), torch.from_numpy(c)).numpy()
        _, d = O.block_distances(x, c, direct=True)
        assert np.all(np.abs(d - r) <= 2 * np.spacing(np.maximum(np.abs(r), 1e-30).astype(np.float32)))
        got = O.encode(x, np.arange(x.shape[1]), c[None], direct=True)[0][:, 0]
        want = np.argmin(r, axis=1)
        for i in np.nonzero(got != want)[0]:
            a, b = d[i, got[i]], d[i, want[i]]
            assert abs(a - b) <= 4 * np.spacing(np.float32(max(min(a, b), 1e-30)))


def _midpoint_keys(seed, n, bd, nc=16):
    """Keys near the midpoints of codeword pairs: the distance formulation decides the winner."""
    rng = np.random.default_rng(seed)
    c = (rng.standard_normal((nc, bd)) * 2).astype(np.float32)
    i, j = rng.integers(0, nc, n), rng.integers(0, nc, n)
    x = (0.5 * (c[i] + c[j]) + rng.standard_normal((n, bd)) * 1e-6).astype(np.float32)
    return x, c


def test_mode_switch_changes_near_tie_codes_as_torch_does(tmp_path):
    """On midpoint keys the two formulations pick different codewords in some rows; torch's own
    choice follows the row count (direct at <= 25 rows, mm above), and so does the oracle's."""
    xs, cs = zip(*[_midpoint_keys(2000 + s, 25, 2) for s in range(80)])
    ref_direct = _torch_cdist_subprocess(list(zip(xs, cs)), tmp_path, "default")
    n_diff = 0
    for x, c, rd in zip(xs, cs, ref_direct):
        cd = O.encode(x, np.arange(2), c[None], direct=True)[0][:, 0]
        cm = O.encode(x, np.arange(2), c[None], direct=False)[0][:, 0]
        assert np.array_equal(cd, np.argmin(rd, axis=1))
        # the same keys inside a 26-row call take the mm formulation
        x26 = np.concatenate([x, x[:1]])
        rm = torch.cdist(torch.from_numpy(x26), torch.from_numpy(c)).numpy()[:25]
        _assert_only_sqrt_ties(x, c, cm, np.argmin(rm, axis=1))
        n_diff += int((cd != cm).sum())
    assert n_diff > 0, "no midpoint key separated the two formulations"


# ----------------------------------------------------------------------------- rotated mode
def _orthogonal(D, seed):
    g = torch.Generator().manual_seed(seed)
    qm, _ = torch.linalg.qr(torch.randn(D, D, generator=g, dtype=torch.float64))
    return qm.float().numpy()


def test_transform_rows_permutation_matrix_is_the_gather():
    rng = np.random.default_rng(31)
    D = 64
    perm = rng.permutation(D)
    P = np.eye(D, dtype=np.float32)[perm]          # (x @ P^T)[j] = x[perm[j]]
    x = (rng.standard_normal((50, D)) * 3).astype(np.float32)
    assert np.array_equal(O.transform_rows(x, P), O.forward_transform(x, perm))
    assert np.array_equal(O.transform_rows(O.forward_transform(x, perm), P, transpose=True), x)


def test_transform_rows_orthogonal_adjointness_and_transpose_slip():
    rng = np.random.default_rng(32)
    D = 64
    R = _orthogonal(D, 5)
    q = rng.standard_normal((7, D)).astype(np.float32)
    k = rng.standard_normal((40, D)).astype(np.float32)
    lhs = q.astype(np.float64) @ O.transform_rows(k, R, transpose=True).astype(np.float64).T
    rhs = O.transform_rows(q, R).astype(np.float64) @ k.astype(np.float64).T
    assert np.abs(lhs - rhs).max() <= 1e-5 * np.abs(lhs).max()
    # the plausible slip (R in place of R^T) breaks the identity
    slip = O.transform_rows(q, R.T.copy()).astype(np.float64) @ k.astype(np.float64).T
    assert np.abs(lhs - slip).max() > 0.1 * np.abs(lhs).max()
    # torch's matmul (the reference's x @ rotation.T) agrees to fp32 rounding
    ref = (torch.from_numpy(q) @ torch.from_numpy(R).T).numpy()
    assert np.abs(O.transform_rows(q, R) - ref).max() <= 1e-5 * np.abs(ref).max()


def test_rotated_encode_with_permutation_matrix_equals_permutation_encode():
    rng = np.random.default_rng(33)
    D, bd = 64, 2
    perm = rng.permutation(D)
    P = np.eye(D, dtype=np.float32)[perm]
    x, c = _data(34, 3000, D)
    cent = (rng.standard_normal((D // bd, 256, bd))).astype(np.float32)
    a, _ = O.encode(x, perm, cent)
    b, _ = O.encode(x, np.zeros(D, np.int64), cent, rotation=P)  # perm ignored under rotation
    assert np.array_equal(a, b)


# ---------------------------------------------------------------------------
# codebooks past 256 codewords: the reference stores int16 / int32 indices (sunshape/codec.py:78-83);
# its default fitter gives 4,096 codewords at 3 bits/dim and block_dim 4 (sunshape/hf.py:594)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("nc,bd", [(512, 2), (4096, 4), (65536, 1)])
def test_wide_encode_vs_torch_cdist(nc, bd):
    """Indices over 512 / 4,096 / 65,536 codewords against torch.cdist(...).argmin(-1), the reference's
    call: every difference is a sqrt-rounding tie of the pre-sqrt values.  The dtype is the
    reference's compact one (16-bit below 65,536 codewords, int32 from there)."""
    D = 4 * bd
    x, _ = _data(300 + nc, 700, D, nc=1)
    rng = np.random.default_rng(301 + nc)
    cent = (rng.standard_normal((D // bd, nc, bd)) * 1.3).astype(np.float32)
    codes, _ = O.encode(x, np.arange(D), cent)
    assert codes.dtype == (np.uint16 if nc <= 65535 else np.int32)
    for b in range(D // bd):
        xb = np.ascontiguousarray(x[:, b * bd:(b + 1) * bd])
        ref = torch.cdist(torch.from_numpy(xb), torch.from_numpy(cent[b])).argmin(-1).numpy()
        got = codes[:, b].astype(np.int64)
        _assert_only_sqrt_ties(xb, cent[b], got, ref)
        assert (got == ref).mean() > 0.99


def test_wide_encode_agrees_with_byte_encode_and_brute_force():
    """The int32-index entry point equals the uint8 one on a 256-codeword codebook bit for bit (the same
    search), codewords placed at keys give their own (first) index past 256, and duplicated codewords
    resolve to the lowest index; a row-chunked, multi-threaded run equals the single-threaded one."""
    rng = np.random.default_rng(9)
    D, bd = 8, 4
    cent = rng.standard_normal((2, 256, bd)).astype(np.float32)
    x = rng.standard_normal((400, D)).astype(np.float32)
    perm = rng.permutation(D)
    c8, _ = O.encode(x, perm, cent)
    wide = np.zeros((2, 1000, bd), np.float32)
    wide[:, :256] = cent
    wide[:, 256:] = 1e6  # far away: the search over 1,000 codewords must pick the same ones
    cw, _ = O.encode(x, perm, wide)
    assert cw.dtype == np.uint16 and np.array_equal(cw.astype(np.int64), c8.astype(np.int64))
    # keys on codewords 700 (block 0) and 999 (block 1), with 999 duplicated at 300
    wide2 = rng.standard_normal((2, 1000, bd)).astype(np.float32)
    wide2[1, 300] = wide2[1, 999]
    xp = np.concatenate([wide2[0, 700], wide2[1, 999]])[None]
    keys = np.empty_like(xp)
    keys[:, perm] = xp
    got, _ = O.encode(keys, perm, wide2)
    assert got.tolist() == [[700, 300]]
    big = rng.standard_normal((3000, D)).astype(np.float32)
    one, _ = O.encode(big, perm, wide2)
    many, _ = O.encode(big, perm, wide2, threads=5)
    assert np.array_equal(one, many)
