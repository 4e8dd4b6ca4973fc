"""HIP encode vs the oracle, bit-for-bit: golden fixture, block sizes, both kernels,
constructed ties, torch.cdist on this host's CPU, paged slot mapping, config 5."""

import os

import numpy as np
import pytest
import torch

from _util import bf16_from_bits, log, np_of, torch_bf16_from_bits
from oracle import vq_oracle as O
from sunshape_amd import hip_ops, synthetic
from sunshape_amd.codec import SunShapeBlockCodec

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _gpu_encode(keys_np, perm, cent, heavy=None, kernel=0, dtype=torch.float32, pt_dense=True):
    keys = torch.from_numpy(keys_np).to(DEV).to(dtype)
    codes, pt = hip_ops.encode(keys[None, None], torch.from_numpy(perm).to(DEV), torch.from_numpy(cent).to(DEV),
                               heavy=None if heavy is None else list(heavy), pt_dtype=torch.float32,
                               pt_dense=pt_dense, kernel=kernel)
    return np_of(codes[0, 0]), None if pt is None else np_of(pt[0, 0])


@pytest.mark.parametrize("kernel", [1, 2, 3])
def test_encode_golden_fixture_bit_exact(kernel):
    log(f"encode golden kernel={kernel}")
    f = np.load(os.path.join(GOLD, "encode_mixed.npz"))
    keys = torch_bf16_from_bits(f["keys_bf16_bits"], DEV)
    cent = torch.from_numpy(f["centroids"]).to(DEV)
    grid = hip_ops.encode_grid(cent) if kernel == 3 else None
    codes, pt = hip_ops.encode(keys[None, None], torch.from_numpy(f["perm"]).to(DEV), cent,
                               heavy=f["heavy"].tolist(), pt_dtype=torch.float32, pt_dense=True, kernel=kernel,
                               grid=grid)
    assert np.array_equal(np_of(codes[0, 0]), f["codes"])
    assert np.array_equal(np_of(pt[0, 0]), f["passthrough"])


@pytest.mark.parametrize("D,bd", [(64, 1), (64, 2), (48, 3), (128, 4), (64, 8), (128, 8), (64, 16)])
def test_encode_kernels_vs_oracle_bit_exact(D, bd):
    log(f"encode D={D} bd={bd}")
    rng = np.random.default_rng(D * 31 + bd)
    n = 3000
    perm = rng.permutation(D)
    sig = np.exp(rng.uniform(np.log(0.1), np.log(3), D)).astype(np.float32)
    cent = (rng.standard_normal((D // bd, 256, bd)) * sig[perm].reshape(D // bd, 1, bd)).astype(np.float32)
    keys = O.bf16_round((rng.standard_normal((n, D)) * sig).astype(np.float32))
    ref, _ = O.encode(keys, perm, cent)
    got_scan, _ = _gpu_encode(keys, perm, cent, kernel=1, dtype=torch.bfloat16)
    assert np.array_equal(got_scan, ref), int((got_scan != ref).sum())
    if bd <= 10:
        got_mfma, _ = _gpu_encode(keys, perm, cent, kernel=2, dtype=torch.bfloat16)
        assert np.array_equal(got_mfma, ref), int((got_mfma != ref).sum())


def test_encode_constructed_ties_and_exact_rows():
    log("encode constructed ties")
    rng = np.random.default_rng(7)
    D, bd = 32, 2
    perm = rng.permutation(D)
    cent = rng.standard_normal((16, 256, bd)).astype(np.float32)
    cent[:, 200] = cent[:, 17]                                    # duplicates: lower index wins
    cent[:, 201] = np.nextafter(cent[:, 40], np.float32(np.inf))  # one-ulp neighbours
    cent[:, 9] = cent[:, 8] * np.float32(1 + 2 ** -22)
    pick = rng.choice([17, 40, 201, 8, 9, 3], size=(400, 16))
    xp = np.stack([np.concatenate([cent[b, pick[i, b]] for b in range(16)]) for i in range(400)])
    xp[200:] += rng.standard_normal(xp[200:].shape).astype(np.float32) * 1e-3
    keys = O.inverse_transform(xp, perm).astype(np.float32)
    ref, _ = O.encode(keys, perm, cent)
    assert not (ref == 200).any()
    for kernel in (1, 2):
        got, _ = _gpu_encode(keys, perm, cent, kernel=kernel)
        assert np.array_equal(got, ref), (kernel, int((got != ref).sum()))


def test_encode_vs_torch_cdist_on_this_host():
    """torch.cdist on this host's CPU differs only on sqrt-rounding ties (counted)."""
    log("encode vs torch.cdist")
    rng = np.random.default_rng(8)
    bd, n = 2, 50000
    x = O.bf16_round(rng.standard_normal((n, bd)).astype(np.float32))
    c = rng.standard_normal((256, bd)).astype(np.float32)
    got, _ = _gpu_encode(x, np.arange(bd), c[None])
    ref = torch.cdist(torch.from_numpy(x), torch.from_numpy(c)).argmin(-1).numpy()
    bad = np.nonzero(got[:, 0] != ref)[0]
    e2, _ = O.block_distances(x, c)
    for i in bad:
        a, b = e2[i, got[i, 0]], e2[i, ref[i]]
        assert abs(a - b) <= 4 * np.spacing(np.float32(max(min(abs(a), abs(b)), 1e-30))), (i, a, b)
    print(f"[info] rows differing from this host's torch.cdist (sqrt ties): {len(bad)} of {n}")


def test_rotated_encode_vs_torch_cdist_on_this_host():
    """Rotated mode (sunshape/codec.py:247-252, :362-377): the reference encodes argmin
    torch.cdist(x @ R^T, C) with torch's own x @ R^T, whose rounding order is the BLAS library's.  The
    GPU encode (transform_rows' k-ascending chain, then the exact search) differs from it only where
    two codewords' distances are within rounding of each other: each difference is proven a near-tie
    against fp64 distances of the fp64-rotated keys (within 1e-5 relative), and counted."""
    log("rotated encode vs torch.cdist")
    rng = np.random.default_rng(18)
    D, bd, n = 16, 2, 20000
    R, _ = np.linalg.qr(rng.standard_normal((D, D)))
    R = R.astype(np.float32)
    x = O.bf16_round(rng.standard_normal((n, D)).astype(np.float32))
    c = rng.standard_normal((D // bd, 256, bd)).astype(np.float32)
    got, _ = hip_ops.encode(torch.from_numpy(x)[None, None].to(DEV), torch.arange(D, device=DEV),
                            torch.from_numpy(c).to(DEV), rotation=torch.from_numpy(R).to(DEV))
    got = np_of(got)[0, 0].astype(np.int64)
    xr = torch.from_numpy(x) @ torch.from_numpy(R).T  # the reference's forward transform, on this host
    xr64 = x.astype(np.float64) @ R.astype(np.float64).T
    n_diff = 0
    for b in range(D // bd):
        xb = xr[:, b * bd:(b + 1) * bd].contiguous()
        ref = torch.cdist(xb, torch.from_numpy(c[b])).argmin(-1).numpy()
        bad = np.nonzero(got[:, b] != ref)[0]
        n_diff += len(bad)
        for i in bad:
            d = ((xr64[i, b * bd:(b + 1) * bd][None] - c[b].astype(np.float64)) ** 2).sum(-1)
            da, db = d[got[i, b]], d[ref[i]]
            assert abs(da - db) <= 1e-5 * max(da, db, 1e-30), (i, b, da, db)
        assert len(bad) <= n // 100
    # the oracle restates the GPU's transform order: bit-exact with it
    ref_o, _ = O.encode(x, np.arange(D), c, rotation=R)
    assert np.array_equal(got, ref_o.astype(np.int64))
    print(f"[info] rotated-mode codes differing from this host's torch.cdist(x @ R.T, C) (near-ties): "
          f"{n_diff} of {n * (D // bd)}")


def test_encode_paged_slot_mapping_matches_contiguous():
    log("encode paged slot mapping")
    p = synthetic.config5(DEV, B=2, S=96)
    heavy = p["heavy"].tolist()
    codes, pt = hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy)
    page, Hkv, nb = 16, 2, 32
    P = 2 * 96 // page + 3
    g = torch.Generator().manual_seed(3)
    table = torch.randperm(P, generator=g)[: 2 * 96 // page].view(2, -1)
    slots = (table[:, :, None] * page + torch.arange(page)).reshape(2, 96).to(torch.int64).to(DEV)
    cpages = torch.zeros(P, Hkv, page, nb, dtype=torch.uint8, device=DEV)
    ppages = torch.zeros(P, Hkv, page, 4, 2, dtype=torch.bfloat16, device=DEV)
    hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy, codes_out=cpages, pt_out=ppages,
                   slot_mapping=slots)
    t = table.to(DEV)
    for b in range(2):
        got_c = cpages[t[b]].permute(1, 0, 2, 3).reshape(Hkv, 96, nb)
        got_p = ppages[t[b]].permute(1, 0, 2, 3, 4).reshape(Hkv, 96, 4, 2)
        assert torch.equal(got_c, codes[b]) and torch.equal(got_p, pt[b])


def test_config5_full_encode():
    """Full config 5 (16 x 2 x 16384 = 524,288 keys): the MFMA, exact-scan and grid-search encodes
    give the same codes and passthrough values, and every one of the 524,288 code rows (and its
    passthrough values) equals the oracle's, the C oracle running over the host's cores."""
    log("config5 full encode")
    p = synthetic.config5(DEV)
    heavy = p["heavy"].tolist()
    c_mfma, pt = hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy, kernel=2)
    c_scan, pt2 = hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy, kernel=1)
    assert torch.equal(c_mfma, c_scan) and torch.equal(pt, pt2)
    grid = hip_ops.encode_grid(p["centroids"])
    c_grid, pt3 = hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy, kernel=3, grid=grid)
    assert torch.equal(c_grid, c_scan) and torch.equal(pt3, pt2)
    hv = p["heavy"].numpy()
    keys = np_of(p["keys"])
    perm, cent = np_of(p["perm"]), np_of(p["centroids"])
    got, got_pt = np_of(c_mfma), np_of(pt)
    threads = min(16, os.cpu_count() or 1)
    for kv in range(2):  # one codebook per KV head: all 16 x 16384 keys of the head at once
        ref, rpt = O.encode(keys[:, kv].reshape(-1, keys.shape[-1]), perm, cent[kv], hv, threads=threads)
        assert np.array_equal(got[:, kv].reshape(ref.shape), ref), f"kv={kv}"
        assert np.array_equal(got_pt[:, kv].reshape(-1, *got_pt.shape[-2:]), rpt[:, hv]), f"kv={kv}"


# ---------------------------------------------------------------------------
# SunShape-Pro block metric (sunshape/codec.py:375-376)
# ---------------------------------------------------------------------------

def _pro_case(D, bd, seed, n=2500, near_identity=False):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(D)
    sig = np.exp(rng.uniform(np.log(0.1), np.log(3), D)).astype(np.float32)
    cent = (rng.standard_normal((D // bd, 256, bd)) * sig[perm].reshape(D // bd, 1, bd)).astype(np.float32)
    keys = O.bf16_round((rng.standard_normal((n, D)) * sig).astype(np.float32))
    E = rng.standard_normal((D, D)).astype(np.float32)
    if near_identity:
        E = (np.eye(D) + 0.3 * E).astype(np.float32)
    return keys, perm, cent, E


@pytest.mark.parametrize("D,bd", [(64, 2), (64, 4), (64, 8), (48, 3), (64, 16)])
def test_metric_encode_kernels_vs_oracle_bit_exact(D, bd):
    log(f"metric encode D={D} bd={bd}")
    keys, perm, cent, E = _pro_case(D, bd, D * 7 + bd)
    ref, _ = O.encode(keys, perm, cent, metric=E)
    kt = torch.from_numpy(keys).to(DEV).to(torch.bfloat16)[None, None]
    args = (torch.from_numpy(perm).to(DEV), torch.from_numpy(cent).to(DEV))
    Et = torch.from_numpy(E).to(DEV)
    for kernel in ([1, 2] if bd <= 10 else [1]):
        codes, _ = hip_ops.encode(kt, *args, metric=Et, kernel=kernel)
        got = np_of(codes[0, 0])
        assert np.array_equal(got, ref), (kernel, int((got != ref).sum()))


def test_metric_encode_mixed_per_head_and_paged():
    """Heavy blocks (raw values, not E_b x), per-KV-head metrics [Hkv, D, D], paged output."""
    log("metric encode mixed/per-head/paged")
    D, bd, Hkv, S = 64, 2, 2, 160
    keys0, perm, cent0, E0 = _pro_case(D, bd, 91, n=S, near_identity=True)
    keys1, _, cent1, E1 = _pro_case(D, bd, 92, n=S, near_identity=True)
    heavy = np.zeros(D // bd, dtype=bool)
    heavy[[1, 5, 17]] = True
    keys = torch.from_numpy(np.stack([keys0, keys1])).to(DEV).to(torch.bfloat16)[None]
    cent = torch.from_numpy(np.stack([cent0, cent1])).to(DEV)
    Et = torch.from_numpy(np.stack([E0, E1])).to(DEV)
    permt = torch.from_numpy(perm).to(DEV)
    codes, pt = hip_ops.encode(keys, permt, cent, heavy=heavy.tolist(), metric=Et, pt_dtype=torch.float32,
                               pt_dense=True)
    for h, (k, c, E) in enumerate(((keys0, cent0, E0), (keys1, cent1, E1))):
        ref, rpt = O.encode(k, perm, c, heavy, metric=E)
        assert np.array_equal(np_of(codes[0, h]), ref)
        assert np.array_equal(np_of(pt[0, h]), rpt)
    page = 16
    P = S // page + 2
    slots = (torch.randperm(P, generator=torch.Generator().manual_seed(4))[: S // page][:, None] * page
             + torch.arange(page)).reshape(1, S).to(torch.int64).to(DEV)
    cp = torch.zeros(P, Hkv, page, D // bd, dtype=torch.uint8, device=DEV)
    pp = torch.zeros(P, Hkv, page, 3, bd, dtype=torch.float32, device=DEV)
    hip_ops.encode(keys, permt, cent, heavy=heavy.tolist(), metric=Et, codes_out=cp, pt_out=pp, slot_mapping=slots)
    s = slots[0].cpu()
    got = cp[s // page, :, s % page].permute(1, 0, 2)
    assert torch.equal(got, codes[0])


def test_pro_codec_quantize_matches_oracle():
    from sunshape_amd.codec import SunShapeBlockCodec

    log("pro codec quantize")
    D, bd = 64, 4
    keys, perm, cent, E = _pro_case(D, bd, 93, n=1500, near_identity=True)
    codec = SunShapeBlockCodec.from_buffers(torch.from_numpy(perm), torch.from_numpy(cent),
                                            mode="profileperm_localmetric_dsq", metric=torch.from_numpy(E), device=DEV)
    qz = codec.quantize(torch.from_numpy(keys).to(DEV))
    ref, _ = O.encode(keys, perm, cent, metric=E)
    assert np.array_equal(np_of(qz.indices), ref)
    # decode-side arithmetic ignores E: k_hat = C[b, idx] in the original basis
    k_hat = np_of(codec.dequantize(qz))
    assert np.array_equal(k_hat, O.dequantize(ref, cent, perm))


# ---------------------------------------------------------------------------
# grid-search encode (kernel 3, block_dim 2): certified candidate lists from encode_grid
# ---------------------------------------------------------------------------

def _grid_case(D, nc, n, seed, spread=1.0):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(D)
    sig = np.exp(rng.uniform(np.log(0.1), np.log(3), D)).astype(np.float32)
    cent = (rng.standard_normal((D // 2, nc, 2)) * sig[perm].reshape(D // 2, 1, 2)).astype(np.float32)
    keys = O.bf16_round((rng.standard_normal((n, D)) * sig * spread).astype(np.float32))
    return keys, perm, cent


@pytest.mark.parametrize("D,nc,n,spread", [(64, 256, 3000, 1.0), (40, 64, 777, 1.0), (64, 256, 1500, 25.0),
                                           (32, 256, 65, 0.2)])
def test_grid_encode_vs_oracle_bit_exact(D, nc, n, spread):
    """Grid encode == oracle == MFMA encode, bit for bit.  spread 25 puts most keys in the far,
    wide cells (long lists or every codeword scanned); spread 0.2 crowds them into the central cells; D 40 gives
    code rows that are not whole 16-byte pieces; 64 codewords exercise nc < 256."""
    log(f"grid encode D={D} nc={nc} n={n} spread={spread}")
    keys, perm, cent = _grid_case(D, nc, n, D * 7 + nc + int(spread * 10), spread)
    ref, _ = O.encode(keys, perm, cent)
    c = torch.from_numpy(cent).to(DEV)
    grid = hip_ops.encode_grid(c)
    k = torch.from_numpy(keys).to(DEV).to(torch.bfloat16)[None, None]
    codes, _ = hip_ops.encode(k, torch.from_numpy(perm).to(DEV), c, kernel=3, grid=grid)
    got = np_of(codes[0, 0])
    assert np.array_equal(got, ref), int((got != ref).sum())
    if nc == 256:
        m, _ = hip_ops.encode(k, torch.from_numpy(perm).to(DEV), c, kernel=2)
        assert torch.equal(m, codes)
    # auto dispatch takes the grid when one is given
    a, _ = hip_ops.encode(k, torch.from_numpy(perm).to(DEV), c, grid=grid)
    assert torch.equal(a, codes)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("odd_stride", [False, True])
def test_grid_encode_key_paths(dtype, D, odd_stride):
    """Both ways the grid search reads keys: rows of at most 128 bytes on 16-byte boundaries are
    read whole into registers (fp16/bf16 up to D 64, fp32 up to D 32); wider rows and rows at
    odd strides read each element on its own.  Each must equal the oracle bit for bit."""
    log(f"grid encode key path dtype={dtype} D={D} odd_stride={odd_stride}")
    keys, perm, cent = _grid_case(D, 256, 700, 300 + D + int(odd_stride), 1.0)
    kt = torch.from_numpy(keys).to(dtype)
    ref, _ = O.encode(kt.float().numpy(), perm, cent)
    if odd_stride:  # rows 3 elements apart beyond D: not 16-byte aligned
        buf = torch.zeros(keys.shape[0], D + 3, dtype=dtype)
        buf[:, :D] = kt
        k = buf.to(DEV)[:, :D][None, None]
        assert k.stride(2) == D + 3
    else:
        k = kt.to(DEV)[None, None]
    c = torch.from_numpy(cent).to(DEV)
    codes, _ = hip_ops.encode(k, torch.from_numpy(perm).to(DEV), c, kernel=3, grid=hip_ops.encode_grid(c))
    got = np_of(codes[0, 0])
    assert np.array_equal(got, ref), int((got != ref).sum())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D,bd", [(64, 2), (128, 4)])
@pytest.mark.parametrize("odd_stride", [False, True])
def test_mfma_encode_key_paths(dtype, D, bd, odd_stride):
    """Both ways the MFMA encode stages keys: 16-bit rows of 64 or 128 elements on 16-byte
    boundaries come in with 16-byte loads (prefetched a round ahead); fp32 rows and rows at odd
    strides are read element by element, 8 loads in flight per lane.  Each must equal the
    oracle bit for bit, with several rounds per workgroup."""
    log(f"mfma encode key path dtype={dtype} D={D} bd={bd} odd_stride={odd_stride}")
    rng = np.random.default_rng(D + bd + int(odd_stride))
    n = 2500
    perm = rng.permutation(D)
    sig = np.exp(rng.uniform(np.log(0.1), np.log(3), D)).astype(np.float32)
    cent = (rng.standard_normal((D // bd, 256, bd)) * sig[perm].reshape(D // bd, 1, bd)).astype(np.float32)
    kt = torch.from_numpy((rng.standard_normal((n, D)) * sig).astype(np.float32)).to(dtype)
    ref, _ = O.encode(kt.float().numpy(), perm, cent)
    if odd_stride:  # rows 3 elements apart beyond D: not 16-byte aligned
        buf = torch.zeros(n, D + 3, dtype=dtype)
        buf[:, :D] = kt
        k = buf.to(DEV)[:, :D][None, None]
        assert k.stride(2) == D + 3
    else:
        k = kt.to(DEV)[None, None]
    codes, _ = hip_ops.encode(k, torch.from_numpy(perm).to(DEV), torch.from_numpy(cent).to(DEV), kernel=2)
    got = np_of(codes[0, 0])
    assert np.array_equal(got, ref), int((got != ref).sum())


def test_grid_encode_constructed_ties_duplicates_and_heavy():
    """Duplicated codewords (lower index wins), one-ulp neighbours, keys on codewords, keys on cell
    boundaries, and passthrough blocks in both layouts."""
    log("grid encode constructed")
    rng = np.random.default_rng(11)
    D = 32
    perm = rng.permutation(D)
    cent = rng.standard_normal((16, 256, 2)).astype(np.float32)
    cent[:, 200] = cent[:, 17]
    cent[:, 201] = np.nextafter(cent[:, 40], np.float32(np.inf))
    cent[:, 9] = cent[:, 8] * np.float32(1 + 2 ** -22)
    pick = rng.choice([17, 40, 201, 8, 9, 3], size=(600, 16))
    xp = np.stack([np.concatenate([cent[b, pick[i, b]] for b in range(16)]) for i in range(600)])
    xp[200:400] += rng.standard_normal(xp[200:400].shape).astype(np.float32) * 1e-3
    # keys on grid-cell boundaries of each block: header (mid, inv) per dimension; cell edge i at
    # t = -1 + 2i/128 of the map t = u / (1 + |u|), u = (x - mid) inv
    c = torch.from_numpy(cent).to(DEV)
    grid = hip_ops.encode_grid(c)
    hdr = np_of(grid[: 16 * 8 * 4].view(torch.float32)).reshape(16, 8)

    def edge(i, mid, inv):
        t = -1.0 + 2.0 * i / 128
        return np.float32(mid + (t / (1.0 - abs(t))) / inv)

    for r in range(400, 600):
        for b in range(16):
            i0, i1 = rng.integers(1, 128, 2)
            xp[r, 2 * b] = edge(i0, hdr[b, 0], hdr[b, 2])
            xp[r, 2 * b + 1] = edge(i1, hdr[b, 1], hdr[b, 3])
    keys = O.inverse_transform(xp, perm).astype(np.float32)
    heavy = np.zeros(16, dtype=bool)
    heavy[[2, 11]] = True
    ref, rpt = O.encode(keys, perm, cent, heavy)
    k = torch.from_numpy(keys).to(DEV)[None, None]
    for dense in (True, False):
        for pdt in (torch.float32, torch.float16, torch.bfloat16):
            codes, pt = hip_ops.encode(k, torch.from_numpy(perm).to(DEV), c, heavy=heavy.tolist(), pt_dtype=pdt,
                                       pt_dense=dense, kernel=3, grid=grid)
            assert np.array_equal(np_of(codes[0, 0]), ref)
            want = torch.from_numpy(rpt if dense else rpt[:, heavy]).to(pdt)  # the stored dtype's rounding
            assert torch.equal(pt[0, 0].cpu(), want), (dense, pdt)


@pytest.mark.parametrize("kernel,bd,B,S", [(1, 4, 64, 1), (2, 4, 64, 1), (2, 4, 5, 300), (1, 2, 33, 3),
                                           (2, 2, 33, 3), (3, 2, 33, 3), (3, 2, 64, 1)])
def test_short_sequences_fold_batches(kernel, bd, B, S):
    """A decode step's append (one or a few keys per sequence): launches put every sequence of a
    KV head in one key range.  Codes into contiguous rows and into shuffled pages must equal the
    oracle's, per (sequence, KV head)."""
    log(f"folded encode kernel={kernel} bd={bd} B={B} S={S}")
    Hkv, D, page = 8 if bd == 4 else 2, 128 if bd == 4 else 64, 16
    cb = synthetic.make_codebook(Hkv, D, bd, 70 + bd)
    g = torch.Generator().manual_seed(71)
    keys = (torch.randn(B, Hkv, S, D, generator=g) * cb.sigma[:, None, :]).to(torch.bfloat16)
    perm, cent = cb.perm.to(DEV), cb.centroids.to(DEV)
    grid = hip_ops.encode_grid(cent) if kernel == 3 else None
    codes, _ = hip_ops.encode(keys.to(DEV), perm, cent, kernel=kernel, grid=grid)
    got = np_of(codes)
    for b in range(B):
        for h in range(Hkv):
            ref, _ = O.encode(keys[b, h].float().numpy(), cb.perm[h].numpy(), cb.centroids[h].numpy())
            assert np.array_equal(got[b, h], ref), (b, h)
    n_pages = B * ((S + page - 1) // page) + 2
    order = torch.randperm(n_pages, generator=g)
    slots = torch.stack([order[b * ((S + page - 1) // page) + torch.arange(S) // page] * page + torch.arange(S) % page
                         for b in range(B)]).to(torch.int64).to(DEV)
    pages = torch.zeros(n_pages, Hkv, page, D // bd, dtype=torch.uint8, device=DEV)
    hip_ops.encode(keys.to(DEV), perm, cent, codes_out=pages, slot_mapping=slots, kernel=kernel, grid=grid)
    flat = pages.permute(0, 2, 1, 3).reshape(n_pages * page, Hkv, D // bd)
    back = flat[slots.reshape(-1)].reshape(B, S, Hkv, D // bd).permute(0, 2, 1, 3)
    assert torch.equal(back, codes)


def test_grid_encode_paged_matches_contiguous():
    log("grid encode paged")
    p = synthetic.config5(DEV, B=2, S=96)
    heavy = p["heavy"].tolist()
    grid = hip_ops.encode_grid(p["centroids"])
    codes, pt = hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy, kernel=2)
    page, Hkv, nb = 16, 2, 32
    P = 2 * 96 // page + 3
    g = torch.Generator().manual_seed(4)
    table = torch.randperm(P, generator=g)[: 2 * 96 // page].view(2, -1)
    slots = (table[:, :, None] * page + torch.arange(page)).reshape(2, 96).to(torch.int64).to(DEV)
    cpages = torch.zeros(P, Hkv, page, nb, dtype=torch.uint8, device=DEV)
    ppages = torch.zeros(P, Hkv, page, 4, 2, dtype=torch.bfloat16, device=DEV)
    hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy, codes_out=cpages, pt_out=ppages,
                   slot_mapping=slots, kernel=3, grid=grid)
    t = table.to(DEV)
    for b in range(2):
        got_c = cpages[t[b]].permute(1, 0, 2, 3).reshape(Hkv, 96, nb)
        got_p = ppages[t[b]].permute(1, 0, 2, 3, 4).reshape(Hkv, 96, 4, 2)
        assert torch.equal(got_c, codes[b]) and torch.equal(got_p, pt[b])


def test_grid_built_for_another_codebook_still_gives_exact_codes():
    """A grid is only a search aid: used with a codebook it was not built for (here one block
    changed by one ulp, and a wholly different codebook), the blocks whose fingerprint differs
    scan every codeword, so the codes still equal the oracle's."""
    log("grid encode with a stale grid")
    keys, perm, cent = _grid_case(64, 256, 1200, 23)
    c = torch.from_numpy(cent).to(DEV)
    grid = hip_ops.encode_grid(c)
    k = torch.from_numpy(keys).to(DEV).to(torch.bfloat16)[None, None]
    tp = torch.from_numpy(perm).to(DEV)
    cent2 = cent.copy()
    cent2[5, 77, 1] = np.nextafter(cent2[5, 77, 1], np.float32(np.inf))
    other = _grid_case(64, 256, 10, 99)[2]
    for cb in (cent2, other):
        ref, _ = O.encode(keys, perm, cb)
        codes, _ = hip_ops.encode(k, tp, torch.from_numpy(cb).to(DEV), kernel=3, grid=grid)
        assert np.array_equal(np_of(codes[0, 0]), ref)


@pytest.mark.parametrize("bd,nc,kernels,dtype", [(2, 256, (0, 1, 2, 3), torch.float32), (2, 256, (3,), torch.bfloat16),
                                                 (4, 256, (0, 1, 2), torch.float32), (2, 512, (0, 1), torch.float32)])
def test_encode_non_finite_keys_every_kernel(bd, nc, kernels, dtype):
    """Keys with NaN, +-inf and huge finite elements, whose distances are NaN (clamped to 0, so the
    first such codeword wins, as the reference's first argmin of a row holding NaN) or inf, and
    blocks whose codewords are all one point (zeros, as a SunShape-Mixed codec's passthrough
    blocks hold, or another constant: the grid has no cells there), and a block of codewords near
    1e13 (no grid either): every encode kernel equals the
    oracle bit for bit.  The grid sends such keys to its end cells, which scan every codeword; the
    MFMA screen makes every codeword a candidate of a key whose norm is not finite."""
    log(f"encode non-finite keys bd={bd} nc={nc} kernels={kernels} {dtype}")
    D = 64
    rng = np.random.default_rng(31 + bd + nc)
    perm = rng.permutation(D)
    sig = np.exp(rng.uniform(np.log(0.1), np.log(3), D)).astype(np.float32)
    cent = (rng.standard_normal((D // bd, nc, bd)) * sig[perm].reshape(D // bd, 1, bd)).astype(np.float32)
    cent[3] = 0.0
    cent[11] = np.float32(-1.25)
    hb = D // bd - 2  # codewords past 2^40: such a block gets no grid (its fp32 chain could overflow)
    cent[hb] *= np.float32(1e13)
    keys = (rng.standard_normal((1500, D)) * sig).astype(np.float32)
    keys[:, perm[hb * bd:(hb + 1) * bd]] *= np.float32(1e13)
    bad = rng.integers(0, keys.size, 400)
    keys.reshape(-1)[bad] = rng.choice(np.array([np.nan, np.inf, -np.inf, 1e30, -1e30, 3e38], dtype=np.float32),
                                       bad.size)
    kt = torch.from_numpy(keys).to(dtype)
    ref, _ = O.encode(kt.float().numpy(), perm, cent)
    c = torch.from_numpy(cent).to(DEV)
    tp = torch.from_numpy(perm).to(DEV)
    k = kt.to(DEV)[None, None]
    for kernel in kernels:
        grid = hip_ops.encode_grid(c) if kernel == 3 else None
        codes, _ = hip_ops.encode(k, tp, c, kernel=kernel, grid=grid)
        got = np_of(codes[0, 0])
        assert np.array_equal(got, ref), (kernel, int((got != ref).sum()))


def test_grid_encode_many_blocks_in_chunks():
    """64 light blocks exceed one workgroup's LDS: the search splits them into block chunks
    (one workgroup per chunk), and the codes still equal the oracle's."""
    log("grid encode at 64 light blocks")
    keys, perm, cent = _grid_case(128, 256, 1500, 17)
    ref, _ = O.encode(keys, perm, cent)
    c = torch.from_numpy(cent).to(DEV)
    grid = hip_ops.encode_grid(c)
    k = torch.from_numpy(keys).to(DEV).to(torch.bfloat16)[None, None]
    for kernel in (0, 3):
        codes, _ = hip_ops.encode(k, torch.from_numpy(perm).to(DEV), c, kernel=kernel, grid=grid)
        assert np.array_equal(np_of(codes[0, 0]), ref)


def test_paged_encode_rejects_mis_shaped_passthrough_pages():
    """Paged outputs are written through the slot mapping; a passthrough page buffer whose slot
    count, block_dim or row packing does not match is refused before any launch."""
    log("paged encode pt_out validation")
    p = synthetic.config5(DEV, B=1, S=16)
    heavy = p["heavy"].tolist()
    slots = torch.arange(16, dtype=torch.int64, device=DEV).view(1, 16)
    cpages = torch.zeros(2, 2, 16, 32, dtype=torch.uint8, device=DEV)
    for bad in (torch.zeros(2, 2, 16, 32, 2, device=DEV),          # dense slots for the compact layout
                torch.zeros(2, 2, 16, 4, 3, device=DEV),           # wrong block_dim
                torch.zeros(2, 2, 16, 2, 4, device=DEV).transpose(3, 4)):  # rows not packed
        with pytest.raises(RuntimeError, match="pt_out"):
            hip_ops.encode(p["keys"], p["perm"], p["centroids"], heavy=heavy, codes_out=cpages, pt_out=bad,
                           slot_mapping=slots)


def test_grid_encode_rejections():
    log("grid encode rejections")
    cent = torch.randn(8, 256, 4, device=DEV)
    with pytest.raises(RuntimeError, match="block_dim 2"):
        hip_ops.encode_grid(cent)
    keys, perm, cent2 = _grid_case(16, 256, 20, 5)
    k = torch.from_numpy(keys).to(DEV)[None, None]
    with pytest.raises(RuntimeError, match="grid"):
        hip_ops.encode(k, torch.from_numpy(perm).to(DEV), torch.from_numpy(cent2).to(DEV), kernel=3)
    small = torch.zeros(16, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="too small"):
        hip_ops.encode(k, torch.from_numpy(perm).to(DEV), torch.from_numpy(cent2).to(DEV), kernel=3, grid=small)


def test_grid_encode_where_rounding_slack_decides():
    """Codebooks clustered far from the origin, keys near codeword midpoints: the reference's fp32
    mm rounding decides many winners, and many are listed only because of the grid's rounding
    slack M_C (tests/test_grid_search.py).  The grid encode still equals the oracle bit for bit."""
    log("grid encode, rounding slack decides")
    from test_grid_search import far_cluster_case

    cents, xs = [], []
    for seed in (0, 3, 12, 21):
        c, x, _, _ = far_cluster_case(seed, n=20000)
        cents.append(c)
        xs.append(x)
    cent = np.stack(cents)                       # [4 blocks, 8 codewords, 2]
    keys = np.concatenate(xs, axis=1)            # [n, 8]: block b's coordinates in dims 2b, 2b + 1
    perm = np.arange(8)
    ref, _ = O.encode(keys, perm, cent)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    grid = hip_ops.encode_grid(t(cent))
    got, _ = hip_ops.encode(t(keys)[None, None], t(perm), t(cent), kernel=3, grid=grid)
    assert np.array_equal(np_of(got[0, 0]), ref), int((np_of(got[0, 0]) != ref).sum())
    scan, _ = hip_ops.encode(t(keys)[None, None], t(perm), t(cent), kernel=1)
    assert np.array_equal(np_of(scan[0, 0]), ref)


def test_per_head_grid_is_a_slice_of_the_per_kv_head_grid():
    """The grid is head-major: head h's part of a grid built for [Hkv, nb, nc, 2] codebooks is
    byte for byte the grid built for that head's codebook alone, and the codec hands a one-head
    view that slice (no second grid)."""
    log("encode grid: per-head slices of a per-KV-head grid")
    g = torch.Generator().manual_seed(21)
    cent = (torch.randn(3, 32, 256, 2, generator=g) * torch.linspace(0.5, 2.0, 32).view(1, 32, 1, 1)).to(DEV)
    full = hip_ops.encode_grid(cent)
    per = full.view(3, -1)
    for h in range(3):
        assert torch.equal(per[h], hip_ops.encode_grid(cent[h].contiguous())), f"head {h}"
    codec = SunShapeBlockCodec.from_buffers(torch.stack([torch.randperm(64, generator=g) for _ in range(3)]),
                                            cent.cpu(), device=DEV)
    whole = codec.encode_search_grid(codec.centroids)
    for h in range(3):
        view = codec.encode_search_grid(codec.codebook(h))
        assert view.data_ptr() == whole.data_ptr() + h * per.shape[1] and view.numel() == per.shape[1]
        assert torch.equal(view, per[h])
    assert len(codec._grid_cache) == 1


def test_encode_grid_budget_32_layers():
    """A 32-layer model with per-KV-head block_dim-2 codecs (20 MiB of grid per layer, 640 MiB in all)
    under a 128 MiB grid budget: the cached grids never exceed the budget, and every layer's codes
    equal the exhaustive encode's."""
    from sunshape_amd import codec as C

    log("encode grid budget, 32 layers")
    B, Hkv, S, D, bd = 2, 2, 1500, 64, 2
    old = C._GRID_BUDGET[0]
    codecs = []  # every layer's codec stays alive, as in a loaded model
    try:
        C.set_encode_grid_budget(128 << 20)
        for layer in range(32):
            cb = synthetic.make_codebook(Hkv, D, bd, 700 + layer)
            codec = SunShapeBlockCodec.from_buffers(cb.perm, cb.centroids, device=DEV)
            codecs.append(codec)
            g = torch.Generator().manual_seed(800 + layer)
            keys = (torch.randn(B, Hkv, S, D, generator=g) * cb.sigma[:, None, :]).to(torch.bfloat16).to(DEV)
            grid = codec.encode_search_grid(codec.centroids)
            assert grid is not None and C.encode_grid_footprint() <= 128 << 20
            with_grid, _ = hip_ops.encode(keys, codec.permutation, codec.centroids, grid=grid)
            exhaustive, _ = hip_ops.encode(keys, codec.permutation, codec.centroids, kernel=1)
            assert torch.equal(with_grid, exhaustive), f"layer {layer}"
        assert 120 << 20 <= C.encode_grid_footprint() <= 128 << 20  # the 6 most recent layers' grids
    finally:
        C.set_encode_grid_budget(old)


@pytest.mark.parametrize("bd,kernel", [(4, 0), (2, 0), (2, 1)])
def test_encode_args_replayed_as_a_serving_loop(bd, kernel):
    """The append pattern of a serving loop: ssq_encode arguments built once with
    hip_ops.encode_args (paged outputs through a slot mapping), each step's keys and slots written
    into the tensors the arguments point into, and the call replayed through the C ABI.  Every
    step's codes (and, with passthrough blocks, values) land in its slots, bit-exact with the
    oracle's encode of that step's keys.  block_dim 2 runs the grid search with the codec's grid
    (kernel 0) or the exact scan (kernel 1); block_dim 4 the MFMA encode."""
    import ctypes

    from sunshape_amd import _native as N

    log(f"encode_args replay bd={bd} kernel={kernel}")
    B, Hkv, D, page, P = 4, 2, 64, 16, 64
    nb = D // bd
    cb = synthetic.make_codebook(Hkv, D, bd, 150 + bd)
    heavy = synthetic.heavy_blocks_by_sigma(cb.sigma, cb.perm, bd, 3).tolist() if bd == 2 else None
    perm, cent = cb.perm.to(DEV), cb.centroids.to(DEV)
    grid = hip_ops.encode_grid(cent, Hkv) if bd == 2 and kernel == 0 else None
    code_pages = torch.zeros(P, Hkv, page, nb, dtype=torch.uint8, device=DEV)
    pt_pages = None if heavy is None else torch.zeros(P, Hkv, page, sum(heavy), bd, dtype=torch.bfloat16, device=DEV)
    table = torch.randperm(P, generator=torch.Generator().manual_seed(151))[:B * 4].view(B, 4)
    g = torch.Generator().manual_seed(152)

    def draw(step):
        keys = (torch.randn(B, Hkv, 1, D, generator=g) * cb.sigma[:, None, :]).to(torch.bfloat16)
        pos = 20 + step  # each sequence's next position
        slots = (table[:, pos // page] * page + pos % page).view(B, 1).to(torch.int64)
        return keys, slots

    keys0, slots0 = draw(0)
    a, _, _, keep = hip_ops.encode_args(keys0.to(DEV), perm, cent, heavy=heavy, codes_out=code_pages,
                                        pt_out=pt_pages, slot_mapping=slots0.to(DEV), kernel=kernel, grid=grid)
    keys_buf, slot_buf = keep[0], keep[5]
    stream = torch.cuda.current_stream(DEV).cuda_stream
    hv = None if heavy is None else np.array(heavy)
    for step in range(6):
        keys, slots = draw(step) if step else (keys0, slots0)
        keys_buf.copy_(keys.to(DEV).view_as(keys_buf))
        slot_buf.copy_(slots.to(DEV))
        N.check(N.lib().ssq_encode(ctypes.byref(a), ctypes.c_void_p(stream)))
        torch.cuda.synchronize()
        pg, off = slots[:, 0] // page, slots[:, 0] % page
        got = np_of(code_pages[pg.to(DEV), :, off.to(DEV)])  # [B, Hkv, nb]
        for b in range(B):
            for h in range(Hkv):
                rc, rpt = O.encode(keys[b, h].float().numpy(), cb.perm[h].numpy(), cb.centroids[h].numpy(), hv)
                assert np.array_equal(got[b, h], rc[0]), f"step {step} b={b} h={h}"
                if hv is not None:
                    gpt = np_of(pt_pages[int(pg[b]), h, int(off[b])].float())
                    assert np.array_equal(gpt, rpt[0][hv]), f"passthrough step {step} b={b} h={h}"
