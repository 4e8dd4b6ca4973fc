"""A seeded sweep of encode problems against the oracle, bit for bit: each case draws head_dim,
block_dim, codebook size (16 to 1,024 codewords), shared or per-KV-head codebooks, key dtype,
passthrough blocks (compact or dense, in the key dtype, bf16 or fp32), the SunShape-Pro block
metric or the rotated mode's R, torch.cdist's direct distance (at most 25 rows and codewords),
and contiguous or paged output through a slot mapping, with some keys set exactly onto
codewords.  Every encode kernel that accepts the problem runs it (the planner's pick, 1 exact
scan, 2 MFMA screen, 3 grid search where a grid applies: block_dim 2, no metric); the others must
refuse with SSQ_ERR_UNSUPPORTED.  Reference: sunshape/codec.py:362-385 via the oracle."""

import numpy as np
import pytest
import torch

from _util import log, np_of
from oracle import vq_oracle as O
from sunshape_amd import _native as N
from sunshape_amd import hip_ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PAGE = 16
DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _draw(seed):
    rng = np.random.default_rng(seed)
    D = int(rng.choice([48, 64, 128]))
    bd = int(rng.choice([b for b in (1, 2, 3, 4, 8, 16) if D % b == 0 and D // b <= 128]))
    nb = D // bd
    c = dict(seed=seed, D=D, bd=bd, nb=nb, nc=int(rng.choice([16, 64, 256, 256, 256, 1024])),
             Hkv=int(rng.choice([1, 2])), B=int(rng.integers(1, 3)), S=int(rng.integers(1, 600)),
             per_head=bool(rng.integers(0, 2)), kdt=str(rng.choice(["bf16", "bf16", "f16", "f32"])),
             n_heavy=int(rng.choice([0, 0, 1, 4])), dense=bool(rng.integers(0, 2)),
             ptdt=str(rng.choice(["key", "bf16", "f32"])), mode=str(rng.choice(["perm", "perm", "metric", "rotated"])),
             paged=bool(rng.integers(0, 3) == 0))
    if c["paged"]:
        c["dense"] = False  # pages take the compact layout
    c["direct"] = False
    if c["nc"] <= 25 and rng.integers(0, 2):  # a call torch.cdist evaluates directly
        c["S"], c["direct"] = int(rng.integers(1, 26)), True
    return c


def _round(x, dt):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dt).float().numpy()


@pytest.mark.parametrize("seed", list(range(700, 760)))
def test_encode_sweep_vs_oracle(seed):
    c = _draw(seed)
    log(f"encode sweep {c}")
    D, bd, nb, nc, Hkv, B, S = (c[k] for k in ("D", "bd", "nb", "nc", "Hkv", "B", "S"))
    rng = np.random.default_rng(seed + 1)
    kdt = DTYPES[c["kdt"]]
    sig = np.exp(rng.uniform(np.log(0.1), np.log(3), (Hkv, D))).astype(np.float32)
    perm = np.stack([rng.permutation(D) for _ in range(Hkv)])
    cent = (rng.standard_normal((Hkv, nb, nc, bd)) * np.take_along_axis(sig, perm, 1).reshape(Hkv, nb, 1, bd))
    cent = cent.astype(np.float32)
    if not c["per_head"]:
        perm, cent = perm[:1].repeat(Hkv, 0), cent[:1].repeat(Hkv, 0)
    metric = rot = None
    if c["mode"] == "metric":
        metric = (np.eye(D) + 0.3 * rng.standard_normal((Hkv if c["per_head"] else 1, D, D)) / np.sqrt(D))
        metric = metric.astype(np.float32).repeat(1 if c["per_head"] else Hkv, 0)
    elif c["mode"] == "rotated":
        rot = np.linalg.qr(rng.standard_normal((D, D)))[0].astype(np.float32)
    keys = (rng.standard_normal((B, Hkv, S, D)) * sig[None, :, None]).astype(np.float32)
    if c["mode"] == "perm":  # some key blocks sit exactly on a codeword (distance 0)
        for kv in range(Hkv):
            t, blk = rng.integers(0, S, 8), rng.integers(0, nb, 8)
            for tt, bb in zip(t, blk):
                keys[0, kv, tt, perm[kv, bb * bd:(bb + 1) * bd]] = cent[kv, bb, rng.integers(0, nc)]
    keys = _round(keys, kdt)
    heavy = None
    hidx = []
    if c["n_heavy"]:
        hidx = sorted(rng.choice(nb, min(c["n_heavy"], nb - 1 if nb > 1 else 0), replace=False).tolist())
        heavy = [i in hidx for i in range(nb)] if hidx else None
    ptdt = kdt if c["ptdt"] == "key" else DTYPES[c["ptdt"]]

    # oracle, per (batch, KV head): codes [B, Hkv, S, nb], passthrough [B, Hkv, S, nb, bd]
    ref_codes = np.zeros((B, Hkv, S, nb), np.int64)
    ref_pt = np.zeros((B, Hkv, S, nb, bd), np.float32)
    for kv in range(Hkv):
        rows = keys[:, kv].reshape(B * S, D)
        rc, rp = O.encode(rows, perm[kv], cent[kv], None if heavy is None else np.array(heavy),
                          metric=None if metric is None else metric[kv], direct=c["direct"], rotation=rot)
        ref_codes[:, kv] = rc.astype(np.int64).reshape(B, S, nb)
        if rp is not None:
            ref_pt[:, kv] = rp.reshape(B, S, nb, bd)

    kt = torch.from_numpy(keys).to(DEV).to(kdt)
    pt_ = torch.from_numpy(perm if c["per_head"] else perm[0]).to(DEV)
    ct_ = torch.from_numpy(cent if c["per_head"] else cent[0]).to(DEV)
    mt_ = None if metric is None else torch.from_numpy(metric if c["per_head"] else metric[0]).to(DEV)
    rt_ = None if rot is None else torch.from_numpy(rot).to(DEV)
    grid = None
    if bd == 2 and nc <= 256 and metric is None:
        grid = hip_ops.encode_grid(ct_, Hkv)
    kernels = (0, 1, 2, 3) if grid is not None else (0, 1, 2)
    ran = []
    for kernel in kernels:
        kw = dict(heavy=heavy, pt_dtype=ptdt, pt_dense=c["dense"], metric=mt_, kernel=kernel,
                  grid=grid if kernel in (0, 3) else None, direct=c["direct"], rotation=rt_)
        if c["paged"]:
            n_pages = (B * S + PAGE - 1) // PAGE + 2
            slots = torch.randperm(n_pages * PAGE, generator=torch.Generator().manual_seed(seed))[:B * S].view(B, S)
            codes_out = torch.full((n_pages, Hkv, PAGE, nb), 7, dtype=hip_ops.index_dtype(nc), device=DEV)
            pt_out = None
            if hidx:
                pt_out = torch.full((n_pages, Hkv, PAGE, len(hidx), bd), -3.0, dtype=ptdt, device=DEV)
            kw.update(slot_mapping=slots.to(DEV), codes_out=codes_out, pt_out=pt_out)
        try:
            codes, pt = hip_ops.encode(kt, pt_, ct_, **kw)
        except N.SunShapeKernelError as e:
            assert e.status == N.SSQ_ERR_UNSUPPORTED and kernel >= 2, (kernel, e.status, str(e))
            continue
        ran.append(kernel)
        got = np_of(codes)
        if got.dtype == np.int16:
            got = got.view(np.uint16)
        got = got.astype(np.int64)
        gpt = None if pt is None else np_of(pt.float())
        if c["paged"]:  # gather each token's slot back into [B, Hkv, S, ...]
            sl = slots.numpy()
            pg, off = sl // PAGE, sl % PAGE
            got = np.stack([got[pg[b], :, off[b]] for b in range(B)]).transpose(0, 2, 1, 3)
            if gpt is not None:
                gpt = np.stack([gpt[pg[b], :, off[b]] for b in range(B)]).transpose(0, 2, 1, 3, 4)
        light = [i for i in range(nb) if i not in hidx]
        diff = got[..., light] != ref_codes[..., light]
        assert not diff.any(), f"kernel {kernel}: {int(diff.sum())} codes differ"
        if hidx:
            assert (got[..., hidx] == 0).all(), f"kernel {kernel}: heavy block codes must be 0"
            want = _round(ref_pt, ptdt)
            if c["dense"]:
                assert np.array_equal(gpt[..., hidx, :], want[..., hidx, :]), f"kernel {kernel}: passthrough"
                assert (gpt[..., light, :] == 0).all(), f"kernel {kernel}: dense light slots must be 0"
            else:
                assert np.array_equal(gpt, want[..., hidx, :]), f"kernel {kernel}: passthrough"
        else:
            assert pt is None or not c["n_heavy"]
    log(f"kernels run: {ran}")
    assert 0 in ran and 1 in ran
