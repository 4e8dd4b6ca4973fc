"""A seeded sweep of decode problems against the oracle: each case draws its layout (contiguous
rows or vLLM-style pages with ragged lengths), head_dim, block_dim, codebook size (16 to 1,024
codewords: byte and 16-bit codes), KV heads, query heads per KV head, new tokens, value dtype,
passthrough blocks, additive mask (random with a finite bias, or causal), split count and code
storage (bytes, 16-bit, or int32 words of 4 to 8 bits), and compares output, lse and raw scores
with the reference semantics
(sunshape/vllm_attn_backend.py:216-253 via the oracle) within the north-star tolerances.  The
hand-picked tests cover each kernel's shapes; this sweep covers their combinations, on the
planner's pick and on every kernel forced (1 generic, 2 MFMA LUT, 3 MFMA contiguous, 4
4x4-MFMA scores) that accepts the problem: one that does not returns SSQ_ERR_UNSUPPORTED.  On
contiguous rows the scores-only entry point (gqa_scores) runs the same problem without values
or mask, on every kernel that accepts it."""

import math

import numpy as np
import pytest
import torch

from _util import BF16_TOL, SCORE_TOL, assert_rel, log, np_of
from oracle import vq_oracle as O
from sunshape_amd import _native as N
from sunshape_amd import hip_ops, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PAGE = 16


def _draw(seed, more=False):
    """One problem; ``more`` widens it: head_dim 256, a value width apart from head_dim, up to six
    new tokens (so more query rows than one workgroup takes), and masks given as broadcast views."""
    rng = np.random.default_rng(seed)
    D = int(rng.choice([64, 128, 256] if more else [64, 128]))
    bd = int(rng.choice([b for b in (1, 2, 4, 8) if D // b <= 64]))
    nb = D // bd
    c = dict(seed=seed, D=D, bd=bd, nb=nb, nc=int(rng.choice([16, 64, 256, 256, 1024])),
             Hkv=int(rng.choice([1, 2])), G=int(rng.choice([1, 2, 4, 7, 8])), B=int(rng.integers(1, 4)),
             Lq=int(rng.choice([1, 1, 2, 3])), T=int(rng.integers(1, 700)), paged=bool(rng.integers(0, 2)),
             vdt=torch.bfloat16 if rng.integers(0, 3) else torch.float16,
             n_heavy=int(rng.choice([0, 0, 1, 3])) if nb >= 4 else 0, splits=int(rng.choice([0, 0, 1, 3])))
    c["mask"] = ["none", "random", "causal"][int(rng.integers(0, 3))]
    c["bits"] = 0  # sub-byte packed code words (int32) where the codebook fits
    if c["nc"] <= 256 and rng.integers(0, 3) == 0:
        c["bits"] = int(rng.integers(int(math.log2(c["nc"])), 9))
    c["Dv"], c["mask_view"] = D, "full"
    if more:
        c["Dv"] = int(rng.choice([64, 128] + ([256] if D == 256 else [])))
        c["Lq"] = int(rng.integers(1, 7))
        c["mask_view"] = str(rng.choice(["full", "per_batch", "per_head"]))
    return c


def _paginate(codes, v, stored, lens, gen):
    """Scatter contiguous rows into shuffled 16-token pages (codes [P, Hkv, 16, nb], values
    [P, Hkv, Dv, 16], passthrough [P, Hkv, 16, slots, bd]); slots past a length stay garbage."""
    B, Hkv, T, nb = codes.shape
    n = (T + PAGE - 1) // PAGE
    table = torch.randperm(B * n, generator=gen).view(B, n).to(torch.int32)
    cp = torch.zeros((B * n, Hkv, PAGE, nb), dtype=codes.dtype)
    vp = torch.full((B * n, Hkv, v.shape[-1], PAGE), float("nan"), dtype=v.dtype)
    pp = None if stored is None else torch.full((B * n, Hkv, PAGE) + tuple(stored.shape[-2:]), float("nan"),
                                                dtype=stored.dtype)
    for b in range(B):
        for j in range(n):
            pg, t0, t1 = int(table[b, j]), j * PAGE, min((j + 1) * PAGE, int(lens[b]))
            if t1 <= t0:
                continue
            cp[pg, :, :t1 - t0] = codes[b, :, t0:t1]
            vp[pg, :, :, :t1 - t0] = v[b, :, t0:t1].transpose(-1, -2)
            if pp is not None:
                pp[pg, :, :t1 - t0] = stored[b, :, t0:t1]
    return cp, vp, pp, table


@pytest.mark.parametrize("seed", list(range(900, 960)))
def test_decode_sweep_vs_oracle(seed):
    _sweep_case(_draw(seed))


@pytest.mark.parametrize("seed", list(range(1000, 1040)))
def test_decode_sweep_more_shapes_vs_oracle(seed):
    _sweep_case(_draw(seed, more=True))


def _sweep_case(c):
    log(f"decode sweep {c}")
    D, bd, nb, nc, Hkv, G, B, Lq, T, Dv = (c[k] for k in ("D", "bd", "nb", "nc", "Hkv", "G", "B", "Lq", "T", "Dv"))
    seed = c["seed"]
    Hq = Hkv * G
    gen = torch.Generator().manual_seed(seed)
    cb = synthetic.make_codebook(Hkv, D, bd, seed, n_centroids=nc)
    q = torch.randn(B, Hq, Lq, D, generator=gen).to(torch.bfloat16)
    codes = torch.randint(0, nc, (B, Hkv, T, nb), generator=gen, dtype=torch.int32)
    codes = codes.to(torch.uint8 if nc <= 256 else torch.int16)
    v = torch.randn(B, Hkv, T, Dv, generator=gen).to(c["vdt"])
    heavy = None
    ptd = stored = None
    if c["n_heavy"]:
        hidx = sorted(torch.randperm(nb, generator=gen)[:c["n_heavy"]].tolist())
        heavy = [i in hidx for i in range(nb)]
        ptd = torch.zeros(B, Hkv, T, nb, bd)
        ptd[:, :, :, hidx] = torch.randn(B, Hkv, T, len(hidx), bd, generator=gen).to(torch.bfloat16).float()
        stored = ptd[:, :, :, hidx].to(torch.bfloat16).contiguous()
    lens = [T] + [max(1, T - 37 * (i + 1)) for i in range(B - 1)] if c["paged"] else [T] * B
    span = ((T + PAGE - 1) // PAGE) * PAGE if c["paged"] else T
    mask = None
    if c["mask"] == "random":
        # per_batch / per_head: one mask row set per sequence or per query head, handed to the
        # kernel as a broadcast (stride-0) view
        mshape = {"full": (B, Hq), "per_batch": (B, 1), "per_head": (1, Hq)}[c["mask_view"]]
        mask = torch.where(torch.rand(*mshape, Lq, span, generator=gen) < 0.2, float("-inf"), 0.0)
        mask[..., 0] = 0.0
        mask[0, 0] += -1.5
    elif c["mask"] == "causal":
        pos = torch.arange(span)
        last = T - Lq + torch.arange(Lq)
        mask = torch.zeros(1, 1, Lq, span).masked_fill(pos[None, :] > last[:, None], float("-inf")).expand(B, Hq, Lq,
                                                                                                        span)
        mask = mask.contiguous()
    scale = 1 / math.sqrt(D)
    bits = c["bits"]

    def dev_codes(x):
        x = x.to(DEV)
        return hip_ops.pack_codes(x, bits) if bits else x

    dmask = None if mask is None else mask.to(DEV).expand(B, Hq, Lq, span)
    mask = None if mask is None else mask.expand(B, Hq, Lq, span).contiguous()
    kw = dict(scale=scale, num_splits=c["splits"], heavy=heavy, mask=dmask, return_lse=True, return_scores=True,
              code_bits=bits)
    args = (q.to(DEV), dev_codes(codes), v.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    if c["paged"]:
        cp, vp, pp, table = _paginate(codes, v, stored, lens, gen)
        kw.update(block_table=table.to(DEV), seq_lens=torch.tensor(lens, dtype=torch.int32).to(DEV),
                  pt=None if pp is None else pp.to(DEV))
        args = (q.to(DEV), dev_codes(cp), vp.to(DEV), cb.perm.to(DEV), cb.centroids.to(DEV))
    else:
        kw.update(pt=None if stored is None else stored.to(DEV))
    runs = {}
    for kernel in (0, 1, 2, 3, 4):
        try:
            runs[kernel] = [np_of(t) for t in hip_ops.decode(*args, kernel=kernel, **kw)]
        except N.SunShapeKernelError as e:
            assert e.status == N.SSQ_ERR_UNSUPPORTED and kernel >= 2, (kernel, e.status, str(e))
    log(f"kernels run: {sorted(runs)}")
    assert 0 in runs and 1 in runs
    sruns = {}
    if not c["paged"]:
        for kernel in (0, 1, 2, 3, 4):
            try:
                sruns[kernel] = np_of(hip_ops.gqa_scores(args[0], args[1], args[3], args[4], scale=scale, heavy=heavy,
                                                         pt=kw["pt"], code_bits=bits, num_splits=c["splits"],
                                                         kernel=kernel))
            except N.SunShapeKernelError as e:
                assert e.status == N.SSQ_ERR_UNSUPPORTED and kernel >= 2, (kernel, e.status, str(e))
        log(f"scores-only kernels run: {sorted(sruns)}")
        assert 0 in sruns and 1 in sruns
    vdt = "bf16" if c["vdt"] == torch.bfloat16 else "f16"
    hv = np.array(heavy) if heavy else None
    for b in range(B):
        L = lens[b]
        m = None if mask is None else mask[b:b + 1, ..., :L].numpy()
        ro, rs, rl = O.decode_attention(q[b:b + 1].float().numpy(), codes[b:b + 1, :, :L].numpy().astype(np.int64),
                                        v[b:b + 1, :, :L].float().numpy(), cb.centroids.numpy(), cb.perm.numpy(),
                                        scale, "bf16", vdt, mask=m, heavy=hv,
                                        pt_values=None if hv is None else ptd[b:b + 1, :, :L].numpy(),
                                        return_scores=True)
        fin = np.isfinite(rs)
        rows = np.isfinite(rl)  # a row whose every score is masked has no defined output
        if sruns:  # scores-only launches carry no mask
            rs0 = rs if m is None else O.decode_attention(
                q[b:b + 1].float().numpy(), codes[b:b + 1, :, :L].numpy().astype(np.int64),
                v[b:b + 1, :, :L].float().numpy(), cb.centroids.numpy(), cb.perm.numpy(), scale, "bf16", vdt,
                heavy=hv, pt_values=None if hv is None else ptd[b:b + 1, :, :L].numpy(), return_scores=True)[1]
            for kernel, so in sruns.items():
                assert_rel(so[b:b + 1], rs0, SCORE_TOL, f"scores-only kernel {kernel} b={b}")
        for kernel, (o, l, sc) in runs.items():
            what = f"kernel {kernel} b={b}"
            assert np.array_equal(np.isfinite(sc[b:b + 1, ..., :L]), fin), f"finite scores {what}"
            assert_rel(sc[b:b + 1, ..., :L][fin], rs[fin], SCORE_TOL, f"scores {what}")
            assert np.array_equal(np.isfinite(l[b:b + 1]), rows), f"finite lse {what}"
            assert_rel(l[b:b + 1][rows], rl[rows], SCORE_TOL, f"lse {what}")
            assert_rel(o[b:b + 1][rows], ro[rows], BF16_TOL, f"out {what}")
