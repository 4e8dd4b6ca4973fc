"""CPU checks of the grid-search encode's claims (no GPU): a key always lies in the (widened) cell
the search kernel computes for it; the builder's pre-selection (dmin(C, c_j)^2 <= min_k dmax(C, c_k)^2
+ M) holds the oracle's winner; and the winner meets every half-plane condition the builder clips a
cell with (|x - c_j|^2 - |x - c_k|^2 <= M_jk for each pre-selected k) at the key itself, so the
key lies in the winner's clipped polygon and the winner is listed.

The grid is this library's search structure (no reference counterpart); the winner it must
contain is the reference's first argmin (sunshape/codec.py:362-385), computed here by the
oracle's brute force over every codeword.
"""

import numpy as np
import pytest

from oracle import vq_oracle as O

KG = 128
MARGIN = 0.001
U24 = 2.0 ** -24
G = 1.001 * 4 * 2.0 ** -23


def cell_edge(t, mid, scale):
    """fp64 cell edge at map value t (the builder's inverse map)."""
    t = np.asarray(t, dtype=np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        x = mid + scale * (t / (1.0 - np.abs(t)))
    return np.where(t <= -1.0, -np.inf, np.where(t >= 1.0, np.inf, x))


def kernel_cell(x, mid, inv, rcp_ulps=0):
    """The search kernel's fp32 cell index; its reciprocal may be off by rcp_ulps units."""
    x = np.asarray(x, dtype=np.float32)
    u = (x - np.float32(mid)).astype(np.float32) * np.float32(inv)
    u = u.astype(np.float32)
    d = (np.float32(1.0) + np.abs(u)).astype(np.float32)
    r = (np.float32(1.0) / d).astype(np.float32)
    for _ in range(abs(rcp_ulps)):
        r = np.nextafter(r, np.float32(np.inf) if rcp_ulps > 0 else np.float32(0)).astype(np.float32)
    t = (u * r).astype(np.float32)
    f = np.floor(((t + np.float32(1.0)).astype(np.float32) * np.float32(0.5 * KG)).astype(np.float32))
    return np.clip(f, 0, KG - 1).astype(np.int64)


def widened(i, mid, inv):
    w = 2.0 / KG
    sc = 1.0 / np.float64(np.float32(inv))
    return cell_edge(-1 + w * (i - MARGIN), np.float64(np.float32(mid)), sc), \
        cell_edge(-1 + w * (i + 1 + MARGIN), np.float64(np.float32(mid)), sc)


@pytest.mark.parametrize("mid,inv", [(0.0, 1.0), (0.37, 2.9), (-5.0, 0.013), (1e3, 40.0), (2e-3, 3e4)])
def test_key_lies_in_its_widened_cell(mid, inv):
    """Keys at every cell edge (and a few ulps either side), random keys and far keys, with the
    reciprocal rounded either way: the computed cell's widened range holds the key."""
    rng = np.random.default_rng(int(abs(mid) * 7 + inv * 3))
    mid, inv = np.float32(mid), np.float32(inv)
    sc = 1.0 / np.float64(inv)
    edges = cell_edge(-1 + 2.0 * np.arange(1, KG) / KG, np.float64(mid), sc).astype(np.float32)
    xs = [edges]
    for k in (1, 2, 5):
        xs += [np.nextafter(edges, np.float32(np.inf)), np.nextafter(edges, np.float32(-np.inf))]
        edges = xs[-2]
    xs.append((np.float64(mid) + rng.standard_normal(20000) * sc * 3).astype(np.float32))
    xs.append((np.float64(mid) + rng.standard_normal(2000) * sc * 1e4).astype(np.float32))
    x = np.concatenate(xs).astype(np.float32)
    x = x[np.isfinite(x)]
    for ulps in (-1, 0, 1):
        f = kernel_cell(x, mid, inv, ulps)
        a, b = widened(f, mid, inv)
        bad = ~((a <= x) & (x <= b))
        assert not bad.any(), (ulps, x[bad][:5], f[bad][:5])


def cell_lists(c, mid, inv):
    """The builder's candidate lists for one block: counts [KG, KG] and a membership mask
    [KG, KG, nc] (fp64, the criterion dmin(C, c_j)^2 <= min_k dmax(C, c_k)^2 + M_C)."""
    a0, b0 = widened(np.arange(KG), mid[0], inv[0])
    a1, b1 = widened(np.arange(KG), mid[1], inv[1])
    A0, B0 = a0[:, None, None], b0[:, None, None]
    A1, B1 = a1[None, :, None], b1[None, :, None]
    cx, cy = c[None, None, :, 0].astype(np.float64), c[None, None, :, 1].astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        dx = np.maximum(np.abs(A0 - cx), np.abs(B0 - cx))
        dy = np.maximum(np.abs(A1 - cy), np.abs(B1 - cy))
        dmm = np.min(dx * dx + dy * dy, axis=2)
        R2 = np.maximum(A0 ** 2, B0 ** 2)[..., 0] + np.maximum(A1 ** 2, B1 ** 2)[..., 0]
        R = np.sqrt(R2)
        nrm = np.float32(c[:, 0].astype(np.float64) ** 2 + c[:, 1].astype(np.float64) ** 2).max()
        Rc = np.sqrt(np.float64(nrm)) * (1 + 2.0 ** -20)
        S, N2 = (R + Rc) ** 2, R2 + Rc * Rc
        M = 1.01 * (4.002 * U24 * N2 + 2.0002 * G * S + (dmm + 2.001 * U24 * N2 + G * S) * 2.0 ** -21)
        bound = dmm + M
        ex = np.maximum(np.maximum(A0 - cx, cx - B0), 0)
        ey = np.maximum(np.maximum(A1 - cy, cy - B1), 0)
        member = (ex * ex + ey * ey) <= bound[..., None]
    member |= ~np.isfinite(bound)[..., None]  # an unbounded cell lists everything: "scan all"
    return member.sum(2), member


def bounded_cell(x, mid, inv):
    """Per key: is its cell bounded (the unbounded end cells are scanned exhaustively)?"""
    f0, f1 = kernel_cell(x[:, 0], mid[0], inv[0]), kernel_cell(x[:, 1], mid[1], inv[1])
    a0, b0 = widened(f0, mid[0], inv[0])
    a1, b1 = widened(f1, mid[1], inv[1])
    return np.isfinite(a0) & np.isfinite(b0) & np.isfinite(a1) & np.isfinite(b1)


def winner_in_polygon(c, mid, inv, x, win, slack=True):
    """Per key: does the winner meet every half-plane condition of its cell's clipping at the
    key itself, 2 (c_k - c_w) . x <= M_wk + |c_k|^2 - |c_w|^2 for each pre-selected competitor k
    (fp64, as the builder)?  Keys in unbounded end cells (scanned exhaustively) count as held.
    slack=False drops the rounding margin M (a planted mistake the far cluster case exposes)."""
    f0, f1 = kernel_cell(x[:, 0], mid[0], inv[0]), kernel_cell(x[:, 1], mid[1], inv[1])
    a0, b0 = widened(f0, mid[0], inv[0])
    a1, b1 = widened(f1, mid[1], inv[1])
    cd = c.astype(np.float64)
    cx, cy = cd[None, :, 0], cd[None, :, 1]
    A0, B0, A1, B1 = a0[:, None], b0[:, None], a1[:, None], b1[:, None]
    ok = np.ones(len(x), dtype=bool)
    fin = np.isfinite(a0) & np.isfinite(b0) & np.isfinite(a1) & np.isfinite(b1)
    with np.errstate(invalid="ignore", over="ignore"):
        dmax = np.maximum(np.abs(A0 - cx), np.abs(B0 - cx)) ** 2 + np.maximum(np.abs(A1 - cy), np.abs(B1 - cy)) ** 2
        dmin = np.maximum(np.maximum(A0 - cx, cx - B0), 0) ** 2 + np.maximum(np.maximum(A1 - cy, cy - B1), 0) ** 2
        dmm = dmax.min(1)
        R2 = np.maximum(a0 ** 2, b0 ** 2) + np.maximum(a1 ** 2, b1 ** 2)
        R = np.sqrt(R2)
        nrm = np.float32(cd[:, 0] ** 2 + cd[:, 1] ** 2).max()
        Rc = np.sqrt(np.float64(nrm)) * (1 + 2.0 ** -20)
        S, N2 = (R + Rc) ** 2, R2 + Rc * Rc
        M0 = 1.01 * (4.002 * U24 * N2 + 2.0002 * G * S + (2.001 * U24 * N2 + G * S) * 2.0 ** -21)
        Mk = 1.01 * 2.0 ** -21
        if not slack:
            M0, Mk = 0.0 * M0, 0.0
        bound = dmm + M0 + Mk * dmm
        pre = dmin <= bound[:, None]
        cw = cd[win]
        nk = (cd ** 2).sum(1)[None, :]
        nw = (cw ** 2).sum(1)[:, None]
        xd = x.astype(np.float64)
        lhs = 2 * ((cx - cw[:, 0:1]) * xd[:, 0:1] + (cy - cw[:, 1:2]) * xd[:, 1:2])
        rhs = M0[:, None] + Mk * dmax + nk - nw
        held = (lhs <= rhs) | ~pre
    held[np.arange(len(x)), win] = True
    ok = held.all(1) | ~fin
    return ok


@pytest.mark.parametrize("seed,nc", [(0, 256), (1, 256), (2, 64), (3, 17)])
def test_cell_lists_hold_the_oracle_winner(seed, nc):
    """Random codebook (with duplicated and one-ulp-apart codewords); keys near Voronoi edges
    (midpoints of codeword pairs), on codewords, on cell edges and at random: the oracle's first
    argmin is in the key's cell list whenever that list is short enough to be used."""
    rng = np.random.default_rng(seed)
    c = (rng.standard_normal((nc, 2)) * np.array([1.0, 0.3])).astype(np.float32)
    if nc > 20:
        c[nc - 1] = c[3]
        c[nc - 2] = np.nextafter(c[5], np.float32(np.inf))
    lo, hi = c.min(0).astype(np.float64), c.max(0).astype(np.float64)
    mid = (0.5 * (lo + hi)).astype(np.float32)
    inv = (1.0 / c.astype(np.float64).std(0)).astype(np.float32)
    cnt, member = cell_lists(c, mid, inv)
    n = 6000
    i, j = rng.integers(0, nc, n), rng.integers(0, nc, n)
    keys = [(0.5 * (c[i].astype(np.float64) + c[j])).astype(np.float32), c[i]]
    keys.append((c[i] + rng.standard_normal((n, 2)) * 1e-3).astype(np.float32))
    keys.append((rng.standard_normal((n, 2)) * c.std(0) * 2).astype(np.float32))
    e0 = cell_edge(-1 + 2.0 * rng.integers(1, KG, n) / KG, np.float64(mid[0]), 1.0 / np.float64(inv[0]))
    e1 = cell_edge(-1 + 2.0 * rng.integers(1, KG, n) / KG, np.float64(mid[1]), 1.0 / np.float64(inv[1]))
    keys.append(np.stack([e0, e1], 1).astype(np.float32))
    x = np.concatenate(keys).astype(np.float32)
    win = O.encode(x, np.arange(2), c[None])[0][:, 0].astype(np.int64)
    f0, f1 = kernel_cell(x[:, 0], mid[0], inv[0]), kernel_cell(x[:, 1], mid[1], inv[1])
    bounded = bounded_cell(x, mid, inv)  # unbounded end cells: the builder scans them all
    assert bounded.mean() > 0.9
    held = member[f0, f1, win]
    assert held[bounded].all(), np.flatnonzero(bounded & ~held)[:10]
    poly = winner_in_polygon(c, mid, inv, x, win)
    assert poly.all(), np.flatnonzero(~poly)[:10]


def _lists_without_slack(c, mid, inv):
    """cell_lists with M_C = 0: dmin(C, c_j)^2 <= min_k dmax(C, c_k)^2 only."""
    a0, b0 = widened(np.arange(KG), mid[0], inv[0])
    a1, b1 = widened(np.arange(KG), mid[1], inv[1])
    A0, B0 = a0[:, None, None], b0[:, None, None]
    A1, B1 = a1[None, :, None], b1[None, :, None]
    cx, cy = c[None, None, :, 0].astype(np.float64), c[None, None, :, 1].astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        dx = np.maximum(np.abs(A0 - cx), np.abs(B0 - cx))
        dy = np.maximum(np.abs(A1 - cy), np.abs(B1 - cy))
        dmm = np.min(dx * dx + dy * dy, axis=2)
        ex = np.maximum(np.maximum(A0 - cx, cx - B0), 0)
        ey = np.maximum(np.maximum(A1 - cy, cy - B1), 0)
        member = (ex * ex + ey * ey) <= dmm[..., None]
    member |= ~np.isfinite(dmm)[..., None]
    return member


def far_cluster_case(seed, n=20000):
    """A small codebook clustered far from the origin (|c| ~ 1e2-1e3, spread ~0.01-1) and keys near
    the midpoints of codeword pairs: the reference's mm formulation cancels |x|^2 against 2 x.c,
    so its fp32 rounding, not the exact distance, decides many of these keys."""
    rng = np.random.default_rng(seed)
    nc = 8
    base = np.float32(rng.uniform(200, 3000))
    c = (base + rng.standard_normal((nc, 2)) * np.float32(rng.uniform(0.01, 1))).astype(np.float32)
    i, j = rng.integers(0, nc, n), rng.integers(0, nc, n)
    x = (0.5 * (c[i].astype(np.float64) + c[j]) + rng.standard_normal((n, 2)) * 1e-4).astype(np.float32)
    lo, hi = c.min(0).astype(np.float64), c.max(0).astype(np.float64)
    mid = (0.5 * (lo + hi)).astype(np.float32)
    inv = (1.0 / c.astype(np.float64).std(0)).astype(np.float32)
    return c, x, mid, inv


@pytest.mark.parametrize("seed", [0, 3, 12])
def test_rounding_slack_decides_lists_and_they_hold_the_winner(seed):
    """Inputs where the slack M_C matters: on a far-from-origin cluster it adds codewords to many
    lists, and for many keys the reference's fp32 winner is in the list only because of it.  With
    it every used list holds the winner; without it some would not."""
    c, x, mid, inv = far_cluster_case(seed)
    cnt, member = cell_lists(c, mid, inv)
    bare = _lists_without_slack(c, mid, inv)
    assert (member != bare).any()
    win = O.encode(x, np.arange(2), c[None])[0][:, 0].astype(np.int64)
    f0, f1 = kernel_cell(x[:, 0], mid[0], inv[0]), kernel_cell(x[:, 1], mid[1], inv[1])
    used = bounded_cell(x, mid, inv)
    assert used.mean() > 0.5
    held = member[f0, f1, win]
    assert held[used].all(), np.flatnonzero(used & ~held)[:10]
    only_with_slack = used & held & ~bare[f0, f1, win]
    assert only_with_slack.sum() > 100, int(only_with_slack.sum())
    # the clipping's half-planes: the winner meets them all with the margin, and without it many
    # winners would be cut from their own cell's list
    assert winner_in_polygon(c, mid, inv, x, win).all()
    cut = ~winner_in_polygon(c, mid, inv, x, win, slack=False)
    assert cut.sum() > 100, int(cut.sum())
