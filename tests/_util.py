"""Helpers shared by the GPU parity tests.

Tolerances (north-star): fp32 scores within 1e-4 and bf16 outputs within 2e-2,
measured norm-relative: max|got - ref| <= tol * max|ref| over the compared tensor.
Encode indices are compared bit-for-bit.
"""

from __future__ import annotations

import sys

import numpy as np
import torch

SCORE_TOL = 1e-4
BF16_TOL = 2e-2


def log(msg: str) -> None:
    """Name the case before any GPU step (flushed, so it survives a lost box)."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def np_of(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.numpy()


def assert_rel(got, ref, tol, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    scale = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    assert err <= tol * scale, f"{what}: max abs err {err:.3e} > {tol} * {scale:.3e}"
    return err / scale if scale else 0.0


def bf16_from_bits(bits) -> np.ndarray:
    return (np.asarray(bits).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)


def torch_bf16_from_bits(bits, device) -> torch.Tensor:
    return torch.from_numpy(np.asarray(bits).astype(np.int16)).view(torch.bfloat16).to(device)
