"""CPU restatement of SunShape's VQ-key decode-attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or, for the baseline, as
the timed CPU path).  The product package ``sunshape_amd`` never imports it and
has no CPU fallback.

Each function names the reference file:line it restates (paths relative to the
gauravsaini/sunshape tree).  Arithmetic follows the reference's eager PyTorch
path in fp32; fp64 is used only where the reference's result is a correctly
rounded fp32 value anyway (the LUT einsum is checked against fp64 with a
tolerance, not bit-for-bit).

Pinning (tests/test_oracle_*.py) -- what checks each function:
  forward/inverse transform   adjointness identity q . inv(k) == fwd(q) . k, exact
  lut_build                   fp64 einsum closed form; brute-force loops; one-hot queries
  scores_from_lut             == dequantize + matmul (two formulations), power-of-two
                              scale closed form, brute force on tiny inputs
  dequantize                  round trip encode(centroid rows) -> same rows
  bf16_round                  bit-for-bit against torch's .to(bfloat16)
  decode_attention            fp64 textbook softmax attention; torch.softmax/matmul
                              (the library calls the reference makes)
  encode (C library)          bit-for-bit against torch.cdist(...).argmin(-1) and
                              torch's pre-sqrt mm formulation; direct mode against torch's
                              scalar cdist kernel (<= 25 rows) bit for bit
  transform_rows              permutation matrices reproduce the gather exactly; orthogonal R
                              gives q . inv(k) == fwd(q) . k; R vs R^T distinguished; torch
                              matmul within fp32 rounding
  gather_pages                inverse of the page scatter used to build the layout
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


# ----------------------------------------------------------------------------
# dtype emulation
# ----------------------------------------------------------------------------

def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 -> bf16 (round-to-nearest-even) and return as fp32.

    torch's float->bfloat16 conversion (c10::BFloat16 round_to_nearest_even).
    NaN inputs are not produced on this path and are left unspecified.
    """
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return rounded.astype(np.uint32).view(np.float32).reshape(a.shape)


def f16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "f16":
        return f16_round(x)
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)


# ----------------------------------------------------------------------------
# codec transforms (sunshape/codec.py)
# ----------------------------------------------------------------------------

def invert_permutation(perm: np.ndarray) -> np.ndarray:
    """sunshape/codec.py:86-89."""
    perm = np.asarray(perm, dtype=np.int64)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.shape[-1], dtype=np.int64)
    return inv


def forward_transform(x: np.ndarray, perm: np.ndarray) -> np.ndarray:
    """x[..., perm]  (sunshape/codec.py:92-95, :247-252, permutation modes)."""
    return np.asarray(x)[..., np.asarray(perm, dtype=np.int64)]


def inverse_transform(x: np.ndarray, perm: np.ndarray) -> np.ndarray:
    """x[..., inv_perm]  (sunshape/codec.py:254-259)."""
    return np.asarray(x)[..., invert_permutation(perm)]


# ----------------------------------------------------------------------------
# LUT build + score gather-sum (sunshape/triton_kernels.py)
# ----------------------------------------------------------------------------

def query_scale(q: np.ndarray, scale: Optional[float], qdtype: str) -> np.ndarray:
    """``query_slice * float(scale)`` in the query dtype, then ``.to(float32)``.

    sunshape/vllm_attn_backend.py:235-236 multiplies the bf16/f16 query by a
    Python float: torch computes float(q) * float(scale) in fp32 and rounds the
    product to the query dtype.  sunshape/triton_kernels.py:429-430 upcasts.
    """
    q = np.asarray(q, dtype=np.float32)
    if scale is None:
        return q
    return round_to(q * np.float32(scale), qdtype)


def lut_build(qp: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """LUT[r, b, c] = sum_d qp[r, b*bd + d] * C[b, c, d].

    sunshape/triton_kernels.py:381-408 (``einsum("qbd,bcd->qbc")`` in fp32).
    Computed in fp64 and rounded once; the reference's einsum is within an ulp
    or two of this, which the tolerance-based comparisons absorb.
    qp: [R, D] query already in the codec basis.  centroids: [nb, nc, bd].
    """
    qp = np.asarray(qp, dtype=np.float64)
    c = np.asarray(centroids, dtype=np.float64)
    nb, nc, bd = c.shape
    qb = qp.reshape(qp.shape[0], nb, bd)
    return np.einsum("rbd,bcd->rbc", qb, c).astype(np.float32)


def scores_from_lut(lut: np.ndarray, codes: np.ndarray,
                    heavy: Optional[np.ndarray] = None,
                    qp: Optional[np.ndarray] = None,
                    pt_values: Optional[np.ndarray] = None) -> np.ndarray:
    """score[r, t] = sum_b LUT[r, b, codes[t, b]], fp32, blocks accumulated in order.

    sunshape/triton_kernels.py:174-196 (precomputed kernel: ``acc += dot_vals``
    for b = 0..nb-1 starting from zero).  Heavy (passthrough) blocks -- which the
    reference only scores through dequantize + matmul (codec.py:392-395,
    triton_kernels.py:300-311) -- contribute qp_b . pt_b in the same block order.
    lut: [R, nb, nc]; codes: [T, nb] integer; pt_values: [T, nb, bd] dense.
    """
    lut = np.asarray(lut, dtype=np.float32)
    codes = np.asarray(codes).astype(np.int64)
    R, nb, _ = lut.shape
    T = codes.shape[0]
    acc = np.zeros((R, T), dtype=np.float32)
    for b in range(nb):
        if heavy is not None and heavy[b]:
            bd = pt_values.shape[-1]
            qb = np.asarray(qp, dtype=np.float64)[:, b * bd:(b + 1) * bd]
            contrib = (qb @ np.asarray(pt_values, dtype=np.float64)[:, b, :].T).astype(np.float32)
        else:
            contrib = lut[:, b, :][:, codes[:, b]]
        acc = (acc + contrib).astype(np.float32)
    return acc


def dequantize(codes: np.ndarray, centroids: np.ndarray, perm: np.ndarray,
               heavy: Optional[np.ndarray] = None,
               pt_values: Optional[np.ndarray] = None,
               rotation: Optional[np.ndarray] = None) -> np.ndarray:
    """k_hat = inverse_transform(concat_b C[b, codes[:, b]] or passthrough).

    sunshape/codec.py:387-398.  Returns fp32 [T, D] in the original basis.
    rotation: the rotated mode's R [D, D]; the inverse transform is then k_hat @ R
    (sunshape/codec.py:257-258) and ``perm`` is ignored.
    """
    codes = np.asarray(codes).astype(np.int64)
    c = np.asarray(centroids, dtype=np.float32)
    nb, _, bd = c.shape
    T = codes.shape[0]
    k_hat = np.zeros((T, nb * bd), dtype=np.float32)
    for b in range(nb):
        if heavy is not None and heavy[b]:
            if pt_values is None:
                raise ValueError("Mixed-precision quantized keys are missing passthrough values.")
            k_hat[:, b * bd:(b + 1) * bd] = pt_values[:, b, :]
        else:
            k_hat[:, b * bd:(b + 1) * bd] = c[b][codes[:, b]]
    if rotation is not None:
        return transform_rows(k_hat, rotation, transpose=True)
    return inverse_transform(k_hat, perm)


def attention_scores(q: np.ndarray, codes: np.ndarray, centroids: np.ndarray, perm: np.ndarray,
                     heavy: Optional[np.ndarray] = None,
                     pt_values: Optional[np.ndarray] = None,
                     rotation: Optional[np.ndarray] = None) -> np.ndarray:
    """``sunshape_attention_scores(codec, q, quantized)``: unscaled fp32 [R, T].

    sunshape/triton_kernels.py:570-609 with the precomputed-LUT kernel
    (:416-482): q -> forward transform -> fp32 -> LUT -> gather-sum.
    rotation: the rotated mode's R [D, D]; the forward transform is then q @ R^T
    (sunshape/codec.py:250-251, applied at triton_kernels.py:427-428) and ``perm`` is ignored.
    """
    if rotation is not None:
        qp = transform_rows(np.asarray(q, dtype=np.float32), rotation)
        lut = lut_build(qp, centroids)
        return scores_from_lut(lut, codes, heavy, qp, pt_values)
    qp = forward_transform(np.asarray(q, dtype=np.float32), perm)
    lut = lut_build(qp, centroids)
    return scores_from_lut(lut, codes, heavy, qp, pt_values)


# ----------------------------------------------------------------------------
# decode attention (sunshape/vllm_attn_backend.py:216-253)
# ----------------------------------------------------------------------------

def select_mask_slice(mask: Optional[np.ndarray], b: int, h0: int, h1: int, batch: int):
    """sunshape/vllm_attn_backend.py:197-213."""
    if mask is None:
        return None
    if mask.ndim == 2:
        return mask[None]
    if mask.ndim == 3:
        if mask.shape[0] == batch:
            return mask[b][None]
        return mask[h0:h1]
    return mask[b, h0:h1]


def softmax_f32(s: np.ndarray) -> np.ndarray:
    """torch.softmax over the last dim in fp32 (max-subtracted exp, sum, divide)."""
    s = np.asarray(s, dtype=np.float32)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp((s - m).astype(np.float64)).astype(np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float64).astype(np.float32)).astype(np.float32)


def decode_attention(q: np.ndarray, codes: np.ndarray, v: np.ndarray,
                     centroids: np.ndarray, perm: np.ndarray,
                     scale: Optional[float], qdtype: str, vdtype: str,
                     mask: Optional[np.ndarray] = None,
                     heavy: Optional[np.ndarray] = None,
                     pt_values: Optional[np.ndarray] = None,
                     return_scores: bool = False,
                     rotation: Optional[np.ndarray] = None):
    """Fused-decode semantics of ``_apply_quantized_attention``.

    sunshape/vllm_attn_backend.py:216-253, one (batch, kv head) at a time:
      q = query[b, kv*G:(kv+1)*G] * scale          (query dtype)       :232-236
      scores = sunshape_attention_scores(...)      (fp32, [G*Lq, T])   :238-239
      scores += mask slice                                             :241-249
      probs = softmax(scores, -1).to(value.dtype)                      :251
      out = probs @ V[b, kv]                       (fp32 accumulate)   :252
    q: [B, Hq, Lq, D] (values already representable in qdtype);
    codes: [B, Hkv, T, nb]; v: [B, Hkv, T, Dv];
    centroids: [Hkv, nb, nc, bd] or [nb, nc, bd]; perm: [Hkv, D] or [D];
    pt_values: [B, Hkv, T, nb, bd] dense (zeros on light blocks) or None.
    Returns out fp32 [B, Hq, Lq, Dv] (already rounded to vdtype), and when
    return_scores: scores fp32 [B, Hq, Lq, T] and lse fp32 [B, Hq, Lq].
    rotation: the rotated mode's R [D, D] in place of the permutation (attention_scores).
    """
    q = np.asarray(q, dtype=np.float32)
    B, Hq, Lq, D = q.shape
    _, Hkv, T, _ = codes.shape
    Dv = v.shape[-1]
    G = Hq // Hkv
    out = np.zeros((B, Hq, Lq, Dv), dtype=np.float32)
    all_scores = np.zeros((B, Hq, Lq, T), dtype=np.float32) if return_scores else None
    lse = np.zeros((B, Hq, Lq), dtype=np.float32) if return_scores else None
    for b in range(B):
        for kv in range(Hkv):
            cen = centroids[kv] if centroids.ndim == 4 else centroids
            pm = perm[kv] if np.ndim(perm) == 2 else perm
            qs = query_scale(q[b, kv * G:(kv + 1) * G], scale, qdtype)      # [G, Lq, D]
            qf = qs.reshape(G * Lq, D)
            pt = None if pt_values is None else pt_values[b, kv]
            s = attention_scores(qf, codes[b, kv], cen, pm, heavy, pt, rotation).reshape(G, Lq, T)
            ms = select_mask_slice(mask, b, kv * G, (kv + 1) * G, B)
            if ms is not None:
                s = (s + np.asarray(ms, dtype=np.float32)).astype(np.float32)
            if return_scores:
                all_scores[b, kv * G:(kv + 1) * G] = s
                m = s.max(-1)
                lse[b, kv * G:(kv + 1) * G] = (m + np.log(np.exp((s - m[..., None]).astype(np.float64)).sum(-1))).astype(np.float32)
            p = round_to(softmax_f32(s), vdtype)
            vv = np.asarray(v[b, kv], dtype=np.float32)
            o = (p.astype(np.float64) @ vv.astype(np.float64)).astype(np.float32)
            out[b, kv * G:(kv + 1) * G] = round_to(o, vdtype)
    if return_scores:
        return out, all_scores, lse
    return out


# ----------------------------------------------------------------------------
# sub-byte packed codes (sunshape/triton_kernels.py:250-266 reads this layout)
# ----------------------------------------------------------------------------

def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """uint8 [..., nb] -> int32 [..., ceil(nb / vpe)], vpe = 32 // bits.

    Block b = p*vpe + v sits in bits [v*bits, (v+1)*bits) of word p, so that the
    reference's reader ``(packed[t, p] >> (v * bits)) & ((1 << bits) - 1)``
    (sunshape/triton_kernels.py:251-266) returns it.
    """
    codes = np.asarray(codes, dtype=np.uint8)
    nb = codes.shape[-1]
    vpe = 32 // bits
    nw = (nb + vpe - 1) // vpe
    words = np.zeros(codes.shape[:-1] + (nw,), dtype=np.uint64)
    for b in range(nb):
        p, v = divmod(b, vpe)
        words[..., p] |= (codes[..., b].astype(np.uint64) & ((1 << bits) - 1)) << np.uint64(v * bits)
    return words.astype(np.uint32).view(np.int32)


def unpack_codes(words: np.ndarray, nb: int, bits: int) -> np.ndarray:
    """The reference reader (sunshape/triton_kernels.py:251-266) applied to every block."""
    w = np.asarray(words).view(np.uint32).astype(np.uint64)
    vpe = 32 // bits
    out = np.empty(w.shape[:-1] + (nb,), dtype=np.uint8)
    for b in range(nb):
        p, v = divmod(b, vpe)
        out[..., b] = (w[..., p] >> np.uint64(v * bits)) & np.uint64((1 << bits) - 1)
    return out


# ----------------------------------------------------------------------------
# paged layout (vLLM-style pages; no counterpart in the reference)
# ----------------------------------------------------------------------------

def gather_pages_codes(code_pages: np.ndarray, block_table: np.ndarray, seq_len: int) -> np.ndarray:
    """Pages [P, Hkv, page, nb] + block table row -> contiguous [Hkv, seq_len, nb]."""
    page = code_pages.shape[2]
    n = (seq_len + page - 1) // page
    g = code_pages[np.asarray(block_table[:n], dtype=np.int64)]          # [n, Hkv, page, nb]
    g = np.transpose(g, (1, 0, 2, 3)).reshape(code_pages.shape[1], n * page, code_pages.shape[3])
    return g[:, :seq_len]


def gather_pages_values(v_pages: np.ndarray, block_table: np.ndarray, seq_len: int) -> np.ndarray:
    """V pages [P, Hkv, Dv, page] (vLLM's value layout) -> contiguous [Hkv, seq_len, Dv]."""
    page = v_pages.shape[3]
    n = (seq_len + page - 1) // page
    g = v_pages[np.asarray(block_table[:n], dtype=np.int64)]             # [n, Hkv, Dv, page]
    g = np.transpose(g, (1, 0, 3, 2)).reshape(v_pages.shape[1], n * page, v_pages.shape[2])
    return g[:, :seq_len]


# ----------------------------------------------------------------------------
# encode (C library; sunshape/codec.py:362-385)
# ----------------------------------------------------------------------------

def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "build", "liboracle_vq.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle C library not built: {path} (run `make -C oracle`)")
        lib = ctypes.CDLL(path)
        vp = ctypes.c_void_p
        lib.oracle_encode.argtypes = [vp, ctypes.c_int64, ctypes.c_int, vp, vp,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp]
        lib.oracle_encode.restype = None
        lib.oracle_encode_metric.argtypes = [vp, ctypes.c_int64, ctypes.c_int, vp, vp, vp,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp]
        lib.oracle_encode_metric.restype = None
        lib.oracle_block_dist.argtypes = [vp, ctypes.c_int64, vp, ctypes.c_int, ctypes.c_int, vp, vp]
        lib.oracle_block_dist.restype = None
        lib.oracle_block_dist_ex.argtypes = [vp, ctypes.c_int64, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
        lib.oracle_block_dist_ex.restype = None
        lib.oracle_encode_ex.argtypes = [vp, ctypes.c_int64, ctypes.c_int, vp, vp, vp, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp]
        lib.oracle_encode_ex.restype = None
        lib.oracle_encode_wide.argtypes = [vp, ctypes.c_int64, ctypes.c_int, vp, vp, vp, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp]
        lib.oracle_encode_wide.restype = None
        lib.oracle_transform_rows.argtypes = [vp, ctypes.c_int64, ctypes.c_int, vp, ctypes.c_int, vp]
        lib.oracle_transform_rows.restype = None
        _LIB = lib
    return _LIB


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def transform_rows(x: np.ndarray, M: np.ndarray, transpose: bool = False) -> np.ndarray:
    """x @ M^T (rotated mode's forward transform, sunshape/codec.py:250-251) or, with transpose,
    x @ M (its inverse, :257-258), fp32 with the k-ascending fused order of oracle/vq_encode.c."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = np.ascontiguousarray(M, dtype=np.float32)
    shape = x.shape
    D = shape[-1]
    if M.shape != (D, D):
        raise ValueError(f"matrix must be [{D}, {D}]")
    flat = x.reshape(-1, D)
    out = np.empty_like(flat)
    _lib().oracle_transform_rows(_ptr(flat), flat.shape[0], D, _ptr(M), 1 if transpose else 0, _ptr(out))
    return out.reshape(shape)


def index_dtype(n_centroids: int):
    """Stored index dtype: sunshape/codec.py:78-83 (_compact_index_dtype), with the 16-bit case
    unsigned so indices up to 65535 keep their value (the reference's int16 holds the same bits)."""
    return np.uint8 if n_centroids <= 256 else np.uint16 if n_centroids <= 65535 else np.int32


def encode(keys: np.ndarray, perm: np.ndarray, centroids: np.ndarray,
           heavy: Optional[np.ndarray] = None, metric: Optional[np.ndarray] = None,
           direct: bool = False, rotation: Optional[np.ndarray] = None, threads: int = 1):
    """``codec.quantize(keys)``: codes [N, nb] (index_dtype), passthrough fp32 [N, nb, bd] or None.

    sunshape/codec.py:362-385; exact arithmetic in oracle/vq_encode.c.
    keys: [N, D] values (bf16 keys pass as their exact fp32 upcast).
    metric: the codec's E [D, D] (SunShape-Pro block metric; only its diagonal
    bd x bd blocks are read, as codec.py:375-376 slices them), None = identity.
    direct: torch.cdist's direct distance (both inputs at most 25 rows) in place of its
    mm formulation.
    rotation: the rotated mode's R [D, D]: keys go through x @ R^T (transform_rows) and
    ``perm`` is ignored (sunshape/codec.py:364, :250-251).
    threads: row chunks encoded on that many host threads (the C code runs without the GIL);
    the result does not depend on it.
    """
    keys = np.ascontiguousarray(keys, dtype=np.float32)
    if rotation is not None:
        keys = transform_rows(keys, rotation)
        perm = np.arange(keys.shape[1])
    perm = np.ascontiguousarray(perm, dtype=np.int64)
    cen = np.ascontiguousarray(centroids, dtype=np.float32)
    nb, nc, bd = cen.shape
    n, D = keys.shape
    wide = nc > 256
    codes = np.empty((n, nb), dtype=np.int32 if wide else np.uint8)
    hv = None
    pt = None
    if heavy is not None and np.any(heavy):
        hv = np.ascontiguousarray(np.asarray(heavy, dtype=bool).astype(np.uint8))
        pt = np.empty((n, nb, bd), dtype=np.float32)
    met = None if metric is None else np.ascontiguousarray(metric, dtype=np.float32)
    if met is not None and met.shape != (D, D):
        raise ValueError(f"metric must be [{D}, {D}]")
    fn = _lib().oracle_encode_wide if wide else _lib().oracle_encode_ex

    def run(lo: int, hi: int) -> None:
        if hi > lo:
            fn(_ptr(keys[lo:hi]), hi - lo, D, _ptr(perm), _ptr(cen), _ptr(met), 1 if direct else 0, nb, nc, bd,
               _ptr(hv), _ptr(codes[lo:hi]), None if pt is None else _ptr(pt[lo:hi]))

    if threads > 1 and n > 1:
        from concurrent.futures import ThreadPoolExecutor

        step = (n + threads - 1) // threads
        with ThreadPoolExecutor(threads) as ex:
            list(ex.map(lambda lo: run(lo, min(lo + step, n)), range(0, n, step)))
    else:
        run(0, n)
    return (codes.astype(index_dtype(nc)) if wide else codes), pt


def block_distances(x: np.ndarray, c: np.ndarray, direct: bool = False):
    """Pre-sqrt and post-sqrt cdist matrices for one block (x [n, bd], c [nc, bd]); direct: the
    direct evaluation torch.cdist takes when both inputs have at most 25 rows."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    c = np.ascontiguousarray(c, dtype=np.float32)
    n, bd = x.shape
    nc = c.shape[0]
    e2 = np.empty((n, nc), dtype=np.float32)
    d = np.empty((n, nc), dtype=np.float32)
    _lib().oracle_block_dist_ex(_ptr(x), n, _ptr(c), nc, bd, 1 if direct else 0, _ptr(e2), _ptr(d))
    return e2, d


# ----------------------------------------------------------------------------
# synthetic-config helpers used by the checker
# ----------------------------------------------------------------------------

def lse_merge(m: np.ndarray, l: np.ndarray, o: np.ndarray):
    """Combine split partials (max, sum-exp, unnormalised out) along axis 0."""
    M = m.max(0)
    w = np.exp((m - M).astype(np.float64))
    L = (l * w).sum(0)
    O = (o * w[..., None]).sum(0) / L[..., None]
    return O.astype(np.float32), (M + np.log(L)).astype(np.float32)


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("annotations", "ctypes", "math", "os", "np", "Optional")]
