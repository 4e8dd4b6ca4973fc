"""Torch-tensor wrappers over the sunshape_amd C ABI.

Every function takes device tensors, checks shapes/dtypes/strides on the host,
launches on the tensors' current HIP stream and returns freshly allocated
outputs (the caller's inputs are never written).  Codec arrays may be shared by
all KV heads (the reference's per-layer codec: perm [D], centroids
[nb, nc, bd]) or given per KV head (perm [Hkv, D], centroids [Hkv, nb, nc, bd]).
"""

from __future__ import annotations

import ctypes
import types
from typing import Optional, Sequence

import torch

from . import _native as N


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _on_gpu(name: str, t: torch.Tensor) -> None:
    _require(t.is_cuda, f"{name} must be a HIP device tensor (got device {t.device}); this library has no CPU path")


def _codec_arrays(perm: torch.Tensor, cent: torch.Tensor, head_dim: int, n_kv: Optional[int]):
    """Validate codec arrays; return (perm, cent, perm_sh, cent_sh, bd, nb, nc)."""
    _on_gpu("permutation", perm)
    _on_gpu("centroids", cent)
    _require(perm.dtype == torch.int64, "permutation must be int64")
    _require(cent.dtype == torch.float32, "centroids must be float32")
    perm = perm.contiguous()
    cent = cent.contiguous()
    if cent.ndim == 3:
        nb, nc, bd = cent.shape
        cent_sh = 0
    elif cent.ndim == 4:
        _, nb, nc, bd = cent.shape
        _require(n_kv is None or cent.shape[0] == n_kv, f"centroids hold {cent.shape[0]} KV heads, expected {n_kv}")
        cent_sh = nb * nc * bd
    else:
        raise RuntimeError(f"Expected codec.centroids.ndim == 3 (or 4 for per-KV-head codebooks), got {cent.ndim}.")
    if perm.ndim == 1:
        perm_sh = 0
        _require(perm.shape[0] == head_dim, f"permutation length {perm.shape[0]} != head_dim {head_dim}")
    else:
        _require(perm.ndim == 2 and perm.shape[1] == head_dim, "permutation must be [D] or [Hkv, D]")
        _require(n_kv is None or perm.shape[0] == n_kv, f"permutation holds {perm.shape[0]} KV heads, expected {n_kv}")
        perm_sh = head_dim
    _require(nb * bd == head_dim, f"centroids [{nb}, {nc}, {bd}] do not tile head_dim {head_dim}")
    return perm, cent, perm_sh, cent_sh, bd, nb, nc


def transform_rows(x: torch.Tensor, mat: torch.Tensor, *, transpose: bool = False,
                   scale: Optional[float] = None) -> torch.Tensor:
    """fp32 ``xs @ mat.T`` (or ``xs @ mat`` with transpose) over the last dim, xs = x, or x * scale
    rounded to x's dtype (the decode's query scaling).  The rotated mode's transforms,
    sunshape/codec.py:247-259: forward ``x @ rotation.T``, inverse ``x @ rotation``.
    """
    _on_gpu("x", x)
    _on_gpu("rotation", mat)
    D = x.shape[-1]
    _require(mat.shape == (D, D), f"rotation must be [{D}, {D}], got {tuple(mat.shape)}")
    mat = mat.to(torch.float32).contiguous()
    flat = x.reshape(-1, D)
    flat = flat if flat.stride(-1) == 1 else flat.contiguous()
    out = torch.empty((flat.shape[0], D), device=x.device, dtype=torch.float32)
    if flat.shape[0]:
        with torch.cuda.device(x.device):  # the library reads the current device
            N.check(N.lib().ssq_transform_rows(N.ptr(flat), N.dtype_code(flat.dtype), flat.stride(0), flat.shape[0], D,
                                               1 if scale is not None else 0, float(scale or 0.0), N.ptr(mat),
                                               1 if transpose else 0, N.ptr(out), out.stride(0), N.stream_of(x.device)))
    return out.view(*x.shape[:-1], D)


_IDENT: dict = {}


def _identity_like(perm: torch.Tensor) -> torch.Tensor:
    """The identity permutation in perm's shape ([D] or [Hkv, D]): under a rotation the kernels see
    queries and keys already in the codec basis."""
    key = (perm.device, tuple(perm.shape))
    t = _IDENT.get(key)
    if t is None:
        t = torch.arange(perm.shape[-1], device=perm.device, dtype=torch.int64).expand(perm.shape).contiguous()
        _IDENT[key] = t
    return t


def lut_build(q: torch.Tensor, perm: torch.Tensor, cent: torch.Tensor, scale: Optional[float] = None) -> torch.Tensor:
    """LUT[r, b, c] = q_perm[r, b-block] . C[b, c]  (fp32 [R, nb, nc]).

    Reference: sunshape/triton_kernels.py:381-408 (``_precompute_query_centroid_dots``).
    """
    _on_gpu("query", q)
    _require(q.ndim == 2, f"Expected query.ndim == 2, got {q.ndim}.")
    q = q if q.stride(-1) == 1 else q.contiguous()
    R, D = q.shape
    perm, cent, _, _, bd, nb, nc = _codec_arrays(perm, cent, D, None)
    _require(perm.ndim == 1 and cent.ndim == 3, "lut_build takes one codec (perm [D], centroids [nb, nc, bd])")
    out = torch.empty((R, nb, nc), device=q.device, dtype=torch.float32)
    if R == 0:
        return out
    with torch.cuda.device(q.device):  # the library reads the current device
        rc = N.lib().ssq_lut_build(N.ptr(q), N.dtype_code(q.dtype), q.stride(0), R, D, N.ptr(perm), N.ptr(cent), bd, nc,
                                   1 if scale is not None else 0, float(scale or 0.0), N.ptr(out), N.stream_of(q.device))
    N.check(rc)
    return out


def index_dtype(n_centroids: int) -> torch.dtype:
    """The stored index dtype: uint8 up to 256 codewords, int16 up to 65535, int32 beyond
    (sunshape/codec.py:78-83, _compact_index_dtype).  The kernels read int16 codes as unsigned."""
    if n_centroids <= 256:
        return torch.uint8
    if n_centroids <= 65535:
        return torch.int16
    return torch.int32


def words_per_row(n_blocks: int, bits: int) -> int:
    """uint32 words of one packed code row: ceil(nb / (32 // bits))."""
    vpe = 32 // bits
    return (n_blocks + vpe - 1) // vpe


def _check_codes(codes: torch.Tensor, nb: int, code_bits: int, nc: int = 256) -> None:
    if code_bits == 0:
        want = index_dtype(nc)
        _require(codes.dtype == want, f"codes must be {want} for n_centroids={nc}, got {codes.dtype}")
        _require(codes.shape[-1] == nb, f"codes must be [.., {nb}] {want}")
    else:
        _require(nc <= 256, f"n_centroids={nc} takes 16- or 32-bit codes, not packed words")
        _require(1 <= code_bits <= 8, "code_bits must be 0 (uint8) or 1..8 (packed words)")
        nw = words_per_row(nb, code_bits)
        _require(codes.dtype == torch.int32, f"packed codes must be int32 words, got {codes.dtype}")
        _require(codes.shape[-1] == nw, f"packed codes must be [.., {nw}] int32 for nb={nb}, bits={code_bits}")


def pack_codes(codes: torch.Tensor, bits: int, *, check: bool = True) -> torch.Tensor:
    """uint8 codes [..., nb] -> int32 words [..., ceil(nb / (32 // bits))].

    Word p holds blocks p*vpe .. p*vpe + vpe - 1 (vpe = 32 // bits), block p*vpe + v in bits
    [v*bits, (v+1)*bits): the layout sunshape/triton_kernels.py:250-266 unpacks.  With ``check``
    (a device reduction and one sync) codes >= 2**bits raise instead of losing their high bits.
    """
    _on_gpu("codes", codes)
    _require(codes.dtype == torch.uint8 and codes.ndim >= 1, "pack_codes takes uint8 codes [..., nb]")
    _require(1 <= bits <= 8, "bits must be in [1, 8]")
    if check and codes.numel() and bits < 8:
        _require(int(codes.max()) < (1 << bits), f"codes do not fit in {bits} bits")
    nb = codes.shape[-1]
    flat = codes.reshape(-1, nb)
    flat = flat if flat.stride(-1) == 1 else flat.contiguous()
    out = torch.empty((flat.shape[0], words_per_row(nb, bits)), device=codes.device, dtype=torch.int32)
    with torch.cuda.device(codes.device):  # the library reads the current device
        N.check(N.lib().ssq_pack_codes(N.ptr(flat), flat.stride(0), flat.shape[0], nb, bits, N.ptr(out), out.stride(0),
                                       N.stream_of(codes.device)))
    return out.view(*codes.shape[:-1], out.shape[-1])


def unpack_codes(packed: torch.Tensor, n_blocks: int, bits: int) -> torch.Tensor:
    """Inverse of pack_codes: int32 words [..., nw] -> uint8 codes [..., n_blocks]."""
    _on_gpu("packed", packed)
    _check_codes(packed, n_blocks, bits)
    nw = packed.shape[-1]
    flat = packed.reshape(-1, nw)
    flat = flat if flat.stride(-1) == 1 else flat.contiguous()
    out = torch.empty((flat.shape[0], n_blocks), device=packed.device, dtype=torch.uint8)
    with torch.cuda.device(packed.device):  # the library reads the current device
        N.check(N.lib().ssq_unpack_codes(N.ptr(flat), flat.stride(0), flat.shape[0], n_blocks, bits, N.ptr(out),
                                         out.stride(0), N.stream_of(packed.device)))
    return out.view(*packed.shape[:-1], n_blocks)


def _pt_args(heavy: Optional[Sequence[bool]], pt: Optional[torch.Tensor], pt_dense: bool):
    w0, w1 = N.heavy_mask_words(heavy)
    if not (w0 or w1):
        return (0, 0), None, 0, N.SSQ_F32
    _require(pt is not None, "Mixed-precision quantized keys are missing passthrough values.")
    _on_gpu("passthrough_values", pt)
    _require(pt.stride(-1) == 1 and pt.stride(-2) == pt.shape[-1], "passthrough values must be contiguous per token")
    return (w0, w1), pt, 1 if pt_dense else 0, N.dtype_code(pt.dtype)


def attention_scores(q: torch.Tensor, codes: torch.Tensor, perm: torch.Tensor, cent: torch.Tensor,
                     heavy: Optional[Sequence[bool]] = None, pt: Optional[torch.Tensor] = None,
                     pt_dense: bool = True, code_bits: int = 0, kernel: int = 0,
                     rotation: Optional[torch.Tensor] = None) -> torch.Tensor:
    """scores[r, t] = q_r . k_hat_t in fp32 (q in the original basis, unscaled).

    q [R, D]; codes uint8 [T, nb] (or int32 packed words [T, nw] with code_bits);
    pt [T, nb, bd] (dense) or [T, n_heavy, bd].  rotation: the rotated mode's R [D, D]; q is then
    taken to the codec basis by q @ R^T (transform_rows) and perm is not used.
    Reference: sunshape/triton_kernels.py:570-609 and sunshape/codec.py:403-422.
    """
    _on_gpu("query", q)
    _on_gpu("indices", codes)
    _require(q.ndim == 2, f"Expected query.ndim == 2, got {q.ndim}.")
    _require(codes.ndim == 2, f"Expected quantized_key.indices.ndim == 2, got {codes.ndim}.")
    if rotation is not None:
        q = transform_rows(q, rotation)
        perm = _identity_like(perm)
    q = q if q.stride(-1) == 1 else q.contiguous()
    codes = codes if codes.stride(-1) == 1 else codes.contiguous()
    R, D = q.shape
    T = codes.shape[0]
    perm, cent, perm_sh, cent_sh, bd, nb, nc = _codec_arrays(perm, cent, D, None)
    _require(perm.ndim == 1 and cent.ndim == 3, "attention_scores takes one codec (perm [D], centroids [nb, nc, bd])")
    if code_bits == 0:
        want = index_dtype(nc)
        _require(codes.dtype == want, f"indices must be {want} codes (n_centroids={nc}), got {codes.dtype}")
        _require(codes.shape[1] == nb, "Quantized key block count does not match codec: "
                 f"indices.shape[1]={codes.shape[1]}, codec.n_blocks={nb}.")
    _check_codes(codes, nb, code_bits, nc)
    if R == 0 or T == 0:
        return torch.empty((R, T), device=q.device, dtype=torch.float32)
    hm, pt, ptd, _ = _pt_args(heavy, pt, pt_dense)
    # one KV head, one query row per head: the torch operator's [B, Hq, Lq, D] / [B, Hkv, T, ..] views
    try:
        out = N.torch_ops().scores(q[None, :, None], codes[None, None], perm, cent, None, N.signed64(hm[0]),
                                   N.signed64(hm[1]), None if pt is None else pt[None, None], bool(ptd),
                                   int(code_bits), 0, int(kernel))
    except RuntimeError as e:
        raise N.kernel_error(e) from None
    return out.view(R, T)


def gqa_scores(q: torch.Tensor, codes: torch.Tensor, perm: torch.Tensor, cent: torch.Tensor, *,
               scale: Optional[float] = None, heavy: Optional[Sequence[bool]] = None,
               pt: Optional[torch.Tensor] = None, pt_dense: bool = False, code_bits: int = 0,
               num_splits: int = 0, kernel: int = 0, rotation: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Raw scores for every (batch, query head) in one launch: fp32 [B, Hq, Lq, T].

    q [B, Hq, Lq, D]; codes [B, Hkv, T, nb] uint8; query head h reads KV head
    h // (Hq/Hkv).  With ``scale`` the query is scaled in its own dtype first
    (sunshape/vllm_attn_backend.py:235-236) -- the logits the decode softmaxes.
    rotation: the rotated mode's R [D, D] (see decode).
    """
    for name, t in (("query", q), ("codes", codes)):
        _on_gpu(name, t)
    if rotation is not None:
        q = transform_rows(q, rotation, scale=scale)
        scale = None
        perm = _identity_like(perm)
    _require(q.ndim == 4 and codes.ndim == 4, "gqa_scores expects q [B, Hq, Lq, D] and codes [B, Hkv, T, nb]")
    q = q if q.stride(-1) == 1 else q.contiguous()
    codes = codes if codes.stride(-1) == 1 else codes.contiguous()
    B, Hq, Lq, D = q.shape
    Hkv, T = codes.shape[1], codes.shape[2]
    _require(codes.shape[0] == B, "Quantized key batch size does not match query batch size.")
    _require(Hq % Hkv == 0, "Query head count must be divisible by kv-head count.")
    perm, cent, perm_sh, cent_sh, bd, nb, nc = _codec_arrays(perm, cent, D, Hkv)
    _check_codes(codes, nb, code_bits, nc)
    if T == 0:
        return torch.empty((B, Hq, Lq, T), device=q.device, dtype=torch.float32)
    hm, pt, ptd, _ = _pt_args(heavy, pt, pt_dense)
    try:
        return N.torch_ops().scores(q, codes, perm, cent, None if scale is None else float(scale), N.signed64(hm[0]),
                                    N.signed64(hm[1]), pt, bool(ptd), int(code_bits), int(num_splits), int(kernel))
    except RuntimeError as e:
        raise N.kernel_error(e) from None


def decode(q: torch.Tensor, codes: torch.Tensor, v: torch.Tensor, perm: torch.Tensor, cent: torch.Tensor, *,
           scale: Optional[float] = None,
           mask: Optional[torch.Tensor] = None,
           heavy: Optional[Sequence[bool]] = None, pt: Optional[torch.Tensor] = None, pt_dense: bool = False,
           block_table: Optional[torch.Tensor] = None, seq_lens: Optional[torch.Tensor] = None,
           return_lse: bool = False, return_scores: bool = False,
           num_splits: int = 0, kernel: int = 0, code_bits: int = 0, no_alloc: bool = False,
           rotation: Optional[torch.Tensor] = None):
    """Fused VQ-key decode attention for all batches and KV heads in one launch.

    q [B, Hq, Lq, D].  Contiguous layout: codes [B, Hkv, T, nb] uint8, v [B, Hkv, T, Dv],
    pt [B, Hkv, T, slots, bd].  Paged layout (block_table given): codes [P, Hkv, page, nb],
    v [P, Hkv, Dv, page] (vLLM's value layout), pt [P, Hkv, page, slots, bd],
    block_table [B, max_pages] int32, seq_lens [B] int32.
    mask: additive, broadcastable to [B, Hq, Lq, T] (converted to fp32).
    code_bits: 0 for uint8 codes, 1..8 for int32 words from pack_codes (last dim nw).
    Returns out [B, Hq, Lq, Dv] in v's dtype, plus lse [B, Hq, Lq] / raw scores [B, Hq, Lq, T]
    (fp32) when requested; paged, T = max_pages * page and a sequence's slots past its length
    hold -inf.
    no_alloc: run through ssq_decode_noalloc (split workspace in the library's per-device scratch
    instead of a torch allocation; calls that overlap on one device race).
    rotation: the rotated mode's R [D, D] (sunshape/codec.py:250-251): the scaled query goes to the
    codec basis as fp32 (q * scale in q's dtype) @ R^T, the reference's order, and perm is not used.
    Reference: sunshape/vllm_attn_backend.py:216-253.
    """
    for name, t in (("query", q), ("codes", codes), ("value", v)):
        _on_gpu(name, t)
    if rotation is not None:
        _require(q.ndim == 4, "Quantized attention expects query/value tensors with shape [batch, heads, seq, dim].")
        q = transform_rows(q, rotation, scale=scale)
        scale = None
        perm = _identity_like(perm)
    hm0, hm1 = N.mask_words_signed(heavy)
    if mask is not None:
        _on_gpu("attn_mask", mask)
    try:
        out, lse, scores = N.torch_ops().decode(
            q, codes, v, perm, cent, None if scale is None else float(scale), mask, hm0, hm1, pt, bool(pt_dense),
            block_table, seq_lens, bool(return_lse), bool(return_scores), int(num_splits), int(kernel),
            int(code_bits), bool(no_alloc))
    except RuntimeError as e:
        raise N.kernel_error(e) from None
    if not (return_lse or return_scores):
        return out
    res = [out]
    if return_lse:
        res.append(lse)
    if return_scores:
        res.append(scores)
    return tuple(res)


def _encode_prepare(keys, perm, cent, heavy, pt_dtype, pt_dense, codes_out, pt_out, slot_mapping, metric, rotation):
    """Validated encode inputs and the outputs to write (allocated unless given): a namespace of
    keys, perm, cent, perm_sh, cent_sh, bd, nb, nc, w0, w1, metric, metric_sh, codes, pt, pt_dtype,
    c_str, p_str, page, slot_mapping."""
    _on_gpu("key_states", keys)
    _require(keys.ndim == 4, "quantize_key_states expects key_states with shape [batch, kv_heads, seq_len, head_dim].")
    if rotation is not None:  # the rotated mode's forward transform, fp32 keys @ R^T (codec.py:363-364)
        keys = transform_rows(keys, rotation)
        perm = _identity_like(perm)
    keys = keys if keys.stride(-1) == 1 else keys.contiguous()
    B, Hkv, S, D = keys.shape
    perm, cent, perm_sh, cent_sh, bd, nb, nc = _codec_arrays(perm, cent, D, Hkv)
    w0, w1 = N.heavy_mask_words(heavy)
    n_heavy = bin(w0).count("1") + bin(w1).count("1")
    pt_dtype = pt_dtype or keys.dtype
    metric_sh = 0
    if metric is not None:
        _on_gpu("metric", metric)
        metric = metric.to(torch.float32).contiguous()
        _require(metric.shape[-2:] == (D, D) and metric.ndim in (2, 3), f"metric must be [{D}, {D}] or [Hkv, {D}, {D}]")
        if metric.ndim == 3:
            _require(metric.shape[0] == Hkv, f"per-head metric holds {metric.shape[0]} heads, keys have {Hkv}")
            metric_sh = D * D
    idt = index_dtype(nc)
    if slot_mapping is None:
        if codes_out is not None:  # caller's buffer (e.g. a slice of a preallocated cache)
            _on_gpu("codes_out", codes_out)
            _require(codes_out.dtype == idt and tuple(codes_out.shape) == (B, Hkv, S, nb)
                     and codes_out.stride(3) == 1, f"codes_out must be {idt} [{B}, {Hkv}, {S}, {nb}] with unit last stride")
            codes = codes_out
        else:
            codes = torch.empty((B, Hkv, S, nb), device=keys.device, dtype=idt)
        pt = None
        if n_heavy:
            if pt_out is not None:
                _on_gpu("pt_out", pt_out)
                slots = nb if pt_dense else n_heavy
                _require(tuple(pt_out.shape) == (B, Hkv, S, slots, bd) and pt_out.stride(4) == 1
                         and pt_out.stride(3) == bd, f"pt_out must be [{B}, {Hkv}, {S}, {slots}, {bd}] with packed rows")
                _require(not pt_dense, "pt_out takes the compact passthrough layout")
                pt = pt_out
                pt_dtype = pt.dtype
            elif pt_dense:
                pt = torch.zeros((B, Hkv, S, nb, bd), device=keys.device, dtype=pt_dtype)
            else:
                pt = torch.empty((B, Hkv, S, n_heavy, bd), device=keys.device, dtype=pt_dtype)
        c_str = (codes.stride(0), codes.stride(1), codes.stride(2))
        p_str = (pt.stride(0), pt.stride(1), pt.stride(2)) if pt is not None else (0, 0, 0)
        page = 0
    else:
        _on_gpu("slot_mapping", slot_mapping)
        _require(slot_mapping.dtype == torch.int64 and slot_mapping.shape == (B, S) and slot_mapping.stride(1) == 1,
                 "slot_mapping must be int64 [B, S]")
        _require(codes_out is not None and codes_out.dtype == idt and codes_out.ndim == 4
                 and codes_out.shape[1] == Hkv and codes_out.shape[3] == nb and codes_out.stride(3) == 1,
                 f"paged encode needs codes_out [P, Hkv, page, nb] {idt}")
        codes = codes_out
        page = codes_out.shape[2]
        pt = pt_out
        if n_heavy:
            slots = nb if pt_dense else n_heavy
            _require(pt is not None and pt.ndim == 5 and pt.shape[1] == Hkv and pt.shape[2] == page
                     and pt.shape[3] == slots and pt.shape[4] == bd and pt.stride(4) == 1 and pt.stride(3) == bd,
                     f"paged encode needs pt_out [P, Hkv, {page}, {slots}, {bd}] with packed rows")
            _on_gpu("pt_out", pt)
            pt_dtype = pt.dtype
        c_str = (codes.stride(0), codes.stride(1), codes.stride(2))
        p_str = (pt.stride(0), pt.stride(1), pt.stride(2)) if pt is not None else (0, 0, 0)
    return types.SimpleNamespace(keys=keys, perm=perm, cent=cent, perm_sh=perm_sh, cent_sh=cent_sh, bd=bd, nb=nb, nc=nc,
                                 w0=w0, w1=w1, metric=metric, metric_sh=metric_sh, codes=codes, pt=pt,
                                 pt_dtype=pt_dtype, c_str=c_str, p_str=p_str, page=page, slot_mapping=slot_mapping)


def encode_args(keys: torch.Tensor, perm: torch.Tensor, cent: torch.Tensor, *,
           heavy: Optional[Sequence[bool]] = None, pt_dtype: Optional[torch.dtype] = None, pt_dense: bool = False,
           codes_out: Optional[torch.Tensor] = None, pt_out: Optional[torch.Tensor] = None,
           slot_mapping: Optional[torch.Tensor] = None, metric: Optional[torch.Tensor] = None, kernel: int = 0,
           grid: Optional[torch.Tensor] = None, direct: bool = False, rotation: Optional[torch.Tensor] = None):
    """Validated ssq_encode arguments for encode(): (args, codes, pt, tensors the args point into).

    For callers that replay one launch many times through the C ABI (a benchmark, a serving
    loop); keep the returned tensors alive while the args are in use.

    Passthrough values (heavy blocks) are [B, Hkv, S, n_heavy, bd] (compact) or
    [B, Hkv, S, nb, bd] zero-filled (pt_dense, the reference's layout).  With
    slot_mapping [B, S] (int64) the outputs go into caller-provided pages:
    codes_out [P, Hkv, page, nb], pt_out [P, Hkv, page, slots, bd].  Without it, codes_out /
    pt_out (compact) may be given as [B, Hkv, S, ...] views to write into instead of allocating.
    metric: SunShape-Pro block metric E [D, D] or per KV head [Hkv, D, D] (fp32); distances are
    taken between E_b x and E_b c (sunshape/codec.py:375-376).  None = identity.
    grid: search grid from encode_grid(cent) (block_dim 2, no metric); with it the encode
    evaluates only each key's certified candidates (same codes).  kernel: 0 auto, 1 exact scan,
    2 MFMA screen, 3 grid search.
    Reference: sunshape/codec.py:362-385, sunshape/vllm_attn_backend.py:101-123.
    """
    e = _encode_prepare(keys, perm, cent, heavy, pt_dtype, pt_dense, codes_out, pt_out, slot_mapping, metric,
                        rotation)
    keys, perm, cent, metric, codes, pt, c_str, p_str = e.keys, e.perm, e.cent, e.metric, e.codes, e.pt, e.c_str, e.p_str
    a = N.EncodeArgs(
        keys=N.ptr(keys), k_dtype=N.dtype_code(keys.dtype), k_sb=keys.stride(0), k_sh=keys.stride(1), k_ss=keys.stride(2),
        batch=keys.shape[0], num_kv_heads=keys.shape[1], seq_len=keys.shape[2], head_dim=keys.shape[3],
        perm=N.ptr(perm), perm_sh=e.perm_sh, cent=N.ptr(cent), cent_sh=e.cent_sh,
        metric=N.ptr(metric), metric_sh=e.metric_sh,
        block_dim=e.bd, n_blocks=e.nb, n_centroids=e.nc,
        codes=N.ptr(codes), c_sb=c_str[0], c_sh=c_str[1], c_st=c_str[2],
        pt=N.ptr(pt), pt_dtype=N.dtype_code(e.pt_dtype), pt_dense=1 if pt_dense else 0,
        pt_sb=p_str[0], pt_sh=p_str[1], pt_st=p_str[2],
        slot_mapping=N.ptr(slot_mapping), sm_sb=slot_mapping.stride(0) if slot_mapping is not None else 0,
        page_size=e.page, kernel=int(kernel), direct_dist=1 if direct else 0,
    )
    if grid is not None and not direct:
        _on_gpu("grid", grid)
        _require(grid.dtype == torch.uint8 and grid.is_contiguous(), "grid must be the uint8 tensor from encode_grid")
        a.grid, a.grid_bytes = N.ptr(grid), grid.numel()
    a.heavy_mask[0], a.heavy_mask[1] = e.w0, e.w1
    return a, codes, pt, (keys, perm, cent, metric, grid, slot_mapping)


def cdist_direct(rows_per_call: int, n_centroids: int) -> bool:
    """Whether torch.cdist evaluates the reference's distances directly rather than by its mm
    formulation: both of its inputs have at most 25 rows (ATen's cdist, compute mode
    use_mm_for_euclid_dist_if_necessary).  rows_per_call is the key count of one reference cdist
    call: N for codec.quantize(keys[N, D]), seq_len for quantize_key_states (one call per batch
    and KV head), B * Hkv * S for the HF cache layer's flattened keys."""
    return rows_per_call <= 25 and n_centroids <= 25


def encode(keys: torch.Tensor, perm: torch.Tensor, cent: torch.Tensor, *,
           heavy: Optional[Sequence[bool]] = None, pt_dtype: Optional[torch.dtype] = None, pt_dense: bool = False,
           codes_out: Optional[torch.Tensor] = None, pt_out: Optional[torch.Tensor] = None,
           slot_mapping: Optional[torch.Tensor] = None, metric: Optional[torch.Tensor] = None, kernel: int = 0,
           grid: Optional[torch.Tensor] = None, direct: bool = False, rotation: Optional[torch.Tensor] = None):
    """Nearest-codeword encode of keys [B, Hkv, S, D] -> (codes [B, Hkv, S, nb], pt or None); codes are
    uint8, or int16 / int32 past 256 codewords (index_dtype).

    Passthrough values (heavy blocks) are [B, Hkv, S, n_heavy, bd] (compact) or
    [B, Hkv, S, nb, bd] zero-filled (pt_dense, the reference's layout).  With
    slot_mapping [B, S] (int64) the outputs go into caller-provided pages:
    codes_out [P, Hkv, page, nb], pt_out [P, Hkv, page, slots, bd].  Without it, codes_out /
    pt_out (compact) may be given as [B, Hkv, S, ...] views to write into instead of allocating.
    metric: SunShape-Pro block metric E [D, D] or per KV head [Hkv, D, D] (fp32); distances are
    taken between E_b x and E_b c (sunshape/codec.py:375-376).  None = identity.
    grid: search grid from encode_grid(cent) (block_dim 2, no metric); with it the encode
    evaluates only each key's certified candidates (same codes).  kernel: 0 auto, 1 exact scan,
    2 MFMA screen, 3 grid search.
    direct: torch.cdist's direct distance in place of its mm formulation (see cdist_direct; the
    exact scan serves it and the grid is not used).
    rotation: the rotated mode's R [D, D]: keys are encoded as fp32 keys @ R^T and perm is not used;
    passthrough values are then the transformed values, as the reference stores them.
    Reference: sunshape/codec.py:362-385, sunshape/vllm_attn_backend.py:101-123.
    """
    e = _encode_prepare(keys, perm, cent, heavy, pt_dtype, pt_dense, codes_out, pt_out, slot_mapping, metric,
                        rotation)
    if grid is not None and not direct:
        _on_gpu("grid", grid)
        _require(grid.dtype == torch.uint8 and grid.is_contiguous(), "grid must be the uint8 tensor from encode_grid")
    try:
        N.torch_ops().encode_into(e.keys, e.perm, e.cent, N.signed64(e.w0), N.signed64(e.w1), bool(pt_dense), e.codes,
                                  e.pt, e.slot_mapping, e.metric, None if direct else grid, int(kernel), bool(direct))
    except RuntimeError as exc:
        raise N.kernel_error(exc) from None
    return e.codes, e.pt


def _grid_args(cent: torch.Tensor, num_kv_heads: int):
    nb, nc = cent.shape[-3], cent.shape[-2]
    return N.EncodeArgs(num_kv_heads=int(cent.shape[0] if cent.ndim == 4 else num_kv_heads), cent=N.ptr(cent),
                        cent_sh=nb * nc * 2 if cent.ndim == 4 else 0, block_dim=2, n_blocks=nb, n_centroids=nc,
                        head_dim=2 * nb)


def encode_grid_bytes(cent: torch.Tensor, num_kv_heads: int = 1) -> int:
    """Device bytes of encode_grid(cent) (0 where the grid does not apply), without building it."""
    if cent.ndim not in (3, 4) or cent.shape[-1] != 2:
        return 0
    return int(N.lib().ssq_encode_grid_bytes(ctypes.byref(_grid_args(cent, num_kv_heads))))


def encode_grid(cent: torch.Tensor, num_kv_heads: int = 1) -> torch.Tensor:
    """Search grid for encode(..., grid=) from codebooks [nb, nc, 2] or [Hkv, nb, nc, 2] (fp32).

    Built once per codebook (a uint8 buffer of 320 KiB per block and head); rebuild it
    whenever the codebook changes.  No counterpart in the reference: a search structure of this
    library, whose encode results equal the exhaustive ones bit for bit.
    """
    _on_gpu("centroids", cent)
    cent = cent.to(torch.float32).contiguous()
    _require(cent.ndim in (3, 4) and cent.shape[-1] == 2, "the encode grid serves block_dim 2 codebooks")
    a = _grid_args(cent, num_kv_heads)
    lib = N.lib()
    size = lib.ssq_encode_grid_bytes(ctypes.byref(a))
    _require(size > 0, "the encode grid serves block_dim 2 codebooks with at most 128 blocks of 256 codewords")
    grid = torch.empty(size, device=cent.device, dtype=torch.uint8)
    with torch.cuda.device(cent.device):  # the library reads the current device
        N.check(lib.ssq_encode_grid_build(ctypes.byref(a), N.ptr(grid), size, N.stream_of(cent.device)))
    return grid


def dequantize(codes: torch.Tensor, perm: torch.Tensor, cent: torch.Tensor, *,
               heavy: Optional[Sequence[bool]] = None, pt: Optional[torch.Tensor] = None,
               pt_dense: bool = True, rotation: Optional[torch.Tensor] = None) -> torch.Tensor:
    """k_hat fp32 [T, D] in the original basis from codes [T, nb] (uint8, or int16 / int32 past 256
    codewords: index_dtype).

    rotation: the rotated mode's R [D, D]: the codewords are taken back by k_hat @ R
    (sunshape/codec.py:257-258) and perm is not used.
    Reference: sunshape/codec.py:387-398.
    """
    if rotation is not None:
        k_rot = dequantize(codes, _identity_like(perm), cent, heavy=heavy, pt=pt, pt_dense=pt_dense)
        return transform_rows(k_rot, rotation, transpose=True)
    _on_gpu("indices", codes)
    _require(cent.ndim == 3 and perm.ndim == 1, "dequantize takes one codec (perm [D], centroids [nb, nc, bd])")
    nb, nc, bd = cent.shape
    _require(codes.ndim == 2 and codes.dtype == index_dtype(nc), f"indices must be {index_dtype(nc)} [T, nb]")
    codes = codes if codes.stride(-1) == 1 else codes.contiguous()
    D = nb * bd
    perm, cent, _, _, bd, nb, nc = _codec_arrays(perm, cent, D, None)
    _require(codes.shape[1] == nb, f"indices.shape[1]={codes.shape[1]} != n_blocks={nb}")
    T = codes.shape[0]
    out = torch.empty((T, D), device=codes.device, dtype=torch.float32)
    (w0, w1), pt, ptd, ptdt = _pt_args(heavy, pt, pt_dense)
    hm = (ctypes.c_uint64 * 2)(w0, w1)
    with torch.cuda.device(codes.device):  # the library reads the current device
        N.check(N.lib().ssq_dequantize(N.ptr(codes), codes.stride(0), T, N.ptr(perm), N.ptr(cent), D, bd, nc,
                                       ctypes.cast(hm, ctypes.c_void_p), ptd, N.ptr(pt), ptdt,
                                       0 if pt is None else pt.stride(0), N.ptr(out), out.stride(0),
                                       N.stream_of(codes.device)))
    return out
