"""SunShape block codec (drop-in for ``sunshape.codec``), backed by HIP kernels.

Same buffers, constructor arguments, ``SunShapeQuantized`` payload and method
names as the reference (sunshape/codec.py:28-34, :205-259, :362-422).  Encode,
dequantize and scoring run on the GPU through the sunshape_amd C ABI; there is
no CPU path.  Offline calibration (``fit``: k-means, DSQ, permutation search,
sunshape/codec.py:261-360) is outside this library: codecs come from a fitted
bundle (``sunshape_amd.hf.SunShapeBundle``) or from ``from_buffers``.

Extension: ``num_kv_heads`` allocates per-KV-head codebooks
(centroids [Hkv, nb, nc, bd], permutation [Hkv, D]); methods then take a
``kv_head`` index.  ``num_kv_heads=None`` is the reference's one-codec-per-layer
layout.
"""

from __future__ import annotations

import math
import os
import threading
import weakref
from collections import OrderedDict
from typing import NamedTuple, Optional

import torch

from . import hip_ops

# Encode search grids are cached per codec and codebook, within one process-wide byte budget shared
# by every codec (a model has one codec per layer): the least recently used grids are dropped to
# make room, and a grid larger than the whole budget is not built (that encode then scans every
# codeword: the same codes, more time).  SUNSHAPE_AMD_GRID_BUDGET_MB sets the budget (default
# 1024 MiB); set_encode_grid_budget changes it at run time.
_GRID_BUDGET = [int(os.environ.get("SUNSHAPE_AMD_GRID_BUDGET_MB", "1024")) << 20]
_GRID_LRU: "OrderedDict[tuple, tuple]" = OrderedDict()  # (id(codec), slot) -> (weakref to codec, bytes)
_GRID_LOCK = threading.RLock()  # the LRU and every codec's grid cache, across threads that encode


def _grid_lru_live():
    """Drop entries whose codec is gone or no longer holds the grid; yield (key, codec, slot, bytes)."""
    for key in list(_GRID_LRU):
        ref, nbytes = _GRID_LRU[key]
        codec = ref()
        if codec is None or key[1] not in codec._grid_cache:
            del _GRID_LRU[key]
            continue
        yield key, codec, key[1], nbytes


def encode_grid_footprint() -> int:
    """Device bytes held by cached encode search grids, over every codec of the process."""
    with _GRID_LOCK:
        return sum(n for *_, n in _grid_lru_live())


def set_encode_grid_budget(nbytes: int) -> None:
    """Process-wide byte budget for cached encode search grids; grids past it are dropped, least
    recently used first."""
    with _GRID_LOCK:
        _GRID_BUDGET[0] = int(nbytes)
        _grid_lru_evict(_GRID_BUDGET[0])


def _grid_lru_evict(limit: int) -> None:
    with _GRID_LOCK:
        used = encode_grid_footprint()
        for key, codec, slot, nbytes in list(_grid_lru_live()):
            if used <= limit:
                break
            codec._grid_cache.pop(slot, None)
            del _GRID_LRU[key]
            used -= nbytes

PERMUTATION_MODES = frozenset({"profileperm_baseline", "profileperm_localmetric_dsq", "profileperm_mixed_precision"})
# modes whose fitted E is the identity (sunshape/codec.py:279-312): encode takes no metric
IDENTITY_METRIC_MODES = frozenset({"profileperm_baseline", "profileperm_mixed_precision", "identity_baseline"})
# SunShape-Pro / legacy modes: encode compares E_b x with E_b c (sunshape/codec.py:375-376)
METRIC_MODES = frozenset({"profileperm_localmetric_dsq", "legacy_strict"})


class SunShapeQuantized(NamedTuple):
    """Quantized keys of one (sequence, KV head): sunshape/codec.py:28-34."""

    indices: torch.Tensor
    head_dim: int
    block_dim: int
    n_blocks: int
    passthrough_blocks: torch.Tensor | None = None
    passthrough_values: torch.Tensor | None = None


def _compact_index_dtype(n_centroids: int) -> torch.dtype:
    """sunshape/codec.py:78-83."""
    if n_centroids <= 256:
        return torch.uint8
    if n_centroids <= 65535:
        return torch.int16
    return torch.int32


def _invert_permutation(perm: torch.Tensor) -> torch.Tensor:
    """sunshape/codec.py:86-89 (row-wise for [Hkv, D])."""
    inv = torch.empty_like(perm)
    ar = torch.arange(perm.shape[-1], device=perm.device, dtype=perm.dtype)
    inv.scatter_(-1, perm, ar.expand_as(perm).contiguous())
    return inv


def _apply_permutation(x: torch.Tensor, perm: Optional[torch.Tensor]) -> torch.Tensor:
    """sunshape/codec.py:92-95."""
    if perm is None or perm.numel() == 0:
        return x
    return x[..., perm]


def _default_device() -> torch.device:
    return torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu")


class SunShapeBlockCodec(torch.nn.Module):
    """Block VQ codec with a fixed ProfilePerm permutation and per-block codebooks."""

    def __init__(
        self,
        head_dim: int,
        block_dim: int = 8,
        n_centroids: int = 256,
        c: float = 5.0,
        n_refine_dsq: int = 3,
        mode: str = "profileperm_baseline",
        use_rotation: bool = False,
        rotation_seed: int = 0,
        device: torch.device | None = None,
        num_kv_heads: int | None = None,
    ):
        super().__init__()
        if head_dim % block_dim != 0:
            raise ValueError("head_dim must be divisible by block_dim")
        self.head_dim = head_dim
        self.block_dim = block_dim
        self.n_blocks = head_dim // block_dim
        self.n_centroids = n_centroids
        self.c = c
        self.mode = "rotated" if use_rotation else mode
        self.n_refine_dsq = 3 if n_refine_dsq is None else int(n_refine_dsq)
        self.use_rotation = self.mode == "rotated"
        self.num_kv_heads = num_kv_heads
        self.device = torch.device(device) if device is not None else _default_device()
        dev = self.device
        hk = () if num_kv_heads is None else (int(num_kv_heads),)
        self.register_buffer("E", torch.eye(head_dim, device=dev))
        self.register_buffer("E_inv", torch.eye(head_dim, device=dev))
        self.register_buffer("centroids", torch.zeros(*hk, self.n_blocks, n_centroids, block_dim, device=dev))
        self.register_buffer("dsq_block_affinity", torch.ones(self.n_blocks, device=dev))
        self.register_buffer("dsq_active_blocks", torch.ones(self.n_blocks, device=dev, dtype=torch.bool))
        self.register_buffer("mixed_high_precision_blocks", torch.zeros(self.n_blocks, device=dev, dtype=torch.bool))
        self.register_buffer("mixed_block_mass", torch.zeros(self.n_blocks, device=dev))
        identity = torch.arange(head_dim, device=dev, dtype=torch.long).expand(*hk, head_dim).contiguous()
        self.register_buffer("permutation", identity.clone())
        self.register_buffer("inv_permutation", identity.clone())
        self.register_buffer("rotation", torch.eye(head_dim, device=dev))
        self._heavy_cache: tuple[int, tuple[bool, ...]] | None = None
        # encode search grids (this library's extension, no reference counterpart), per
        # codebook tensor passed to the encode; see encode_search_grid
        self.use_encode_grid = True
        self._grid_cache: dict = {}

    # ------------------------------------------------------------------ helpers
    @classmethod
    def from_buffers(cls, permutation: torch.Tensor, centroids: torch.Tensor, *,
                     mode: str = "profileperm_baseline",
                     mixed_high_precision_blocks: torch.Tensor | None = None,
                     metric: torch.Tensor | None = None,
                     device: torch.device | None = None) -> "SunShapeBlockCodec":
        """Codec from a fitted permutation ([D] or [Hkv, D]) and codebook ([nb, nc, bd] or [Hkv, nb, nc, bd]).

        metric: the SunShape-Pro block metric E ([D, D], or [Hkv, D, D] per KV head); E_inv is
        set to its pseudo-inverse as the reference's fit does (sunshape/codec.py:303-304).
        """
        nkv = centroids.shape[0] if centroids.ndim == 4 else None
        nb, nc, bd = centroids.shape[-3:]
        dev = torch.device(device) if device is not None else centroids.device
        codec = cls(head_dim=nb * bd, block_dim=bd, n_centroids=nc, mode=mode, device=dev, num_kv_heads=nkv)
        codec.centroids.copy_(centroids.to(dev, torch.float32))
        perm = permutation.to(dev, torch.long)
        if nkv is not None and perm.ndim == 1:
            perm = perm.expand(nkv, -1)
        codec.permutation.copy_(perm)
        codec.inv_permutation.copy_(_invert_permutation(codec.permutation))
        if mixed_high_precision_blocks is not None:
            codec.mixed_high_precision_blocks.copy_(mixed_high_precision_blocks.to(dev, torch.bool))
        if metric is not None:
            E = metric.to(dev, torch.float32).contiguous()
            if E.shape[-2:] != (nb * bd, nb * bd) or E.ndim not in (2, 3):
                raise ValueError(f"metric must be [{nb * bd}, {nb * bd}] or [Hkv, {nb * bd}, {nb * bd}]")
            codec.E = E
            codec.E_inv = torch.linalg.pinv(E.cpu()).to(dev)
        return codec

    def heavy_blocks(self) -> tuple[bool, ...] | None:
        """Passthrough mask as a host tuple (None unless SunShape-Mixed with heavy blocks).

        Cached against the buffer's version counter so the hot path does not sync.
        """
        if self.mode != "profileperm_mixed_precision":
            return None
        buf = self.mixed_high_precision_blocks
        ver = buf._version
        if self._heavy_cache is None or self._heavy_cache[0] != ver or len(self._heavy_cache[1]) != buf.numel():
            self._heavy_cache = (ver, tuple(bool(x) for x in buf.tolist()))
        mask = self._heavy_cache[1]
        return mask if any(mask) else None

    def effective_permutation(self, kv_head: int | None = None) -> torch.Tensor:
        """The permutation _forward_transform applies (identity outside the ProfilePerm modes)."""
        if self.mode in PERMUTATION_MODES:
            perm = self.permutation
        else:
            perm = torch.arange(self.head_dim, device=self.permutation.device, dtype=torch.long)
            if self.num_kv_heads is not None:
                perm = perm.expand(self.num_kv_heads, -1).contiguous()
        if kv_head is not None and perm.ndim == 2:
            perm = perm[kv_head]
        return perm

    def encode_metric(self, kv_head: int | None = None) -> torch.Tensor | None:
        """The block metric E the encode applies (SunShape-Pro), or None for identity-metric modes.

        [D, D] (or [Hkv, D, D] for per-head metrics; kv_head selects one).  Only the diagonal
        bd x bd blocks are read, as sunshape/codec.py:375-376 slices them.
        """
        if self.mode not in METRIC_MODES:
            return None
        E = self.E
        if kv_head is not None and E.ndim == 3:
            E = E[kv_head]
        return E

    def encode_search_grid(self, cent: torch.Tensor) -> torch.Tensor | None:
        """The search grid for ``hip_ops.encode(..., grid=)`` over ``cent`` (this codec's
        codebook, or one KV head of it), or None where the grid does not apply (block_dim other
        than 2, a block metric, or ``use_encode_grid = False``).

        No counterpart in the reference: a search structure whose encode results equal the
        exhaustive search bit for bit.  Built on first use and rebuilt when the centroid buffer
        changes (new storage or an in-place write, seen through its version counter).

        Footprint: 20 B per cell, 128 x 128 cells per block and codebook head (320 KiB; a lookup
        reads the first 4 B of a cell), plus a 32-byte header per block: 20 MiB for the config-5
        layer (2 heads x 32 blocks), 160 MiB for a Llama-3-8B layer at 4 bits/dim (8 heads x 64
        blocks).  A
        per-KV-head codebook has one grid: a single head's view (``codebook(kv_head)``) gets
        that head's slice of it (the layout is head-major), not a grid of its own.  Set
        ``use_encode_grid = False`` to run the exhaustive encode without any grid.  Every codec's
        grids count against one process-wide budget (``set_encode_grid_budget``,
        ``encode_grid_footprint``; 1 GiB unless SUNSHAPE_AMD_GRID_BUDGET_MB says otherwise): the
        least recently used are dropped first, and an encode whose grid is dropped or would not
        fit scans every codeword instead (the same codes).
        """
        if not self.use_encode_grid or self.block_dim != 2 or self.mode in METRIC_MODES:
            return None
        if cent.shape[-2] > 256 or cent.shape[-3] > 128:
            return None
        buf = self.centroids
        if buf.ndim == 4 and cent.ndim == 3 and cent.shape == buf.shape[1:] and buf.is_contiguous():
            step = buf[0].numel() * buf.element_size()
            off = cent.data_ptr() - buf.data_ptr()
            if off % step == 0 and 0 <= off // step < buf.shape[0] and cent.is_contiguous():
                full = self.encode_search_grid(buf)  # one head of the per-KV-head grid
                return None if full is None else full.view(buf.shape[0], -1)[off // step]
        slot = (cent.data_ptr(), tuple(cent.shape))
        key = (buf.data_ptr(), buf._version)
        lru_key = (id(self), slot)
        with _GRID_LOCK:
            hit = self._grid_cache.get(slot)
            if hit is not None and hit[0] == key:
                if lru_key in _GRID_LRU:
                    _GRID_LRU.move_to_end(lru_key)
                return hit[1]
            self._grid_cache.pop(slot, None)  # stale (the codebook changed): its bytes are freed below
            _GRID_LRU.pop(lru_key, None)
            nbytes = hip_ops.encode_grid_bytes(cent)
            if nbytes > _GRID_BUDGET[0]:
                return None  # larger than the whole budget: the exhaustive encode (same codes)
            _grid_lru_evict(_GRID_BUDGET[0] - nbytes)
            hit = (key, hip_ops.encode_grid(cent))
            self._grid_cache[slot] = hit
            _GRID_LRU[lru_key] = (weakref.ref(self), nbytes)
            return hit[1]

    def rotation_matrix(self) -> torch.Tensor | None:
        """The rotated mode's dense R [D, D] (forward transform x @ R^T, inverse x @ R,
        sunshape/codec.py:247-259), or None in the other modes."""
        return self.rotation if self.use_rotation else None

    def codebook(self, kv_head: int | None = None) -> torch.Tensor:
        cent = self.centroids
        if kv_head is not None and cent.ndim == 4:
            cent = cent[kv_head]
        return cent

    def _select_head(self, kv_head: int | None):
        if self.num_kv_heads is not None and kv_head is None:
            raise RuntimeError("per-KV-head codec: pass kv_head=")
        return self.effective_permutation(kv_head), self.codebook(kv_head)

    def unsupported_reason(self) -> str | None:
        """Why the HIP kernels cannot serve this codec (None when they can)."""
        if self.n_centroids > 1 << 20:
            return f"n_centroids={self.n_centroids} exceeds the kernels' 2^20 codewords per block."
        return None

    # --------------------------------------------------------------- transforms
    def _forward_transform(self, x: torch.Tensor, kv_head: int | None = None) -> torch.Tensor:
        """sunshape/codec.py:247-252."""
        if self.mode in PERMUTATION_MODES:
            return _apply_permutation(x, self.effective_permutation(kv_head))
        if self.use_rotation:
            return x @ self.rotation.T
        return x

    def _inverse_transform(self, x: torch.Tensor, kv_head: int | None = None) -> torch.Tensor:
        """sunshape/codec.py:254-259."""
        if self.mode in PERMUTATION_MODES:
            inv = self.inv_permutation
            if kv_head is not None and inv.ndim == 2:
                inv = inv[kv_head]
            return _apply_permutation(x, inv)
        if self.use_rotation:
            return x @ self.rotation
        return x

    def fit(self, *args, **kwargs):
        raise NotImplementedError(
            "SunShapeBlockCodec.fit (offline k-means/DSQ calibration) is not part of sunshape_amd; "
            "load fitted codecs with SunShapeBundle.load or SunShapeBlockCodec.from_buffers"
        )

    # ------------------------------------------------------------ encode/decode
    def quantize(self, keys: torch.Tensor, kv_head: int | None = None) -> SunShapeQuantized:
        """Nearest-codeword encode on the GPU (sunshape/codec.py:362-385).

        Returns indices [N, nb] in the reference's compact dtype (uint8 up to 256
        codewords, int16 up to 65535, int32 beyond; sunshape/codec.py:78-83); in
        SunShape-Mixed mode the heavy blocks' indices are 0 and passthrough_values is
        the reference's dense fp32 [N, nb, bd] (zeros on light blocks).
        """
        reason = self.unsupported_reason()
        if reason is not None:
            raise RuntimeError(reason)
        perm, cent = self._select_head(kv_head)
        keys = keys.to(self.device)
        if keys.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            keys = keys.float()
        heavy = self.heavy_blocks()
        metric = self.encode_metric(kv_head)
        if metric is not None and metric.ndim == 3:
            raise RuntimeError("per-KV-head metric: pass kv_head=")
        flat = keys.reshape(1, 1, -1, self.head_dim)
        codes, pt = hip_ops.encode(flat, perm, cent, heavy=heavy, pt_dtype=torch.float32, pt_dense=True,
                                   metric=metric, grid=self.encode_search_grid(cent),
                                   direct=hip_ops.cdist_direct(flat.shape[2], self.n_centroids),
                                   rotation=self.rotation_matrix())
        mixed = self.mode == "profileperm_mixed_precision"
        return SunShapeQuantized(
            indices=codes.reshape(-1, self.n_blocks),
            head_dim=self.head_dim,
            block_dim=self.block_dim,
            n_blocks=self.n_blocks,
            passthrough_blocks=self.mixed_high_precision_blocks.detach().clone() if mixed else None,
            passthrough_values=None if pt is None else pt.reshape(-1, self.n_blocks, self.block_dim),
        )

    def dequantize(self, quantized: SunShapeQuantized, kv_head: int | None = None) -> torch.Tensor:
        """sunshape/codec.py:387-398: fp32 [N, D] in the original basis."""
        reason = self.unsupported_reason()
        if reason is not None:
            raise RuntimeError(reason)
        perm, cent = self._select_head(kv_head)
        heavy = None
        if quantized.passthrough_blocks is not None:
            heavy = tuple(bool(x) for x in quantized.passthrough_blocks.tolist())
            if not any(heavy):
                heavy = None
        pt = quantized.passthrough_values
        if heavy is not None and pt is None:
            raise ValueError("Mixed-precision quantized keys are missing passthrough values.")
        idx = quantized.indices
        want = _compact_index_dtype(self.n_centroids)
        if idx.dtype != want:  # e.g. int64 indices: the stored dtype's bits (16-bit codes read unsigned)
            idx = idx.to(want)
        return hip_ops.dequantize(idx, perm, cent, heavy=heavy, pt=pt,
                                  pt_dense=pt is not None and pt.shape[-2] == self.n_blocks,
                                  rotation=self.rotation_matrix())

    def forward(self, keys: torch.Tensor, kv_head: int | None = None) -> torch.Tensor:
        return self.dequantize(self.quantize(keys, kv_head), kv_head)

    def attention_scores(self, query: torch.Tensor, quantized: SunShapeQuantized, kv_head: int | None = None) -> torch.Tensor:
        """sunshape/codec.py:403-422: q . k_hat (fp32 [n_qh, T]) from the codes, on the GPU."""
        from .kernels import sunshape_attention_scores_strict

        return sunshape_attention_scores_strict(self, query.to(self.device), quantized, kv_head=kv_head)

    def heldout_logit_mse(self, q_test: torch.Tensor, k_test: torch.Tensor, kv_head: int | None = None) -> float:
        """sunshape/codec.py:424-429."""
        q_test = q_test.to(self.device).float()
        k_test = k_test.to(self.device).float()
        delta = k_test - self.forward(k_test, kv_head)
        return ((q_test * delta).sum(dim=1).square()).mean().item()

    def kl_attention(self, q_test: torch.Tensor, k_test: torch.Tensor, kv_head: int | None = None) -> float:
        """sunshape/codec.py:431-442."""
        q_test = q_test.to(self.device).float()
        k_test = k_test.to(self.device).float()
        k_hat = self.forward(k_test, kv_head)
        scale = math.sqrt(self.head_dim)
        p = torch.softmax((q_test @ k_test.T) / scale, dim=-1)
        qd = torch.softmax((q_test @ k_hat.T) / scale, dim=-1)
        return (p * (torch.log(p + 1e-9) - torch.log(qd + 1e-9))).sum(dim=-1).mean().item()

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        # a per-KV-head SunShape-Pro metric is stored as [Hkv, D, D] (from_buffers); size E / E_inv
        # from the payload so such a codec reloads (the reference's layout is [D, D])
        for name in ("E", "E_inv"):
            t = state_dict.get(prefix + name)
            cur = getattr(self, name)
            if t is not None and t.ndim == 3 and t.shape[-2:] == cur.shape[-2:] and tuple(t.shape) != tuple(cur.shape):
                setattr(self, name, torch.empty(tuple(t.shape), device=cur.device, dtype=cur.dtype))
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)
        self._heavy_cache = None
        self._grid_cache = {}
