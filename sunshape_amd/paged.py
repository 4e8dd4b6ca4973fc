"""vLLM-style paged KV cache for SunShape-compressed keys.

No counterpart in the reference: its quantized keys are one contiguous [T, nb] code
tensor per (batch, KV head) (sunshape/vllm_attn_backend.py:99-123), and it has no paged
layout.  This is the caller on the write side of the decode kernel:

* key pages   [P, Hkv, page, nb] codes (uint8, or int16 / int32 past 256 codewords), filled by the encode kernel through
  a slot mapping (token slot = page * page_size + offset), no dense key tensor;
* passthrough [P, Hkv, page, n_heavy, bd] for SunShape-Mixed heavy blocks;
* value pages [P, Hkv, Dv, page] -- vLLM's dim-major value layout, which the
  MFMA decode kernel reads as B-operand fragments directly;
* per-sequence block tables and lengths, with a simple free-page allocator.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import hip_ops


class PagedSunShapeCache:
    def __init__(self, codec, *, num_pages: int, num_kv_heads: int, value_dim: int, page_size: int = 16,
                 value_dtype: torch.dtype = torch.bfloat16, passthrough_dtype: torch.dtype = torch.bfloat16,
                 device: Optional[torch.device] = None):
        reason = codec.unsupported_reason()
        if reason is not None:
            raise RuntimeError(reason)
        self.codec = codec
        self.device = torch.device(device) if device is not None else codec.device
        self.page_size = int(page_size)
        self.num_pages = int(num_pages)
        self.num_kv_heads = int(num_kv_heads)
        self.value_dim = int(value_dim)
        nb, bd = codec.n_blocks, codec.block_dim
        self.code_pages = torch.zeros(num_pages, num_kv_heads, page_size, nb, device=self.device,
                                      dtype=hip_ops.index_dtype(self.codec.n_centroids))
        self.v_pages = torch.zeros(num_pages, num_kv_heads, value_dim, page_size, dtype=value_dtype, device=self.device)
        heavy = codec.heavy_blocks()
        self.heavy = heavy
        self.pt_pages = None
        if heavy is not None:
            self.pt_pages = torch.zeros(num_pages, num_kv_heads, page_size, sum(heavy), bd, dtype=passthrough_dtype,
                                        device=self.device)
        self._free = list(range(num_pages - 1, -1, -1))
        self.block_tables: dict[int, list[int]] = {}
        self.seq_lens: dict[int, int] = {}

    # ------------------------------------------------------------------ pages
    def _ensure_capacity(self, seq_id: int, new_len: int) -> None:
        table = self.block_tables.setdefault(seq_id, [])
        need = (new_len + self.page_size - 1) // self.page_size
        while len(table) < need:
            if not self._free:
                raise RuntimeError("PagedSunShapeCache is out of pages")
            table.append(self._free.pop())

    def free(self, seq_id: int) -> None:
        for pg in self.block_tables.pop(seq_id, []):
            self._free.append(pg)
        self.seq_lens.pop(seq_id, None)

    def slot_mapping(self, seq_ids: list[int], num_new: int) -> torch.Tensor:
        """Allocate room for num_new tokens per sequence; return int64 slots [len(seq_ids), num_new]."""
        rows = []
        for sid in seq_ids:
            start = self.seq_lens.get(sid, 0)
            self._ensure_capacity(sid, start + num_new)
            table = self.block_tables[sid]
            rows.append([table[(start + i) // self.page_size] * self.page_size + (start + i) % self.page_size
                         for i in range(num_new)])
            self.seq_lens[sid] = start + num_new
        return torch.tensor(rows, dtype=torch.int64, device=self.device)

    # ------------------------------------------------------------------ append / decode
    def append(self, seq_ids: list[int], key_states: torch.Tensor, value_states: torch.Tensor) -> torch.Tensor:
        """Encode keys [B, Hkv, S, D] into the code pages and write values [B, Hkv, S, Dv]; returns the slots."""
        B, Hkv, S, _ = key_states.shape
        if Hkv != self.num_kv_heads or value_states.shape[:3] != key_states.shape[:3]:
            raise RuntimeError("key/value shapes do not match the cache")
        slots = self.slot_mapping(seq_ids, S)
        perm = self.codec.effective_permutation()
        # as quantize_key_states: one reference cdist per (sequence, KV head) over its S new keys
        hip_ops.encode(key_states.to(self.device), perm, self.codec.centroids, heavy=self.heavy,
                       codes_out=self.code_pages, pt_out=self.pt_pages, slot_mapping=slots,
                       metric=self.codec.encode_metric(), grid=self.codec.encode_search_grid(self.codec.centroids),
                       direct=hip_ops.cdist_direct(S, self.codec.n_centroids),
                       rotation=self.codec.rotation_matrix())
        flat = slots.reshape(-1)
        page, off = flat // self.page_size, flat % self.page_size
        vals = value_states.to(self.device, self.v_pages.dtype).permute(0, 2, 1, 3).reshape(B * S, Hkv, self.value_dim)
        self.v_pages[page, :, :, off] = vals
        return slots

    def tables(self, seq_ids: list[int]) -> tuple[torch.Tensor, torch.Tensor]:
        """(block_table [B, max_pages] int32, seq_lens [B] int32) for these sequences."""
        width = max(len(self.block_tables.get(s, [])) for s in seq_ids) or 1
        bt = torch.zeros(len(seq_ids), width, dtype=torch.int32)
        for i, s in enumerate(seq_ids):
            t = self.block_tables.get(s, [])
            bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
        lens = torch.tensor([self.seq_lens.get(s, 0) for s in seq_ids], dtype=torch.int32)
        return bt.to(self.device), lens.to(self.device)

    def decode(self, seq_ids: list[int], query: torch.Tensor, *, scale: Optional[float] = None,
               return_lse: bool = False):
        """Fused decode of query [B, Hq, Lq, D] against the cached sequences."""
        bt, lens = self.tables(seq_ids)
        return hip_ops.decode(query, self.code_pages, self.v_pages, self.codec.effective_permutation(),
                              self.codec.centroids, scale=scale, heavy=self.heavy, pt=self.pt_pages,
                              pt_dense=False, block_table=bt, seq_lens=lens, return_lse=return_lse,
                              rotation=self.codec.rotation_matrix())
