"""Paged KV cache for the Qwen3 model: one page pool per layer, pages shared by
all requests, a host-side page list per request.

Follows the reference's ``TinyKvPagedPool`` / ``TinyKvPagedCache``
(``cache/paged.py:21-559``) and its per-layer pools (``models/qwen3.py:272-283``):
a pool holds ``key_pages``/``value_pages [P, num_kv_heads, page_size, D]``;
token ``j`` of a request lives in slot ``j % page_size`` of the request's page
``j // page_size``.  Here every pool is allocated once at its full size (HBM
is large) instead of grown geometrically, and one free list serves all layers
(a request holds the same page ids in every layer).  Prefix caching and int8
pages are not built.
"""

from __future__ import annotations

from typing import Dict, List, Sequence

import torch


class PagedKVCache:
    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, num_pages: int,
                 page_size: int, dtype: torch.dtype = torch.bfloat16, device="cuda"):
        if num_pages <= 0 or page_size <= 0:
            raise ValueError("PagedKVCache: num_pages and page_size must be positive")
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_pages = num_pages
        self.page_size = page_size
        self.dtype = dtype
        self.device = torch.device(device)
        # one page past the pool takes the writes of padding rows and of
        # graph warm-up/capture runs; it is never handed to a request
        self.scratch_page = num_pages
        shape = (num_pages + 1, num_kv_heads, page_size, head_dim)
        self.key_pages = [torch.zeros(shape, dtype=dtype, device=self.device)
                          for _ in range(num_layers)]
        self.value_pages = [torch.zeros(shape, dtype=dtype, device=self.device)
                            for _ in range(num_layers)]
        self._free: List[int] = list(range(num_pages - 1, -1, -1))
        self.pages: Dict[int, List[int]] = {}
        self.lens: Dict[int, int] = {}

    # ---------------------------------------------------------------- requests

    def add(self, seq_id: int) -> None:
        if seq_id in self.pages:
            raise ValueError(f"sequence {seq_id} already has a cache")
        self.pages[seq_id] = []
        self.lens[seq_id] = 0

    def free(self, seq_id: int) -> None:
        """Return the request's pages to the pool."""
        self._free.extend(reversed(self.pages.pop(seq_id)))
        del self.lens[seq_id]

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def pages_needed(self, seq_id: int, n_new: int) -> int:
        total = self.lens[seq_id] + n_new
        return max(0, -(-total // self.page_size) - len(self.pages[seq_id]))

    def reserve(self, seq_id: int, n_new: int) -> None:
        """Make room for ``n_new`` more tokens of the request."""
        need = self.pages_needed(seq_id, n_new)
        if need > len(self._free):
            raise RuntimeError(f"PagedKVCache: out of pages ({need} needed, "
                               f"{len(self._free)} free)")
        for _ in range(need):
            self.pages[seq_id].append(self._free.pop())

    # ---------------------------------------------------------------- one step

    def slot_mapping(self, seq_ids: Sequence[int], n_new: int):
        """(page ids, slots) of the next ``n_new`` tokens of every request, in
        request-major order, as device tensors (after ``reserve``)."""
        pages, slots = [], []
        ps = self.page_size
        for s in seq_ids:
            plist, start = self.pages[s], self.lens[s]
            for j in range(start, start + n_new):
                pages.append(plist[j // ps])
                slots.append(j % ps)
        dev = self.device
        return (torch.tensor(pages, dtype=torch.int32, device=dev),
                torch.tensor(slots, dtype=torch.int32, device=dev))

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor, page_ids: torch.Tensor,
              slots: torch.Tensor) -> None:
        """Store ``k``/``v [B, L, num_kv_heads, D]`` at the mapped slots (for
        callers that compute k/v themselves; the model's fused q/k kernel
        stores them directly)."""
        kk = k.reshape(-1, self.num_kv_heads, self.head_dim).to(self.dtype)
        vv = v.reshape(-1, self.num_kv_heads, self.head_dim).to(self.dtype)
        page_ids, slots = page_ids.long(), slots.long()
        self.key_pages[layer][page_ids, :, slots, :] = kk
        self.value_pages[layer][page_ids, :, slots, :] = vv

    def advance(self, seq_ids: Sequence[int], n_new: int) -> None:
        for s in seq_ids:
            self.lens[s] += n_new

    def block_table(self, seq_ids: Sequence[int], extra: int = 0, width: int | None = None):
        """``block_table [B, width]`` (-1 past a request's pages; width defaults
        to the longest page list) and ``context_lens [B]`` (current length +
        ``extra``) as int32 tensors."""
        width = width or max(1, max(len(self.pages[s]) for s in seq_ids))
        rows = [self.pages[s] + [-1] * (width - len(self.pages[s])) for s in seq_ids]
        dev = self.device
        return (torch.tensor(rows, dtype=torch.int32, device=dev),
                torch.tensor([self.lens[s] + extra for s in seq_ids], dtype=torch.int32,
                             device=dev))
