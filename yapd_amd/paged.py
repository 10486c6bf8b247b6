"""Paged KV pool, page tables and the attention plan (host side of kernel (a)).

The reference gives each sample a static slice of ``ceil(max_seq/16)`` pages
(engines/flashinfer.py:104-116) and re-plans the attention metadata in Python
per block (engines/flashinfer.py:346-411, 1506-1556).  Here every layer owns a
zero-filled pool ``[pages, 2, H, 16*64]`` (layout in csrc/kv_layout.h), rows
map positions to pages through an int32 table that may be any permutation of
pool pages, and the attention work list is built once per block by the
native planner (``yapd_attn_plan``) and uploaded.
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import numpy as np
import torch

from . import kernels

PAGE_SIZE = 16
HEAD_DIM = 64


def to_device_async(data, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """Host data (list or array) on ``device`` without a host synchronisation: staged through
    pinned memory and copied on the current stream (a copy from pageable memory would wait for
    every kernel already queued)."""
    t = torch.as_tensor(np.asarray(data), dtype=dtype)
    if torch.device(device).type != "cuda":
        return t.to(device)
    return t.pin_memory().to(device, non_blocking=True)


def copy_from_host_async(dst: torch.Tensor, data) -> None:
    """``dst.copy_(data)`` for host data (list or array) without a host synchronisation: staged
    through pinned memory and copied on the current stream.  Not for use inside a graph capture
    (the copy would keep reading a recycled staging buffer on every replay)."""
    t = torch.as_tensor(np.asarray(data)).to(dst.dtype)
    if dst.device.type != "cuda":
        dst.copy_(t)
        return
    dst.copy_(t.pin_memory(), non_blocking=True)


class PagedKV:
    """Per-layer page pools plus a host-side page allocator and device page table."""

    def __init__(self, *, n_layers: int, n_rows: int, pages_per_row: int, n_heads: int,
                 device: torch.device, n_pages: Optional[int] = None, shuffle_seed: Optional[int] = None):
        self.n_layers = int(n_layers)
        self.n_rows = int(n_rows)
        self.pages_per_row = int(pages_per_row)
        self.n_heads = int(n_heads)
        self.device = torch.device(device)
        self.n_pages = int(n_pages) if n_pages is not None else self.n_rows * self.pages_per_row
        kernels.require(self.n_pages >= self.n_rows * self.pages_per_row, "pool smaller than rows * pages_per_row")
        self.pools: List[torch.Tensor] = [
            torch.zeros(self.n_pages, 2, self.n_heads, PAGE_SIZE * HEAD_DIM, dtype=torch.bfloat16,
                        device=self.device)
            for _ in range(self.n_layers)
        ]
        order = np.arange(self.n_pages, dtype=np.int32)
        if shuffle_seed is not None:
            order = np.random.default_rng(shuffle_seed).permutation(self.n_pages).astype(np.int32)
        take = order[: self.n_rows * self.pages_per_row]
        self.table_host = take.reshape(self.n_rows, self.pages_per_row).copy()
        self.table = torch.from_numpy(self.table_host).to(self.device)

    @property
    def bytes_per_layer(self) -> int:
        return self.pools[0].numel() * 2

    def swap_rows(self, a: int, b: int) -> None:
        """Exchange page-table rows ``a`` and ``b`` (host mirror and device table): each row's KV
        moves with its pages, nothing is copied.  Device work is stream-ordered, no host sync."""
        if a == b:
            return
        self.table_host[[a, b]] = self.table_host[[b, a]]
        tmp = self.table[a].clone()
        self.table[a].copy_(self.table[b])
        self.table[b].copy_(tmp)

    def copy_row_pages(self, src_row: int, dst_row: int, n_positions: int) -> None:
        """Copy the pages holding positions ``[0, n_positions)`` of one row to another, every layer."""
        npg = (n_positions + PAGE_SIZE - 1) // PAGE_SIZE
        src = to_device_async(self.table_host[src_row, :npg], torch.int64, self.device)
        dst = to_device_async(self.table_host[dst_row, :npg], torch.int64, self.device)
        for pool in self.pools:
            pool.index_copy_(0, dst, pool.index_select(0, src))


class AttnPlan:
    """Device work list + split-KV workspace for one set of per-row kv lengths."""

    def __init__(self, kv_len: Sequence[int], bl: int, n_heads: int, device: torch.device,
                 target_items: int = 192, min_split_keys: int = 1024):
        work, merge, n_slots = kernels.attn_plan(kv_len, target_items=target_items, min_split_keys=min_split_keys)
        self.kv_len_host = [int(x) for x in kv_len]
        self.work = to_device_async(work, torch.int32, device)
        self.merge = to_device_async(merge, torch.int32, device) if merge.shape[0] else None
        self.n_slots = n_slots
        self.kv_len = to_device_async(self.kv_len_host, torch.int32, device)
        if n_slots:
            self.part_o = torch.empty(n_slots, bl, n_heads, HEAD_DIM, dtype=torch.float32, device=device)
            self.part_ml = torch.empty(n_slots, bl, n_heads, 2, dtype=torch.float32, device=device)
        else:
            self.part_o = self.part_ml = None

    def run(self, q: torch.Tensor, pool: torch.Tensor, table: torch.Tensor, out: torch.Tensor,
            scale: float, causal: bool = False) -> None:
        kernels.require(max(self.kv_len_host) <= table.shape[1] * PAGE_SIZE,
                        "page table maps fewer positions than kv_len")
        kernels.attn_paged_block(q, pool, table, self.kv_len, self.work, self.merge, self.part_o, self.part_ml,
                                 out, scale, causal=causal)
