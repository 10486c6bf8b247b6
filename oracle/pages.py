"""Oracle: paged-KV index math and pool gather/scatter.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference gives every sample a static slice of pages
(engines/flashinfer.py:104-116) and computes write indices and the attention
plan from it (engines/flashinfer.py:318-344, 346-411).  Here the same math is
restated for an arbitrary page table ``table[row][j]`` = pool page that holds
positions ``[j*ps, (j+1)*ps)`` of ``row``; the reference's static slices are
the special case ``table[row][j] = row*P + j``.

Pool layout (the engine's own, chosen for the MI355X attention kernel):
one layer's pool is ``[pages, 2, heads, ps*hd]`` bf16.  Plane 0 holds K
head-major and token-major inside a head (element ``t*hd + d``); plane 1
holds V transposed inside a head (element ``d*ps + t``), so a lane can read
consecutive tokens of one V column with a single vector load.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple, Union

import numpy as np
import torch


def page_write_indices(table: Sequence[Sequence[int]], cache_starts: Union[int, Sequence[int]], bl: int,
                       ps: int = 16) -> Tuple[np.ndarray, np.ndarray]:
    """Flat (page, slot) for the ``B*bl`` block tokens (engines/flashinfer.py:318-344).

    ``cache_starts`` is one start for every row or a per-row list, as in the
    reference; with the identity table ``table[r][j] = r*P + j`` this is the
    reference's ``r*P + pos//ps``, ``pos % ps``."""
    if isinstance(cache_starts, (int, np.integer)):
        cache_starts = [int(cache_starts)] * len(table)
    pages: List[int] = []
    slots: List[int] = []
    for r, cs in enumerate(cache_starts):
        for j in range(bl):
            pos = cs + j
            pages.append(int(table[r][pos // ps]))
            slots.append(pos % ps)
    return np.asarray(pages, dtype=np.int64), np.asarray(slots, dtype=np.int64)


def plan(table: Sequence[Sequence[int]], kv_lens: Union[int, Sequence[int]], bl: int, ps: int = 16):
    """``qo_indptr``, ``kv_indptr``, ``kv_indices``, ``last_page_len`` (engines/flashinfer.py:346-411):
    each row's ``ceil(kv_len/ps)`` pages in table order, ``last_page_len = kv_len % ps or ps``."""
    if isinstance(kv_lens, (int, np.integer)):
        kv_lens = [int(kv_lens)] * len(table)
    B = len(kv_lens)
    qo = np.zeros(B + 1, dtype=np.int32)
    kvi = np.zeros(B + 1, dtype=np.int32)
    idx: List[int] = []
    last = np.zeros(B, dtype=np.int32)
    for b in range(B):
        pu = (kv_lens[b] + ps - 1) // ps
        qo[b + 1] = qo[b] + bl
        kvi[b + 1] = kvi[b] + pu
        idx.extend(int(p) for p in table[b][:pu])
        rem = kv_lens[b] % ps
        last[b] = rem if rem > 0 else ps
    return qo, kvi, np.asarray(idx, dtype=np.int32), last


def pool_write(pool: torch.Tensor, table, cache_starts, k: torch.Tensor, v: torch.Tensor,
               ps: int = 16) -> None:
    """Scatter K/V of ``B*bl`` tokens (``[N, H, hd]``) into ``pool`` ``[P, 2, H, ps*hd]``."""
    H, hd = k.shape[1], k.shape[2]
    bl = k.shape[0] // len(cache_starts)
    pages, slots = page_write_indices(table, cache_starts, bl, ps)
    for n in range(k.shape[0]):
        p, t = int(pages[n]), int(slots[n])
        for h in range(H):
            pool[p, 0, h].view(ps, hd)[t] = k[n, h]
            pool[p, 1, h].view(hd, ps)[:, t] = v[n, h]


def pool_gather(pool: torch.Tensor, table_row: Sequence[int], kv_len: int,
                ps: int = 16) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dense ``K, V`` ``[kv_len, H, hd]`` of one row, walking its page list."""
    H = pool.shape[2]
    hd = pool.shape[3] // ps
    npg = (kv_len + ps - 1) // ps
    ks = []
    vs = []
    for j in range(npg):
        p = int(table_row[j])
        ks.append(pool[p, 0].view(H, ps, hd).permute(1, 0, 2))      # [ps, H, hd]
        vs.append(pool[p, 1].view(H, hd, ps).permute(2, 0, 1))      # [ps, H, hd]
    K = torch.cat(ks, 0)[:kv_len].contiguous()
    V = torch.cat(vs, 0)[:kv_len].contiguous()
    return K, V
