"""Engine protocol consumed by the block-diffusion decode loop.

Same surface as chatterbox_flash/engines/base.py:42-141 so ``HipEngine`` is
a drop-in: lifecycle ``reset`` -> ``prefix_forward`` -> optional
``capture_cuda_graph`` -> per block, per denoise step ``set_shift_ctx`` +
``block_forward_graph`` (or ``block_forward``) -> commit via
``block_forward`` -> ``advance_cache``.
"""

from __future__ import annotations

from typing import List, Optional, Protocol, Tuple, Union, runtime_checkable

import torch
from torch import Tensor

CacheStarts = Union[int, List[int]]


@runtime_checkable
class InferenceEngine(Protocol):
    has_cuda_graph: bool

    @property
    def cache_len(self) -> int: ...

    def reset(self) -> None: ...

    def can_reuse(self, max_seq_len: int, dtype: torch.dtype, *, batch_size: int,
                  page_size: int = 16) -> bool: ...

    def prefix_forward(self, prefix_emb_or_list: Union[Tensor, List[Tensor]]) -> Tensor: ...

    def block_forward(self, block_emb: Tensor, cache_starts: CacheStarts) -> Tensor: ...

    def block_forward_graph(self, block_emb: Tensor,
                            cache_starts: CacheStarts) -> Tuple[Tensor, Optional[Tensor]]: ...

    def advance_cache(self, block_len: int) -> None: ...

    def set_shift_ctx(self, ctx: Tensor) -> None: ...

    def capture_cuda_graph(self, block_size: int, *,
                           speech_head: Optional[torch.nn.Linear] = None) -> None: ...
