"""PagedCache: a ``transformers.Cache`` whose storage is the paged pool in HBM.

Same classes and engine interface as the reference (memforge_ml/runtime/
paged_cache.py:27-274). Every layer's ``update`` scatters the new K/V into the
sequence's physical blocks with the KV-write kernel; it returns either just
the new tokens (``lazy_read``, for the block-wise backend that reads the pool
itself) or the whole context gathered by the gather kernel. Growth is
block-granular and ``rollback(n)`` is O(1).

The reference's optional append-only decode mirror (``view_capacity``) is not
part of this build: it trades the memory paging saves for a contiguous copy,
which the varlen kernel makes unnecessary.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from memforge_amd.runtime.kv_pool import PagedKVPool


class PagedCacheLayer(CacheLayerMixin):
    """One attention layer's view of the shared paged pool."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, owner: "PagedCache", layer_idx: int):
        super().__init__()
        self.owner = owner
        self.layer_idx = layer_idx
        self.position = 0
        self.is_initialized = True

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args,
               **kwargs) -> Tuple[torch.Tensor, torch.Tensor]:
        if key_states.shape[0] != 1:
            raise ValueError(
                f"PagedCache is a single-sequence cache; got batch size {key_states.shape[0]}. "
                "Batched decoding goes through ContinuousBatchingEngine instead."
            )
        num_new = key_states.shape[-2]
        start, end = self.position, self.position + num_new
        self.owner.pool.write_flat(self.layer_idx, self.owner.flat_indices(start, end), key_states, value_states)
        self.position = end
        if self.owner.lazy_read and num_new == 1:
            return key_states, value_states
        return self.owner.pool.gather_flat(self.layer_idx, self.owner.flat_indices(0, end))

    def get_mask_sizes(self, query_length: int) -> Tuple[int, int]:
        return self.position + query_length, 0

    def get_seq_length(self) -> int:
        return self.position

    def get_max_length(self) -> int:
        return self.owner.pool.capacity_tokens

    def reset(self) -> None:
        self.position = 0

    def crop(self, tokens_to_remove: int) -> None:
        self.position = max(0, self.position - abs(tokens_to_remove))


class PagedCache(Cache):
    """Single-sequence KV cache over the shared pool. The engine calls
    ``set_block_table`` when the allocator grows the table and ``begin_step``
    before each forward pass."""

    def __init__(self, pool: PagedKVPool, block_table: List[int], device: Optional[str] = None,
                 view_capacity: Optional[int] = None, lazy_read: bool = False):
        if lazy_read and view_capacity:
            raise ValueError(
                "lazy_read and view_capacity are mutually exclusive: the mirror "
                "materialises the context, lazy mode avoids materialising it"
            )
        if view_capacity:
            raise NotImplementedError(
                "the contiguous decode mirror (view_capacity) is not part of memforge_amd; "
                "the varlen kernel reads the pool directly"
            )
        self.pool = pool
        self.device_str = device or pool.spec.device
        self._block_table: torch.Tensor = PagedKVPool.block_table_tensor(block_table, self.device_str)
        self._table_list: List[int] = list(block_table)
        self._index_memo: Dict[Tuple[int, int], Tuple[torch.Tensor, torch.Tensor]] = {}
        self._flat_memo: Dict[Tuple[int, int], torch.Tensor] = {}
        self.lazy_read = bool(lazy_read)
        self.view_cache = None
        super().__init__(layers=[PagedCacheLayer(self, i) for i in range(pool.spec.num_layers)])

    # ------------------------------------------------------- engine interface

    def set_block_table(self, block_table: List[int]) -> None:
        """Re-bind to a (possibly grown) logical -> physical block table."""
        if list(block_table) != self._table_list:
            self._table_list = list(block_table)
            self._block_table = PagedKVPool.block_table_tensor(self._table_list, self.device_str)
            self._index_memo.clear()
            self._flat_memo.clear()

    def begin_step(self, block_table: Optional[List[int]] = None) -> None:
        if block_table is not None:
            self.set_block_table(block_table)
        self._index_memo.clear()
        self._flat_memo.clear()

    def seed_position(self, num_cached_tokens: int) -> None:
        """Declare the first ``num_cached_tokens`` positions resident (prefix hit
        or an earlier prefill chunk); writes resume after them."""
        if num_cached_tokens < 0:
            raise ValueError(f"num_cached_tokens must be non-negative, got {num_cached_tokens}")
        for layer in self.layers:
            layer.position = num_cached_tokens
        self._index_memo.clear()
        self._flat_memo.clear()

    def indices(self, start: int, end: int) -> Tuple[torch.Tensor, torch.Tensor]:
        key = (start, end)
        if key not in self._index_memo:
            self._index_memo[key] = self.pool.slot_indices(self._block_table, start, end)
        return self._index_memo[key]

    def flat_indices(self, start: int, end: int) -> torch.Tensor:
        key = (start, end)
        if key not in self._flat_memo:
            self._flat_memo[key] = self.pool.flat_indices(self._block_table, start, end)
        return self._flat_memo[key]

    @property
    def block_table(self) -> List[int]:
        return list(self._table_list)

    def block_table_tensor_cached(self) -> torch.Tensor:
        return self._block_table

    @property
    def position(self) -> int:
        return self.layers[0].position

    def rollback(self, num_tokens: int) -> None:
        """Discard the last ``num_tokens`` positions by moving the cursor: O(1)."""
        if num_tokens <= 0:
            return
        for layer in self.layers:
            layer.crop(num_tokens)
        self._index_memo.clear()
        self._flat_memo.clear()

    def reset(self) -> None:
        for layer in self.layers:
            layer.reset()
        self._index_memo.clear()
        self._flat_memo.clear()

    def num_blocks_needed(self, total_tokens: int) -> int:
        bs = self.pool.block_size
        return (total_tokens + bs - 1) // bs
