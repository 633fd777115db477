"""The standalone PagedAttention operator on the MI355X.

Same classes and contracts as the reference (memforge_ml/models/
paged_attention.py:12-141): ``PagedKVCache`` keeps K and V in per-head
physical blocks ``(num_blocks, num_heads, block_size, head_dim)``;
``PagedAttention.forward`` attends every query row to the first
``context_len`` tokens read through the block table, with no causal mask and
no grouped-query expansion, returning ``(1, query_len, num_heads * head_dim)``.
Writes, reads and the attention itself run as HIP kernels through the C ABI
(mf_kv_write, mf_kv_gather, mf_paged_attention); the softmax accumulates in
fp32 inside the attention kernel.
"""

from __future__ import annotations

import math
from typing import List, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

from memforge_amd import _native as nat
from memforge_amd.kernels._varlen import run_varlen


def _default_device() -> str:
    return "cuda"


class PagedKVCache:
    """Physical K/V blocks, shape per block ``(num_heads, block_size, head_dim)``."""

    def __init__(self, num_blocks: int, block_size: int, num_heads: int, head_dim: int,
                 dtype: torch.dtype = torch.float32, device: Optional[str] = None):
        device = device if device is not None else _default_device()
        if torch.device(device).type != "cuda":
            raise ValueError(
                f"memforge_amd keeps the paged KV cache in GPU memory; got device {device!r} "
                "(there is no CPU path)"
            )
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        shape = (num_blocks, num_heads, block_size, head_dim)
        self.key_cache = torch.zeros(shape, dtype=dtype, device=device)
        self.value_cache = torch.zeros(shape, dtype=dtype, device=device)

    def _view(self) -> nat.PoolView:
        # built once per (key_cache, value_cache) pair: the strides checks and
        # the view are the same on every call
        pv = getattr(self, "_pool_view", None)
        if pv is None or pv.k is not self.key_cache or pv.v is not self.value_cache:
            pv = nat.PoolView.from_bhsd(self.key_cache, self.value_cache)
            self._pool_view = pv
        return pv

    def _blocks(self, block_table: List[int], needed: int) -> np.ndarray:
        """The first ``needed`` physical block ids as the reference's tensor
        indexing reads them: a negative id counts from the end of the cache,
        and an id outside [-num_blocks, num_blocks) raises torch's IndexError
        (``self.key_cache[physical_block_id]``, paged_attention.py:65, 87)."""
        ids = np.asarray(list(block_table)[:needed], dtype=np.int64)
        bad = (ids < -self.num_blocks) | (ids >= self.num_blocks)
        if bad.any():
            raise IndexError(f"index {int(ids[bad][0])} is out of bounds for dimension 0 with size "
                             f"{self.num_blocks}")
        return np.where(ids < 0, ids + self.num_blocks, ids)

    def _slots(self, block_table: List[int], start: int, count: int) -> torch.Tensor:
        pos = np.arange(start, start + count, dtype=np.int64)
        table = self._blocks(block_table, (start + count + self.block_size - 1) // self.block_size)
        slots = table[pos // self.block_size] * self.block_size + pos % self.block_size
        return nat.upload([slots], self.device)[0]

    def write_kv(self, key_states: torch.Tensor, value_states: torch.Tensor,
                 block_table: List[int], start_pos: int) -> None:
        """Write ``(1, num_heads, seq_len, head_dim)`` K/V at positions
        start_pos.. through the block table (paged_attention.py:45-67). Tokens
        before the first one past the table are written before the
        IndexError, as the reference's per-token loop does."""
        seq_len = key_states.shape[2]
        fits = min(seq_len, max(0, len(block_table) * self.block_size - start_pos))
        if fits > 0:
            nat.kv_write(key_states[0, :, :fits].permute(1, 0, 2), value_states[0, :, :fits].permute(1, 0, 2),
                         self._slots(block_table, start_pos, fits), self._view())
        if fits < seq_len:
            logical = (start_pos + fits) // self.block_size
            raise IndexError(
                f"Logical block {logical} exceeds allocated block table length {len(block_table)}"
            )

    def read_kv(self, block_table: List[int], total_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """The first ``total_len`` tokens as ``(num_heads, total_len, head_dim)``
        (paged_attention.py:69-97)."""
        if total_len <= 0:
            raise RuntimeError("read_kv needs at least one token (torch.cat of an empty block list)")
        needed = (total_len + self.block_size - 1) // self.block_size
        if needed > len(block_table):
            raise IndexError("list index out of range")
        keys = torch.empty((self.num_heads, total_len, self.head_dim), dtype=self.dtype, device=self.device)
        values = torch.empty_like(keys)
        nat.kv_gather(self._view(), self._slots(block_table, 0, total_len),
                      keys.permute(1, 0, 2), values.permute(1, 0, 2))
        return keys, values


class PagedAttention(nn.Module):
    """``softmax(Q K^T * scale) V`` against the paged cache (paged_attention.py:100-141)."""

    def __init__(self, scale: Optional[float] = None):
        super().__init__()
        self.scale = scale

    def forward(self, query: torch.Tensor, paged_kv: PagedKVCache, block_table: List[int],
                context_len: int) -> torch.Tensor:
        head_dim = query.shape[-1]
        scale = self.scale or (1.0 / math.sqrt(head_dim))
        if context_len <= 0:
            raise RuntimeError("PagedAttention needs at least one context token")
        if (context_len + paged_kv.block_size - 1) // paged_kv.block_size > len(block_table):
            raise IndexError("list index out of range")
        _, num_heads, q_len, _ = query.shape
        if num_heads != paged_kv.num_heads:
            raise RuntimeError(
                f"query has {num_heads} heads but the paged cache has {paged_kv.num_heads}"
            )
        q = query[0].to(paged_kv.dtype).permute(1, 0, 2)  # (q_len, H, D) view
        out = torch.empty((1, q_len, num_heads * head_dim), dtype=paged_kv.dtype, device=query.device)
        table = paged_kv._blocks(block_table, (context_len + paged_kv.block_size - 1) // paged_kv.block_size)
        run_varlen(q, out[0].view(q_len, num_heads, head_dim), paged_kv._view(), [table.tolist()],
                   [0] * q_len, [context_len - 1] * q_len, scale, num_heads, kv_lens=[context_len])
        return out.to(query.dtype)
