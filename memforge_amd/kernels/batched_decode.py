"""Left-padded batch assembly of paged contexts (the reference's decode/verify
fallback layout, memforge_ml/kernels/batched_decode.py:42-219).

The engine in this package never materialises contexts -- the varlen kernel
reads the pool in place -- but the assembly API is kept for callers that feed
an ordinary padded ``DynamicCache``: each sequence's context is gathered
straight into its left-aligned window of one preallocated buffer by the
gather kernel, and new tokens are scattered back by the KV-write kernel.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch

from memforge_amd import _native as nat


class BatchedDecodeBuffers:
    """Reusable ``(layers, batch, heads, padded_len, head_dim)`` K/V scratch,
    bucketed to ``pad_to`` tokens and zeroed on reuse (batched_decode.py:42-120)."""

    DEFAULT_BUCKET_BLOCKS = 4

    def __init__(self, num_layers: int, block_size: int = 16, pad_to: Optional[int] = None):
        self.num_layers = num_layers
        self.block_size = max(1, block_size)
        self.pad_to = max(1, pad_to if pad_to else self.block_size * self.DEFAULT_BUCKET_BLOCKS)
        self._cache: Dict[Tuple[int, int], Tuple[torch.Tensor, torch.Tensor]] = {}

    def padded_len(self, max_len: int) -> int:
        return ((max_len + self.pad_to - 1) // self.pad_to) * self.pad_to

    def acquire(self, batch: int, max_len: int, num_heads: int, head_dim: int, dtype: torch.dtype,
                device: str) -> Tuple[torch.Tensor, torch.Tensor, int]:
        padded = self.padded_len(max_len)
        key = (batch, padded)
        entry = self._cache.get(key)
        if entry is None:
            shape = (self.num_layers, batch, num_heads, padded, head_dim)
            entry = (torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device))
            self._cache[key] = entry
        else:
            entry[0].zero_()
            entry[1].zero_()
        return entry[0], entry[1], padded

    def clear(self) -> None:
        self._cache.clear()

    @property
    def num_cached_shapes(self) -> int:
        return len(self._cache)


def assemble_batch(pool, buffers: BatchedDecodeBuffers, block_tables: Sequence[torch.Tensor],
                   context_lengths: Sequence[int]) -> Tuple[List[Tuple[torch.Tensor, torch.Tensor]], torch.Tensor, int]:
    """Gather a batch's contexts into one left-padded buffer: returns per-layer
    ``(keys, values)`` of ``(batch, heads, padded_len, head_dim)``, the
    ``(batch, padded_len)`` attention mask and the padded length
    (batched_decode.py:123-191)."""
    batch = len(context_lengths)
    if batch == 0:
        raise ValueError("assemble_batch requires at least one sequence")
    if len(block_tables) != batch:
        raise ValueError(f"{len(block_tables)} block tables for {batch} sequences")
    max_len = max(context_lengths)
    heads, dim = pool.spec.num_kv_heads, pool.spec.head_dim
    keys, values, padded = buffers.acquire(batch, max_len, heads, dim, pool.key_pool.dtype, pool.spec.device)
    flat = [pool.flat_indices(t, 0, c) for t, c in zip(block_tables, context_lengths)]
    for layer in range(pool.spec.num_layers):
        view = pool.layer_view(layer)
        for row, (index, ctx) in enumerate(zip(flat, context_lengths)):
            if ctx == 0:
                continue
            start = padded - ctx
            nat.kv_gather(view, index, keys[layer, row, :, start:padded, :].permute(1, 0, 2),
                          values[layer, row, :, start:padded, :].permute(1, 0, 2))
    mask = torch.zeros((batch, padded), dtype=torch.long, device=pool.spec.device)
    for row, ctx in enumerate(context_lengths):
        mask[row, padded - ctx:] = 1
    return [(keys[i], values[i]) for i in range(pool.spec.num_layers)], mask, padded


def scatter_new_tokens(pool, block_tables: Sequence[torch.Tensor], context_lengths: Sequence[int],
                       new_keys: Sequence[torch.Tensor], new_values: Sequence[torch.Tensor]) -> None:
    """Write each row's one new token back to its own blocks at position
    ``context_lengths[row]`` (batched_decode.py:194-219): one KV-write launch
    per layer for the whole batch."""
    slots = torch.cat([pool.flat_indices(t, c, c + 1) for t, c in zip(block_tables, context_lengths)])
    for layer in range(pool.spec.num_layers):
        k, v = new_keys[layer], new_values[layer]  # (batch, heads, 1, dim)
        nat.kv_write(k[:, :, 0, :], v[:, :, 0, :], slots, pool.layer_view(layer))
