"""Paged KV gather and scatter through the HIP copy kernels.

Same functions and contracts as the reference's
memforge_ml/kernels/paged_gather.py:42-117; the copies run as
``mf_kv_gather`` / ``mf_kv_write`` on the MI355X, bit-identical to
``index_select`` / ``index_copy_`` of the flattened pool.
"""

from __future__ import annotations

from typing import Tuple

import torch

from memforge_amd import _native as nat


def flat_slot_index(physical: torch.Tensor, slots: torch.Tensor, block_size: int) -> torch.Tensor:
    """``physical * block_size + slot`` as one contiguous int64 index
    (paged_gather.py:42-55)."""
    return (physical.to(torch.int64) * block_size + slots.to(torch.int64)).contiguous()


def _layer_view(key_pool: torch.Tensor, value_pool: torch.Tensor, layer_idx: int) -> nat.PoolView:
    return nat.PoolView.from_bshd(key_pool[layer_idx], value_pool[layer_idx])


def gather_kv(key_pool: torch.Tensor, value_pool: torch.Tensor, layer_idx: int,
              flat_index: torch.Tensor, block_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """One layer's K/V at ``flat_index`` as contiguous ``(1, heads, tokens, head_dim)``
    (paged_gather.py:58-89)."""
    num_blocks, slots_per_block = key_pool.shape[1], key_pool.shape[2]
    assert slots_per_block == block_size, (
        f"pool block size {slots_per_block} does not match {block_size}"
    )
    heads, dim = key_pool.shape[3], key_pool.shape[4]
    t = flat_index.numel()
    k = torch.empty((1, heads, t, dim), dtype=key_pool.dtype, device=key_pool.device)
    v = torch.empty_like(k)
    nat.kv_gather(_layer_view(key_pool, value_pool, layer_idx), flat_index.reshape(-1),
                  k[0].permute(1, 0, 2), v[0].permute(1, 0, 2))
    return k, v


def scatter_kv(key_pool: torch.Tensor, value_pool: torch.Tensor, layer_idx: int,
               flat_index: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
               block_size: int) -> None:
    """Write ``(1, heads, tokens, head_dim)`` K/V into the pool in place,
    converting to the pool dtype (paged_gather.py:92-117)."""
    nat.kv_write(keys[0].permute(1, 0, 2), values[0].permute(1, 0, 2), flat_index.reshape(-1),
                 _layer_view(key_pool, value_pool, layer_idx))
