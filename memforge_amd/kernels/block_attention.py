"""Single-query paged attention (the decode case) on the MI355X.

The contract of the reference's ``paged_attention_blockwise``
(memforge_ml/kernels/block_attention.py:51-145): one query position
``(1, H, 1, D)`` against the first ``context_length`` tokens of one sequence,
grouped-query heads sharing KV heads, fp32 accumulation, output in the query
dtype. It is the varlen kernel with one row.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from memforge_amd import _native as nat
from memforge_amd.kernels._varlen import as_table_list, run_varlen


def paged_attention_blockwise(query: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
                              layer_idx: int, block_table: torch.Tensor, context_length: int,
                              block_size: int, scale: Optional[float] = None) -> torch.Tensor:
    if query.shape[0] != 1 or query.shape[2] != 1:
        raise ValueError(f"expected a single query position (1, H, 1, D), got {tuple(query.shape)}")
    if context_length <= 0:
        raise ValueError(f"context_length must be positive, got {context_length}")
    num_heads, head_dim = query.shape[1], query.shape[3]
    num_kv_heads = key_pool.shape[3]
    if num_heads % num_kv_heads != 0:
        raise ValueError(f"{num_heads} query heads is not a multiple of {num_kv_heads} kv heads")
    num_logical = (context_length + block_size - 1) // block_size
    table = as_table_list(block_table)
    if num_logical > len(table):
        raise IndexError(f"context of {context_length} tokens needs {num_logical} blocks, "
                         f"block table has {len(table)}")
    nat.require_device(query, key_pool)
    dtype = key_pool.dtype
    q = query[0].to(dtype).permute(1, 0, 2)  # (1, H, D)
    out = torch.empty((1, num_heads, 1, head_dim), dtype=dtype, device=query.device)
    run_varlen(q, out[0].permute(1, 0, 2), nat.PoolView.from_bshd(key_pool[layer_idx], value_pool[layer_idx]),
               [table], [0], [context_length - 1], scale, num_kv_heads)
    return out.to(query.dtype)


def reference_attention(query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                        scale: Optional[float] = None) -> torch.Tensor:
    """Standard single-query attention over a materialised ``(1, Hkv, T, D)``
    context with grouped-query expansion, in dense torch ops; the reference
    ``paged_attention_blockwise`` is proved against (block_attention.py:148-174)."""
    num_heads, head_dim = query.shape[1], query.shape[3]
    group = num_heads // keys.shape[1]
    scale = scale if scale is not None else 1.0 / math.sqrt(head_dim)
    k = keys.to(torch.float32)
    v = values.to(torch.float32)
    if group > 1:
        k = k.repeat_interleave(group, dim=1)
        v = v.repeat_interleave(group, dim=1)
    scores = torch.matmul(query.to(torch.float32), k.transpose(2, 3).contiguous()) * scale
    weights = torch.softmax(scores, dim=-1)
    return torch.matmul(weights, v.contiguous()).to(query.dtype)
