"""Varlen paged attention for packed multi-sequence passes on the MI355X.

The contract of the reference (memforge_ml/kernels/varlen_attention.py:60-395):
query rows packed as ``(1, H, T_total, D)`` in any order; row r belongs to
``seq_ids[r]`` (an index into ``block_tables``) and attends to that
sequence's keys at positions ``0..positions[r]`` inclusive, with grouped-query
heads sharing a KV head. Output rows come back in input order, in the query
dtype. Both reference entry points -- the block-wise ``paged_attention_varlen``
and the gather-then-softmax ``paged_attention_varlen_materialised`` -- are the
same function, and here both are the one HIP kernel (mf_paged_attention),
which walks the pool block by block with an fp32 online softmax.
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch

from memforge_amd import _native as nat
from memforge_amd.kernels._varlen import as_table_list, run_varlen

MASK_FILL = float("-inf")


def group_by_sequence(seq_ids: Sequence[int]) -> List[Tuple[int, List[int]]]:
    """Packed rows per sequence in first-seen order (varlen_attention.py:60-76)."""
    order: List[int] = []
    rows: dict = {}
    for row, seq_id in enumerate(seq_ids):
        if seq_id not in rows:
            rows[seq_id] = []
            order.append(seq_id)
        rows[seq_id].append(row)
    return [(seq_id, rows[seq_id]) for seq_id in order]


def _validate(query: torch.Tensor, num_kv_heads: int, seq_ids, positions, block_tables, block_size,
              materialised: bool):
    if query.shape[0] != 1:
        raise ValueError(f"expected a packed batch of 1, got {tuple(query.shape)}")
    total = query.shape[2]
    if len(seq_ids) != total or len(positions) != total:
        raise ValueError(f"{total} query tokens but {len(seq_ids)} seq_ids and {len(positions)} positions")
    if total == 0:
        raise ValueError("paged_attention_varlen requires at least one query token")
    if any(p < 0 for p in positions):
        raise ValueError(f"negative query position in {list(positions)}")
    num_heads = query.shape[1]
    if num_heads % num_kv_heads != 0:
        raise ValueError(f"{num_heads} query heads is not a multiple of {num_kv_heads} kv heads")
    tables = [as_table_list(t) for t in block_tables]
    for seq_id, rows in group_by_sequence(seq_ids):
        if seq_id < 0 or seq_id >= len(tables):
            raise IndexError(f"seq_id {seq_id} has no block table (got {len(tables)})")
        last_key = max(positions[r] for r in rows)
        needed = (last_key + 1 + block_size - 1) // block_size
        if needed > len(tables[seq_id]):
            raise IndexError(
                f"sequence {seq_id} reads up to position {last_key}, needing "
                f"{needed} blocks, but its block table has {len(tables[seq_id])} entries"
            )
    return tables


def _run(query, key_pool_layer, value_pool_layer, tables, seq_ids, positions, scale):
    num_kv_heads = key_pool_layer.shape[2]
    dtype = key_pool_layer.dtype
    q = query[0].to(dtype).permute(1, 0, 2)  # (T, H, D)
    total, heads, dim = q.shape
    out = torch.empty((1, heads, total, dim), dtype=dtype, device=query.device)
    run_varlen(q, out[0].permute(1, 0, 2), nat.PoolView.from_bshd(key_pool_layer, value_pool_layer),
               tables, list(seq_ids), list(positions), scale, num_kv_heads)
    return out.to(query.dtype)


def paged_attention_varlen(query: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
                           layer_idx: int, block_tables: Sequence[torch.Tensor], seq_ids: Sequence[int],
                           positions: Sequence[int], block_size: int,
                           scale: Optional[float] = None) -> torch.Tensor:
    """Attention for a packed run of query tokens from several sequences
    (varlen_attention.py:78-235). Pools are ``(layers, blocks, slots, kv_heads, head_dim)``."""
    nat.require_device(query, key_pool)
    if key_pool.shape[2] != block_size:
        raise ValueError(f"pool block size {key_pool.shape[2]} does not match {block_size}")
    tables = _validate(query, key_pool.shape[3], seq_ids, positions, block_tables, block_size, False)
    return _run(query, key_pool[layer_idx], value_pool[layer_idx], tables, seq_ids, positions, scale)


def paged_attention_varlen_materialised(query: torch.Tensor, pool, layer_idx: int,
                                        block_tables: Sequence[torch.Tensor], seq_ids: Sequence[int],
                                        positions: Sequence[int],
                                        scale: Optional[float] = None) -> torch.Tensor:
    """The same function with the reference's pool-object signature
    (varlen_attention.py:291-395)."""
    nat.require_device(query, pool.key_pool)
    tables = _validate(query, pool.key_pool.shape[3], seq_ids, positions, block_tables, pool.block_size, True)
    return _run(query, pool.key_pool[layer_idx], pool.value_pool[layer_idx], tables, seq_ids, positions, scale)


def reference_varlen_attention(query: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
                               layer_idx: int, block_tables: Sequence[torch.Tensor], seq_ids: Sequence[int],
                               positions: Sequence[int], block_size: int,
                               scale: Optional[float] = None) -> torch.Tensor:
    """What the kernel must equal, computed the obvious way with dense torch
    ops (varlen_attention.py:238-288): per row, materialise its visible keys
    token by token and run one plain softmax. Shares no code with the kernel;
    meant for tests."""
    num_heads, head_dim = query.shape[1], query.shape[3]
    num_kv_heads = key_pool.shape[3]
    group = num_heads // num_kv_heads
    scale = scale if scale is not None else 1.0 / math.sqrt(head_dim)
    total = query.shape[2]
    out = torch.zeros((num_heads, total, head_dim), dtype=torch.float32, device=query.device)
    for row in range(total):
        table = as_table_list(block_tables[seq_ids[row]])
        visible = positions[row] + 1
        pos = torch.arange(visible)
        phys = torch.tensor(table, dtype=torch.long)[pos // block_size].to(query.device)
        keys = key_pool[layer_idx, phys, (pos % block_size).to(query.device)].float()
        values = value_pool[layer_idx, phys, (pos % block_size).to(query.device)].float()
        if group > 1:
            keys = keys.repeat_interleave(group, dim=1)
            values = values.repeat_interleave(group, dim=1)
        q = query[0, :, row, :].float()
        scores = torch.matmul(keys.permute(1, 0, 2).contiguous(), q.unsqueeze(-1)).squeeze(-1) * scale
        weights = torch.softmax(scores, dim=-1)  # (heads, visible)
        out[:, row, :] = torch.matmul(weights.unsqueeze(1), values.permute(1, 0, 2).contiguous()).squeeze(1)
    return out.unsqueeze(0).to(query.dtype)
