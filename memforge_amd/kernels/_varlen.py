"""Host-side launcher of the varlen paged-attention kernel from per-sequence
descriptions (Python lists or tensors of block ids, per-row sequence ids and
positions). Shared by every attention entry point of the package; the engine
uses its own pre-packed path instead of this one."""

from __future__ import annotations

import math
from typing import List, Optional, Sequence

import numpy as np
import torch

from memforge_amd import _native as nat


def as_table_list(table) -> List[int]:
    if isinstance(table, torch.Tensor):
        return [int(x) for x in table.reshape(-1).tolist()]
    return [int(x) for x in table]


def padded_tables_host(tables: Sequence[Sequence[int]]) -> np.ndarray:
    """Block tables as one zero-padded int32 (B, max_blocks) array."""
    width = max(1, max((len(t) for t in tables), default=1))
    out = np.zeros((max(1, len(tables)), width), dtype=np.int32)
    for i, t in enumerate(tables):
        if len(t):
            out[i, : len(t)] = np.asarray(t, dtype=np.int64).astype(np.int32)
    return out


def padded_tables(tables: Sequence[Sequence[int]], device) -> torch.Tensor:
    return nat.upload([padded_tables_host(tables)], device)[0]


def run_varlen(q_rows: torch.Tensor, out_rows: torch.Tensor, pool: nat.PoolView,
               tables: Sequence[Sequence[int]], seq_ids: Sequence[int], positions: Sequence[int],
               scale: Optional[float], num_kv_heads: int, kv_lens: Optional[Sequence[int]] = None,
               pool_lens: Optional[Sequence[int]] = None, new_k_rows: Optional[torch.Tensor] = None,
               new_v_rows: Optional[torch.Tensor] = None) -> None:
    """Attention for packed rows in any order.

    q_rows / out_rows: (T, Hq, D) device views. Row r belongs to table
    ``seq_ids[r]`` and sees keys 0..positions[r]. ``kv_lens`` (per table)
    defaults to max position + 1 of that table's rows. With ``pool_lens`` the
    keys at or above pool_lens[s] are the in-flight rows of sequence s's own
    query rows, in position order.
    """
    dev = q_rows.device
    T, hq, d = q_rows.shape
    groups = {}
    order: List[int] = []
    for r, s in enumerate(seq_ids):
        if s not in groups:
            groups[s] = []
            order.append(s)
        groups[s].append(r)
    row_map: List[int] = []
    cu = [0]
    kvl: List[int] = []
    for s in order:
        rows = sorted(groups[s], key=lambda r: positions[r])
        row_map.extend(rows)
        cu.append(len(row_map))
        kvl.append(kv_lens[s] if kv_lens is not None else max(positions[r] for r in rows) + 1)
    identity = row_map == list(range(T))
    # every block id the kernel will read must address the pool
    bs, nblocks = pool.block_size, pool.num_blocks
    for i, s in enumerate(order):
        keys = kvl[i] if pool_lens is None else min(kvl[i], pool_lens[s])
        need = (keys + bs - 1) // bs
        if need > len(tables[s]):
            raise IndexError(f"sequence {s} needs {need} blocks but its block table has {len(tables[s])}")
        ids = np.asarray(tables[s][:need], dtype=np.int64)
        if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= nblocks):
            raise IndexError(f"block table of sequence {s} names a block outside the pool of {nblocks}")
    nat.require_device(q_rows, out_rows, pool.k)
    # a large decode step on 16-token blocks runs as one round of slices
    sliceable = identity and pool_lens is None and pool.block_size == 16
    items, merges, counts, sliced = nat.plan_host(cu, kvl, hq, num_kv_heads, d, q_rows.dtype, dev,
                                                  decode_slices=sliceable)
    # tables, plan, cu/kv lengths, positions, row map and pool lengths cross
    # to the device in one copy (none when the same bytes crossed before on
    # this stream), and the launch addresses them inside that one buffer
    tables_host = padded_tables_host([tables[s] for s in order])
    parts = [tables_host, *nat.plan_upload_parts(items, merges),
             np.asarray(cu + kvl, dtype=np.int32), np.asarray(list(positions), dtype=np.int64)]
    if not identity:
        parts.append(np.asarray(row_map, dtype=np.int32))
    if pool_lens is not None:
        parts.append(np.asarray([pool_lens[s] for s in order], dtype=np.int32))
    buf, offsets = nat.upload_packed_cached(parts, dev)
    nat.paged_attention_packed(
        q_rows, out_rows, pool, buf, offsets, len(order), tables_host.shape[1], counts,
        scale if scale is not None else 1.0 / math.sqrt(d), num_kv_heads,
        has_row_map=not identity, has_pool_lens=pool_lens is not None,
        new_k_rows=new_k_rows, new_v_rows=new_v_rows, sliced=sliced,
    )
