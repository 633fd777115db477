"""Paged-pool addressing, KV write/gather and ragged packing (test infrastructure only).

Every function restates one piece of the reference's behaviour on plain
Python/numpy data so the device kernels can be compared against it
bit-exactly.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np


def flat_slot_index(physical: Sequence[int], slots: Sequence[int], block_size: int) -> np.ndarray:
    """``physical * block_size + slot`` (memforge_ml/kernels/paged_gather.py:42-55)."""
    return np.asarray(physical, dtype=np.int64) * block_size + np.asarray(slots, dtype=np.int64)


def slot_indices(block_table: Sequence[int], start: int, end: int,
                 block_size: int) -> Tuple[np.ndarray, np.ndarray]:
    """(physical block, slot) for token range [start, end), with the reference's
    IndexError text (memforge_ml/runtime/kv_pool.py:92-110)."""
    table = np.asarray(block_table, dtype=np.int64)
    positions = np.arange(start, end, dtype=np.int64)
    logical = positions // block_size
    slots = positions % block_size
    if logical.size and int(logical.max()) >= table.size:
        raise IndexError(
            f"logical block {int(logical.max())} is outside a block table of "
            f"{table.size} entries (token range {start}:{end})"
        )
    return table[logical], slots


def slot_mapping(block_table: Sequence[int], start: int, end: int, block_size: int) -> np.ndarray:
    """Flat pool slots of [start, end): ``flat_indices``, i.e. slot_indices plus
    the flat index (memforge_ml/runtime/kv_pool.py:116-130)."""
    physical, slots = slot_indices(block_table, start, end, block_size)
    return flat_slot_index(physical, slots, block_size)


def varlen_write_index(block_tables: Sequence[Sequence[int]], seq_ids: Sequence[int],
                       positions: Sequence[int], block_size: int) -> np.ndarray:
    """One flat write slot per packed token, each through its own sequence's
    table, with the reference's checks and messages
    (memforge_ml/runtime/varlen_cache.py:161-191)."""
    flat: List[int] = []
    for seq_id, position in zip(seq_ids, positions):
        if seq_id < 0 or seq_id >= len(block_tables):
            raise IndexError(f"seq_id {seq_id} has no block table (got {len(block_tables)})")
        if position < 0:
            raise ValueError(f"negative position {position}")
        table = list(block_tables[seq_id])
        logical = position // block_size
        if logical >= len(table):
            raise IndexError(
                f"position {position} needs logical block {logical} but "
                f"sequence {seq_id} has a block table of {len(table)}"
            )
        flat.append(int(table[logical]) * block_size + position % block_size)
    if len(set(flat)) != len(flat):
        raise ValueError(
            "two packed tokens map to the same pool slot; the step's "
            "sequence ids and positions overlap"
        )
    return np.asarray(flat, dtype=np.int64)


def kv_write(pool_layer: np.ndarray, slots: np.ndarray, rows: np.ndarray) -> None:
    """``pool[layer].view(N*bs, H, D)[slots] = rows`` (index_copy_ semantics,
    memforge_ml/kernels/paged_gather.py:92-117). ``pool_layer`` is
    (N, bs, H, D); ``rows`` is (T, H, D) already in the pool's dtype (or bit
    pattern). Negative slots are skipped, as the device kernel does."""
    n, bs, h, d = pool_layer.shape
    flat = pool_layer.reshape(n * bs, h, d)
    keep = np.asarray(slots) >= 0
    flat[np.asarray(slots)[keep]] = rows[keep]


def kv_gather(pool_layer: np.ndarray, slots: np.ndarray) -> np.ndarray:
    """``index_select`` of flat slots -> (T, H, D) (paged_gather.py:58-89)."""
    n, bs, h, d = pool_layer.shape
    return pool_layer.reshape(n * bs, h, d)[np.asarray(slots)].copy()


def ragged_pack(entries: Sequence[Tuple[int, int, int, Sequence[int], Sequence[int]]],
                block_size: int, max_blocks: int) -> dict:
    """Brute-force restatement of the engine's per-step packing.

    Each entry is ``(q_len, start_pos, kv_len, block_table, tokens)`` in plan
    order (prefill entries, then decode entries: continuous_engine.py:874-905).
    Row r of entry e carries token ``tokens[i]``, position ``start_pos + i``
    (continuous_engine.py:810-833, 892-896) and slot
    ``table[p // bs] * bs + p % bs`` (varlen_cache.py:173-179); a row whose
    block lies past its table gets slot -1 and is reported.
    """
    token_ids: List[int] = []
    positions: List[int] = []
    seq_slot: List[int] = []
    slots: List[int] = []
    cu = [0]
    kv_lens: List[int] = []
    tables = np.zeros((len(entries), max_blocks), dtype=np.int32)
    overflow_rows: List[int] = []
    for e, (q_len, start, kv_len, table, tokens) in enumerate(entries):
        for k, blk in enumerate(list(table)[:max_blocks]):
            tables[e, k] = blk
        for i in range(q_len):
            p = start + i
            r = len(token_ids)
            token_ids.append(int(tokens[i]))
            positions.append(p)
            seq_slot.append(e)
            logical = p // block_size
            if p < 0 or logical >= len(table):
                if p >= 0:
                    overflow_rows.append(r)
                slots.append(-1)
            else:
                slots.append(int(table[logical]) * block_size + p % block_size)
        cu.append(len(token_ids))
        kv_lens.append(kv_len)
    dup_rows: List[int] = []
    seen = set()
    for r, s in enumerate(slots):
        if s < 0:
            continue
        if s in seen:
            dup_rows.append(r)
        seen.add(s)
    return {
        "token_ids": np.asarray(token_ids, dtype=np.int64),
        "positions": np.asarray(positions, dtype=np.int64),
        "seq_slot": np.asarray(seq_slot, dtype=np.int32),
        "slot_mapping": np.asarray(slots, dtype=np.int64),
        "cu_seqlens": np.asarray(cu, dtype=np.int32),
        "kv_lens": np.asarray(kv_lens, dtype=np.int32),
        "block_tables": tables,
        "first_overflow_row": overflow_rows[0] if overflow_rows else -1,
        "first_duplicate_row": dup_rows[0] if dup_rows else -1,
    }
