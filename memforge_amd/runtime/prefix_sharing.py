"""Pool-side half of prefix sharing: the copy-on-write block copy and the
sharing figures (same functions as the reference, memforge_ml/runtime/
prefix_sharing.py:28-98). Which blocks are shared is decided by the C++
``PrefixCache`` and ``BlockAllocator``; this file only moves K/V and reports.
"""

from __future__ import annotations

import itertools
from typing import Any, Dict, Iterable, List, Optional, Sequence, Tuple

from memforge_amd import _native
from memforge_amd.runtime.kv_pool import PagedKVPool


def copy_block(pool: PagedKVPool, src: int, dst: int) -> None:
    """Copy block ``src`` to ``dst`` in every layer, K and V, with one
    ``mf_kv_copy_blocks`` launch; a no-op on itself. Must run before the
    write that triggered the copy-on-write."""
    if src == dst:
        return
    copy_blocks(pool, [(src, dst)])


def copy_blocks(pool: PagedKVPool, pairs: Sequence[Tuple[int, int]]) -> None:
    """Several copy-on-write moves in one launch (up to 32 pairs per launch).
    Raises if an index is out of range, a block is written twice, or a written
    block is also read."""
    pairs = [(int(s), int(d)) for s, d in pairs]
    if not pairs:
        return
    _native.kv_copy_blocks(pool.key_pool, pool.value_pool, pairs)


def block_owners(runtimes: Iterable[Tuple[int, List[int]]], total_blocks: int) -> Dict[str, List[int]]:
    """Every in-range physical block mapped to all sequences whose table holds
    it (a sequence once per table entry), owners sorted; keys are the block
    ids as strings (JSON), in block order."""
    holdings = sorted((int(b), int(seq_id)) for seq_id, table in runtimes for b in table
                      if 0 <= int(b) < total_blocks)
    return {str(block): [seq for _, seq in group]
            for block, group in itertools.groupby(holdings, key=lambda h: h[0])}


def sharing_telemetry(allocator: Any, pool: PagedKVPool, prefix_cache: Optional[Any],
                      owners: Optional[Dict[str, List[int]]] = None) -> Dict[str, Any]:
    """Sharing figures with a stable shape (zeros when sharing is off).
    ``memory_saved_mb`` = blocks saved (sum of references minus distinct
    allocated blocks) x the pool's bytes per block."""
    saved = allocator.get_num_blocks_saved()
    payload: Dict[str, Any] = {
        "shared_blocks": allocator.get_num_shared_blocks(),
        "blocks_saved": saved,
        "memory_saved_mb": round(saved * pool.bytes_per_block / (1024 * 1024), 3),
        "cached_prefix_blocks": prefix_cache.num_cached_blocks() if prefix_cache else 0,
        "prefix_hit_rate": round(prefix_cache.hit_rate(), 4) if prefix_cache else 0.0,
        "prefix_cache_hits": prefix_cache.num_hits() if prefix_cache else 0,
        "prefix_cache_misses": prefix_cache.num_misses() if prefix_cache else 0,
        "prefix_sharing_enabled": prefix_cache is not None,
    }
    if owners is not None:
        payload["block_owners"] = owners
    return payload
