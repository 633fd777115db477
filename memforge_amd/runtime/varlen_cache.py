"""A cache for one packed multi-sequence forward pass (prefill chunks, decodes
and verify rows in one row of tokens).

Same classes as the reference (memforge_ml/runtime/varlen_cache.py:42-203):
each packed token's K/V goes to its own sequence's slot through one flat write
index (the slot_mapping), and ``update`` returns the inputs unchanged -- the
varlen kernel reads the pool itself. Here the write index is built on the GPU
by the ragged-pack kernel, duplicate slots are caught with its device bitmap,
and the write is the KV-write kernel.

Two extra constructors serve the engine: ``from_slot_mapping`` wraps a
slot_mapping the engine's own ragged pack already produced, and ``verify``
writes nothing during the pass (the candidates are attended in flight) but
keeps each layer's new K/V so only the confirmed prefix is scattered after
rejection sampling.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from memforge_amd import _native as nat
from memforge_amd.kernels._varlen import as_table_list


class VarlenPackedCacheLayer(CacheLayerMixin):
    """One layer's view of a packed, multi-sequence write."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, owner: "VarlenPackedCache", layer_idx: int):
        super().__init__()
        self.owner = owner
        self.layer_idx = layer_idx
        self.is_initialized = True

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args,
               **kwargs) -> Tuple[torch.Tensor, torch.Tensor]:
        if key_states.shape[0] != 1:
            raise ValueError(f"VarlenPackedCache takes one packed row, got batch {key_states.shape[0]}")
        if key_states.shape[-2] != self.owner.num_tokens:
            raise ValueError(f"{key_states.shape[-2]} key states for {self.owner.num_tokens} packed tokens")
        if self.owner.hold_new_kv:
            self.owner.new_kv[self.layer_idx] = (key_states, value_states)
        elif self.owner.write_in_attention:
            # the layer's attention launch writes these rows itself
            # (mf_paged_attention_kv_write), reading them in flight meanwhile
            pass
        else:
            timer = self.owner.timer
            began = timer.start(self.layer_idx) if timer is not None else None
            self.owner.pool.write_flat(self.layer_idx, self.owner.write_index, key_states, value_states)
            if timer is not None:
                timer.stop("kv_write", began)
        return key_states, value_states

    def get_mask_sizes(self, query_length: int) -> Tuple[int, int]:
        return query_length, 0

    def get_seq_length(self) -> int:
        return 0

    def get_max_length(self) -> int:
        return self.owner.pool.capacity_tokens

    def reset(self) -> None:
        pass

    def crop(self, tokens_to_remove: int) -> None:
        raise NotImplementedError(
            "VarlenPackedCache holds no per-sequence cursor to crop; roll back "
            "the owning sequences' PagedCache positions instead"
        )


def _runs(seq_ids: Sequence[int], positions: Sequence[int]) -> List[Tuple[int, int, int]]:
    """Maximal runs of consecutive rows of one sequence at consecutive positions:
    (seq_id, start_position, length)."""
    runs: List[Tuple[int, int, int]] = []
    for s, p in zip(seq_ids, positions):
        if runs and runs[-1][0] == s and runs[-1][1] + runs[-1][2] == p:
            runs[-1] = (s, runs[-1][1], runs[-1][2] + 1)
        else:
            runs.append((s, p, 1))
    return runs


def _slot_bitmap(pool) -> torch.Tensor:
    """Per-pool duplicate-slot bitmap, all-zero between ragged-pack calls."""
    bm = getattr(pool, "_mf_slot_bitmap", None)
    words = (pool.capacity_tokens + 31) // 32
    if bm is None or bm.numel() < words:
        bm = torch.zeros(words, dtype=torch.int32, device=pool.key_pool.device)
        pool._mf_slot_bitmap = bm
    return bm


def build_write_index(pool, block_tables: Sequence, seq_ids: Sequence[int],
                      positions: Sequence[int]) -> torch.Tensor:
    """One flat pool slot per packed token through its own sequence's table,
    with the reference's checks and messages (varlen_cache.py:161-191)."""
    bs = pool.block_size
    tables = [as_table_list(t) for t in block_tables]
    for seq_id, position in zip(seq_ids, positions):
        if seq_id < 0 or seq_id >= len(tables):
            raise IndexError(f"seq_id {seq_id} has no block table (got {len(tables)})")
        if position < 0:
            raise ValueError(f"negative position {position}")
        logical = position // bs
        if logical >= len(tables[seq_id]):
            raise IndexError(
                f"position {position} needs logical block {logical} but "
                f"sequence {seq_id} has a block table of {len(tables[seq_id])}"
            )
    runs = _runs(seq_ids, positions)
    entries, flat_tables = [], []
    for s, start, n in runs:
        entries.append([n, start, start + n, len(flat_tables), len(tables[s]), 0])
        flat_tables.extend(tables[s])
    dev = pool.key_pool.device
    ints = torch.tensor([x for e in entries for x in e] + flat_tables, dtype=torch.int32).to(dev)
    ne = len(entries) * nat.ENTRY_INTS
    # the pass only needs slots: every entry reads dummy token ids from one zero run
    zeros = torch.zeros(max(n for _, _, n in runs), dtype=torch.int32, device=dev)
    packed = nat.ragged_pack(ints[:ne].view(-1, nat.ENTRY_INTS), ints[ne:], zeros, len(seq_ids), bs, 1,
                             _slot_bitmap(pool), pool.capacity_tokens)
    status = packed.status.tolist()
    if status[0] & nat.PACK_DUPLICATE_SLOT:
        raise ValueError(
            "two packed tokens map to the same pool slot; the step's "
            "sequence ids and positions overlap"
        )
    if status[0]:
        raise RuntimeError(f"ragged pack rejected the write index (status {status})")
    return packed.slot_mapping


class VarlenPackedCache(Cache):
    """Cache for a single fused forward pass over tokens from many sequences."""

    # a sampled pass's event record (engine telemetry); None: nothing is timed
    timer = None
    # the pass's attention writes each layer's new rows (see from_slot_mapping)
    write_in_attention = False

    def __init__(self, pool, num_layers: int, block_tables: Sequence[torch.Tensor], seq_ids: Sequence[int],
                 positions: Sequence[int]):
        if len(seq_ids) != len(positions):
            raise ValueError(f"{len(seq_ids)} seq_ids but {len(positions)} positions")
        if not seq_ids:
            raise ValueError("a packed pass needs at least one token")
        self.pool = pool
        self.block_tables = list(block_tables)
        self.seq_ids = list(seq_ids)
        self.positions = list(positions)
        self.num_tokens = len(seq_ids)
        self.hold_new_kv = False
        self.new_kv: List[Optional[Tuple[torch.Tensor, torch.Tensor]]] = [None] * num_layers
        self.write_index = build_write_index(pool, self.block_tables, self.seq_ids, self.positions)
        super().__init__(layers=[VarlenPackedCacheLayer(self, i) for i in range(num_layers)])

    @classmethod
    def from_slot_mapping(cls, pool, num_layers: int, slot_mapping: torch.Tensor,
                          write_in_attention: bool = False) -> "VarlenPackedCache":
        """Wrap a slot_mapping already built on the device by the ragged pack.
        With ``write_in_attention`` ``update`` writes nothing: the pass's
        attention binding carries the slot_mapping and every layer's
        attention launch writes the rows it is handed (one launch instead of
        a write and an attention per layer); only valid under such a binding."""
        self = cls.__new__(cls)
        self.pool = pool
        self.block_tables, self.seq_ids, self.positions = [], [], []
        self.num_tokens = int(slot_mapping.numel())
        self.hold_new_kv = False
        self.write_in_attention = bool(write_in_attention)
        self.new_kv = [None] * num_layers
        self.write_index = slot_mapping
        Cache.__init__(self, layers=[VarlenPackedCacheLayer(self, i) for i in range(num_layers)])
        return self

    @classmethod
    def verify(cls, pool, num_layers: int, num_tokens: int) -> "VarlenPackedCache":
        """A pass that writes nothing and keeps each layer's new K/V in
        ``new_kv`` (the speculative verify: candidates are attended in flight)."""
        self = cls.__new__(cls)
        self.pool = pool
        self.block_tables, self.seq_ids, self.positions = [], [], []
        self.num_tokens = num_tokens
        self.hold_new_kv = True
        self.new_kv = [None] * num_layers
        self.write_index = None
        Cache.__init__(self, layers=[VarlenPackedCacheLayer(self, i) for i in range(num_layers)])
        return self

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return 0

    def get_max_cache_shape(self) -> Optional[int]:
        return self.pool.capacity_tokens

    def reset(self) -> None:
        pass

    def __len__(self) -> int:
        return len(self.layers)
