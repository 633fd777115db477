"""Hugging Face attention-registry backend ``memforge_paged`` on the MI355X.

Same registry name, bindings and routing as the reference
(memforge_ml/kernels/attention_backend.py:54-465): an unmodified HF model is
pointed at ``memforge_paged``; the engine binds the pool and the pass's
addressing in a thread-local slot for the duration of a forward (thread-local,
not contextvars, because the server steps the engine in an executor thread);
``paged_attention_forward`` then serves every layer with the varlen HIP kernel
reading K/V straight out of the pool.

Routing:
  * a varlen binding (packed multi-sequence pass) always takes the kernel and
    raises on a shape mismatch -- a fallback would attend across sequences;
  * a single-sequence binding takes the kernel for one query position under a
    permissive mask with a non-empty context, and otherwise falls back to eager
    attention over the key/value it was handed (prefill, padded batches);
  * no binding: eager attention.

The mask registry entry builds nothing while a varlen binding is active (the
kernel masks from positions) and otherwise aliases transformers' eager mask
builder, so a fallback still gets a causal mask.
"""

from __future__ import annotations

import math
import threading
from contextlib import contextmanager
from typing import Any, List, Optional, Sequence, Tuple

import numpy as np
import torch

from memforge_amd import _native as nat
from memforge_amd.kernels._varlen import as_table_list, padded_tables_host, run_varlen
from memforge_amd.kernels.block_attention import paged_attention_blockwise

BACKEND_NAME = "memforge_paged"

_state = threading.local()


class _Binding:
    """Pool + one sequence's cache; the context length is read from the cache
    at attention time, after this step's key was written (attention_backend.py:59-87)."""

    __slots__ = ("pool", "cache", "used", "fallbacks")

    def __init__(self, pool, cache):
        self.pool = pool
        self.cache = cache
        self.used = 0
        self.fallbacks = 0

    @property
    def block_table(self) -> torch.Tensor:
        return self.cache.block_table_tensor_cached()

    @property
    def context_length(self) -> int:
        return self.cache.position


class _VarlenBinding:
    """Addressing for a packed multi-sequence pass (attention_backend.py:90-122).

    Built from per-row lists (the reference's constructor) or from an already
    packed step (``from_packed``, the engine). The device metadata -- grouped
    row order, cu_seqlens, kv_lens, positions, padded block tables and the
    attention work plan -- is built once and shared by every layer.
    ``pool_lens`` turns the pass into a verify pass: keys at or above
    pool_lens[s] are the layer's in-flight key/value rows, not pool slots. A
    host sequence is uploaded with the rest of the metadata; a device tensor
    must already be in the grouped sequence order.
    """

    __slots__ = ("pool", "block_tables", "seq_ids", "positions", "block_wise", "used", "_meta",
                 "pool_lens", "num_rows", "timer", "write_slots")

    def __init__(self, pool, block_tables, seq_ids, positions, block_wise=False, pool_lens=None):
        self.pool = pool
        self.block_tables = list(block_tables)
        self.seq_ids = list(seq_ids)
        self.positions = list(positions)
        self.block_wise = bool(block_wise)
        self.used = 0
        self._meta = None
        self.pool_lens = pool_lens
        self.num_rows = len(self.seq_ids)
        self.timer = None  # a sampled pass's event record (engine telemetry)
        self.write_slots = None

    @classmethod
    def from_packed(cls, pool, meta: dict, num_rows: int, pool_lens: Optional[torch.Tensor] = None,
                    write_slots: Optional[torch.Tensor] = None):
        """A prepared binding. ``write_slots`` (the step's slot_mapping, with a
        cache made by ``VarlenPackedCache.from_slot_mapping(...,
        write_in_attention=True)``): every layer's attention launch also writes
        the new K/V rows it is handed into the pool and reads each sequence's
        new keys from those rows (the step's rows are every sequence's new
        tokens, ending its context)."""
        b = cls.__new__(cls)
        b.pool = pool
        b.block_tables = []
        b.seq_ids = []
        b.positions = []
        b.block_wise = False
        b.used = 0
        b._meta = meta
        b.pool_lens = pool_lens
        b.num_rows = num_rows
        b.timer = None
        b.write_slots = write_slots
        return b

    def meta(self, num_q_heads: int, head_dim: int, dtype: torch.dtype, device) -> dict:
        if self._meta is not None:
            return self._meta
        tables = [as_table_list(t) for t in self.block_tables]
        groups, order = {}, []
        for r, s in enumerate(self.seq_ids):
            if s < 0 or s >= len(tables):
                raise IndexError(f"seq_id {s} has no block table (got {len(tables)})")
            if s not in groups:
                groups[s] = []
                order.append(s)
            groups[s].append(r)
        row_map, cu, kvl = [], [0], []
        for s in order:
            rows = sorted(groups[s], key=lambda r: self.positions[r])
            row_map.extend(rows)
            cu.append(len(row_map))
            kvl.append(max(self.positions[r] for r in rows) + 1)
            needed = (kvl[-1] + self.pool.block_size - 1) // self.pool.block_size
            if needed > len(tables[s]):
                raise IndexError(
                    f"sequence {s} reads up to position {kvl[-1] - 1}, needing {needed} blocks, "
                    f"but its block table has {len(tables[s])} entries"
                )
        identity = row_map == list(range(len(row_map)))
        # a large decode step on 16-token blocks runs as one round of slices
        sliceable = identity and self.pool_lens is None and self.pool.block_size == 16
        items, merges, counts, sliced = nat.plan_host(cu, kvl, num_q_heads, self.pool.spec.num_kv_heads,
                                                      head_dim, dtype, device, decode_slices=sliceable)
        # everything the launch reads crosses to the device in one copy
        parts = [padded_tables_host([tables[s] for s in order]), *nat.plan_upload_parts(items, merges),
                 np.asarray(cu + kvl, dtype=np.int32), np.asarray(list(self.positions), dtype=np.int64)]
        if not identity:
            parts.append(np.asarray(row_map, dtype=np.int32))
        host_pool_lens = self.pool_lens is not None and not isinstance(self.pool_lens, torch.Tensor)
        if host_pool_lens:
            parts.append(np.asarray([int(self.pool_lens[s]) for s in order], dtype=np.int32))
        dev = nat.upload(parts, device)
        if host_pool_lens:
            self.pool_lens = dev[-1]
        plan = nat.plan_from_parts(items, merges, counts, dev[1], dev[2], sliced)
        self._meta = {
            "block_tables": dev[0],
            "cu_seqlens": dev[3][: len(cu)],
            "kv_lens": dev[3][len(cu):],
            "positions": dev[4],
            "row_map": None if identity else dev[5],
            "plan": plan,
        }
        return self._meta


def _current() -> Optional[_Binding]:
    return getattr(_state, "binding", None)


def _current_varlen() -> Optional[_VarlenBinding]:
    return getattr(_state, "varlen", None)


@contextmanager
def paged_attention_context(pool, cache):
    """Bind the pool and one sequence's cache for the enclosed forward; nests."""
    previous = _current()
    binding = _Binding(pool, cache)
    _state.binding = binding
    try:
        yield binding
    finally:
        _state.binding = previous


@contextmanager
def varlen_attention_context(pool, block_tables, seq_ids, positions, block_wise=False):
    """Bind a packed multi-sequence pass for the enclosed forward; nests."""
    previous = _current_varlen()
    binding = _VarlenBinding(pool, block_tables, seq_ids, positions, block_wise=block_wise)
    _state.varlen = binding
    try:
        yield binding
    finally:
        _state.varlen = previous


@contextmanager
def bind_varlen(binding: _VarlenBinding):
    """Bind a prepared varlen binding (the engine's pre-packed steps)."""
    previous = _current_varlen()
    _state.varlen = binding
    try:
        yield binding
    finally:
        _state.varlen = previous


def _mask_is_permissive(attention_mask: Optional[torch.Tensor]) -> bool:
    if attention_mask is None:
        return True
    if attention_mask.dtype == torch.bool:
        return bool(attention_mask.all())
    return bool(torch.all(attention_mask == 0))


def _varlen_forward(module, query, key, value, scaling, binding: _VarlenBinding) -> torch.Tensor:
    if query.shape[0] != 1 or query.shape[2] != binding.num_rows:
        raise ValueError(
            f"varlen pass expected one packed row of {binding.num_rows} tokens, got {tuple(query.shape)}"
        )
    _, hq, total, d = query.shape
    pool = binding.pool
    dtype = pool.key_pool.dtype
    meta = binding.meta(hq, d, dtype, query.device)
    q_rows = query[0].to(dtype).permute(1, 0, 2)
    out = torch.empty((1, total, hq, d), dtype=dtype, device=query.device)
    layer = module.layer_idx
    nk = nv = None
    if binding.pool_lens is not None:
        nk = key[0].to(dtype).permute(1, 0, 2)
        nv = value[0].to(dtype).permute(1, 0, 2)
    timer = binding.timer
    began = timer.start(layer) if timer is not None else None
    if binding.write_slots is not None:
        # the launch reads K and V rows with one pair of strides
        wk, wv = key[0].to(dtype).permute(1, 0, 2), value[0].to(dtype).permute(1, 0, 2)
        if not nat.same_layout(wk, wv):
            wk, wv = wk.contiguous(), wv.contiguous()
        nat.paged_attention_kv_write(
            q_rows, out[0], pool.layer_view(layer), meta["block_tables"], meta["cu_seqlens"],
            meta["kv_lens"], meta["positions"], meta["plan"],
            scaling if scaling is not None else 1.0 / math.sqrt(d), pool.spec.num_kv_heads, wk, wv,
            binding.write_slots,
        )
        if timer is not None:
            timer.stop("attention_kv_write", began)
        return out.to(query.dtype)
    nat.paged_attention(
        q_rows, out[0], pool.layer_view(layer), meta["block_tables"], meta["cu_seqlens"],
        meta["kv_lens"], meta["positions"], meta["plan"],
        scaling if scaling is not None else 1.0 / math.sqrt(d), pool.spec.num_kv_heads,
        row_map=meta["row_map"], pool_lens=binding.pool_lens, new_k_rows=nk, new_v_rows=nv,
    )
    if timer is not None:
        timer.stop("attention", began)
    return out.to(query.dtype)


def paged_attention_forward(module: Any, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            attention_mask: Optional[torch.Tensor] = None, scaling: Optional[float] = None,
                            dropout: float = 0.0, **kwargs: Any) -> Tuple[torch.Tensor, None]:
    """The function registered as ``memforge_paged`` (attention_backend.py:195-272).
    Returns ``(batch, q_len, heads, head_dim)`` as transformers expects."""
    varlen = _current_varlen()
    if varlen is not None:
        varlen.used += 1
        return _varlen_forward(module, query, key, value, scaling, varlen), None

    binding = _current()
    single_query = query.shape[0] == 1 and query.shape[2] == 1
    if binding is not None and single_query and _mask_is_permissive(attention_mask) and binding.context_length > 0:
        binding.used += 1
        out = paged_attention_blockwise(query, binding.pool.key_pool, binding.pool.value_pool,
                                        module.layer_idx, binding.block_table, binding.context_length,
                                        binding.pool.block_size, scale=scaling)
        return _to_attention_output_layout(out), None

    if binding is not None:
        binding.fallbacks += 1
    return _eager_attention(module, query, key, value, attention_mask, scaling), None


def _to_attention_output_layout(attn_output: torch.Tensor) -> torch.Tensor:
    """(batch, heads, q_len, head_dim) -> (batch, q_len, heads, head_dim) (attention_backend.py:275-292)."""
    return attn_output.transpose(1, 2).contiguous()


def _eager_attention(module, query, key, value, attention_mask, scaling) -> torch.Tensor:
    """Plain attention with grouped-query expansion for unbound calls
    (attention_backend.py:295-328); softmax in fp32."""
    num_heads, head_dim = query.shape[1], query.shape[3]
    scaling = scaling if scaling is not None else 1.0 / math.sqrt(head_dim)
    group = num_heads // key.shape[1]
    k, v = key, value
    if group > 1:
        k = k.repeat_interleave(group, dim=1)
        v = v.repeat_interleave(group, dim=1)
    scores = torch.matmul(query, k.transpose(2, 3).contiguous()) * scaling
    if attention_mask is not None:
        scores = scores + attention_mask[:, :, :, : k.shape[-2]]
    else:
        scores = _apply_implicit_causal_mask(scores)
    weights = torch.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype)
    return _to_attention_output_layout(torch.matmul(weights, v))


def _apply_implicit_causal_mask(scores: torch.Tensor) -> torch.Tensor:
    """Right-aligned causality when transformers passes no mask
    (attention_backend.py:331-357)."""
    q_len, kv_len = scores.shape[-2], scores.shape[-1]
    if q_len <= 1:
        return scores
    causal = torch.ones(q_len, kv_len, dtype=torch.bool, device=scores.device).tril(diagonal=kv_len - q_len)
    return scores.masked_fill(~causal, torch.finfo(scores.dtype).min)


def _mask_builder(*args, **kwargs):
    """Mask registry entry: nothing to build for a packed pass (the kernel masks
    from positions), eager's mask otherwise."""
    if _current_varlen() is not None:
        return None
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS

    return ALL_MASK_ATTENTION_FUNCTIONS["eager"](*args, **kwargs)


def register() -> bool:
    """Add the backend and its mask builder to transformers' registries;
    idempotent, False when the registries are missing (attention_backend.py:360-401)."""
    try:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    except ImportError:
        return False
    try:
        if BACKEND_NAME not in ALL_ATTENTION_FUNCTIONS:
            ALL_ATTENTION_FUNCTIONS[BACKEND_NAME] = paged_attention_forward
    except Exception:
        return False
    try:
        from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS

        if BACKEND_NAME not in ALL_MASK_ATTENTION_FUNCTIONS:
            ALL_MASK_ATTENTION_FUNCTIONS[BACKEND_NAME] = _mask_builder
    except Exception:
        return False
    return True


def enable_on(model) -> bool:
    """Point a model at this backend permanently; False if registration failed."""
    if not register():
        return False
    for holder in _attn_config_holders(model):
        holder._attn_implementation = BACKEND_NAME
    return True


def is_enabled_on(model) -> bool:
    return getattr(model.config, "_attn_implementation", None) == BACKEND_NAME


def _attn_config_holders(model) -> List[Any]:
    holders = [model.config]
    for attr in ("text_config", "decoder"):
        sub = getattr(model.config, attr, None)
        if sub is not None and hasattr(sub, "_attn_implementation"):
            holders.append(sub)
    return holders


@contextmanager
def backend_enabled_on(model):
    """Route ``model``'s attention through this backend for the enclosed block
    only; yields False and changes nothing without the registries
    (attention_backend.py:436-465)."""
    if not register():
        yield False
        return
    holders = _attn_config_holders(model)
    previous = [getattr(h, "_attn_implementation", None) for h in holders]
    for holder in holders:
        holder._attn_implementation = BACKEND_NAME
    try:
        yield True
    finally:
        for holder, original in zip(holders, previous):
            holder._attn_implementation = original
