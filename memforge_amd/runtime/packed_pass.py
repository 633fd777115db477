"""One eager packed varlen pass of a model over a paged pool.

Every contributing sequence adds a run of query tokens at consecutive
positions ``start .. start + len - 1`` whose K/V are written through its block
table. The descriptors, tables, token ids and attention plan are staged in
pinned memory and cross PCIe in one copy; the ragged-pack kernel builds token ids, positions,
slot_mapping, cu_seqlens and padded tables on the device; each layer's
attention is one launch that writes the layer's new K/V through slot_mapping
and attends with the pool read in place (the new keys read from the rows
themselves) -- or, unfused, the KV-write kernel in the cache update followed
by the attention launch. This is the reference's fused varlen step
(memforge_ml/runtime/continuous_engine.py:782-905) with the gather, the padding
and the Python list building moved onto the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence

import numpy as np
import torch

from memforge_amd import _native as nat
from memforge_amd.kernels import attention_backend
from memforge_amd.runtime.varlen_cache import VarlenPackedCache


@dataclass
class PackedPassResult:
    logits: torch.Tensor      # (len(keep_rows), vocab), rows in keep_rows order
    cu_seqlens: np.ndarray    # (B + 1,) host prefix sums of the query lengths
    kv_lens: List[int]        # keys each sequence's attention read
    num_tokens: int           # packed query rows
    layers_used: int          # layers whose attention ran through the varlen kernel


@torch.no_grad()
def packed_forward(model, pool, tokens: Sequence[Sequence[int]], starts: Sequence[int],
                   tables: Sequence[Sequence[int]], keep_rows: Sequence[int], timer=None,
                   fuse_kv_write: bool = True) -> PackedPassResult:
    """Run ``model`` once over every sequence's ``tokens`` (written at
    ``starts[i]`` onward through ``tables[i]``) and return the logits of the
    packed rows ``keep_rows``. Raises IndexError when a run does not fit its
    table, and RuntimeError when a layer did not use the varlen kernel. With
    ``timer`` (a sampled pass's event record) every layer's KV write and
    attention launch is bracketed by HIP events. With ``fuse_kv_write`` each
    layer's KV write rides in its attention launch (mf_paged_attention_kv_write)
    instead of running as a launch of its own."""
    bs = pool.block_size
    spec = pool.spec
    B = len(tokens)
    q_lens = [len(t) for t in tokens]
    kv_lens = [int(s) + q for s, q in zip(starts, q_lens)]
    for i, (kv, t) in enumerate(zip(kv_lens, tables)):
        if kv > len(t) * bs:
            raise IndexError(f"entry {i} needs {kv} slots but its block table has {len(t)} blocks of {bs}")
    max_blocks = max(len(t) for t in tables)
    T = int(sum(q_lens))
    cu = np.zeros(B + 1, dtype=np.int64)
    np.cumsum(q_lens, out=cu[1:])

    ent = np.empty((B, nat.ENTRY_INTS), dtype=np.int32)
    t_off = np.zeros(B, dtype=np.int64)
    t_off[1:] = np.cumsum([len(t) for t in tables])[:-1]
    ent[:, 0] = q_lens
    ent[:, 1] = starts
    ent[:, 2] = kv_lens
    ent[:, 3] = t_off
    ent[:, 4] = [len(t) for t in tables]
    ent[:, 5] = cu[:-1]
    flat_tables = np.fromiter((b for t in tables for b in t), dtype=np.int32)
    flat_tokens = np.fromiter((tok for run in tokens for tok in run), dtype=np.int32)
    nat.check_pack_entries(ent, flat_tables, len(flat_tokens), T, pool.num_blocks)
    items, merges, counts = nat.plan_attention_host(cu.tolist(), kv_lens, model.config.num_attention_heads,
                                                    spec.num_kv_heads, spec.head_dim, pool.key_pool.dtype)
    keep_np = np.asarray(list(keep_rows), dtype=np.int64)
    # descriptors, tables, tokens, the attention plan and the kept rows cross
    # to the device in one copy
    d_ent, d_tables, d_tokens, d_items, d_merges, keep = nat.upload(
        [ent, flat_tables, flat_tokens, *nat.plan_upload_parts(items, merges), keep_np], spec.device)
    packed = nat.ragged_pack(d_ent, d_tables, d_tokens, T, bs, max_blocks, num_slots=pool.capacity_tokens)
    attn_plan = nat.plan_from_parts(items, merges, counts, d_items, d_merges)
    meta = {"block_tables": packed.block_tables, "cu_seqlens": packed.cu_seqlens,
            "kv_lens": packed.kv_lens, "positions": packed.positions, "row_map": None,
            "plan": attn_plan}
    fuse = fuse_kv_write and pool.key_pool.dtype == model.dtype
    binding = attention_backend._VarlenBinding.from_packed(pool, meta, T,
                                                           write_slots=packed.slot_mapping if fuse else None)
    cache = VarlenPackedCache.from_slot_mapping(pool, spec.num_layers, packed.slot_mapping, write_in_attention=fuse)
    binding.timer = cache.timer = timer
    with attention_backend.backend_enabled_on(model) as routed:
        if not routed:
            raise RuntimeError("the packed pass needs the attention registry")
        with attention_backend.bind_varlen(binding):
            out = model(input_ids=packed.token_ids.view(1, T), position_ids=packed.positions.view(1, T),
                        past_key_values=cache, use_cache=True, logits_to_keep=keep)
    if binding.used != spec.num_layers:
        raise RuntimeError(f"packed pass: {binding.used} of {spec.num_layers} layers used the kernel")
    return PackedPassResult(out.logits[0], cu, kv_lens, T, binding.used)
