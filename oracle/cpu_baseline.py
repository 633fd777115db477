"""The reference's CPU paths, ported to torch-on-CPU for the ``cpu_baseline``
legs of bench.py (test infrastructure only; never shipped, never the thing
measured on the GPU).

* ``decode_attention_cpu`` -- the reference's CPU decode-attention path: per
  sequence and layer one flat ``index_select`` of its context and a permute
  (``gather_kv``, memforge_ml/kernels/paged_gather.py:58-89, slot mapping
  from memforge_ml/runtime/kv_pool.py:92-130), KV heads repeated for
  grouped-query attention, and a plain softmax attention over the
  materialised context (``paged_attention_varlen_materialised``,
  memforge_ml/kernels/varlen_attention.py:291-395). Used for C5.
* ``operator_cpu`` -- the standalone operator ``PagedAttention.forward``
  (memforge_ml/models/paged_attention.py:69-141): per-block slices of the
  ``(blocks, heads, slots, dim)`` cache concatenated (``read_kv``), then
  ``softmax(q k^T * scale)`` in fp32 cast to the query dtype, times V. C1.
* ``varlen_cpu`` -- ``paged_attention_varlen_materialised`` for packed rows
  of many sequences (varlen_attention.py:291-395): per sequence one gather,
  scores for all its rows, the causal mask (key position <= row position),
  softmax, value product. C2 and C3.
* ``greedy_cpu`` -- greedy generation with a transformers model on the CPU,
  one request after another, each with its own DynamicCache: the CPU
  baseline of the end-to-end engine (C4), whose reference runs the same
  transformers forward (memforge_ml/runtime/continuous_engine.py:131-155
  takes ``device='cpu'``).

All compute in float32.
"""

from __future__ import annotations

import math
from typing import List, Sequence

import torch


def decode_attention_cpu(q: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
                         tables: Sequence[Sequence[int]], ctx: Sequence[int],
                         block_size: int) -> torch.Tensor:
    """q (B, Hq, D); pools (N, bs, Hkv, D) on the CPU. Returns (B, Hq, D)."""
    B, hq, d = q.shape
    n, bs, hkv, _ = key_pool.shape
    group = hq // hkv
    scale = 1.0 / math.sqrt(d)
    flat_k = key_pool.view(n * bs, hkv, d)
    flat_v = value_pool.view(n * bs, hkv, d)
    out = torch.empty_like(q)
    for b in range(B):
        c = int(ctx[b])
        pos = torch.arange(c)
        table = torch.as_tensor(tables[b][: (c + bs - 1) // bs], dtype=torch.long)
        flat = table[pos // block_size] * block_size + pos % block_size
        k = torch.index_select(flat_k, 0, flat).permute(1, 0, 2)  # (Hkv, c, D)
        v = torch.index_select(flat_v, 0, flat).permute(1, 0, 2)
        if group > 1:
            k = k.repeat_interleave(group, dim=0)
            v = v.repeat_interleave(group, dim=0)
        s = torch.einsum("hd,htd->ht", q[b], k) * scale
        w = torch.softmax(s, dim=-1)
        out[b] = torch.einsum("ht,htd->hd", w, v)
    return out


def operator_cpu(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                 block_table: Sequence[int], context_len: int) -> torch.Tensor:
    """One ``PagedAttention.forward`` call: query (1, H, q_len, D), caches
    (N, H, bs, D). Returns (1, q_len, H * D)."""
    bs = key_cache.shape[2]
    ks, vs = [], []
    for logical in range((context_len + bs - 1) // bs):
        take = min(bs, context_len - logical * bs)
        ks.append(key_cache[block_table[logical], :, :take, :])
        vs.append(value_cache[block_table[logical], :, :take, :])
    keys, values = torch.cat(ks, dim=1), torch.cat(vs, dim=1)
    q = query[0]
    scores = torch.matmul(q, keys.transpose(-1, -2)) * (1.0 / math.sqrt(q.shape[-1]))
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype)
    out = torch.matmul(probs, values)
    h, ql, d = out.shape
    return out.transpose(0, 1).reshape(1, ql, h * d)


def varlen_cpu(q: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
               tables: Sequence[Sequence[int]], cu_seqlens: Sequence[int], positions: Sequence[int],
               block_size: int) -> torch.Tensor:
    """Packed rows q (T, Hq, D); pools (N, bs, Hkv, D); the rows of sequence s
    are cu_seqlens[s]..cu_seqlens[s+1]-1. Returns (T, Hq, D)."""
    T, hq, d = q.shape
    n, bs, hkv, _ = key_pool.shape
    group = hq // hkv
    scale = 1.0 / math.sqrt(d)
    flat_k = key_pool.view(n * bs, hkv, d)
    flat_v = value_pool.view(n * bs, hkv, d)
    pos_all = torch.as_tensor(list(positions), dtype=torch.long)
    out = torch.empty((T, hq, d), dtype=torch.float32)
    for s in range(len(cu_seqlens) - 1):
        r0, r1 = int(cu_seqlens[s]), int(cu_seqlens[s + 1])
        rows_pos = pos_all[r0:r1]
        c = int(rows_pos.max()) + 1
        keys_at = torch.arange(c)
        table = torch.as_tensor(tables[s][: (c + bs - 1) // bs], dtype=torch.long)
        flat = table[keys_at // block_size] * block_size + keys_at % block_size
        k = torch.index_select(flat_k, 0, flat).permute(1, 0, 2)
        v = torch.index_select(flat_v, 0, flat).permute(1, 0, 2)
        if group > 1:
            k = k.repeat_interleave(group, dim=0)
            v = v.repeat_interleave(group, dim=0)
        scores = torch.einsum("rhd,htd->hrt", q[r0:r1], k) * scale
        visible = keys_at[None, :] <= rows_pos[:, None]
        scores = scores.masked_fill(~visible[None], float("-inf"))
        out[r0:r1] = torch.einsum("hrt,htd->rhd", torch.softmax(scores, dim=-1), v)
    return out


@torch.no_grad()
def greedy_cpu(model, prompts: Sequence[Sequence[int]], new_tokens: int) -> List[List[int]]:
    """Greedy generation on the CPU, one request after another."""
    from transformers.cache_utils import DynamicCache

    results = []
    for prompt in prompts:
        cache = DynamicCache()
        out = model(input_ids=torch.tensor([list(prompt)]), past_key_values=cache, use_cache=True)
        toks: List[int] = []
        while len(toks) < new_tokens:
            toks.append(int(out.logits[0, -1].argmax()))
            if len(toks) < new_tokens:
                out = model(input_ids=torch.tensor([[toks[-1]]]), past_key_values=cache, use_cache=True)
        results.append(toks)
    return results
