"""The reference's CPU decode-attention path, ported to torch-on-CPU for the
``cpu_baseline`` leg of bench.py (test infrastructure only; never shipped).

Per sequence and layer the reference reads its context out of the pool with
one flat ``index_select`` and a permute (``gather_kv``,
memforge_ml/kernels/paged_gather.py:58-89, slot mapping from
memforge_ml/runtime/kv_pool.py:92-130), repeats KV heads for grouped-query
attention and runs a plain softmax attention over the materialised context
(``paged_attention_varlen_materialised``, memforge_ml/kernels/
varlen_attention.py:291-395). That is exactly what this does, in float32.
"""

from __future__ import annotations

import math
from typing import Sequence

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
