"""Paged / varlen attention in float64 (test infrastructure only).

The semantics are those of ``reference_varlen_attention``
(memforge_ml/kernels/varlen_attention.py:238-288): packed query row r of
sequence ``seq_ids[r]`` attends, per query head, to that sequence's keys at
positions 0..positions[r] inclusive, read through its block table
(``table[p // bs]``, slot ``p % bs``), with grouped-query heads sharing a KV
head by ``repeat_interleave`` (query head qh reads kv head qh // G). Scores are
``q . k * scale`` with scale defaulting to 1/sqrt(D) (varlen_attention.py:334).

The computation is vectorised per sequence (one gather of its visible keys,
one masked softmax) rather than per row, which is the same function as the
row-by-row form and lets the oracle finish in seconds at the benchmark
shapes.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np


def _gather_keys(pool_layer: np.ndarray, table: Sequence[int], n: int, block_size: int) -> np.ndarray:
    """Keys 0..n-1 of one sequence from a (N, bs, Hkv, D) pool layer."""
    pos = np.arange(n)
    phys = np.asarray(table, dtype=np.int64)[pos // block_size]
    return pool_layer[phys, pos % block_size]  # (n, Hkv, D)


def varlen_attention(query: np.ndarray, key_pool: np.ndarray, value_pool: np.ndarray,
                     block_tables: Sequence[Sequence[int]], seq_ids: Sequence[int],
                     positions: Sequence[int], block_size: int, scale: Optional[float] = None,
                     pool_lens: Optional[Sequence[int]] = None,
                     new_k: Optional[np.ndarray] = None, new_v: Optional[np.ndarray] = None,
                     new_rows: Optional[Sequence[Sequence[int]]] = None) -> np.ndarray:
    """Packed varlen attention, float64.

    query: (Hq, T, D); key_pool/value_pool: one layer, (N, bs, Hkv, D).
    In-flight keys (the verify pass, memforge_ml/runtime/batched_speculative.py:
    645-728, where the candidates' K/V are attended without being written to the
    pool): when ``pool_lens`` is given, sequence s's key at position
    p >= pool_lens[s] is row ``new_rows[s][p - pool_lens[s]]`` of new_k/new_v
    ((T, Hkv, D)). Returns (Hq, T, D) float64.
    """
    hq, total, d = query.shape
    hkv = key_pool.shape[2]
    if hq % hkv:
        raise ValueError(f"{hq} query heads is not a multiple of {hkv} kv heads")
    group = hq // hkv
    scale = scale if scale is not None else 1.0 / math.sqrt(d)
    q64 = query.astype(np.float64)
    out = np.zeros((hq, total, d), dtype=np.float64)
    rows_of = {}
    for r, s in enumerate(seq_ids):
        rows_of.setdefault(s, []).append(r)
    for s, rows in rows_of.items():
        rows = np.asarray(rows)
        pos = np.asarray([positions[r] for r in rows], dtype=np.int64)
        n = int(pos.max()) + 1
        if pool_lens is None:
            keys = _gather_keys(key_pool, block_tables[s], n, block_size).astype(np.float64)
            vals = _gather_keys(value_pool, block_tables[s], n, block_size).astype(np.float64)
        else:
            pl = min(pool_lens[s], n)
            kp = _gather_keys(key_pool, block_tables[s], pl, block_size).astype(np.float64)
            vp = _gather_keys(value_pool, block_tables[s], pl, block_size).astype(np.float64)
            extra = list(new_rows[s][: n - pl])
            keys = np.concatenate([kp, new_k[extra].astype(np.float64)], axis=0)
            vals = np.concatenate([vp, new_v[extra].astype(np.float64)], axis=0)
        keys = np.repeat(keys, group, axis=1)  # (n, Hq, D)
        vals = np.repeat(vals, group, axis=1)
        q = q64[:, rows, :]  # (Hq, R, D)
        scores = np.einsum("hrd,thd->hrt", q, keys) * scale
        visible = np.arange(n)[None, :] <= pos[:, None]  # (R, n)
        scores = np.where(visible[None], scores, -np.inf)
        scores -= scores.max(axis=-1, keepdims=True)
        w = np.exp(scores)
        w /= w.sum(axis=-1, keepdims=True)
        out[:, rows, :] = np.einsum("hrt,thd->hrd", w, vals)
    return out


def paged_operator(query: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                   block_table: Sequence[int], context_len: int, scale: Optional[float] = None,
                   round_probs=None) -> np.ndarray:
    """The standalone operator ``PagedAttention.forward``
    (memforge_ml/models/paged_attention.py:108-141) in float64.

    query (1, H, q_len, D); caches (N, H, bs, D). No causal mask and no GQA:
    every query row attends to all ``context_len`` keys. ``scale`` follows
    ``self.scale or 1/sqrt(D)`` (so 0.0 and None both mean the default).
    ``round_probs`` optionally rounds the softmax to the query dtype before the
    value product, as ``.to(query.dtype)`` does at paged_attention.py:133.
    Returns (1, q_len, H*D).
    """
    _, h, q_len, d = query.shape
    scale = scale or (1.0 / math.sqrt(d))
    bs = key_cache.shape[2]
    nblocks = (context_len + bs - 1) // bs
    ks, vs = [], []
    for logical in range(nblocks):
        phys = block_table[logical]
        take = min(bs, context_len - logical * bs)
        ks.append(key_cache[phys, :, :take, :])
        vs.append(value_cache[phys, :, :take, :])
    keys = np.concatenate(ks, axis=1).astype(np.float64)  # (H, ctx, D)
    vals = np.concatenate(vs, axis=1).astype(np.float64)
    q = query[0].astype(np.float64)  # (H, q_len, D)
    scores = np.einsum("hqd,htd->hqt", q, keys) * scale
    scores -= scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    if round_probs is not None:
        p = round_probs(p)
    out = np.einsum("hqt,htd->hqd", p, vals)  # (H, q_len, D)
    return out.transpose(1, 0, 2).reshape(1, q_len, h * d)
