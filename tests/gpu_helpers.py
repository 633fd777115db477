"""Helpers shared by the GPU parity tests: build device inputs from logical
(per-sequence) descriptions and call the C ABI through ``memforge_amd._native``."""

from __future__ import annotations

from collections import OrderedDict
from typing import List, Optional, Sequence

import numpy as np
import torch

from memforge_amd import _native as nat


def to_np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy()


def random_tables(gen: torch.Generator, num_blocks: int, lengths: Sequence[int], block_size: int) -> List[List[int]]:
    """Non-contiguous tables: one seeded permutation of the pool, consumed in order."""
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    tables, k = [], 0
    for n in lengths:
        nb = (n + block_size - 1) // block_size
        tables.append(perm[k:k + nb])
        k += nb
    assert k <= num_blocks, "pool too small for the requested contexts"
    return tables


def pad_tables(tables: Sequence[Sequence[int]], device) -> torch.Tensor:
    width = max(1, max((len(t) for t in tables), default=1))
    out = np.zeros((max(1, len(tables)), width), dtype=np.int32)
    for i, t in enumerate(tables):
        out[i, : len(t)] = np.asarray(t, dtype=np.int32)
    return torch.from_numpy(out).to(device)


def gpu_varlen(q: torch.Tensor, kpool: torch.Tensor, vpool: torch.Tensor,
               tables: Sequence[Sequence[int]], seq_ids: Sequence[int], positions: Sequence[int],
               scale: Optional[float] = None, partition_tiles: int = 0,
               pool_lens: Optional[Sequence[int]] = None, new_k: Optional[torch.Tensor] = None,
               new_v: Optional[torch.Tensor] = None, layout: str = "bshd",
               fused: bool = False) -> torch.Tensor:
    """Varlen paged attention through the C ABI.

    q: (Hq, T, D) on the device; pools one layer (N, bs, Hkv, D) ("bshd") or
    (N, Hkv, bs, D) ("bhsd"). Rows may be packed in any order; they are
    grouped by sequence through row_map. For a verify pass, ``pool_lens[s]``
    splits sequence s's keys between the pool and the in-flight rows
    ``new_k``/``new_v`` ((T, Hkv, D)), which are that sequence's own rows in
    position order. Returns (Hq, T, D).
    """
    dev = q.device
    hq, T, d = q.shape
    pool = nat.PoolView.from_bshd(kpool, vpool) if layout == "bshd" else nat.PoolView.from_bhsd(kpool, vpool)
    hkv = pool.num_heads
    groups: "OrderedDict[int, List[int]]" = OrderedDict()
    for r, s in enumerate(seq_ids):
        groups.setdefault(s, []).append(r)
    seqs = list(groups)
    row_map: List[int] = []
    cu = [0]
    kv_lens = []
    for s in seqs:
        rows = sorted(groups[s], key=lambda r: positions[r])
        row_map.extend(rows)
        cu.append(len(row_map))
        kv_lens.append(max(positions[r] for r in rows) + 1)
    bt = pad_tables([tables[s] for s in seqs], dev)
    plan = nat.plan_attention(cu, kv_lens, hq, hkv, d, q.dtype, dev, partition_tiles)
    out = torch.full((T, hq, d), float("nan"), dtype=q.dtype, device=dev)
    pl = None
    if pool_lens is not None:
        pl = torch.tensor([pool_lens[s] for s in seqs], dtype=torch.int32, device=dev)
    nat.paged_attention(
        q.permute(1, 0, 2), out, pool, bt,
        torch.tensor(cu, dtype=torch.int32, device=dev),
        torch.tensor(kv_lens, dtype=torch.int32, device=dev),
        torch.tensor(list(positions), dtype=torch.int64, device=dev),
        plan, scale if scale is not None else 1.0 / float(np.sqrt(d)), hkv,
        row_map=torch.tensor(row_map, dtype=torch.int32, device=dev),
        pool_lens=pl, new_k_rows=new_k, new_v_rows=new_v, fused_merge=fused,
    )
    return out.permute(1, 0, 2)


def gpu_decode_slices(q: torch.Tensor, kpool: torch.Tensor, vpool: torch.Tensor,
                      tables: Sequence[Sequence[int]], positions: Sequence[int], num_cus: int,
                      kv_lens: Optional[Sequence[int]] = None, scale: Optional[float] = None):
    """One decode row per sequence (row s is sequence s) through a decode
    slice plan made for a GPU of ``num_cus`` compute units -- a small count
    makes few waves per round, so even a small batch is cut into several
    slices and split sequences. q: (Hq, B, D); pools one layer
    (N, 16, Hkv, D). Returns ((Hq, B, D) output, plan)."""
    dev = q.device
    hq, B, d = q.shape
    pool = nat.PoolView.from_bshd(kpool, vpool)
    hkv = pool.num_heads
    cu = list(range(B + 1))
    kvl = list(kv_lens) if kv_lens is not None else [p + 1 for p in positions]
    made = nat.plan_slices_host(cu, kvl, hq, hkv, d, q.dtype, num_cus, min_tiles=0)
    assert made is not None, "not a decode step"
    items, merges, counts = made
    dev_items, dev_merges = nat.upload(nat.plan_upload_parts(items, merges), dev)
    plan = nat.plan_from_parts(items, merges, counts, dev_items, dev_merges, sliced=True)
    out = torch.full((B, hq, d), float("nan"), dtype=q.dtype, device=dev)
    nat.paged_attention(
        q.permute(1, 0, 2), out, pool, pad_tables(tables, dev),
        torch.tensor(cu, dtype=torch.int32, device=dev), torch.tensor(kvl, dtype=torch.int32, device=dev),
        torch.tensor(list(positions), dtype=torch.int64, device=dev),
        plan, scale if scale is not None else 1.0 / float(np.sqrt(d)), hkv,
    )
    return out.permute(1, 0, 2), plan


def assert_close_bf16(got: np.ndarray, want: np.ndarray, max_abs: float = 2e-2, mean_rel: float = 1e-2):
    err = np.abs(got - want)
    assert np.isfinite(got).all(), "non-finite output"
    assert err.max() <= max_abs, f"max-abs {err.max():.3e} > {max_abs}"
    rel = err.mean() / max(np.abs(want).mean(), 1e-30)
    assert rel <= mean_rel, f"mean-rel {rel:.3e} > {mean_rel}"
