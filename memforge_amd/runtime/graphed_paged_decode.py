"""HIP-graphed paged decode step.

Same class and step contract as the reference's GraphedPagedDecoder
(memforge_ml/runtime/graphed_paged_decode.py:112-266): decode one token for
each of B sequences against the paged pool as one graph replay, with
everything that varies between steps held in device buffers that the graph
reads. The reference graphs a gather of every context plus the model's sdpa
attention; here the graph holds the packed varlen pass itself -- the ragged
pack and, per layer, one attention launch that writes the layer's new K/V
through slot_mapping and attends with the pool read in place -- so nothing is
gathered or padded by context length.

What makes the attention capturable is mf_paged_attention_counted: its grids
are sized by a capacity fixed at capture time, and the live item and merge
counts are read from device memory, so each step's plan -- made on the host
from that step's context lengths -- is swapped in by a copy before the
replay. When the longest reachable context fits one cooperative unit (four
waves of 128 key tiles), every step's plan is made merge-free -- at most four
items per (sequence, kv head), no split-K partials -- and the graph holds no
merge launch at all; otherwise the capacity is every sequence at the longest
context split into the smallest partitions the planner uses.

Batches are bucketed to powers of two. Padding rows are empty entries (no
keys, slot -1): they write nothing and attend to nothing, and their logits
are never read.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Sequence

import numpy as np
import torch

from memforge_amd import _native as nat
from memforge_amd.kernels import attention_backend
from memforge_amd.runtime.varlen_cache import VarlenPackedCache

# smallest split-K partition (16-key tiles) the planner chooses by itself
_MIN_PARTITION_TILES = 4


def split_plan_capacity(batch: int, num_kv_heads: int, max_blocks: int, block_size: int, head_dim: int):
    """(narrow items, wide items, merges, partial floats) that hold any decode
    plan of ``batch`` single-row sequences whose tables have at most
    ``max_blocks`` blocks of ``block_size`` keys."""
    tiles = math.ceil(max_blocks * block_size / 16)
    cap_items = batch * num_kv_heads * (math.ceil(tiles / _MIN_PARTITION_TILES) + 4) + 4
    floats = cap_items * 16 * (max(head_dim, 32) + 2)
    return cap_items, 0, batch * num_kv_heads, floats


class _Bucket:
    """Static buffers and the captured graph of one batch size."""

    def __init__(self, owner: "GraphedPagedDecoder", b: int):
        dev = owner.device
        mb = owner.max_blocks
        self.b = b
        self.inputs = torch.zeros(b * nat.ENTRY_INTS + b * mb + b, dtype=torch.int32, device=dev)
        self.entries = self.inputs[: b * nat.ENTRY_INTS].view(b, nat.ENTRY_INTS)
        self.tables = self.inputs[b * nat.ENTRY_INTS: b * nat.ENTRY_INTS + b * mb]
        self.tokens = self.inputs[b * nat.ENTRY_INTS + b * mb:]
        self.host = torch.zeros(self.inputs.numel(), dtype=torch.int32).pin_memory()
        self.packed = nat.PackedStep.allocate(b, b, mb, dev)
        hkv = owner.pool.spec.num_kv_heads
        if owner.merge_free:
            # one single item or one four-wave unit per (sequence, kv head),
            # the single items padded to whole workgroups; nothing to merge
            self.plan = nat.CountedPlan(4 * b * hkv + 4, 0, 0, 0, dev)
        else:
            # a (sequence, kv head) of T 16-key tiles is one item when T <= P,
            # else four per unit of at most 4P tiles (P >= _MIN_PARTITION_TILES),
            # i.e. at most ceil(T / P) + 4 items; the single items are padded to
            # whole workgroups. T counts tiles, not pool blocks: a block of 32
            # keys is two tiles.
            self.plan = nat.CountedPlan(*split_plan_capacity(b, hkv, mb, owner.bs, owner.pool.spec.head_dim),
                                        dev)
        self.keep = torch.arange(b, dtype=torch.long, device=dev)
        meta = {"block_tables": self.packed.block_tables, "cu_seqlens": self.packed.cu_seqlens,
                "kv_lens": self.packed.kv_lens, "positions": self.packed.positions, "row_map": None,
                "plan": self.plan}
        fuse = owner.fuse_kv_write
        self.binding = attention_backend._VarlenBinding.from_packed(
            owner.pool, meta, b, write_slots=self.packed.slot_mapping if fuse else None)
        self.cache = VarlenPackedCache.from_slot_mapping(owner.pool, owner.pool.spec.num_layers,
                                                         self.packed.slot_mapping, write_in_attention=fuse)
        self.graph = None
        self.logits = None
        self.copied = None


class GraphedPagedDecoder:
    """Decode one token for each of B sequences against the paged pool, as a graph."""

    def __init__(self, model, pool, max_batch: int, max_model_len: int, ctx_bucket: int = 32,
                 attn_kernel: str = "gather", num_splits: int = 8, fuse_kv_write: bool = True):
        # ctx_bucket / attn_kernel / num_splits are accepted for the
        # reference's signature: nothing here is padded to a context bucket and
        # there is one attention kernel. fuse_kv_write: every layer's KV write
        # rides in its attention launch (mf_paged_attention_kv_write).
        if not str(pool.spec.device).startswith("cuda"):
            raise ValueError("graphed paged decode needs a GPU device")
        hq = model.config.num_attention_heads
        hkv = pool.spec.num_kv_heads
        if hq % hkv or hq // hkv > 16:
            raise ValueError(f"graphed decode needs at most 16 query heads per kv head, got {hq}/{hkv}")
        if not attention_backend.register():
            raise RuntimeError("the transformers attention registry is required")
        self.model, self.pool = model, pool
        self.fuse_kv_write = bool(fuse_kv_write) and pool.key_pool.dtype == model.dtype
        self.device = pool.spec.device
        self.bs = pool.block_size
        self.max_batch = max(1, int(max_batch))
        # room for the longest context plus a speculative lookahead block
        self.max_blocks = (max_model_len + self.bs - 1) // self.bs + 1
        # every reachable context (in 16-key tiles) fits one cooperative unit:
        # plans can always be merge-free, and the graph needs no merge launch
        self.merge_free = (self.max_blocks * self.bs + 15) // 16 <= 4 * nat.MAX_ITEM_TILES
        self.num_q_heads = hq
        self._mem_pool = torch.cuda.graph_pool_handle()
        self._buckets: Dict[int, _Bucket] = {}
        self.replays = 0
        self.captures = 0

    def _batch_bucket(self, b: int) -> int:
        """Powers of two, capped at max_batch (so any max_batch is a bucket)."""
        p = 1
        while p < b:
            p *= 2
        return min(p, self.max_batch) if b <= self.max_batch else p

    def _forward(self, bk: _Bucket) -> torch.Tensor:
        nat.ragged_pack(bk.entries, bk.tables, bk.tokens, bk.b, self.bs, self.max_blocks, out=bk.packed,
                        num_slots=self.pool.capacity_tokens)
        with attention_backend.backend_enabled_on(self.model) as routed:
            if not routed:
                raise RuntimeError("graphed decode needs the attention registry")
            with attention_backend.bind_varlen(bk.binding):
                out = self.model(input_ids=bk.packed.token_ids.view(1, bk.b),
                                 position_ids=bk.packed.positions.view(1, bk.b),
                                 past_key_values=bk.cache, use_cache=True, logits_to_keep=bk.keep)
        return out.logits[0]

    def _capture(self, bk: _Bucket) -> None:
        # one eager pass on a side stream first (allocator and library
        # warm-up), then the capture; both run this step's staged inputs
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            bk.binding.used = 0
            self._forward(bk)
            if bk.binding.used != self.pool.spec.num_layers:
                raise RuntimeError(f"graphed decode: {bk.binding.used} of {self.pool.spec.num_layers} layers "
                                   "used the varlen kernel")
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self._mem_pool):
            bk.logits = self._forward(bk)
        bk.graph = graph
        self.captures += 1

    def _stage(self, bk: _Bucket, tokens, ctx_lens, tables) -> None:
        n, b, mb = len(tokens), bk.b, self.max_blocks
        if bk.copied is not None:
            bk.copied.synchronize()  # the previous step's copy has left the pinned buffer
        h = bk.host.numpy()
        ent = h[: b * nat.ENTRY_INTS].reshape(b, nat.ENTRY_INTS)
        tab = h[b * nat.ENTRY_INTS: b * nat.ENTRY_INTS + b * mb].reshape(b, mb)
        tok = h[b * nat.ENTRY_INTS + b * mb:]
        ent[:] = 0
        ent[:, 0] = 1                       # one query row per entry
        ent[:, 5] = np.arange(b)            # token offset
        ent[:, 3] = np.arange(b) * mb       # table offset
        tok[:] = 0
        for i in range(n):
            t = tables[i]
            if len(t) > mb:
                raise ValueError(f"block table of {len(t)} blocks exceeds the graphed width {mb}")
            ctx = int(ctx_lens[i])
            if ctx + 1 > len(t) * self.bs:
                raise IndexError(f"row {i}: position {ctx} is past its block table of {len(t)} blocks")
            ent[i, 1] = ctx
            ent[i, 2] = ctx + 1
            ent[i, 4] = len(t)
            tab[i, : len(t)] = t
            tok[i] = int(tokens[i])
        if n and (tab[:n].min() < 0 or tab[:n].max() >= self.pool.num_blocks):
            raise IndexError(f"a block table names a block outside the pool of {self.pool.num_blocks}")
        bk.inputs.copy_(bk.host, non_blocking=True)
        bk.copied = torch.cuda.Event()
        bk.copied.record()
        kv = [int(c) + 1 for c in ctx_lens] + [0] * (b - n)
        plan_args = (list(range(b + 1)), kv, self.num_q_heads, self.pool.spec.num_kv_heads,
                     self.pool.spec.head_dim, self.pool.key_pool.dtype)
        items, merges, counts = nat.plan_attention_host(*plan_args)
        if self.merge_free and counts[2] > 0:
            # the planner's pick splits a range: take the smallest partition
            # whose units hold the longest context whole instead
            longest = (max(kv) + 15) // 16
            part = _MIN_PARTITION_TILES
            while 4 * part < longest:
                part *= 2
            items, merges, counts = nat.plan_attention_host(*plan_args, partition_tiles=part)
        bk.plan.update(items, merges, counts)

    def bucket(self, n: int) -> _Bucket:
        """The static buffers (and graph, once captured) for a batch of ``n``."""
        if n == 0:
            raise ValueError("step() needs at least one sequence")
        b = self._batch_bucket(n)
        if b > self.max_batch:
            raise ValueError(f"batch {n} exceeds max_batch {self.max_batch}")
        bk = self._buckets.get(b)
        if bk is None:
            bk = self._buckets[b] = _Bucket(self, b)
        return bk

    @torch.no_grad()
    def logits_view(self, tokens: Sequence[int], ctx_lens: Sequence[int],
                    block_tables: Sequence[Sequence[int]],
                    device_tokens: Optional[torch.Tensor] = None, timer=None) -> torch.Tensor:
        """Like ``step`` but returns a view of the graph's output, valid until
        the next call. With ``device_tokens`` (n integers on the GPU, e.g. the
        previous step's argmax) the input tokens are taken from there by a
        device copy, and ``tokens`` is ignored: nothing waits for the host.
        With ``timer`` (a sampled pass's event record) the replay is bracketed
        by HIP events."""
        n = len(ctx_lens)
        if device_tokens is None and len(tokens) != n:
            raise ValueError(f"{len(tokens)} tokens for {n} rows")
        bk = self.bucket(n)
        tables = [t.tolist() if isinstance(t, torch.Tensor) else list(t) for t in block_tables]
        self._stage(bk, tokens if device_tokens is None else [0] * n, ctx_lens, tables)
        if device_tokens is not None:
            bk.tokens[:n].copy_(device_tokens.view(-1)[:n])
        if bk.graph is None:
            self._capture(bk)
        began = timer.start_whole() if timer is not None else None
        bk.graph.replay()
        if timer is not None:
            timer.stop("decode_graph", began)
        self.replays += 1
        return bk.logits[:n]

    @torch.no_grad()
    def step(self, tokens: Sequence[int], ctx_lens: Sequence[int],
             block_tables: Sequence[torch.Tensor]) -> torch.Tensor:
        """Decode one token per row. ``ctx_lens[i]`` tokens are already cached
        for row i; the new token is written at that position (its block must
        already be allocated). Returns fresh logits ``(n, vocab)``."""
        return self.logits_view(tokens, ctx_lens, block_tables).clone()
