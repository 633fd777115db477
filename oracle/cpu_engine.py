"""The reference engine's CPU path, ported to torch-on-CPU for the C4
``cpu_baseline`` leg of bench.py (test infrastructure only; never shipped,
never the thing measured on the GPU).

One ``step`` of the reference engine (memforge_ml/runtime/continuous_engine.py:
516-595) with its CPU data path:

* the host scheduler decides the step (this repo's ``memforge_c``, the
  reference's C++ scheduler, block for block: admission, block tables, the
  finish rule);
* each prefill entry runs its own forward (``_run_prefill``,
  continuous_engine.py:596-700) and its K/V go into the sequence's pool blocks.
  The reference writes them through ``PagedCache.update`` during that forward;
  here the forward uses a DynamicCache and the K/V are scattered into the
  pool after it: the same rows, copied once;
* every decoding sequence runs in ONE batched forward (``_run_decode_batched``,
  continuous_engine.py:1062-1170): per layer each sequence's whole context is
  gathered from the pool into one preallocated, zeroed, left-padded buffer
  (``assemble_batch``, memforge_ml/kernels/batched_decode.py:123-191, padded to
  a multiple of 4 blocks), the model sees it as a DynamicCache with an
  ``attention_mask`` over the padding, explicit ``position_ids`` and
  ``cache_position``, and afterwards the new K/V of every sequence is
  scattered back into its blocks (kv_pool.py:134-149);
* greedy tokens, one argmax per row (runtime/sampling.py:43-75).

Pool layout and dtypes follow the reference's ``PagedKVPool``
(``(layers, blocks, block_size, kv_heads, head_dim)``, kv_pool.py:61-74).
"""

from __future__ import annotations

from typing import Dict, List, Sequence

import torch


class CpuBatchedEngine:
    """The reference's continuous-batching step on the CPU, greedy only."""

    PAD_BLOCKS = 4  # BatchedDecodeBuffers.DEFAULT_BUCKET_BLOCKS (batched_decode.py:67)

    def __init__(self, model, num_blocks: int, block_size: int = 16, max_num_seqs: int = 8,
                 max_prefill_tokens_per_step: int = 0):
        from memforge_amd import memforge_c

        cfg = model.config
        self.model = model
        self.bs = block_size
        self.layers = cfg.num_hidden_layers
        self.hkv = cfg.num_key_value_heads
        self.d = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        dtype = next(model.parameters()).dtype
        shape = (self.layers, num_blocks, block_size, self.hkv, self.d)
        self.key_pool = torch.zeros(shape, dtype=dtype)
        self.value_pool = torch.zeros(shape, dtype=dtype)
        self.allocator = memforge_c.BlockAllocator(num_blocks, block_size)
        self.scheduler = memforge_c.Scheduler(self.allocator, max_num_seqs, None, max_prefill_tokens_per_step, 0)
        self.forward_passes = 0

    # ---------------------------------------------------------------- pool I/O

    def _flat(self, table: Sequence[int], start: int, end: int) -> torch.Tensor:
        """Flat slot ids of positions [start, end) (kv_pool.py:92-130)."""
        pos = torch.arange(start, end)
        t = torch.as_tensor(list(table), dtype=torch.long)
        return t[pos // self.bs] * self.bs + pos % self.bs

    def _write(self, layer: int, flat: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: (kv_heads, T, D) -> the pool's flat (slots, kv_heads, D) view."""
        self.key_pool[layer].view(-1, self.hkv, self.d).index_copy_(0, flat, k.permute(1, 0, 2))
        self.value_pool[layer].view(-1, self.hkv, self.d).index_copy_(0, flat, v.permute(1, 0, 2))

    # ------------------------------------------------------------------ steps

    @torch.no_grad()
    def _prefill(self, tokens: List[int], table: Sequence[int], start: int, end: int) -> int:
        from transformers.cache_utils import DynamicCache

        cache = DynamicCache()
        if start > 0:  # a prefix already in the pool: seed the cache with it
            flat = self._flat(table, 0, start)
            data = []
            for layer in range(self.layers):
                k = self.key_pool[layer].view(-1, self.hkv, self.d).index_select(0, flat).permute(1, 0, 2)
                v = self.value_pool[layer].view(-1, self.hkv, self.d).index_select(0, flat).permute(1, 0, 2)
                data.append((k[None].contiguous(), v[None].contiguous()))
            cache = DynamicCache(ddp_cache_data=data)
        pos = torch.arange(start, end)
        out = self.model(input_ids=torch.tensor([tokens[start:end]]), past_key_values=cache, use_cache=True,
                         position_ids=pos[None], cache_position=pos)
        self.forward_passes += 1
        flat = self._flat(table, start, end)
        for layer in range(self.layers):
            entry = cache.layers[layer]
            self._write(layer, flat, entry.keys[0, :, start:end], entry.values[0, :, start:end])
        return int(out.logits[0, -1].argmax())

    @torch.no_grad()
    def _decode_batched(self, rows: List[tuple]) -> List[int]:
        """rows: (last token, context length, block table) per decoding sequence."""
        from transformers.cache_utils import DynamicCache

        batch = len(rows)
        ctx = [c for _, c, _ in rows]
        pad_to = self.bs * self.PAD_BLOCKS
        padded = (max(ctx) + pad_to - 1) // pad_to * pad_to
        dtype = self.key_pool.dtype
        keys = torch.zeros((self.layers, batch, self.hkv, padded, self.d), dtype=dtype)
        values = torch.zeros_like(keys)
        flats = [self._flat(t, 0, c) for _, c, t in rows]
        for layer in range(self.layers):
            src_k = self.key_pool[layer].view(-1, self.hkv, self.d)
            src_v = self.value_pool[layer].view(-1, self.hkv, self.d)
            for r, (flat, c) in enumerate(zip(flats, ctx)):
                keys[layer, r, :, padded - c:] = src_k.index_select(0, flat).permute(1, 0, 2)
                values[layer, r, :, padded - c:] = src_v.index_select(0, flat).permute(1, 0, 2)
        mask = torch.zeros((batch, padded + 1), dtype=torch.long)
        for r, c in enumerate(ctx):
            mask[r, padded - c:] = 1
        cache = DynamicCache(ddp_cache_data=[(keys[i], values[i]) for i in range(self.layers)])
        out = self.model(input_ids=torch.tensor([[t] for t, _, _ in rows]), attention_mask=mask,
                         position_ids=torch.tensor([[c] for c in ctx]),
                         past_key_values=cache, cache_position=torch.arange(padded, padded + 1), use_cache=True)
        self.forward_passes += 1
        for layer in range(self.layers):
            nk = cache.layers[layer].keys[:, :, -1]
            nv = cache.layers[layer].values[:, :, -1]
            for r, (_, c, t) in enumerate(rows):
                self._write(layer, self._flat(t, c, c + 1), nk[r][:, None], nv[r][:, None])
        return out.logits[:, -1].argmax(dim=-1).tolist()

    def generate(self, prompts: Sequence[Sequence[int]], new_tokens: int) -> List[List[int]]:
        """Greedy generation of ``new_tokens`` per prompt, all submitted at once."""
        tokens: Dict[int, List[int]] = {}
        out: Dict[int, List[int]] = {}
        for i, p in enumerate(prompts):
            self.scheduler.add_sequence(i, list(p), new_tokens)
            tokens[i] = list(p)
            out[i] = []

        def emit(seq_id: int, tok: int) -> None:
            tokens[seq_id].append(tok)
            out[seq_id].append(tok)
            self.scheduler.update_sequence(seq_id, tok, False)

        while self.scheduler.has_unfinished_sequences():
            result = self.scheduler.step()
            decodes = []
            for info in result.running_sequences:
                sid = info.seq_id
                if len(out[sid]) >= new_tokens:
                    continue
                table = list(info.block_table)
                if info.is_prefill:
                    total = len(tokens[sid])
                    cached = int(info.num_cached_tokens)
                    end = int(info.prefill_chunk_end) or total
                    end = min(end, total)
                    if end <= cached:
                        continue
                    tok = self._prefill(tokens[sid], table, cached, end)
                    if end >= total:
                        emit(sid, tok)
                else:
                    decodes.append((sid, (tokens[sid][-1], len(tokens[sid]) - 1, table)))
            if decodes:
                for (sid, _), tok in zip(decodes, self._decode_batched([r for _, r in decodes])):
                    emit(sid, tok)
        return [out[i] for i in range(len(prompts))]
