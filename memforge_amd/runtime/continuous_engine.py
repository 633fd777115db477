"""ContinuousBatchingEngine on the MI355X.

Same public surface as the reference engine (memforge_ml/runtime/
continuous_engine.py:131-1613): submit / abort / step / run_until_idle /
generate / result_for / drain_events / telemetry, with the C++ scheduler and
block allocator (``memforge_c``) deciding every step which sequences run and
which physical blocks they own.

What differs is the execution of a step. The reference runs prefill chunks
and decodes as separate passes (a padded, gathered batch for decode; an
optional fused varlen pass). Here EVERY step is one packed pass through the
model, because the varlen HIP kernel serves prefill chunks and decodes alike:

1. the scheduler's step output becomes one descriptor per contributing
   sequence (prefill entries first, then decodes, in scheduler order, as in the
   reference's fused step), staged in pinned memory and copied to the GPU in
   one transfer together with the block tables and the step's token ids;
2. the ragged-pack kernel builds token ids, positions, slot_mapping,
   cu_seqlens and padded block tables on the device;
3. the model runs once over the packed row; each layer's cache update is the
   KV-write kernel through slot_mapping and its attention the varlen kernel
   reading the pool in place -- nothing is gathered or padded;
4. only each sequence's last row goes through the LM head, and greedy
   sampling is one device argmax and one device-to-host copy per step.

Speculative decoding (draft model + lookahead) verifies all candidate runs in
one varlen pass with the candidates attended in flight, resolves every row
with one rejection-sampling launch (consuming torch's generators exactly as
the per-row reference does), and writes every row's confirmed K/V with one
KV-write launch per layer.

Per-request bookkeeping works on runs of tokens: a pass commits each
request's new tokens together (one token, or a speculative round's confirmed
run), with one clock reading per step, and detokenises incrementally over a
short window instead of re-decoding the whole output for every token.
"""

from __future__ import annotations

import logging
import threading
import time
import warnings
from collections import deque
from dataclasses import dataclass, field
from typing import Any, Deque, Dict, List, Optional, Sequence

import numpy as np
import torch

from memforge_amd import _native as nat
from memforge_amd.kernels import attention_backend
from memforge_amd.runtime.batched_speculative import (
    BatchedGraphedDraftPool,
    BatchedGraphedDraftState,
    DraftState,
    confirmed_slot_mapping,
    propose_draft_tokens,
    resolve_round,
    resolve_rounds_global_rng,
    scatter_accepted_kv,
    scatter_confirmed_rows,
    verify_pass,
)
from memforge_amd.runtime.engine_telemetry import DataPathMeter, device_figures
from memforge_amd.runtime.graphed_paged_decode import GraphedPagedDecoder
from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool
from memforge_amd.runtime.packed_pass import packed_forward
from memforge_amd.runtime.prefix_sharing import block_owners, copy_block, sharing_telemetry
from memforge_amd.runtime.sampling import SamplingParams, sample_logits

LOGGER = logging.getLogger(__name__)

try:
    from memforge_amd import memforge_c

    HAS_CPP_ENGINE = True
except ImportError:  # pragma: no cover - only on an unbuilt checkout
    memforge_c = None
    HAS_CPP_ENGINE = False


@dataclass
class TokenEvent:
    """A single emitted token."""

    seq_id: int
    index: int
    token_id: int
    text: str
    source: str = "target"  # "target" | "draft" | "resample"


class SequenceCursor:
    """Where a running sequence's resident KV ends and which blocks hold it
    (the engine-side state the reference keeps in each sequence's PagedCache)."""

    __slots__ = ("block_table", "position", "_table_tensor")

    def __init__(self, block_table: List[int], position: int = 0):
        self.block_table = list(block_table)
        self.position = position
        self._table_tensor = None

    def rebind(self, block_table: List[int]) -> None:
        if list(block_table) != self.block_table:
            self.block_table = list(block_table)
            self._table_tensor = None

    def block_table_tensor(self, device) -> torch.Tensor:
        if self._table_tensor is None:
            self._table_tensor = torch.tensor(self.block_table, dtype=torch.long, device=device)
        return self._table_tensor


@dataclass
class SequenceRuntime:
    """Python-side state for one in-flight sequence (the C++ side owns memory)."""

    seq_id: int
    prompt_ids: List[int]
    params: SamplingParams
    tokens: List[int]
    cache: Optional[SequenceCursor] = None
    generated: List[int] = field(default_factory=list)
    sources: List[str] = field(default_factory=list)
    events: Deque[TokenEvent] = field(default_factory=deque)
    generator: Optional[torch.Generator] = None
    submitted_at: float = field(default_factory=time.perf_counter)
    first_token_at: Optional[float] = None
    finished_at: Optional[float] = None
    finish_reason: Optional[str] = None
    num_prefills: int = 0
    num_preemptions: int = 0
    decoded_chars: int = 0
    draft: Optional[DraftState] = None
    num_draft_proposed: int = 0
    num_draft_accepted: int = 0
    # incremental detokenisation window: generated[text_from:] is what the
    # next decode looks at, generated[text_from:text_to] what was already shown
    text_from: int = 0
    text_to: int = 0

    @property
    def done(self) -> bool:
        return self.finish_reason is not None

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_ids)


@dataclass
class StepReport:
    """Telemetry for one iteration-level scheduler step."""

    step_index: int
    num_running: int
    num_waiting: int
    num_prefill: int
    num_decode: int
    tokens_emitted: int
    finished: List[int]
    preempted: List[int]
    aborted: List[int]
    free_blocks: int
    total_blocks: int
    memory_utilization: float
    step_latency_ms: float
    events: List[TokenEvent]


class _AbortRequests:
    """Sequence ids another thread asked to abandon. The stepping thread takes
    them all at the top of a step, so an abort never lands in the middle of one
    (a step may be writing into the sequence's blocks)."""

    __slots__ = ("_lock", "_ids")

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._ids: set = set()

    def add(self, seq_id: int) -> None:
        with self._lock:
            self._ids.add(seq_id)

    def take(self) -> List[int]:
        with self._lock:
            ids, self._ids = self._ids, set()
        return sorted(ids)

    def __bool__(self) -> bool:
        with self._lock:
            return bool(self._ids)


class _ThroughputWindow:
    """Tokens emitted over the last ``seconds`` of activity, kept as one
    (first token time, last token time, count) mark per commit instead of one
    timestamp per token. The rate is tokens over the span from the oldest
    mark's first token to the newest mark's last, so a window holding one
    multi-token commit still has a span, as the reference's per-token stamps
    do (memforge_ml/runtime/continuous_engine.py:1422-1430)."""

    __slots__ = ("seconds", "_marks", "_count")

    def __init__(self, seconds: float):
        self.seconds = seconds
        self._marks: Deque = deque()
        self._count = 0

    def mark(self, first: float, last: float, count: int) -> None:
        if count:
            self._marks.append((first, last, count))
            self._count += count

    def rate(self, now: float) -> float:
        horizon = now - self.seconds
        while self._marks and self._marks[0][1] < horizon:
            self._count -= self._marks.popleft()[2]
        if self._count < 2:
            return 0.0
        span = self._marks[-1][1] - self._marks[0][0]
        return round(self._count / span, 2) if span > 0 else 0.0


def _share(part: float, whole: float, digits: int) -> float:
    return round(part / whole, digits) if whole else 0.0


class ContinuousBatchingEngine:
    def __init__(self, model, tokenizer, *, block_size: int = 16, num_blocks: Optional[int] = None,
                 kv_budget_mb: float = 512.0, max_num_seqs: int = 16, max_model_len: int = 2048,
                 dtype: Optional[torch.dtype] = None, device: Optional[str] = None,
                 batched_decode: bool = True, enable_prefix_sharing: bool = True,
                 decode_view_cache: bool = False, view_cache_budget_mb: float = 512.0,
                 block_attention: bool = False, max_prefill_tokens_per_step: int = 0,
                 draft_model=None, lookahead_k: int = 0, fused_prefill: bool = False,
                 paged_attn_kernel: str = "gather", draft_cuda_graph=False, paged_cuda_graph=False,
                 telemetry_sample_every: int = 16, fused_kv_write: bool = True):
        if not HAS_CPP_ENGINE:
            raise RuntimeError("The native memforge_c extension is required; build it with "
                               "`python -m memforge_amd._build`")
        if decode_view_cache:
            raise NotImplementedError("the contiguous decode mirror is not part of memforge_amd")
        self.model = model
        # each layer's KV write rides in its attention launch (one launch per
        # layer instead of two); needs the pool in the model's dtype
        self._fused_kv_write = bool(fused_kv_write)
        self.tokenizer = tokenizer
        self.device = device or str(next(model.parameters()).device)
        if torch.device(self.device).type != "cuda":
            raise ValueError(f"memforge_amd runs the engine on the GPU; got device {self.device!r}")
        self.dtype = dtype or next(model.parameters()).dtype
        self.block_size = block_size
        self.max_num_seqs = max_num_seqs
        self.max_model_len = max_model_len
        # Accepted for API compatibility: every step is one packed varlen pass,
        # which is what the reference's batched_decode / block_attention /
        # fused_prefill / paged kernel options choose between.
        self.batched_decode = batched_decode
        self.fused_prefill = True
        self.block_attention = True
        self.decode_view_cache = False

        self.spec = ModelKVSpec.from_config(model.config, self.dtype, self.device)
        if num_blocks is None:
            num_blocks = PagedKVPool.blocks_for_budget(self.spec, block_size, kv_budget_mb)
        self.pool = PagedKVPool(self.spec, num_blocks=num_blocks, block_size=block_size)

        self.allocator = memforge_c.BlockAllocator(num_blocks, block_size)
        self.prefix_cache = memforge_c.PrefixCache(self.allocator, block_size) if enable_prefix_sharing else None
        self.max_prefill_tokens_per_step = max(0, int(max_prefill_tokens_per_step))
        self.draft_model = draft_model
        self.lookahead_k = max(0, int(lookahead_k)) if draft_model is not None else 0
        lookahead_slots = self.lookahead_k + 1 if self.lookahead_k > 0 else 0
        self.scheduler = memforge_c.Scheduler(self.allocator, max_num_seqs, self.prefix_cache,
                                              self.max_prefill_tokens_per_step, lookahead_slots)
        if not attention_backend.register():
            raise RuntimeError("the transformers attention registry is required")
        # Pure-decode steps replay a captured HIP graph of the packed pass
        # (False | True | "auto", as the reference's paged_cuda_graph; "auto"
        # is on whenever the model's head grouping allows it).
        self._paged_graph = None
        if paged_cuda_graph:
            if paged_cuda_graph != "auto" or self._graph_heads_ok(model):
                self._paged_graph = GraphedPagedDecoder(model, self.pool, max_batch=max_num_seqs,
                                                        max_model_len=max_model_len,
                                                        fuse_kv_write=fused_kv_write)

        # Draft proposals (False | "batched" | "batched-unrolled" | "auto" |
        # True, as the reference's draft_cuda_graph): the batched forms draft
        # every running sequence in K+1 graph replays per round (one replay
        # when unrolled), with the greedy feedback on the device. "auto" picks
        # "batched" whenever the draft's head grouping allows it. True, the
        # reference's superseded per-sequence graphs, runs as "batched".
        self._draft_pool = None
        if draft_cuda_graph == "auto":
            draft_cuda_graph = "batched" if (draft_model is not None
                                             and self._graph_heads_ok(draft_model)) else False
        if draft_cuda_graph is True:
            warnings.warn(
                "draft_cuda_graph=True (one graph per sequence) is superseded by 'batched', which "
                "drafts the whole batch per replay; it runs as 'batched'. Pass draft_cuda_graph="
                "'batched' or 'auto'.", DeprecationWarning, stacklevel=2)
            draft_cuda_graph = "batched"
        if draft_cuda_graph and draft_model is not None and self.lookahead_k > 0:
            if draft_cuda_graph not in ("batched", "batched-unrolled"):
                raise ValueError(f"draft_cuda_graph must be False, True, 'auto', 'batched' or "
                                 f"'batched-unrolled', got {draft_cuda_graph!r}")
            self._draft_pool = BatchedGraphedDraftPool(
                draft_model, max_len=max_model_len, num_slots=max_num_seqs, device=self.device,
                unroll=draft_cuda_graph == "batched-unrolled")
        # every speculative step resolves its rows with one kernel launch; the
        # one-row-at-a-time form stays selectable for differential tests
        self._batched_resolve = True

        self.eos_token_ids = self._resolve_eos_ids()
        self.runtimes: Dict[int, SequenceRuntime] = {}
        self._next_seq_id = 1
        self._step_index = 0
        for name in ("total_tokens_generated", "total_prefill_tokens", "total_steps", "total_forward_passes",
                     "total_preemptions", "total_cached_prefix_tokens", "total_cow_copies",
                     "total_prefill_chunks", "total_fused_steps", "total_fused_tokens",
                     "total_draft_tokens_proposed", "total_draft_tokens_accepted", "total_speculative_rounds",
                     "total_speculative_sequence_rounds", "total_blockwise_layers", "total_blockwise_fallbacks",
                     # sum over passes of every sequence's kv length / of packed query rows
                     "total_attended_kv_tokens", "total_packed_rows"):
            setattr(self, name, 0)
        self.engine_started_at = time.perf_counter()
        self._aborts = _AbortRequests()
        self._throughput = _ThroughputWindow(5.0)
        weight_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
        self._meter = DataPathMeter(self.spec, model.config.num_attention_heads, block_size, weight_bytes,
                                    every=telemetry_sample_every)

    @property
    def throughput_window_s(self) -> float:
        return self._throughput.seconds

    @throughput_window_s.setter
    def throughput_window_s(self, seconds: float) -> None:
        self._throughput.seconds = float(seconds)

    # ------------------------------------------------------------------ setup

    @staticmethod
    def _graph_heads_ok(model) -> bool:
        """The captured decode pass handles up to 16 query heads per KV head."""
        cfg = model.config
        hq = cfg.num_attention_heads
        hkv = getattr(cfg, "num_key_value_heads", None) or hq
        return hq % hkv == 0 and hq // hkv <= 16

    def _resolve_eos_ids(self) -> set:
        ids = set()
        cfg_eos = getattr(self.model.config, "eos_token_id", None)
        for candidate in (cfg_eos, getattr(self.tokenizer, "eos_token_id", None)):
            if isinstance(candidate, int):
                ids.add(candidate)
            elif isinstance(candidate, (list, tuple)):
                ids.update(int(c) for c in candidate)
        return ids

    def describe(self) -> Dict[str, Any]:
        return {
            "engine": "C++ native (memforge_c) + HIP data path (libmemforge_hip)",
            "model": getattr(self.model.config, "name_or_path", "unknown"),
            "device": self.device,
            "dtype": str(self.dtype),
            "max_num_seqs": self.max_num_seqs,
            "max_model_len": self.max_model_len,
            "batched_decode": True,
            "prefix_sharing": self.prefix_cache is not None,
            "decode_view_cache": False,
            "block_attention": True,
            "paged_cuda_graph": self._paged_graph is not None,
            "max_prefill_tokens_per_step": self.max_prefill_tokens_per_step,
            "chunked_prefill": self.max_prefill_tokens_per_step > 0,
            "eos_token_ids": sorted(self.eos_token_ids),
            "kv_pool": self.pool.describe(),
            "data_path": {
                "library": nat.LIB_PATH.name,
                "arch": "gfx950",
                "step": "one packed varlen pass (ragged pack, then per layer "
                        + ("one launch for the KV write and the paged attention)" if self._fused_kv_write
                           else "the KV write and the paged attention)"),
                "speculative_resolve": "one mf_spec_verify launch per round" if self._batched_resolve
                                       else "one row at a time",
                "telemetry_sample_every": self._meter.every,
            },
        }

    # ------------------------------------------------------------- submission

    def submit(self, prompt, params: Optional[SamplingParams] = None) -> int:
        """Enqueue a request; nothing runs until ``step()`` (continuous_engine.py:381-414)."""
        params = params or SamplingParams()
        if isinstance(prompt, str):
            prompt_ids = self.tokenizer(prompt, return_tensors=None)["input_ids"]
        else:
            prompt_ids = list(prompt)
        if not prompt_ids:
            raise ValueError("cannot submit an empty prompt")
        headroom = self.max_model_len - len(prompt_ids)
        if headroom <= 0:
            raise ValueError(f"prompt of {len(prompt_ids)} tokens leaves no room under "
                             f"max_model_len={self.max_model_len}")
        params = params.clamped(headroom)
        seq_id = self._next_seq_id
        self._next_seq_id += 1
        generator = None
        if params.seed is not None:
            generator = torch.Generator(device="cpu").manual_seed(params.seed)
        self.runtimes[seq_id] = SequenceRuntime(seq_id=seq_id, prompt_ids=list(prompt_ids), params=params,
                                                tokens=list(prompt_ids), generator=generator)
        self.scheduler.add_sequence(seq_id, list(prompt_ids), params.max_new_tokens)
        return seq_id

    def abort(self, seq_id: int) -> bool:
        """Ask, from any thread, for a running request to be abandoned; it is
        applied at the top of the next step. False if it is unknown or done."""
        rt = self.runtimes.get(seq_id)
        if rt is None or rt.done:
            return False
        self._aborts.add(seq_id)
        return True

    def _process_pending_aborts(self) -> None:
        for seq_id in self._aborts.take():
            rt = self.runtimes.get(seq_id)
            if rt is not None and not rt.done:
                self.scheduler.abort_sequence(seq_id)
                self._finish(rt, "aborted")

    # ------------------------------------------------------------------ steps

    def has_work(self) -> bool:
        if self._aborts:
            return True
        return self.scheduler.has_unfinished_sequences() or any(not rt.done for rt in self.runtimes.values())

    @property
    def speculation_enabled(self) -> bool:
        return self.draft_model is not None and self.lookahead_k > 0

    def step(self) -> StepReport:
        """Run exactly one iteration-level scheduling + execution step."""
        t0 = time.perf_counter()
        self._process_pending_aborts()
        result = self.scheduler.step()
        self._step_index += 1
        self.total_steps += 1

        for seq_id in result.aborted_sequence_ids:
            rt = self.runtimes.get(seq_id)
            if rt is not None and not rt.done:
                self._finish(rt, "aborted_unschedulable")
        for seq_id in result.preempted_sequence_ids:
            rt = self.runtimes.get(seq_id)
            if rt is not None and rt.cache is not None:
                rt.cache = None
                # a waiting sequence holds no draft slot; the next round
                # re-feeds its draft from the start
                self._release_draft(rt)
                rt.num_preemptions += 1
                self.total_preemptions += 1

        prefill_infos = [i for i in result.running_sequences if i.is_prefill]
        decode_infos = [i for i in result.running_sequences if not i.is_prefill]
        events: List[TokenEvent] = []

        plan: List[dict] = []
        for info in prefill_infos:
            entry = self._prepare_prefill(info)
            if entry is not None:
                plan.append(entry)
        n_prefill = len(plan)
        spec_rts: List[SequenceRuntime] = []
        for info in decode_infos:
            rt = self.runtimes.get(info.seq_id)
            if rt is None or rt.done or rt.cache is None:
                continue
            self._begin_write_step(rt, info)
            if self.speculation_enabled and self._speculation_headroom(rt):
                spec_rts.append(rt)
            else:
                plan.append({"rt": rt, "kind": "decode", "tokens": [rt.tokens[-1]],
                             "start": rt.cache.position, "table": rt.cache.block_table})
        if plan:
            # a sampled step is timed the way it runs: kernel by kernel when
            # eager, as a whole replay when graphed (sampling never changes
            # which path a step takes, so it never changes the results)
            sampled = self._meter.arm()
            if n_prefill == 0 and self._paged_graph is not None:
                events.extend(self._run_graphed(plan, sampled))
            else:
                events.extend(self._run_packed(plan, sampled))
                if n_prefill and len(plan) > n_prefill:
                    self.total_fused_steps += 1
        if spec_rts:
            events.extend(self._run_speculative(spec_rts))

        for seq_id in result.finished_sequence_ids:
            rt = self.runtimes.get(seq_id)
            if rt is not None and not rt.done:
                self._finish(rt, "length")

        return StepReport(
            step_index=self._step_index,
            num_running=len(result.running_sequences),
            num_waiting=result.num_waiting,
            num_prefill=n_prefill,
            num_decode=len(plan) - n_prefill + len(spec_rts),
            tokens_emitted=len(events),
            finished=list(result.finished_sequence_ids),
            preempted=list(result.preempted_sequence_ids),
            aborted=list(result.aborted_sequence_ids),
            free_blocks=result.num_free_blocks,
            total_blocks=result.total_blocks,
            memory_utilization=result.memory_utilization_ratio,
            step_latency_ms=(time.perf_counter() - t0) * 1000.0,
            events=events,
        )

    def _prepare_prefill(self, info) -> Optional[dict]:
        """This step's prefill chunk of one sequence, with the reference's chunk
        arithmetic (continuous_engine.py:603-640, 782-832)."""
        rt = self.runtimes.get(info.seq_id)
        if rt is None or rt.done:
            return None
        table = list(info.block_table)
        if rt.cache is None:
            rt.cache = SequenceCursor(table)
        else:
            rt.cache.rebind(table)
        cached = int(getattr(info, "num_cached_tokens", 0) or 0)
        total = len(rt.tokens)
        chunk_end = int(getattr(info, "prefill_chunk_end", 0) or 0)
        if chunk_end <= 0 or chunk_end > total:
            chunk_end = total
        if cached >= total:
            cached, chunk_end = 0, total
        if chunk_end <= cached:
            return None  # budget exhausted this step; resumes next step
        rt.num_prefills += 1
        rt.cache.position = cached
        return {"rt": rt, "kind": "prefill", "tokens": rt.tokens[cached:chunk_end], "start": cached,
                "table": table, "cached": cached, "chunk_end": chunk_end, "is_final": chunk_end >= total}

    def _begin_write_step(self, rt: SequenceRuntime, info) -> None:
        """Rebind a decoding sequence's table, copying a shared block on write
        (continuous_engine.py:974-1006)."""
        rt.cache.rebind(list(info.block_table))
        if self.prefix_cache is None:
            return
        seq = self.scheduler.get_sequence(rt.seq_id)
        if seq is None:
            return
        cow = self.allocator.prepare_write(seq, rt.cache.position // self.block_size)
        if cow is None:
            return
        old_block, new_block = cow
        copy_block(self.pool, old_block, new_block)
        rt.cache.rebind(list(seq.get_block_table()))
        self.total_cow_copies += 1

    # ------------------------------------------------------------ packed pass

    def _run_packed(self, plan: List[dict], sampled: bool = False) -> List[TokenEvent]:
        """One forward over every entry of ``plan`` (prefill chunks, then decodes)."""
        q_lens = [len(e["tokens"]) for e in plan]
        cu = np.concatenate([[0], np.cumsum(q_lens)])
        # only rows that produce a token go through the LM head
        emit = [i for i, e in enumerate(plan) if e["kind"] == "decode" or e["is_final"]]
        timer = None
        if sampled:
            kv = [e["start"] + n for e, n in zip(plan, q_lens)]
            timer = self._meter.begin(self._meter.layer_bytes(kv, int(cu[-1])))
        try:
            res = packed_forward(self.model, self.pool, [e["tokens"] for e in plan],
                                 [e["start"] for e in plan], [e["table"] for e in plan],
                                 [int(cu[i + 1]) - 1 for i in emit], timer=timer,
                                 fuse_kv_write=self._fused_kv_write)
        except IndexError as exc:
            raise IndexError(f"{exc} (sequences {[e['rt'].seq_id for e in plan]})") from None
        self.total_forward_passes += 1
        self.total_blockwise_layers += res.layers_used
        self.total_fused_tokens += res.num_tokens
        self.total_attended_kv_tokens += int(sum(res.kv_lens))
        self.total_packed_rows += res.num_tokens
        return self._emit(plan, emit, res.logits)

    def _run_graphed(self, plan: List[dict], sampled: bool = False) -> List[TokenEvent]:
        """A decode-only step as one replay of the captured packed pass."""
        ctx = [e["start"] for e in plan]
        timer = None
        if sampled:
            nbytes = self._meter.step_bytes([c + 1 for c in ctx], len(plan))
            timer = self._meter.begin({"decode_graph": nbytes}, whole=True)
        logits = self._paged_graph.logits_view([e["tokens"][0] for e in plan], ctx, [e["table"] for e in plan],
                                               timer=timer)
        self.total_forward_passes += 1
        self.total_blockwise_layers += self.spec.num_layers
        self.total_fused_tokens += len(plan)
        self.total_attended_kv_tokens += sum(c + 1 for c in ctx)
        self.total_packed_rows += len(plan)
        return self._emit(plan, list(range(len(plan))), logits)

    def _emit(self, plan: List[dict], emit: List[int], logits: torch.Tensor) -> List[TokenEvent]:
        """Sample one token for each entry in ``emit`` (indices into ``plan``,
        rows of ``logits``) and do every entry's bookkeeping."""
        greedy = [j for j, i in enumerate(emit) if plan[i]["rt"].params.temperature <= 0.0]
        tokens: Dict[int, int] = {}
        if len(greedy) == len(emit):  # one device argmax, one copy to the host
            tokens = dict(enumerate(logits.argmax(dim=-1).tolist()))
        elif greedy:
            idx = torch.tensor(greedy, dtype=torch.long).to(self.device)
            for j, tok in zip(greedy, logits.index_select(0, idx).argmax(dim=-1).tolist()):
                tokens[j] = int(tok)
        for j, i in enumerate(emit):
            if j not in tokens:
                rt = plan[i]["rt"]
                row = logits[j].float()
                if rt.generator is not None:  # a seeded request draws from its own CPU generator
                    row = row.cpu()
                tokens[j] = sample_logits(row, rt.params, rt.generator)

        now = time.perf_counter()
        events: List[TokenEvent] = []
        j = 0
        for entry in plan:
            rt = entry["rt"]
            if entry["kind"] == "prefill":
                rt.cache.position = entry["chunk_end"]
                self.total_prefill_tokens += len(entry["tokens"])
                self.total_cached_prefix_tokens += entry["cached"]
                self.total_prefill_chunks += 1
                if not entry["is_final"]:
                    continue
                if self.prefix_cache is not None:
                    self.prefix_cache.register_full_blocks(rt.tokens, entry["table"])
            else:
                rt.cache.position += 1
            events.extend(self._commit(rt, (tokens[j],), ("target",), now))
            j += 1
        return events

    # ----------------------------------------------------- speculative decode

    def _speculation_headroom(self, rt: SequenceRuntime) -> bool:
        span = self.lookahead_k + 1
        if rt.cache.position + span > self.max_model_len:
            return False
        return len(rt.generated) + span <= rt.params.max_new_tokens

    def _propose(self, rts: List[SequenceRuntime]):
        """Every row's K draft candidates and their draft distributions."""
        k = self.lookahead_k
        proposals: List[List[int]] = [[] for _ in rts]
        draft_probs: List[List[torch.Tensor]] = [[] for _ in rts]
        for rt in rts:
            if rt.draft is None:
                rt.draft = self._draft_pool.acquire() if self._draft_pool is not None else DraftState()
        if self._draft_pool is not None:
            # K+1 replays per temperature present (the reference requires a
            # single temperature per round; rows keep their order either way)
            groups: Dict[float, List[int]] = {}
            for row, rt in enumerate(rts):
                groups.setdefault(float(rt.params.temperature), []).append(row)
            for temp, rows in groups.items():
                out = self._draft_pool.propose([rts[r].draft for r in rows], [rts[r].tokens for r in rows],
                                               k, temp)
                for r, (cand, probs) in zip(rows, out):
                    proposals[r], draft_probs[r] = cand, probs
        else:
            for row, rt in enumerate(rts):
                proposals[row], draft_probs[row] = propose_draft_tokens(
                    self.draft_model, rt.draft, rt.tokens, k, rt.params.temperature, self.device)
        return proposals, draft_probs

    def _run_speculative(self, rts: List[SequenceRuntime]) -> List[TokenEvent]:
        """Draft proposals, one batched verify pass, rejection, confirmed-prefix
        write (continuous_engine.py:1212-1341)."""
        k = self.lookahead_k
        proposals, draft_probs = self._propose(rts)
        token_counts = [len(rt.tokens) for rt in rts]
        ctx = [rt.cache.position for rt in rts]
        tables = [list(rt.cache.block_table) for rt in rts]
        queries = [[rt.tokens[-1]] + cand for rt, cand in zip(rts, proposals)]
        logits, new_kv = verify_pass(self.model, self.pool, tables, ctx, queries, self.device)
        self.total_forward_passes += 1
        self.total_attended_kv_tokens += sum(c + k + 1 for c in ctx)
        self.total_packed_rows += (k + 1) * len(rts)
        self.total_speculative_rounds += 1
        self.total_speculative_sequence_rounds += len(rts)
        if not self._batched_resolve:
            return self._resolve_rows_one_by_one(rts, proposals, draft_probs, logits, new_kv, ctx, token_counts)

        rounds = resolve_rounds_global_rng(
            [rt.seq_id for rt in rts], proposals,
            torch.stack([torch.stack(p) for p in draft_probs]).float(), logits,
            [rt.params.temperature for rt in rts])
        now = time.perf_counter()
        events: List[TokenEvent] = []
        confirmed: List[int] = []
        for rt, rnd in zip(rts, rounds):
            got = self._commit(rt, rnd.accepted, ["draft" if f else "target" for f in rnd.is_draft], now)
            events.extend(got)
            self._count_round(rt, rnd)
            # a request that stopped has no use for its K/V (its blocks go
            # back to the allocator on the next step): nothing is written
            confirmed.append(0 if rt.done else len(got))
        if any(confirmed):
            slots = confirmed_slot_mapping(tables, ctx, confirmed, k + 1, self.block_size)
            scatter_confirmed_rows(self.pool, new_kv, nat.upload([slots], self.device)[0])
        for rt, rnd, n, count in zip(rts, rounds, confirmed, token_counts):
            if not rt.done:
                rt.cache.position += n
                rt.draft.rollback_to(count + rnd.num_accepted_draft)
        return events

    def _resolve_rows_one_by_one(self, rts, proposals, draft_probs, logits, new_kv, ctx, token_counts):
        """The per-row form of the same step: ``resolve_round`` and
        ``scatter_accepted_kv`` for one row after the other."""
        events: List[TokenEvent] = []
        for row, rt in enumerate(rts):
            rnd = resolve_round(rt.seq_id, proposals[row], draft_probs[row],
                                [x.float() for x in logits[row]], rt.params.temperature)
            table = rt.cache.block_table_tensor(self.device)
            got = self._commit(rt, rnd.accepted, ["draft" if f else "target" for f in rnd.is_draft],
                               time.perf_counter())
            events.extend(got)
            self._count_round(rt, rnd)
            if rt.done:
                continue
            scatter_accepted_kv(self.pool, table, ctx[row], new_kv, row, len(got))
            rt.cache.position += len(got)
            rt.draft.rollback_to(token_counts[row] + rnd.num_accepted_draft)
        return events

    def _count_round(self, rt: SequenceRuntime, rnd) -> None:
        proposed = len(rnd.candidates)
        rt.num_draft_proposed += proposed
        rt.num_draft_accepted += rnd.num_accepted_draft
        self.total_draft_tokens_proposed += proposed
        self.total_draft_tokens_accepted += rnd.num_accepted_draft

    # ------------------------------------------------------------ bookkeeping

    def _release_draft(self, rt: SequenceRuntime) -> None:
        if isinstance(rt.draft, BatchedGraphedDraftState):
            self._draft_pool.release(rt.draft)
        rt.draft = None

    def _commit(self, rt: SequenceRuntime, token_ids: Sequence[int], sources: Sequence[str],
                now: float) -> List[TokenEvent]:
        """Append a run of tokens to one request -- one token from a packed
        pass, or a speculative round's confirmed run -- up to the first that
        ends it: an end-of-sequence token (when the request stops on EOS) or
        the one that spends its token budget. Every appended token is reported
        to the scheduler and gets an event with its new text. Returns the
        events, one per appended token."""
        if rt.done or not token_ids:
            return []
        if rt.first_token_at is None:
            rt.first_token_at = now
        budget = rt.params.max_new_tokens
        stop_ids = self.eos_token_ids if rt.params.stop_on_eos else ()
        produced: List[TokenEvent] = []
        reason = None
        for token_id, source in zip(token_ids, sources):
            token_id = int(token_id)
            ends = token_id in stop_ids
            rt.tokens.append(token_id)
            rt.generated.append(token_id)
            rt.sources.append(source)
            self.scheduler.update_sequence(rt.seq_id, token_id, ends)
            produced.append(TokenEvent(seq_id=rt.seq_id, index=len(rt.generated) - 1, token_id=token_id,
                                       text=self._text_delta(rt), source=source))
            if ends:
                reason = "stop"
            elif len(rt.generated) >= budget:
                reason = "length"
            if reason:
                break
        rt.events.extend(produced)
        self.total_tokens_generated += len(produced)
        # the run's first token counts from the step's clock reading, its
        # last from now
        self._throughput.mark(now, time.perf_counter(), len(produced))
        if reason:
            self._finish(rt, reason)
        return produced

    def _text_delta(self, rt: SequenceRuntime) -> str:
        """The text the newest token adds, decoded over a short window:
        generated[text_from:] against generated[text_from:text_to], the part
        already shown. A window ending in an incomplete character (U+FFFD)
        shows nothing yet; the character appears with the token that completes
        it. Decoding from the window's start token on both sides keeps the
        tokenizer's own handling of leading spaces, so the deltas add up to
        the full decode."""
        shown = self.tokenizer.decode(rt.generated[rt.text_from:rt.text_to], skip_special_tokens=True)
        window = self.tokenizer.decode(rt.generated[rt.text_from:], skip_special_tokens=True)
        if len(window) <= len(shown) or window.endswith("\ufffd"):
            return ""
        rt.text_from, rt.text_to = rt.text_to, len(rt.generated)
        delta = window[len(shown):]
        rt.decoded_chars += len(delta)
        return delta

    def _finish(self, rt: SequenceRuntime, reason: str) -> None:
        if rt.done:
            return
        rt.finish_reason = reason
        rt.finished_at = time.perf_counter()
        self._release_draft(rt)
        rt.cache = None  # the scheduler frees the physical blocks on its next step

    # ----------------------------------------------------------------- output

    def result_for(self, seq_id: int) -> Dict[str, Any]:
        rt = self.runtimes[seq_id]
        end = rt.finished_at if rt.finished_at is not None else time.perf_counter()
        elapsed = end - rt.submitted_at
        first = None if rt.first_token_at is None else rt.first_token_at - rt.submitted_at
        made = len(rt.generated)
        return {
            "seq_id": seq_id,
            "prompt_tokens": rt.prompt_len,
            "generated_tokens": made,
            "text": self.tokenizer.decode(rt.generated, skip_special_tokens=True),
            "token_ids": rt.generated[:],
            "token_sources": rt.sources[:],
            "finish_reason": rt.finish_reason,
            "time_to_first_token_ms": round(first * 1e3, 2) if first else None,
            "total_time_s": round(elapsed, 4),
            "tokens_per_second": round(made / elapsed, 2) if elapsed > 0 else 0.0,
            "num_prefills": rt.num_prefills,
            "num_preemptions": rt.num_preemptions,
        }

    def drain_events(self, seq_id: int) -> List[TokenEvent]:
        """Hand over (and forget) the request's events not yet drained."""
        rt = self.runtimes[seq_id]
        pending, rt.events = rt.events, deque()
        return list(pending)

    def recent_tokens_per_second(self) -> float:
        return self._throughput.rate(time.perf_counter())

    def _counters(self, uptime: float) -> Dict[str, Any]:
        spec_rounds = self.total_speculative_rounds
        return {
            "uptime_s": round(uptime, 2),
            "steps": self.total_steps,
            "forward_passes": self.total_forward_passes,
            "tokens_generated": self.total_tokens_generated,
            "prefill_tokens": self.total_prefill_tokens,
            "tokens_per_second": self.recent_tokens_per_second(),
            "lifetime_tokens_per_second": _share(self.total_tokens_generated, uptime, 2),
            "tokens_per_forward_pass": _share(self.total_tokens_generated, self.total_forward_passes, 3),
            "active_sequences": sum(not rt.done for rt in self.runtimes.values()),
            "waiting_sequences": self.scheduler.get_num_waiting(),
            "running_sequences": self.scheduler.get_num_running(),
            "preemptions": self.total_preemptions,
            "cached_prefix_tokens": self.total_cached_prefix_tokens,
            "cow_copies": self.total_cow_copies,
            "prefill_chunks": self.total_prefill_chunks,
            "fused_steps": self.total_fused_steps,
            "fused_tokens": self.total_fused_tokens,
            "speculative_rounds": spec_rounds,
            "speculative_sequences_per_round": _share(self.total_speculative_sequence_rounds, spec_rounds, 3),
            "draft_tokens_proposed": self.total_draft_tokens_proposed,
            "draft_tokens_accepted": self.total_draft_tokens_accepted,
            "draft_acceptance_rate": _share(self.total_draft_tokens_accepted, self.total_draft_tokens_proposed, 4),
            "blockwise_layer_calls": self.total_blockwise_layers,
            "blockwise_fallbacks": self.total_blockwise_fallbacks,
            "attended_kv_tokens": self.total_attended_kv_tokens,
            "packed_rows": self.total_packed_rows,
        }

    def _features(self) -> Dict[str, Any]:
        graph, drafts = self._paged_graph, self._draft_pool
        return {
            "fused_prefill_enabled": True,
            "chunked_prefill_enabled": self.max_prefill_tokens_per_step > 0,
            "max_prefill_tokens_per_step": self.max_prefill_tokens_per_step,
            "speculation_enabled": self.speculation_enabled,
            "lookahead_k": self.lookahead_k,
            "decode_view_cache_enabled": False,
            "block_attention_enabled": True,
            "paged_cuda_graph_enabled": graph is not None,
            "graph_replays": graph.replays if graph is not None else 0,
            "graph_captures": graph.captures if graph is not None else 0,
            "draft_graph_enabled": drafts is not None,
            "draft_graph_replays": drafts.replays if drafts is not None else 0,
            # the reference's decode mirror is not built: its figures stay at zero
            "view_cache_mb_in_use": 0.0,
            "view_cache_budget_mb": 0.0,
            "view_cache_grants": 0,
            "view_cache_denials": 0,
        }

    def _pool_figures(self) -> Dict[str, Any]:
        total = self.allocator.get_total_blocks()
        free = self.allocator.get_num_free_blocks()
        return {
            "total_blocks": total,
            "free_blocks": free,
            "allocated_blocks": total - free,
            "memory_utilization": round(self.allocator.get_utilization_ratio(), 4),
            "block_size": self.block_size,
            "kv_pool_mb": self.pool.describe()["total_mb"],
        }

    def telemetry(self) -> Dict[str, Any]:
        """Every figure a dashboard reads, under the reference's keys
        (continuous_engine.py:1485-1569), plus the measured data-path
        bandwidth (attention, KV write and graph-replayed decode steps)."""
        figures: Dict[str, Any] = {}
        figures.update(sharing_telemetry(self.allocator, self.pool, self.prefix_cache, owners=self.block_owners()))
        figures.update(device_figures(self.pool))
        figures.update(self._counters(time.perf_counter() - self.engine_started_at))
        figures.update(self._features())
        figures.update(self._pool_figures())
        figures.update(self._meter.snapshot())
        return figures

    def _live_block_tables(self) -> List[Any]:
        return [(seq_id, rt.cache.block_table) for seq_id, rt in self.runtimes.items()
                if not rt.done and rt.cache is not None]

    def block_occupancy(self) -> List[int]:
        """Owner of every physical block (0 = none), one owner per block:
        where tables share a block, the last live request listed holds it."""
        owner = np.zeros(self.allocator.get_total_blocks(), dtype=np.int64)
        for seq_id, table in self._live_block_tables():
            ids = np.asarray(table, dtype=np.int64)
            owner[ids[(ids >= 0) & (ids < owner.size)]] = seq_id
        return owner.tolist()

    def block_owners(self) -> Dict[str, List[int]]:
        return block_owners(self._live_block_tables(), self.allocator.get_total_blocks())

    # ------------------------------------------------------- blocking helpers

    def run_until_idle(self, max_steps: int = 100_000) -> List[StepReport]:
        reports: List[StepReport] = []
        while len(reports) < max_steps and self.has_work():
            reports.append(self.step())
        return reports

    def generate(self, prompts, params: Optional[SamplingParams] = None) -> List[Dict[str, Any]]:
        """Submit one prompt or many, step until all are done, return their results."""
        batch = (prompts,) if isinstance(prompts, str) else tuple(prompts)
        ids = [self.submit(prompt, params) for prompt in batch]
        self.run_until_idle()
        return list(map(self.result_for, ids))
