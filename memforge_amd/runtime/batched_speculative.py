"""Speculative decoding inside continuous batching: verify, resolve, scatter.

Same functions as the reference's verify path (memforge_ml/runtime/
batched_speculative.py:98-124, 645-811), re-built around the varlen kernel:

* ``verify_candidates_batched`` runs ONE target pass over every sequence's
  ``[last_confirmed, d1..dK]`` row as a packed varlen pass. The candidates'
  K/V are attended in flight (the kernel reads keys at or above each
  sequence's context length from the layer's own new K/V rows), so nothing is
  written to the pool during verification and no context is gathered or
  padded.
* ``resolve_round`` is the reference's per-sequence resolve (vocabulary
  clipping, then ``RejectionSampler.verify_tokens`` with the global RNG in the
  reference's order); ``resolve_rounds_batched`` resolves every row in one
  mf_spec_verify launch with caller-supplied randomness.
* ``scatter_accepted_kv`` writes only the confirmed prefix, so rejected
  candidates leave no trace in the pool.

The draft side has two forms. ``propose_draft_tokens`` feeds one sequence
through its own DynamicCache (the reference's eager draft).
``BatchedGraphedDraftPool`` drafts every running sequence together: the draft
model's K/V live in a paged pool of their own, one fixed run of blocks per
slot, and each of a round's K+1 decode steps is one replay of the captured
packed pass, with the greedy argmax fed back to the next step on the device.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
from transformers.cache_utils import DynamicCache

from memforge_amd import _native as nat
from memforge_amd.kernels import attention_backend
from memforge_amd.runtime.graphed_paged_decode import GraphedPagedDecoder, _Bucket
from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool
from memforge_amd.runtime.packed_pass import packed_forward
from memforge_amd.runtime.varlen_cache import VarlenPackedCache
from memforge_amd.speculative.rejection_sampler import RejectionSampler


@dataclass
class DraftState:
    """One sequence's draft-model cache and how far it has been fed."""

    cache: DynamicCache = field(default_factory=DynamicCache)
    position: int = 0

    def reset(self) -> None:
        self.cache = DynamicCache()
        self.position = 0

    def rollback_to(self, position: int) -> None:
        """Forget what the draft conditioned on past ``position`` (batched_speculative.py:62-94)."""
        if position < 0:
            raise ValueError(f"cannot roll a draft back to position {position}")
        extra = self.position - position
        if extra > 0:
            self.cache.crop(-extra)
            self.position = position
        elif extra < 0:
            raise ValueError(f"draft is at {self.position}, behind the requested {position}")


@dataclass
class SpeculativeRound:
    """What one speculative step produced for one sequence."""

    seq_id: int
    candidates: List[int]
    accepted: List[int]
    is_draft: List[bool]
    num_accepted_draft: int

    @property
    def num_confirmed(self) -> int:
        return len(self.accepted)


def _probs_from_logits(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """One position's distribution; a point mass on the argmax at temperature 0
    (batched_speculative.py:112-124)."""
    if temperature <= 0.0:
        out = torch.zeros_like(logits)
        out[int(logits.argmax())] = 1.0
        return out
    return torch.softmax(logits / temperature, dim=-1)


def _probs_from_logits_rows(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    if temperature <= 0.0:
        out = torch.zeros_like(logits)
        out.scatter_(1, logits.argmax(-1, keepdim=True), 1.0)
        return out
    return torch.softmax(logits / temperature, dim=-1)


@torch.no_grad()
def propose_draft_tokens(draft_model, state: DraftState, tokens: Sequence[int], lookahead: int,
                         temperature: float, device: str) -> Tuple[List[int], List[torch.Tensor]]:
    """Run the draft ``lookahead`` times for one sequence (batched_speculative.py:589-642)."""
    pending = list(tokens[state.position:])
    if not pending:
        raise ValueError(f"draft is at position {state.position} with only {len(tokens)} tokens")
    out = draft_model(input_ids=torch.tensor([pending], dtype=torch.long, device=device),
                      past_key_values=state.cache, use_cache=True)
    state.position = len(tokens)
    candidates: List[int] = []
    probs: List[torch.Tensor] = []
    for _ in range(lookahead):
        step_probs = _probs_from_logits(out.logits[0, -1].float(), temperature)
        token = int(step_probs.argmax()) if temperature <= 0.0 else int(
            torch.multinomial(step_probs, num_samples=1).item())
        candidates.append(token)
        probs.append(step_probs)
        out = draft_model(input_ids=torch.tensor([[token]], dtype=torch.long, device=device),
                          past_key_values=state.cache, use_cache=True)
        state.position += 1
    return candidates, probs


class BatchedGraphedDraftState:
    """A sequence's handle on one slot of a ``BatchedGraphedDraftPool``
    (batched_speculative.py:328-344): ``position`` tokens of the sequence have
    their draft K/V in the slot's blocks."""

    def __init__(self, pool: "BatchedGraphedDraftPool", slot: int):
        self.pool = pool
        self.slot = slot
        self.position = 0

    def reset(self) -> None:
        self.position = 0

    def rollback_to(self, position: int) -> None:
        """Forget the draft K/V past ``position``; O(1), the stale rows are
        overwritten by later steps and never read before that."""
        if position < 0:
            raise ValueError(f"cannot roll a draft back to position {position}")
        if position > self.position:
            raise ValueError(f"draft is at {self.position}, behind the requested {position}")
        self.position = position


class BatchedGraphedDraftPool:
    """The draft model for every running sequence at once
    (batched_speculative.py:347-577): a round of K proposals costs K+1 graph
    replays whatever the batch size.

    * The draft's K/V live in a paged pool of its own. Slot i owns the fixed
      blocks ``[i*nb, (i+1)*nb)``, nb = ceil(max_len / 16), so a slot never
      allocates and its table never changes.
    * A decode step is one replay of the captured packed pass (ragged pack,
      every layer's KV write, the counted varlen attention) over the round's
      rows, bucketed to powers of two; padding rows write and read nothing. Rows
      sit at their own positions, and each step's attention plan is made on the
      host from positions it already knows, so nothing waits for the GPU.
    * Greedy proposals never leave the GPU inside a round: each step's argmax is
      copied into the next step's token buffer on the device, and the
      candidates come back in one read at the end.
    * ``unroll=True`` captures a whole greedy round -- K+1 steps and the
      feedback -- as one graph per (bucket, K). Sampling rounds (temperature >
      0) always go step by step.
    * A backlog of tokens the draft has not seen (after a round that confirmed
      several) is fed for all rows together in one eager packed pass.
    """

    def __init__(self, model, max_len: int, num_slots: int, device: str, unroll: bool = False,
                 block_size: int = 16):
        if not str(device).startswith("cuda"):
            raise ValueError("a graphed draft needs a GPU device")
        if num_slots < 1 or max_len < 1:
            raise ValueError("a draft pool needs at least one slot and one position")
        self.model, self.device = model, device
        self.max_len = int(max_len)
        self.num_slots = int(num_slots)
        self.unroll = bool(unroll)
        dtype = next(model.parameters()).dtype
        self.spec = ModelKVSpec.from_config(model.config, dtype, device)
        self.blocks_per_slot = -(-self.max_len // block_size)
        self.kv = PagedKVPool(self.spec, num_blocks=self.num_slots * self.blocks_per_slot,
                              block_size=block_size)
        nb = self.blocks_per_slot
        self._tables = [list(range(i * nb, (i + 1) * nb)) for i in range(self.num_slots)]
        self._decoder = GraphedPagedDecoder(model, self.kv, max_batch=self.num_slots,
                                            max_model_len=self.max_len)
        self._free = list(range(self.num_slots))
        self._ugraph: Dict[Tuple[int, int], torch.cuda.CUDAGraph] = {}
        self._uout: Dict[Tuple[int, int], torch.Tensor] = {}
        self._ubuckets: Dict[Tuple[int, int], List[_Bucket]] = {}
        self.replays = 0

    @property
    def _graph(self) -> Dict[int, torch.cuda.CUDAGraph]:
        """Captured single-step graphs by bucket size."""
        return {b: bk.graph for b, bk in self._decoder._buckets.items() if bk.graph is not None}

    # ------------------------------------------------------------- slots
    def acquire(self) -> BatchedGraphedDraftState:
        if not self._free:
            raise RuntimeError("no free draft slot; raise num_slots to max_num_seqs")
        self._free.sort(reverse=True)  # lowest slot first
        return BatchedGraphedDraftState(self, self._free.pop())

    def release(self, state: BatchedGraphedDraftState) -> None:
        if state.slot in self._free:
            raise ValueError(f"draft slot {state.slot} is already free")
        state.reset()
        self._free.append(state.slot)

    # ------------------------------------------------------------- feeding
    @torch.no_grad()
    def prefill(self, state: BatchedGraphedDraftState, tokens: Sequence[int]) -> None:
        """Feed several tokens into one slot eagerly."""
        self._prefill_many([(state, list(tokens))])

    def _prefill_many(self, runs: List[Tuple[BatchedGraphedDraftState, List[int]]]) -> None:
        runs = [(st, toks) for st, toks in runs if toks]
        if not runs:
            return
        for st, toks in runs:
            if st.position + len(toks) > self.max_len:
                raise ValueError(f"draft context {st.position + len(toks)} exceeds {self.max_len}")
        packed_forward(self.model, self.kv, [toks for _, toks in runs],
                       [st.position for st, _ in runs], [self._tables[st.slot] for st, _ in runs],
                       keep_rows=[0])
        for st, toks in runs:
            st.position += len(toks)

    # ------------------------------------------------------------- rounds
    @torch.no_grad()
    def propose(self, states: Sequence[BatchedGraphedDraftState], tokens_list: Sequence[Sequence[int]],
                lookahead: int, temperature: float):
        """K candidates and the draft's K distributions for every state.

        Any backlog but the last pending token is prefilled first; then the
        last token and each candidate are fed one step at a time, the final
        candidate included, so its K/V survives a fully accepted round
        (batched_speculative.py:514-577). Every state advances by K+1."""
        if len(states) != len(tokens_list):
            raise ValueError(f"{len(states)} states for {len(tokens_list)} token lists")
        if not states:
            return []
        k = int(lookahead)
        backlog = []
        for st, toks in zip(states, tokens_list):
            if st.pool is not self:
                raise ValueError("draft state belongs to another pool")
            pending = list(toks[st.position:])
            if not pending:
                raise ValueError(f"draft is at position {st.position} with only {len(toks)} tokens")
            if len(toks) + k > self.max_len:
                raise ValueError(f"draft round reaches position {len(toks) + k - 1}, past {self.max_len - 1}")
            if len(pending) > 1:
                backlog.append((st, pending[:-1]))
        self._prefill_many(backlog)

        n = len(states)
        pos = [st.position for st in states]
        tables = [self._tables[st.slot] for st in states]
        last = [int(toks[-1]) for toks in tokens_list]
        if self.unroll and temperature <= 0.0 and k > 0:
            cand_dev = self._unrolled_round(n, k, last, pos, tables)
            cand = cand_dev.tolist()  # the round's one read-back
            vocab = self.model.get_output_embeddings().weight.shape[0]
            onehot = torch.zeros((n, k, vocab), dtype=torch.float32, device=self.device)
            onehot.scatter_(2, cand_dev[:, :, None], 1.0)
            for st in states:
                st.position += k + 1
            return [(cand[i], [onehot[i, j] for j in range(k)]) for i in range(n)]

        step_tokens: List[torch.Tensor] = []
        step_probs: List[torch.Tensor] = []
        nxt: Optional[torch.Tensor] = None
        for j in range(k + 1):
            logits = self._decoder.logits_view(last, [p + j for p in pos], tables, device_tokens=nxt)
            self.replays += 1
            if j == k:
                break  # the last step only caches the final candidate's K/V
            probs = _probs_from_logits_rows(logits.float(), temperature)
            nxt = probs.argmax(-1) if temperature <= 0.0 else torch.multinomial(probs, 1)[:, 0]
            step_tokens.append(nxt)
            step_probs.append(probs)
        cand = torch.stack(step_tokens, dim=1).tolist() if k else [[] for _ in range(n)]
        for st in states:
            st.position += k + 1
        return [(cand[i], [step_probs[j][i] for j in range(k)]) for i in range(n)]

    def _unrolled_round(self, n: int, k: int, last: List[int], pos: List[int],
                        tables: List[List[int]]) -> torch.Tensor:
        """A greedy round as one replay: K+1 captured steps, each with its own
        static inputs and plan, the argmax of step j written into step j+1's
        token buffer inside the graph. Returns the (n, K) candidates."""
        b = self._decoder._batch_bucket(n)
        if b > self.num_slots:
            raise ValueError(f"batch {n} exceeds {self.num_slots} draft slots")
        key = (b, k)
        buckets = self._ubuckets.get(key)
        if buckets is None:
            buckets = self._ubuckets[key] = [_Bucket(self._decoder, b) for _ in range(k + 1)]
        for j, bk in enumerate(buckets):
            self._decoder._stage(bk, last if j == 0 else [0] * n, [p + j for p in pos], tables)
        if key not in self._ugraph:
            self._capture_unrolled(key, buckets)
        self._ugraph[key].replay()
        self.replays += 1
        return self._uout[key][:n]

    def _unrolled_body(self, buckets: List[_Bucket]) -> torch.Tensor:
        k = len(buckets) - 1
        cands = torch.empty((buckets[0].b, k), dtype=torch.long, device=self.device)
        for j, bk in enumerate(buckets):
            logits = self._decoder._forward(bk)
            if j < k:
                nxt = logits.argmax(-1)
                cands[:, j].copy_(nxt)
                buckets[j + 1].tokens.copy_(nxt)
        return cands

    def _capture_unrolled(self, key: Tuple[int, int], buckets: List[_Bucket]) -> None:
        # one eager round on a side stream first (allocator and library
        # warm-up; it computes exactly what the replay then recomputes), then
        # the capture
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for bk in buckets:
                bk.binding.used = 0
            self._unrolled_body(buckets)
            for bk in buckets:
                if bk.binding.used != self.spec.num_layers:
                    raise RuntimeError(f"unrolled draft: {bk.binding.used} of {self.spec.num_layers} "
                                       "layers used the varlen kernel")
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self._decoder._mem_pool):
            self._uout[key] = self._unrolled_body(buckets)
        self._ugraph[key] = graph


@torch.no_grad()
def verify_candidates_batched(target_model, pool, buffers, block_tables: Sequence[torch.Tensor],
                              context_lengths: Sequence[int], query_tokens: Sequence[Sequence[int]],
                              device: str) -> Tuple[List[List[torch.Tensor]], List[Tuple[torch.Tensor, torch.Tensor]], int]:
    """One target pass over every sequence's candidate run (batched_speculative.py:645-728).

    Returns per-sequence logits (one tensor per query position), each layer's
    new K/V as ``(batch, kv_heads, query_len, head_dim)`` for
    ``scatter_accepted_kv``, and the widest context. ``buffers`` (the
    reference's padded-batch scratch) is unused: nothing is padded here.
    """
    logits, new_kv = verify_pass(target_model, pool, block_tables, context_lengths, query_tokens, device)
    batch, query_len = logits.shape[0], logits.shape[1]
    per_sequence_logits = [[logits[b, j] for j in range(query_len)] for b in range(batch)]
    return per_sequence_logits, new_kv, max(int(c) for c in context_lengths)


@torch.no_grad()
def verify_pass(target_model, pool, block_tables: Sequence, context_lengths: Sequence[int],
                query_tokens: Sequence[Sequence[int]], device: str) -> Tuple[torch.Tensor, List[Tuple[torch.Tensor, torch.Tensor]]]:
    """``verify_candidates_batched`` with the logits as one ``(batch,
    query_len, vocab)`` tensor (what the batched resolve consumes)."""
    batch = len(context_lengths)
    if batch == 0:
        raise ValueError("verify_candidates_batched requires at least one sequence")
    widths = {len(q) for q in query_tokens}
    if len(widths) != 1:
        raise ValueError(f"all sequences must propose the same count, got {widths}")
    query_len = widths.pop()
    if query_len < 1:
        raise ValueError("each sequence needs at least one query token")
    seq_ids = [b for b in range(batch) for _ in range(query_len)]
    positions = [int(c) + j for c in context_lengths for j in range(query_len)]
    total = len(seq_ids)
    num_layers = pool.spec.num_layers
    cache = VarlenPackedCache.verify(pool, num_layers, total)
    binding = attention_backend._VarlenBinding(pool, block_tables, seq_ids, positions,
                                               pool_lens=[int(c) for c in context_lengths])
    input_ids, position_ids = nat.upload(
        [np.asarray([[t for q in query_tokens for t in q]], dtype=np.int64),
         np.asarray([positions], dtype=np.int64)], device)
    with attention_backend.backend_enabled_on(target_model) as routed:
        if not routed:
            raise RuntimeError("verification needs the attention registry, which is unavailable")
        with attention_backend.bind_varlen(binding):
            out = target_model(input_ids=input_ids, position_ids=position_ids, past_key_values=cache,
                               use_cache=True)
    if binding.used != num_layers:
        raise RuntimeError(f"verify pass: {binding.used} of {num_layers} layers used the varlen kernel")
    logits = out.logits[0].view(batch, query_len, -1)
    new_kv = []
    for k, v in cache.new_kv:
        hkv, d = k.shape[1], k.shape[3]
        new_kv.append((k[0].view(hkv, batch, query_len, d).permute(1, 0, 2, 3),
                       v[0].view(hkv, batch, query_len, d).permute(1, 0, 2, 3)))
    return logits, new_kv


def resolve_round(seq_id: int, candidates: List[int], draft_probs: List[torch.Tensor],
                  target_logits: List[torch.Tensor], temperature: float) -> SpeculativeRound:
    """Clip the target to the draft vocabulary, then rejection-sample
    (batched_speculative.py:731-777)."""
    if draft_probs:
        width = draft_probs[0].shape[-1]
        target_logits = [logit[..., :width] for logit in target_logits]
    target_probs = [_probs_from_logits(logit, temperature) for logit in target_logits]
    accepted, is_draft, num_accepted = RejectionSampler.verify_tokens(candidates, draft_probs, target_probs)
    return SpeculativeRound(seq_id=seq_id, candidates=list(candidates), accepted=list(accepted),
                            is_draft=list(is_draft), num_accepted_draft=num_accepted)


def resolve_rounds_batched(seq_ids: Sequence[int], candidates: torch.Tensor, draft_probs: torch.Tensor,
                           target_logits: torch.Tensor, temperature: float, u_accept: torch.Tensor,
                           exp_noise: torch.Tensor) -> List[SpeculativeRound]:
    """Every row's rejection sampling in one mf_spec_verify launch.

    candidates (B, K) int, draft_probs (B, K, V) fp32, target_logits
    (B, K+1, >= V) -- clipped to V inside the kernel --, u_accept (B, K)
    uniforms and exp_noise (B, V) Exp(1) draws, all on the GPU. Row b uses
    u_accept[b][i] for candidate i and exp_noise[b] for its final draw.
    """
    res = nat.spec_verify(candidates, draft_probs, target_logits, temperature, u_accept, exp_noise)
    tokens = res.tokens.cpu().tolist()
    flags = res.is_draft.cpu().tolist()
    counts = res.count.cpu().tolist()
    nacc = res.num_accepted.cpu().tolist()
    cand = candidates.cpu().tolist()
    return [SpeculativeRound(seq_id=int(s), candidates=cand[b], accepted=tokens[b][: counts[b]],
                             is_draft=[bool(x) for x in flags[b][: counts[b]]], num_accepted_draft=nacc[b])
            for b, s in enumerate(seq_ids)]


def resolve_rounds_global_rng(seq_ids: Sequence[int], candidates: Sequence[Sequence[int]],
                              draft_probs: torch.Tensor, target_logits: torch.Tensor,
                              temperatures: Sequence[float]) -> List[SpeculativeRound]:
    """Every row of a speculative step resolved by ONE mf_spec_verify launch,
    with the same outcome, row for row, as ``resolve_round`` applied to the
    rows in order, up to fp32 near-ties in the final draw (the kernel ranks
    the candidates by fl(w / E) where the reference's ``multinomial`` sees w
    normalised twice first, two more roundings; accept decisions are exact)
    -- including what each consumes of torch's global
    generators (memforge_ml/runtime/continuous_engine.py:1295-1311,
    memforge_ml/speculative/rejection_sampler.py:28-83):

    1. row b's target distribution is ``_probs_from_logits`` at its own
       temperature over the draft's vocabulary width (the same torch softmax,
       row by row);
    2. the acceptance test needs p and q at each candidate, which cross to the
       host in one copy; the host then walks the CPU generator's stream as the
       reference does -- one uniform per examined candidate, row after row,
       stopping a row at its first rejection -- by drawing the most a round can
       use, replaying the walk, and re-drawing from the saved state exactly the
       count the walk used (``torch.rand(n)`` is ``n`` draws of
       ``torch.rand(1)`` on the CPU generator);
    3. each row's final draw takes one Exp(1) vector of the vocabulary's size
       from the GPU generator, in row order, as ``torch.multinomial`` would;
    4. the kernel draws every row at once, with the host's accept decisions
       passed in as forced uniforms (0 accepts, 2 rejects).

    ``draft_probs`` is (B, K, V) fp32 and ``target_logits`` (B, K+1, >= V),
    both on the GPU.
    """
    B = len(candidates)
    if B == 0:
        return []
    K = len(candidates[0])
    if any(len(c) != K for c in candidates):
        raise ValueError("every row must carry the same number of candidates")
    dev = target_logits.device
    V = draft_probs.shape[-1] if K else target_logits.shape[-1]
    logits = target_logits[..., :V].float()
    probs = torch.empty((B, K + 1, V), dtype=torch.float32, device=dev)
    groups: Dict[float, List[int]] = {}
    for b, t in enumerate(temperatures):
        groups.setdefault(float(t), []).append(b)
    for t, rows in groups.items():
        sel = logits if len(rows) == B else logits[rows]
        p = _probs_from_logits_rows(sel.reshape(-1, V), t).view(len(rows), K + 1, V)
        if len(rows) == B:
            probs.copy_(p)
        else:
            probs[rows] = p
    cand = torch.tensor(list(candidates), dtype=torch.int64).view(B, K).to(dev)
    # (2) p and q at each candidate, one copy to the host
    if K:
        pq = torch.stack([probs[:, :K].gather(2, cand[..., None])[..., 0],
                          draft_probs.gather(2, cand[..., None])[..., 0]]).cpu().double().tolist()
    saved = torch.get_rng_state()
    draws = torch.rand(B * K).tolist() if K else []
    forced = np.full((B, K), 2.0, dtype=np.float32)
    used = 0
    for b in range(B):
        for i in range(K):
            r = draws[used]
            used += 1
            if r <= min(1.0, pq[0][b][i] / (pq[1][b][i] + 1e-9)):
                forced[b, i] = 0.0
            else:
                break
    torch.set_rng_state(saved)
    if used:
        torch.rand(used)
    # (3) one Exp(1) vector per row on the GPU generator, in row order, each
    # drawn into a fresh vocabulary-sized tensor exactly as multinomial's
    # ``empty_like(p).exponential_(1)`` draws it
    noise = torch.stack([torch.empty(V, dtype=torch.float32, device=dev).exponential_(1.0) for _ in range(B)])
    # (4) one launch for every row
    u = torch.from_numpy(forced).to(dev)
    dp = draft_probs if K else torch.zeros((B, 0, V), dtype=torch.float32, device=dev)
    res = nat.spec_verify(cand.to(torch.int32), dp, probs, 1.0, u, noise, target_is_probs=True)
    out = torch.cat([res.tokens, res.is_draft.to(torch.int32), res.count[:, None],
                     res.num_accepted[:, None]], dim=1).cpu().tolist()
    rounds = []
    for b, s in enumerate(seq_ids):
        row = out[b]
        n = row[2 * (K + 1)]
        rounds.append(SpeculativeRound(seq_id=int(s), candidates=list(candidates[b]), accepted=row[:n],
                                       is_draft=[bool(x) for x in row[K + 1:K + 1 + n]],
                                       num_accepted_draft=row[2 * (K + 1) + 1]))
    return rounds


def confirmed_slot_mapping(tables: Sequence[Sequence[int]], context_lengths: Sequence[int],
                           confirmed: Sequence[int], width: int, block_size: int) -> np.ndarray:
    """Pool slots for a verify pass's packed rows (``width`` per sequence):
    row j of sequence b goes to position ctx_b + j when j < confirmed[b], and
    nowhere (slot -1) otherwise, so one KV write per layer stores exactly every
    sequence's confirmed prefix (batched_speculative.py:780-811 for all rows)."""
    slots = np.full((len(tables), width), -1, dtype=np.int64)
    for b, (table, ctx, n) in enumerate(zip(tables, context_lengths, confirmed)):
        if n <= 0:
            continue
        pos = np.arange(int(ctx), int(ctx) + int(n), dtype=np.int64)
        blocks = np.asarray(table, dtype=np.int64)[pos // block_size]
        slots[b, :n] = blocks * block_size + pos % block_size
    return slots.reshape(-1)


def scatter_confirmed_rows(pool, new_kv: Sequence[Tuple[torch.Tensor, torch.Tensor]],
                           slots: torch.Tensor) -> None:
    """One KV write per layer for every sequence's confirmed prefix:
    ``new_kv`` as ``verify_candidates_batched`` returns it ((B, kv_heads, width,
    head_dim) per layer), ``slots`` from ``confirmed_slot_mapping`` on the GPU."""
    for layer_idx, (keys, values) in enumerate(new_kv):
        B, H, W, D = keys.shape
        rows_k = keys.permute(0, 2, 1, 3).reshape(B * W, H, D)
        rows_v = values.permute(0, 2, 1, 3).reshape(B * W, H, D)
        nat.kv_write(rows_k, rows_v, slots, pool.layer_view(layer_idx))


def scatter_accepted_kv(pool, block_table: torch.Tensor, context_length: int,
                        new_kv: Sequence[Tuple[torch.Tensor, torch.Tensor]], row: int, num_confirmed: int) -> None:
    """Write only the confirmed prefix of one row's candidate run
    (batched_speculative.py:780-811)."""
    if num_confirmed <= 0:
        return
    flat = pool.flat_indices(block_table, context_length, context_length + num_confirmed)
    for layer_idx, (keys, values) in enumerate(new_kv):
        pool.write_flat(layer_idx, flat, keys[row:row + 1, :, :num_confirmed, :],
                        values[row:row + 1, :, :num_confirmed, :])
