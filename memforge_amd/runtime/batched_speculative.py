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

The draft-side proposal loop is kept minimal (one DynamicCache per sequence);
CUDA-graph draft runners are not part of this build.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import torch
from transformers.cache_utils import DynamicCache

from memforge_amd import _native as nat
from memforge_amd.kernels import attention_backend
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
    binding = attention_backend._VarlenBinding(
        pool, block_tables, seq_ids, positions,
        pool_lens=torch.tensor([int(c) for c in context_lengths], dtype=torch.int32).to(device))
    input_ids = torch.tensor([[t for q in query_tokens for t in q]], dtype=torch.long, device=device)
    position_ids = torch.tensor([positions], dtype=torch.long, device=device)
    with attention_backend.backend_enabled_on(target_model) as routed:
        if not routed:
            raise RuntimeError("verification needs the attention registry, which is unavailable")
        with attention_backend.bind_varlen(binding):
            out = target_model(input_ids=input_ids, position_ids=position_ids, past_key_values=cache,
                               use_cache=True)
    if binding.used != num_layers:
        raise RuntimeError(f"verify pass: {binding.used} of {num_layers} layers used the varlen kernel")
    logits = out.logits[0].view(batch, query_len, -1)
    per_sequence_logits = [[logits[b, j] for j in range(query_len)] for b in range(batch)]
    new_kv = []
    for k, v in cache.new_kv:
        hkv, d = k.shape[1], k.shape[3]
        new_kv.append((k[0].view(hkv, batch, query_len, d).permute(1, 0, 2, 3),
                       v[0].view(hkv, batch, query_len, d).permute(1, 0, 2, 3)))
    return per_sequence_logits, new_kv, max(int(c) for c in context_lengths)


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
