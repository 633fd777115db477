"""How a request turns logits into its next token.

The request-facing names, defaults and outcomes are the reference's
(memforge_ml/runtime/sampling.py:11-75): ``SamplingParams`` with
``clamped``, ``apply_top_p``, ``logits_to_probs``, ``sample_from_probs`` and
``sample_logits``. The distribution is fixed by three rules:

* temperature <= 0 is greedy: all mass on the FIRST maximal logit;
* otherwise softmax(logits / temperature), then the nucleus: in order of
  decreasing probability a token survives while the mass strictly before it
  is at most ``top_p`` (so the most likely token always survives), and the
  survivors are renormalised -- unless nothing would remain, in which case the
  softmax is kept as it is;
* a draw clamps negative weights to zero, renormalises (a uniform draw when
  the weights sum to zero or overflow) and takes one ``torch.multinomial``
  sample from the given generator, so a seeded request consumes its
  generator exactly as the reference does.

The nucleus is applied by rank: each token's rank in the descending order is
computed once, and a row keeps the ranks below its survivor count. The kept
values stay at their vocabulary positions, so the renormalising sum runs over
the same array in the same order as a sort-mask-scatter formulation would.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F


@dataclass
class SamplingParams:
    max_new_tokens: int = 128
    temperature: float = 0.7
    top_p: float = 0.9
    seed: Optional[int] = None
    stop_on_eos: bool = True

    @property
    def greedy(self) -> bool:
        return self.temperature <= 0.0

    def clamped(self, hard_max: int) -> "SamplingParams":
        """A copy whose token budget fits ``hard_max`` (and is at least one)."""
        return dataclasses.replace(self, max_new_tokens=max(1, min(self.max_new_tokens, hard_max)))


def _survivor_counts(ordered: torch.Tensor, top_p: float) -> torch.Tensor:
    """Per row, how many of the descending-ordered probabilities survive the
    nucleus: the mass before a token (an exclusive prefix sum, non-decreasing
    along the row) must be at most top_p."""
    mass_before = ordered.cumsum(dim=-1) - ordered
    return (mass_before <= top_p).sum(dim=-1, keepdim=True)


def apply_top_p(probs: torch.Tensor, top_p: float) -> torch.Tensor:
    """Nucleus filter over a ``(..., vocab)`` probability tensor
    (the reference's sampling.py:33-44 rule)."""
    if top_p >= 1.0:
        return probs
    ordered, order = probs.sort(dim=-1, descending=True)
    keep = _survivor_counts(ordered, top_p)
    ranks = torch.arange(probs.shape[-1], device=probs.device).expand_as(order)
    rank_of = torch.empty_like(order).scatter_(-1, order, ranks)
    kept = probs.masked_fill(rank_of >= keep, 0.0)
    mass = kept.sum(dim=-1, keepdim=True)
    return torch.where(mass > 0, kept / mass, probs)


def logits_to_probs(logits: torch.Tensor, temperature: float, top_p: float) -> torch.Tensor:
    """The distribution a token is drawn from (the reference's sampling.py:47-56)."""
    scores = logits.float()
    if temperature <= 0.0:
        return F.one_hot(scores.argmax(dim=-1), scores.shape[-1]).to(scores.dtype)
    return apply_top_p(torch.softmax(scores / temperature, dim=-1), top_p)


def sample_from_probs(probs: torch.Tensor, generator: Optional[torch.Generator] = None) -> int:
    """One token id from a 1-D weight vector (the reference's sampling.py:59-65)."""
    weights = probs.clamp_min(0.0)
    mass = weights.sum()
    usable = bool(torch.isfinite(mass)) and float(mass) > 0.0
    weights = weights / mass if usable else torch.full_like(weights, 1.0 / weights.numel())
    return int(torch.multinomial(weights, 1, generator=generator))


def sample_logits(logits: torch.Tensor, params: SamplingParams,
                  generator: Optional[torch.Generator] = None) -> int:
    """The next token of one request from its logits row."""
    if params.greedy:
        return int(logits.float().argmax())
    return sample_from_probs(logits_to_probs(logits, params.temperature, params.top_p), generator)
