"""Speculative rejection sampling, with the vocabulary-wide work on the MI355X.

Same API and outcome as the reference (memforge_ml/speculative/
rejection_sampler.py:12-83), including its use of torch's global generators in
the same order: one ``torch.rand(1)`` per examined candidate, then for the
draw that ends the round one Exp(1) vector of the vocabulary's size on the
probabilities' device -- exactly what ``torch.multinomial(p, 1)`` consumes, as
it samples ``argmax(p / E)``. The accept decisions are a handful of scalar
comparisons on the host (they need those host draws); the residual
``max(p - q, 0)``, its normalisations and the ``argmax(w / E)`` over the
vocabulary run in the mf_spec_verify kernel.
"""

from __future__ import annotations

from typing import List, Tuple

import torch

from memforge_amd import _native as nat


def _device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


def _draw(probs_rows: torch.Tensor, draft_rows: torch.Tensor, tokens: List[int], noise: torch.Tensor,
          stop: int, reject: bool) -> int:
    """Final draw of a round through the kernel: candidates before ``stop`` are
    forced accepted (u = 0), the one at ``stop`` forced rejected (u = 2) when
    ``reject``, else every candidate is accepted and the bonus row is drawn."""
    dev = _device()
    k = stop + 1 if reject else stop
    u = torch.zeros((1, k), dtype=torch.float32)
    if reject:
        u[0, stop] = 2.0
    V = probs_rows.shape[-1]
    target = probs_rows[: k + (0 if reject else 1)].to(dev, torch.float32)
    if reject:  # the kernel wants k+1 target rows; the extra row is never read
        target = torch.cat([target, target[-1:]], dim=0)
    res = nat.spec_verify(
        torch.tensor([tokens[:k]], dtype=torch.int32).to(dev) if k else torch.zeros((1, 0), dtype=torch.int32, device=dev),
        draft_rows[:k].to(dev, torch.float32).reshape(1, k, V) if k else torch.zeros((1, 0, V), device=dev),
        target.reshape(1, k + 1, V).contiguous(), 1.0, u.to(dev),
        noise.to(dev, torch.float32).reshape(1, V), target_is_probs=True,
    )
    return int(res.tokens[0, k if not reject else stop].item())


class RejectionSampler:
    @staticmethod
    def sample_from_probs(probs: torch.Tensor) -> int:
        """One token from a 1-D distribution: clamp at 0, renormalise (uniform
        when the sum is 0), multinomial (rejection_sampler.py:12-26)."""
        noise = torch.empty_like(probs, dtype=torch.float32).exponential_(1.0)
        return _draw(probs.reshape(1, -1), torch.zeros((0, probs.numel())), [], noise, 0, False)

    @staticmethod
    def verify_tokens(draft_tokens: List[int], draft_probs: List[torch.Tensor],
                      target_probs: List[torch.Tensor]) -> Tuple[List[int], List[bool], int]:
        """Rejection sampling over K draft tokens (rejection_sampler.py:28-83).
        Returns (accepted tokens, is-draft flags, draft tokens accepted)."""
        k = len(draft_tokens)
        accepted: List[int] = []
        is_draft: List[bool] = []
        if k:
            d = torch.stack([p.float() for p in draft_probs])
            t = torch.stack([p.float() for p in target_probs[:k]])
            idx = torch.tensor(list(draft_tokens), dtype=torch.long, device=d.device).view(-1, 1)
            q = d.gather(1, idx).view(-1).cpu().tolist()
            p = t.gather(1, idx.to(t.device)).view(-1).cpu().tolist()
        for i in range(k):
            acceptance = min(1.0, p[i] / (q[i] + 1e-9))
            r = float(torch.rand(1).item())
            if r <= acceptance:
                accepted.append(int(draft_tokens[i]))
                is_draft.append(True)
                continue
            noise = torch.empty_like(target_probs[i], dtype=torch.float32).exponential_(1.0)
            rows = torch.stack([x.float() for x in target_probs[: i + 1]])
            accepted.append(_draw(rows, torch.stack([x.float() for x in draft_probs[: i + 1]]),
                                  list(draft_tokens), noise, i, True))
            is_draft.append(False)
            return accepted, is_draft, i
        if len(target_probs) > k:
            noise = torch.empty_like(target_probs[k], dtype=torch.float32).exponential_(1.0)
            rows = torch.stack([x.float() for x in target_probs[: k + 1]])
            drafts = torch.stack([x.float() for x in draft_probs]) if k else torch.zeros((0, rows.shape[-1]))
            accepted.append(_draw(rows, drafts, list(draft_tokens), noise, k, False))
            is_draft.append(False)
        return accepted, is_draft, k
