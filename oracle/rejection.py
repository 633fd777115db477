"""Speculative rejection sampling with explicit randomness (test infrastructure only).

The reference draws its randomness from torch's global generator inside the
loop (memforge_ml/speculative/rejection_sampler.py:48-75): one ``torch.rand(1)``
per examined candidate and, for the final draw, ``torch.multinomial(p, 1)``,
which for one sample is ``argmax(p / E)`` with ``E`` an Exp(1) vector the same
size as ``p`` (PyTorch's multinomial fast path). Here both are inputs: ``u[i]``
is the uniform used for candidate i and ``noise`` the Exp(1) vector used for the
one draw that ends the round. Arithmetic follows the reference: probabilities
in float32 (numpy), the acceptance ratio in double (Python floats).
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np


def probs_from_logits(logits: np.ndarray, temperature: float) -> np.ndarray:
    """``_probs_from_logits`` (memforge_ml/runtime/batched_speculative.py:112-124):
    a one-hot on the first argmax at temperature <= 0, else softmax(logits / T)
    in float32."""
    logits = np.asarray(logits, dtype=np.float32)
    if temperature <= 0.0:
        out = np.zeros_like(logits)
        out[int(np.argmax(logits))] = 1.0
        return out
    x = logits / np.float32(temperature)
    e = np.exp(x - x.max())
    return (e / e.sum(dtype=np.float32)).astype(np.float32)


def sample_from_probs(probs: np.ndarray, noise: np.ndarray) -> int:
    """``RejectionSampler.sample_from_probs`` (rejection_sampler.py:12-26) with the
    Exp(1) draws supplied: clamp at 0, renormalise (uniform if the sum is 0),
    then ``argmax(p / E)`` (first index on ties)."""
    p = np.maximum(np.asarray(probs, dtype=np.float32), np.float32(0.0))
    total = p.sum(dtype=np.float32)
    if total == 0:
        p = np.full_like(p, np.float32(1.0) / np.float32(p.shape[0]))
    else:
        p = (p / total).astype(np.float32)
    return int(np.argmax(p / np.asarray(noise, dtype=np.float32)))


def verify_tokens(draft_tokens: Sequence[int], draft_probs: Sequence[np.ndarray],
                  target_probs: Sequence[np.ndarray], u: Sequence[float],
                  noise: np.ndarray) -> Tuple[List[int], List[bool], int]:
    """``RejectionSampler.verify_tokens`` (rejection_sampler.py:28-83) with
    explicit randomness. Returns (accepted tokens, is-draft flags, number of
    draft tokens accepted)."""
    accepted: List[int] = []
    is_draft: List[bool] = []
    k = len(draft_tokens)
    for i in range(k):
        tok = int(draft_tokens[i])
        q = float(np.float32(draft_probs[i][tok]))
        p = float(np.float32(target_probs[i][tok]))
        acceptance = min(1.0, p / (q + 1e-9))
        r = float(np.float32(u[i]))
        if r <= acceptance:
            accepted.append(tok)
            is_draft.append(True)
            continue
        diff = np.maximum(np.asarray(target_probs[i], np.float32) - np.asarray(draft_probs[i], np.float32),
                          np.float32(0.0))
        diff_sum = diff.sum(dtype=np.float32)
        if diff_sum > 0:
            tok2 = sample_from_probs((diff / diff_sum).astype(np.float32), noise)
        else:
            tok2 = sample_from_probs(target_probs[i], noise)
        accepted.append(tok2)
        is_draft.append(False)
        return accepted, is_draft, i
    if len(target_probs) > k:
        accepted.append(sample_from_probs(target_probs[k], noise))
        is_draft.append(False)
    return accepted, is_draft, k


def resolve_round(candidates: Sequence[int], draft_probs: Sequence[np.ndarray],
                  target_logits: Sequence[np.ndarray], temperature: float,
                  u: Sequence[float], noise: np.ndarray) -> Tuple[List[int], List[bool], int]:
    """``resolve_round`` (batched_speculative.py:731-777): clip target logits to
    the draft vocabulary width before the softmax, then verify."""
    if len(draft_probs):
        width = np.asarray(draft_probs[0]).shape[-1]
        target_logits = [np.asarray(t)[..., :width] for t in target_logits]
    target_probs = [probs_from_logits(t, temperature) for t in target_logits]
    return verify_tokens(candidates, draft_probs, target_probs, u, noise)


def verify_tokens_global_rng(draft_tokens, draft_probs, target_probs):
    """``RejectionSampler.verify_tokens`` (rejection_sampler.py:28-83) drawing
    from torch's global generators exactly as the reference does:
    ``torch.rand(1)`` per examined candidate and ``torch.multinomial`` on the
    probabilities' device for the draw that ends the round. Takes and returns
    what the reference does; used to check that a drop-in consumes the same
    random numbers in the same order."""
    import torch

    def draw(probs):
        probs = torch.clamp(probs, min=0.0)
        total = probs.sum()
        probs = torch.ones_like(probs) / probs.shape[0] if total == 0 else probs / total
        return int(torch.multinomial(probs, num_samples=1).item())

    accepted, is_draft = [], []
    for i, tok in enumerate(draft_tokens):
        q = float(draft_probs[i][tok].item())
        p = float(target_probs[i][tok].item())
        acceptance = min(1.0, p / (q + 1e-9))
        if float(torch.rand(1).item()) <= acceptance:
            accepted.append(int(tok))
            is_draft.append(True)
            continue
        diff = torch.clamp(target_probs[i] - draft_probs[i], min=0.0)
        total = diff.sum()
        accepted.append(draw(diff / total) if total > 0 else draw(target_probs[i]))
        is_draft.append(False)
        return accepted, is_draft, i
    if len(target_probs) > len(draft_tokens):
        accepted.append(draw(target_probs[len(draft_tokens)]))
        is_draft.append(False)
    return accepted, is_draft, len(draft_tokens)
