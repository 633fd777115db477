"""Rejection-sampling verify kernel: accepted-token sequences bit-exact against
the oracle's restatement of RejectionSampler.verify_tokens given the same
randomness (uniforms for the accept tests, Exp(1) noise for the final draw)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from memforge_amd import _native as nat
from oracle import rejection as orj

pytestmark = pytest.mark.gpu


def _run_both(device, draft_logits, target_logits, draft_tokens, u, noise, temperature):
    """draft_logits (B, K, V); target_logits (B, K+1, Vt >= V)."""
    B, K, V = draft_logits.shape
    draft_probs = torch.stack([
        torch.from_numpy(np.stack([orj.probs_from_logits(draft_logits[b, i].numpy(), temperature)
                                   for i in range(K)])) for b in range(B)])
    res = nat.spec_verify(draft_tokens.to(device), draft_probs.to(device), target_logits.to(device),
                          temperature, u.to(device), noise.to(device))
    tokens = res.tokens.cpu().numpy()
    flags = res.is_draft.cpu().numpy()
    count = res.count.cpu().numpy()
    nacc = res.num_accepted.cpu().numpy()
    for b in range(B):
        want_tok, want_flags, want_acc = orj.resolve_round(
            draft_tokens[b].tolist(), [draft_probs[b, i].numpy() for i in range(K)],
            [target_logits[b, i].numpy() for i in range(K + 1)], temperature,
            u[b].tolist(), noise[b].numpy())
        n = int(count[b])
        assert tokens[b, :n].tolist() == want_tok, f"row {b}"
        assert [bool(x) for x in flags[b, :n]] == want_flags, f"row {b}"
        assert int(nacc[b]) == want_acc, f"row {b}"
    return count, nacc


def _inputs(seed, B, K, V, Vt=None, agree=0.0):
    """N(0,2) logits (std sqrt(2)); target = agree * draft + noise, so larger
    `agree` gives a higher acceptance rate."""
    gen = torch.Generator().manual_seed(seed)
    Vt = Vt or V
    draft = torch.randn((B, K, V), generator=gen) * math.sqrt(2.0)
    target = torch.randn((B, K + 1, Vt), generator=gen) * math.sqrt(2.0)
    target[:, :K, :V] = agree * draft + (1 - agree) * target[:, :K, :V]
    probs = torch.softmax(draft, dim=-1)
    tokens = torch.multinomial(probs.reshape(B * K, V), 1, generator=gen).reshape(B, K).to(torch.int32)
    u = torch.rand((B, K), generator=gen)
    noise = torch.empty((B, V)).exponential_(1.0, generator=gen)
    return draft, target, tokens, u, noise


@pytest.mark.parametrize("agree", [0.0, 0.9, 1.0])
def test_c3_shape_bit_exact(device, agree):
    """Config 3's rejection step: 16 rows, k=4, vocab 49152, fp32 logits."""
    draft, target, tokens, u, noise = _inputs(0, 16, 4, 49152, agree=agree)
    count, nacc = _run_both(device, draft, target, tokens, u, noise, 1.0)
    if agree == 1.0:
        assert (nacc == 4).all() and (count == 5).all()


@pytest.mark.parametrize("temperature", [0.7, 1.3])
def test_temperatures_and_wider_target_vocab(device, temperature):
    """Target vocabulary wider than the draft's is clipped before the softmax
    (test_vocab_padding.py:6-35)."""
    draft, target, tokens, u, noise = _inputs(1, 8, 3, 3000, Vt=3128, agree=0.8)
    _run_both(device, draft, target, tokens, u, noise, temperature)


def test_greedy_known_answers(device):
    """temperature 0: a candidate equal to the target argmax is always accepted;
    the first that differs is replaced by the target argmax and ends the row
    (test_rejection_sampler.py:5-50, test_batched_speculative.py:320-376)."""
    B, K, V = 3, 4, 50
    gen = torch.Generator().manual_seed(2)
    target = torch.randn((B, K + 1, V), generator=gen)
    greedy = target.argmax(-1)
    draft = torch.randn((B, K, V), generator=gen)
    tokens = greedy[:, :K].clone().to(torch.int32)
    tokens[1, 2] = (greedy[1, 2] + 1) % V   # row 1 diverges at position 2
    tokens[2, 0] = (greedy[2, 0] + 7) % V   # row 2 diverges at once
    # one-hot drafts on the proposed tokens (the greedy draft distribution)
    for b in range(B):
        for i in range(K):
            draft[b, i] = -1e4
            draft[b, i, int(tokens[b, i])] = 0.0
    u = torch.rand((B, K), generator=gen)
    noise = torch.empty((B, V)).exponential_(1.0, generator=gen)
    count, nacc = _run_both(device, draft, target, tokens, u, noise, 0.0)
    assert nacc.tolist() == [4, 2, 0] and count.tolist() == [5, 3, 1]


def test_draw_families_residual_target_uniform(device):
    """The three branches of the final draw, on target probabilities given as
    such: a rejection whose residual max(p - q, 0) has mass draws from it; a
    rejection where the target equals the draft (no residual mass) draws from
    the target; a bonus position with no target mass draws uniformly (the
    smallest Exp(1) draw wins). Checked against the oracle's restatement."""
    B, K, V = 3, 2, 4000
    gen = torch.Generator().manual_seed(5)
    draft = torch.softmax(torch.randn((B, K, V), generator=gen) * 2.0, dim=-1)
    target = torch.softmax(torch.randn((B, K + 1, V), generator=gen) * 2.0, dim=-1)
    tokens = torch.stack([torch.multinomial(draft[b], 1, generator=gen).view(-1) for b in range(B)]).to(torch.int32)
    u = torch.rand((B, K), generator=gen)
    # row 0: reject at once (u = 1 > any ratio below 1), residual has mass
    u[0, 0] = 1.0
    target[0, 0, int(tokens[0, 0])] = 0.5 * float(draft[0, 0, int(tokens[0, 0])])
    # row 1: target equals the draft at position 0, rejected by u = 1 since
    # p / (q + 1e-9) < 1: the residual is zero everywhere
    target[1, 0] = draft[1, 0]
    u[1, 0] = 1.0
    # row 2: both candidates accepted (u = 0), bonus position has no mass
    u[2] = 0.0
    target[2, K] = 0.0
    noise = torch.empty((B, V)).exponential_(1.0, generator=gen)
    res = nat.spec_verify(tokens.to(device), draft.to(device), target.to(device), 1.0, u.to(device),
                          noise.to(device), target_is_probs=True)
    tok = res.tokens.cpu().numpy()
    cnt = res.count.cpu().numpy()
    for b in range(B):
        want, flags, nacc = orj.verify_tokens(tokens[b].tolist(), [draft[b, i].numpy() for i in range(K)],
                                              [target[b, i].numpy() for i in range(K + 1)], u[b].tolist(),
                                              noise[b].numpy())
        assert tok[b, :cnt[b]].tolist() == want, f"row {b}"
    assert cnt.tolist() == [1, 1, 3]
    assert int(tok[2, 2]) == int(torch.argmin(noise[2]))


def test_zero_uniform_accepts_zero_probability_candidates(device):
    """The accept test is r <= min(1, p / (q + 1e-9)) (rejection_sampler.py:55-57),
    so r = 0.0 accepts even a candidate the target gives no mass: p = 0 gives
    a ratio of exactly 0, and 0 <= 0. Row 0 draws u = 0 at every candidate,
    each with p = 0, and keeps all of them plus the bonus; row 1 draws the
    smallest positive uniform at its second candidate, which then fails.
    Checked against the oracle and against the closed form."""
    B, K, V = 2, 3, 1000
    gen = torch.Generator().manual_seed(9)
    draft = torch.softmax(torch.randn((B, K, V), generator=gen) * 2.0, dim=-1)
    target = torch.softmax(torch.randn((B, K + 1, V), generator=gen) * 2.0, dim=-1)
    tokens = torch.stack([torch.multinomial(draft[b], 1, generator=gen).view(-1) for b in range(B)]).to(torch.int32)
    for b in range(B):
        for i in range(K):
            target[b, i, int(tokens[b, i])] = 0.0
    u = torch.zeros((B, K))
    u[1, 1] = float(np.float32(2.0 ** -24))
    noise = torch.empty((B, V)).exponential_(1.0, generator=gen)
    res = nat.spec_verify(tokens.to(device), draft.to(device), target.to(device), 1.0, u.to(device),
                          noise.to(device), target_is_probs=True)
    tok, cnt, nacc = res.tokens.cpu().numpy(), res.count.cpu().numpy(), res.num_accepted.cpu().numpy()
    for b in range(B):
        want, flags, n = orj.verify_tokens(tokens[b].tolist(), [draft[b, i].numpy() for i in range(K)],
                                           [target[b, i].numpy() for i in range(K + 1)], u[b].tolist(),
                                           noise[b].numpy())
        assert tok[b, :cnt[b]].tolist() == want and int(nacc[b]) == n, f"row {b}"
    assert nacc.tolist() == [K, 1] and cnt.tolist() == [K + 1, 2]
    assert tok[0, :K].tolist() == tokens[0].tolist()


def test_greedy_zero_uniform_accepts_a_mismatching_candidate(device):
    """At temperature 0 the target is a one-hot on its argmax, so a candidate
    that differs from it has p = 0 and q = 1 (a one-hot draft); u = 0 still
    accepts it (0 <= 0), where any positive uniform replaces it by the
    argmax (test_greedy_known_answers)."""
    B, K, V = 2, 4, 64
    gen = torch.Generator().manual_seed(12)
    target = torch.randn((B, K + 1, V), generator=gen)
    greedy = target.argmax(-1)
    tokens = ((greedy[:, :K] + 3) % V).to(torch.int32)  # every candidate differs from the argmax
    draft = torch.full((B, K, V), -1e4)
    for b in range(B):
        for i in range(K):
            draft[b, i, int(tokens[b, i])] = 0.0
    u = torch.zeros((B, K))
    u[1, 2] = 0.25
    noise = torch.empty((B, V)).exponential_(1.0, generator=gen)
    count, nacc = _run_both(device, draft, target, tokens, u, noise, 0.0)
    assert nacc.tolist() == [4, 2] and count.tolist() == [5, 3]



def test_repeated_calls_on_one_workspace_and_a_large_batch(device):
    """The binding keeps its scratch between calls: repeated calls give the
    oracle's tokens every time, and a batch of 1,100 rows (over a small
    vocabulary) resolves like a small one."""
    draft, target, tokens, u, noise = _inputs(21, 16, 4, 49152, agree=0.5)
    first = None
    for _ in range(3):
        count, nacc = _run_both(device, draft, target, tokens, u, noise, 1.0)
        first = (count, nacc) if first is None else first
        assert (count == first[0]).all() and (nacc == first[1]).all()
    draft, target, tokens, u, noise = _inputs(22, 1100, 2, 96, agree=0.5)
    _run_both(device, draft, target, tokens, u, noise, 0.9)


@pytest.mark.parametrize("V", [65537, 131080])
def test_vocabularies_past_one_batch_of_chunk_statistics(device, V):
    """Vocabularies over 8 x 8,192 entries: the accept walk combines each
    position's chunk statistics over several batches of loads (the batch past
    the last chunk clamped and masked). A round that rejects and one that
    accepts every candidate both match the oracle."""
    for agree, seed in ((0.0, 31), (1.0, 32)):
        draft, target, tokens, u, noise = _inputs(seed, 3, 3, V, agree=agree)
        _run_both(device, draft, target, tokens, u, noise, 1.0)
