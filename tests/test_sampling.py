"""CPU tests of the sampling rules (memforge_ml/runtime/sampling.py:11-75):
the rank-based nucleus agrees bit for bit with the sort / mask / scatter
formulation of the same rule, greedy is the first argmax, and draws consume a
seeded generator exactly like torch.multinomial on the renormalised weights."""

import pytest
import torch

from memforge_amd.runtime.sampling import (SamplingParams, apply_top_p, logits_to_probs, sample_from_probs,
                                           sample_logits)


def _sort_mask_scatter(probs, top_p):
    """The same nucleus rule written the other way round: sort, zero the
    tokens whose preceding mass exceeds top_p, scatter back, renormalise."""
    if top_p >= 1.0:
        return probs
    ordered, order = torch.sort(probs, descending=True, dim=-1)
    before = torch.cumsum(ordered, dim=-1) - ordered
    ordered = ordered.masked_fill(before > top_p, 0.0)
    back = torch.zeros_like(probs).scatter(-1, order, ordered)
    mass = back.sum(dim=-1, keepdim=True)
    return torch.where(mass > 0, back / mass, probs)


@pytest.mark.parametrize("top_p", [0.0, 1e-6, 0.3, 0.9, 0.999, 1.0])
def test_nucleus_equals_the_sort_mask_scatter_form_bitwise(top_p):
    g = torch.Generator().manual_seed(int(top_p * 1000))
    logits = torch.randn((7, 500), generator=g) * 3
    logits[2, :] = 0.0                  # a row of ties
    logits[3, ::2] = -float("inf")      # half the vocabulary impossible
    probs = torch.softmax(logits, dim=-1)
    assert torch.equal(apply_top_p(probs, top_p), _sort_mask_scatter(probs, top_p))


def test_nucleus_keeps_the_top_token_and_renormalises():
    probs = torch.tensor([[0.5, 0.3, 0.15, 0.05]])
    assert torch.allclose(apply_top_p(probs, 0.0), torch.tensor([[1.0, 0.0, 0.0, 0.0]]))
    assert torch.allclose(apply_top_p(probs, 0.6), torch.tensor([[0.625, 0.375, 0.0, 0.0]]))
    # exact binary fractions: the mass before the third token is 0.75, at
    # most 0.75 (it survives) but above 0.7 (it does not)
    dyadic = torch.tensor([[0.5, 0.25, 0.125, 0.125]])
    assert (apply_top_p(dyadic, 0.75) > 0).sum() == 3
    assert (apply_top_p(dyadic, 0.7) > 0).sum() == 2


def test_greedy_is_a_one_hot_on_the_first_maximum():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0], [0.0, 0.0, 0.0, 0.0]])
    p = logits_to_probs(logits, 0.0, 0.9)
    assert p.tolist() == [[0.0, 1.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0]]
    assert sample_logits(logits[0], SamplingParams(temperature=0.0)) == 1
    assert sample_logits(logits[1], SamplingParams(temperature=-1.0)) == 0


def test_temperature_scales_before_the_softmax():
    logits = torch.randn(64, generator=torch.Generator().manual_seed(1))
    p = logits_to_probs(logits, 0.5, 1.0)
    assert torch.equal(p, torch.softmax(logits / 0.5, dim=-1))


def test_draws_consume_the_generator_like_multinomial():
    w = torch.rand(300, generator=torch.Generator().manual_seed(2))
    for seed in range(5):
        a = sample_from_probs(w, torch.Generator().manual_seed(seed))
        b = int(torch.multinomial(w / w.sum(), 1, generator=torch.Generator().manual_seed(seed)))
        assert a == b
    # negative weights count as zero; all-zero weights draw uniformly
    neg = torch.tensor([-1.0, 0.0, 2.0])
    assert all(sample_from_probs(neg, torch.Generator().manual_seed(s)) == 2 for s in range(10))
    zero = torch.zeros(4)
    picks = {sample_from_probs(zero, torch.Generator().manual_seed(s)) for s in range(40)}
    assert picks == {0, 1, 2, 3}


def test_sampled_tokens_follow_the_nucleus():
    logits = torch.tensor([4.0, 3.9, -5.0, -6.0])
    params = SamplingParams(temperature=1.0, top_p=0.5)
    g = torch.Generator().manual_seed(0)
    assert {sample_logits(logits, params, g) for _ in range(50)} <= {0, 1}


def test_clamped_budget():
    p = SamplingParams(max_new_tokens=100, temperature=0.3, seed=7)
    assert p.clamped(10).max_new_tokens == 10 and p.clamped(500).max_new_tokens == 100
    assert p.clamped(0).max_new_tokens == 1
    c = p.clamped(10)
    assert (c.temperature, c.top_p, c.seed, c.stop_on_eos) == (0.3, 0.9, 7, True) and c is not p
    assert SamplingParams() == SamplingParams(128, 0.7, 0.9, None, True)
