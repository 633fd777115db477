"""GPU tests of the speculative path: the kernel-backed RejectionSampler as a
drop-in (same random numbers consumed in the same order as the reference's
torch code, same tokens), the batched verify pass with candidates attended in
flight, and the confirmed-prefix scatter (the reference's
tests/python/test_rejection_sampler.py, test_batched_speculative.py and
test_vocab_padding.py cover the same behaviour)."""

import numpy as np
import pytest
import torch

from oracle import rejection as orj
from tests.tiny_models import tiny_llama

pytestmark = pytest.mark.gpu


def _dist(g, v, sharp=1.0):
    return torch.softmax(torch.randn(v, generator=g) * sharp, dim=-1)


@pytest.mark.parametrize("seed", range(12))
def test_rejection_sampler_is_a_drop_in_for_the_reference_draws(device, seed):
    """Same seed -> same accepted tokens as the reference algorithm drawing
    from torch's global generators (torch.rand on the host, multinomial on
    the probabilities' device)."""
    from memforge_amd.speculative import RejectionSampler

    g = torch.Generator().manual_seed(1000 + seed)
    k, v = 4, 300
    # draft close to the target for some seeds, far for others
    target = [_dist(g, v, 3.0).to(device) for _ in range(k + 1)]
    mix = (seed % 3) / 2.0
    draft = [(mix * target[i] + (1 - mix) * _dist(g, v, 3.0).to(device)) for i in range(k)]
    tokens = [int(torch.multinomial(d.cpu(), 1, generator=g)) for d in draft]
    torch.manual_seed(seed)
    got = RejectionSampler.verify_tokens(tokens, draft, target)
    torch.manual_seed(seed)
    want = orj.verify_tokens_global_rng(tokens, draft, target)
    assert got == want


@pytest.mark.parametrize("seed", range(6))
def test_sample_from_probs_matches_multinomial(device, seed):
    from memforge_amd.speculative import RejectionSampler

    g = torch.Generator().manual_seed(seed)
    p = _dist(g, 1000, 2.0).to(device)
    p[::7] = 0.0
    torch.manual_seed(seed)
    got = RejectionSampler.sample_from_probs(p * 3.0)
    torch.manual_seed(seed)
    q = torch.clamp(p * 3.0, min=0.0)
    want = int(torch.multinomial(q / q.sum(), 1).item())
    assert got == want
    zero = torch.zeros(50, device=device)
    torch.manual_seed(seed)
    got0 = RejectionSampler.sample_from_probs(zero)
    torch.manual_seed(seed)
    assert got0 == int(torch.multinomial(torch.ones(50, device=device) / 50, 1).item())


def test_perfect_match_accepts_everything_and_adds_a_bonus(device):
    from memforge_amd.speculative import RejectionSampler

    v = 64
    probs = [torch.zeros(v, device=device) for _ in range(4)]
    for i, t in enumerate([5, 9, 11, 3]):
        probs[i][t] = 1.0
    acc, flags, n = RejectionSampler.verify_tokens([5, 9, 11], probs[:3], probs)
    assert acc == [5, 9, 11, 3] and flags == [True, True, True, False] and n == 3


def test_certain_rejection_resamples_from_the_residual(device):
    from memforge_amd.speculative import RejectionSampler

    v = 32
    draft = torch.zeros(v, device=device)
    draft[4] = 1.0
    target = torch.zeros(v, device=device)
    target[7] = 1.0
    acc, flags, n = RejectionSampler.verify_tokens([4, 4], [draft, draft], [target, target, target])
    assert acc == [7] and flags == [False] and n == 0


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_batched_resolve_matches_the_oracle(device, temperature):
    """resolve_rounds_batched (one kernel launch for every row) against the
    oracle's resolve_round with the same explicit uniforms and Exp(1) noise,
    including a target vocabulary wider than the draft's."""
    from memforge_amd.runtime.batched_speculative import resolve_rounds_batched

    g = torch.Generator().manual_seed(7)
    B, K, V, Vt = 6, 3, 200, 232
    draft_probs = torch.softmax(torch.randn((B, K, V), generator=g) * 2, dim=-1)
    target_logits = torch.randn((B, K + 1, Vt), generator=g) * 2
    target_logits[:, :K, :V] += torch.log(draft_probs + 1e-3)  # correlated, so some candidates pass
    cand = torch.stack([torch.multinomial(draft_probs[b], 1, generator=g).view(-1) for b in range(B)])
    u = torch.rand((B, K), generator=g)
    u[0] = 0.0  # row 0 accepts everything
    noise = torch.empty((B, V)).exponential_(1.0, generator=g)
    rounds = resolve_rounds_batched(list(range(B)), cand.to(device), draft_probs.to(device),
                                    target_logits.to(device), temperature, u.to(device), noise.to(device))
    for b in range(B):
        acc, flags, n = orj.resolve_round(cand[b].tolist(), list(draft_probs[b].numpy()),
                                          list(target_logits[b].numpy()), temperature, u[b].tolist(), noise[b].numpy())
        assert rounds[b].accepted == acc and rounds[b].is_draft == flags and rounds[b].num_accepted_draft == n


# ---------------------------------------------------------- batched verification


@pytest.fixture(scope="module")
def model(device):
    return tiny_llama(num_layers=2, seed=0)


def _prefill(model, pool, table, ids):
    from memforge_amd.runtime.paged_cache import PagedCache

    cache = PagedCache(pool, table)
    with torch.no_grad():
        model(input_ids=torch.tensor([ids], device="cuda:0"), past_key_values=cache, use_cache=True)


def test_batched_verification_matches_per_sequence_runs(model):
    from transformers.cache_utils import DynamicCache

    from memforge_amd.runtime.batched_speculative import scatter_accepted_kv, verify_candidates_batched
    from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool

    spec = ModelKVSpec.from_config(model.config, torch.float32, "cuda:0")
    pool = PagedKVPool(spec, num_blocks=64, block_size=4)
    prompts = [[5, 6, 7, 8, 9, 10, 11], [40, 41, 42], [90, 91, 92, 93, 94, 95, 96, 97, 98, 99, 100]]
    tables = [[3, 9, 14, 20], [1, 2], [30, 31, 32, 33, 34]]
    for t, p in zip(tables, prompts):
        _prefill(model, pool, t, p[:-1])
    queries = [[p[-1], 17, 18, 19] for p in prompts]
    before = [pool.gather_flat(0, pool.flat_indices(torch.tensor(t, device="cuda:0"), 0, 4 * len(t)))
              for t in tables]
    logits, new_kv, widest = verify_candidates_batched(
        model, pool, None, [torch.tensor(t, device="cuda:0") for t in tables], [len(p) - 1 for p in prompts],
        queries, "cuda:0")
    assert widest == max(len(p) - 1 for p in prompts)
    assert new_kv[0][0].shape == (3, 2, 4, 16)
    for b, (p, q) in enumerate(zip(prompts, queries)):
        cache = DynamicCache()
        with torch.no_grad():
            out = model(input_ids=torch.tensor([p[:-1] + q], device="cuda:0"), past_key_values=cache).logits[0]
        for j in range(4):
            torch.testing.assert_close(logits[b][j], out[len(p) - 1 + j], atol=2e-5, rtol=1e-4)
    # verification wrote nothing to the pool
    for t, (k0, v0) in zip(tables, before):
        k1, v1 = pool.gather_flat(0, pool.flat_indices(torch.tensor(t, device="cuda:0"), 0, 4 * len(t)))
        assert torch.equal(k0, k1) and torch.equal(v0, v1)
    # only the confirmed prefix is written
    tb = torch.tensor(tables[0], device="cuda:0")
    ctx = len(prompts[0]) - 1
    untouched = pool.gather_flat(1, pool.flat_indices(tb, ctx + 2, ctx + 4))
    scatter_accepted_kv(pool, tb, ctx, new_kv, 0, 2)
    for layer in range(2):
        k, v = pool.gather_flat(layer, pool.flat_indices(tb, ctx, ctx + 2))
        assert torch.equal(k[0], new_kv[layer][0][0, :, :2]) and torch.equal(v[0], new_kv[layer][1][0, :, :2])
    after = pool.gather_flat(1, pool.flat_indices(tb, ctx + 2, ctx + 4))
    assert torch.equal(after[0], untouched[0]) and torch.equal(after[1], untouched[1])
    scatter_accepted_kv(pool, tb, ctx, new_kv, 0, 0)  # a no-op


def test_batched_verification_rejects_bad_batches(model):
    from memforge_amd.runtime.batched_speculative import verify_candidates_batched
    from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool

    pool = PagedKVPool(ModelKVSpec.from_config(model.config, torch.float32, "cuda:0"), num_blocks=8, block_size=4)
    t = [torch.tensor([0, 1], device="cuda:0"), torch.tensor([2, 3], device="cuda:0")]
    with pytest.raises(ValueError):
        verify_candidates_batched(model, pool, None, t, [2, 2], [[1, 2], [1, 2, 3]], "cuda:0")
    with pytest.raises(ValueError):
        verify_candidates_batched(model, pool, None, [], [], [], "cuda:0")


def test_greedy_round_truncates_at_the_first_wrong_candidate(device):
    from memforge_amd.runtime.batched_speculative import resolve_round

    v = 16
    target = [torch.full((v,), -5.0, device=device) for _ in range(4)]
    for i, t in enumerate([3, 8, 2, 6]):
        target[i][t] = 5.0
    draft = [torch.zeros(v, device=device) for _ in range(3)]
    for i, t in enumerate([3, 9, 2]):
        draft[i][t] = 1.0
    r = resolve_round(1, [3, 9, 2], draft, target, 0.0)
    assert r.accepted == [3, 8] and r.is_draft == [True, False] and r.num_accepted_draft == 1


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("temps", [(1.0,), (0.0,), (0.7, 0.0, 1.3)])
def test_global_rng_batched_resolve_equals_row_by_row(device, seed, temps):
    """resolve_rounds_global_rng (one launch for every row) against
    resolve_round applied row after row, from the same global seeds: same
    rounds for every row, and both leave torch's CPU and GPU generators in
    the same state (the batched form consumes exactly what the rows would).
    Target logits are wider than the draft vocabulary (clipped first)."""
    from memforge_amd.runtime.batched_speculative import resolve_round, resolve_rounds_global_rng

    g = torch.Generator().manual_seed(seed)
    B, K, V, Vt = 6, 4, 3000, 3072
    target = (torch.randn((B, K + 1, Vt), generator=g) * 2).to(device)
    mix = (seed % 3) / 2.0
    dlog = torch.randn((B, K, V), generator=g) * 2
    dprobs = torch.softmax(mix * target[:, :K, :V].cpu() + (1 - mix) * dlog, dim=-1).to(device)
    cand = [[int(torch.multinomial(dprobs[b, i].cpu(), 1, generator=g)) for i in range(K)] for b in range(B)]
    t_rows = [temps[b % len(temps)] for b in range(B)]

    torch.manual_seed(seed)
    torch.cuda.manual_seed(seed)
    want = [resolve_round(b, cand[b], list(dprobs[b]), list(target[b]), t_rows[b]) for b in range(B)]
    cpu_after, gpu_after = torch.get_rng_state(), torch.cuda.get_rng_state()

    torch.manual_seed(seed)
    torch.cuda.manual_seed(seed)
    got = resolve_rounds_global_rng(list(range(B)), cand, dprobs, target, t_rows)
    assert [(r.accepted, r.is_draft, r.num_accepted_draft) for r in got] == \
           [(r.accepted, r.is_draft, r.num_accepted_draft) for r in want]
    assert torch.equal(torch.get_rng_state(), cpu_after)
    assert torch.equal(torch.cuda.get_rng_state(), gpu_after)


# torch.manual_seed(0), then torch.rand(ZERO_OFFSET): the next torch.rand(1)
# on the CPU generator is exactly 0.0 (pinned in tests/test_oracle.py)
ZERO_SEED, ZERO_OFFSET = 0, 41102971


@pytest.mark.parametrize("temperature", [1.0, 0.0])
def test_global_rng_resolve_accepts_a_zero_probability_candidate_at_u_zero(device, temperature):
    """The reference accepts a candidate when r <= min(1, p / (q + 1e-9))
    (rejection_sampler.py:55-57), so a draw of exactly 0.0 accepts a candidate
    with p = 0. Row 0's first candidate gets no target mass (a -inf logit, so
    softmax gives exactly 0, or a one-hot argmax elsewhere at temperature 0)
    and the global CPU generator is placed so that its next uniform is 0.0:
    the engine's batched resolve keeps the candidate, as the row-by-row
    resolve and the reference algorithm on the global generators do, and all
    three leave the generators in the same state."""
    from memforge_amd.runtime.batched_speculative import (_probs_from_logits, resolve_round,
                                                          resolve_rounds_global_rng)

    g = torch.Generator().manual_seed(11)
    B, K, V = 3, 4, 500
    target = torch.randn((B, K + 1, V), generator=g) * 2
    dprobs = torch.softmax(torch.randn((B, K, V), generator=g) * 2, dim=-1)
    cand = [[int(torch.multinomial(dprobs[b, i], 1, generator=g)) for i in range(K)] for b in range(B)]
    target[0, 0, cand[0][0]] = float("-inf")
    target, dprobs = target.to(device), dprobs.to(device)
    t_rows = [temperature] * B

    def seeded():
        torch.manual_seed(ZERO_SEED)
        torch.rand(ZERO_OFFSET)
        torch.cuda.manual_seed(5)

    seeded()
    want = [resolve_round(b, cand[b], list(dprobs[b]), list(target[b]), t_rows[b]) for b in range(B)]
    cpu_after, gpu_after = torch.get_rng_state(), torch.cuda.get_rng_state()
    seeded()
    got = resolve_rounds_global_rng(list(range(B)), cand, dprobs, target, t_rows)
    assert [(r.accepted, r.is_draft, r.num_accepted_draft) for r in got] == \
           [(r.accepted, r.is_draft, r.num_accepted_draft) for r in want]
    assert torch.equal(torch.get_rng_state(), cpu_after)
    assert torch.equal(torch.cuda.get_rng_state(), gpu_after)
    assert got[0].accepted[0] == cand[0][0] and got[0].is_draft[0]
    # the reference algorithm itself, row 0, from the same generator state
    seeded()
    probs0 = [_probs_from_logits(target[0, i], temperature) for i in range(K + 1)]
    assert float(probs0[0][cand[0][0]]) == 0.0
    acc, flags, n = orj.verify_tokens_global_rng(cand[0], list(dprobs[0]), probs0)
    assert (acc, flags, n) == (got[0].accepted, got[0].is_draft, got[0].num_accepted_draft)


def test_confirmed_prefix_scatter_writes_only_confirmed_rows(device):
    """One KV write per layer for every row's confirmed prefix: the pool
    holds exactly the rows scatter_accepted_kv would write one sequence at a
    time, and nothing else changes."""
    from memforge_amd.runtime.batched_speculative import (confirmed_slot_mapping, scatter_accepted_kv,
                                                           scatter_confirmed_rows)
    from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool

    spec = ModelKVSpec(num_layers=3, num_kv_heads=2, head_dim=64, dtype=torch.bfloat16, device=str(device))
    bs, W = 16, 5
    a, b = PagedKVPool(spec, 40, bs), PagedKVPool(spec, 40, bs)
    g = torch.Generator().manual_seed(4)
    tables = [[3, 17, 5], [8, 1], [30, 31, 32, 33]]
    ctx = [30, 14, 60]
    confirmed = [5, 0, 2]
    new_kv = [(torch.randn((3, 2, W, 64), generator=g).to(torch.bfloat16).to(device),
               torch.randn((3, 2, W, 64), generator=g).to(torch.bfloat16).to(device)) for _ in range(3)]
    slots = confirmed_slot_mapping(tables, ctx, confirmed, W, bs)
    assert slots.shape == (3 * W,) and (slots[W:2 * W] == -1).all() and (slots[2 * W + 2:] == -1).all()
    scatter_confirmed_rows(a, new_kv, torch.from_numpy(slots).to(device))
    for row in range(3):
        scatter_accepted_kv(b, torch.tensor(tables[row], device=device), ctx[row], new_kv, row, confirmed[row])
    assert torch.equal(a.key_pool, b.key_pool) and torch.equal(a.value_pool, b.value_pool)
    assert int((a.key_pool != 0).any(dim=(0, 2, 3, 4)).sum()) > 0
