"""CPU pins of the oracle: each oracle function is checked against something
that does not restate it -- a library routine (torch's bf16 conversion, SDPA,
``torch.multinomial``, ``index_copy_``), the reference tests' own known
answers, closed forms and invariants, or a Monte Carlo check of the theorem
the algorithm exists for. A planted mistake in the oracle (wrong rounding,
off-by-one causality, wrong GQA head mapping, a dropped renormalisation)
fails at least one of these."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oat
from oracle import bf16 as obf
from oracle import cpu_baseline
from oracle import paging as opg
from oracle import rejection as orj

# ----------------------------------------------------------------------- bf16


def test_bf16_rounding_equals_torch_on_random_and_edge_values():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.3895314e38, -3.3895314e38, 1e-40, -1e-45,
                  1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20], dtype=np.float32),
    ]).astype(np.float32)
    # exact ties at many magnitudes
    ties = (rng.integers(0, 1 << 16, 2000, dtype=np.uint32) << 16) | 0x8000
    x = np.concatenate([x, ties.view(np.float32)])
    x = x[~np.isnan(x) | (np.arange(x.size) == np.argmax(np.isnan(x)))]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = obf.f32_to_bf16_bits(x)
    finite = ~np.isnan(x)
    assert np.array_equal(got[finite], want[finite])
    assert np.all(got[~finite] & 0x7F80 == 0x7F80) and np.all(got[~finite] & 0x7F)  # NaN stays NaN
    assert np.array_equal(obf.round_to_bf16(x)[finite],
                          torch.from_numpy(x).to(torch.bfloat16).float().numpy()[finite])


# ------------------------------------------------------------------ attention


def _pool(rng, n, bs, hkv, d):
    return (rng.standard_normal((n, bs, hkv, d)), rng.standard_normal((n, bs, hkv, d)))


def _dense(pool, table, n, bs):
    pos = np.arange(n)
    return pool[np.asarray(table)[pos // bs], pos % bs]  # (n, Hkv, D)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (6, 1)])
@pytest.mark.parametrize("bs", [1, 4, 16])
def test_varlen_attention_equals_sdpa_causal_slices(hq, hkv, bs):
    """Rows of several sequences packed in any order equal rows of a full
    causal SDPA (torch's own causal mask and GQA mapping) over each sequence."""
    rng = np.random.default_rng(hq * 100 + bs)
    d, lens = 32, [1, 9, 23]
    need = sum((n + bs - 1) // bs for n in lens)
    kp, vp = _pool(rng, need + 3, bs, hkv, d)
    perm = rng.permutation(need + 3)
    tables, k = [], 0
    for n in lens:
        nb = (n + bs - 1) // bs
        tables.append(perm[k:k + nb].tolist())
        k += nb
    # decode of seq 0, a prefill chunk of seq 1 (rows 4..8), full prefill of seq 2; shuffled
    rows = [(0, 0)] + [(1, p) for p in range(4, 9)] + [(2, p) for p in range(23)]
    order = rng.permutation(len(rows))
    rows = [rows[i] for i in order]
    seq_ids = [s for s, _ in rows]
    positions = [p for _, p in rows]
    q = rng.standard_normal((hq, len(rows), d))
    got = oat.varlen_attention(q, kp, vp, tables, seq_ids, positions, bs)
    for s, n in enumerate(lens):
        keys = torch.from_numpy(_dense(kp, tables[s], n, bs)).permute(1, 0, 2)[None]
        vals = torch.from_numpy(_dense(vp, tables[s], n, bs)).permute(1, 0, 2)[None]
        mine = [r for r, (ss, _) in enumerate(rows) if ss == s]
        qfull = torch.zeros((1, hq, n, d), dtype=torch.float64)
        for r in mine:
            qfull[0, :, rows[r][1]] = torch.from_numpy(q[:, r])
        ref = F.scaled_dot_product_attention(qfull, keys, vals, is_causal=True, enable_gqa=hq != hkv)[0]
        for r in mine:
            np.testing.assert_allclose(got[:, r], ref[:, rows[r][1]].numpy(), rtol=1e-12, atol=1e-12)


def test_varlen_attention_closed_forms_and_scale():
    rng = np.random.default_rng(3)
    kp, vp = _pool(rng, 4, 4, 2, 8)
    q = rng.standard_normal((4, 2, 8))
    # a row at position 0 sees exactly one key: output is that value row
    out = oat.varlen_attention(q, kp, vp, [[2], [3]], [0, 1], [0, 0], 4)
    np.testing.assert_allclose(out[:, 0], np.repeat(vp[2, 0], 2, axis=0), rtol=0, atol=1e-15)
    np.testing.assert_allclose(out[:, 1], np.repeat(vp[3, 0], 2, axis=0), rtol=0, atol=1e-15)
    # scale 0 -> uniform weights -> mean of the visible values
    out = oat.varlen_attention(q[:, :1], kp, vp, [[1, 0]], [0], [6], 4, scale=0.0)
    vals = _dense(vp, [1, 0], 7, 4).mean(axis=0)
    np.testing.assert_allclose(out[:, 0], np.repeat(vals, 2, axis=0), atol=1e-14)
    # an explicit scale equals SDPA's ``scale`` argument
    keys = torch.from_numpy(_dense(kp, [1, 0], 7, 4)).permute(1, 0, 2)[None]
    vals_t = torch.from_numpy(_dense(vp, [1, 0], 7, 4)).permute(1, 0, 2)[None]
    out = oat.varlen_attention(q[:, :1], kp, vp, [[1, 0]], [0], [6], 4, scale=0.3)
    ref = F.scaled_dot_product_attention(torch.from_numpy(q[:, :1])[None], keys, vals_t, scale=0.3,
                                         enable_gqa=True)[0]
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-13)


def test_in_flight_keys_equal_keys_written_to_the_pool():
    """A verify pass (keys >= pool_len read from the new rows) equals the same
    pass after those rows are written into the pool."""
    rng = np.random.default_rng(4)
    bs, hkv, d = 4, 2, 16
    kp, vp = _pool(rng, 12, bs, hkv, d)
    tables = [[3, 7, 1, 9], [0, 5, 11, 2]]
    ctx = [6, 9]
    seq_ids = [0] * 4 + [1] * 4
    positions = [6, 7, 8, 9, 9, 10, 11, 12]
    new_k = rng.standard_normal((8, hkv, d))
    new_v = rng.standard_normal((8, hkv, d))
    q = rng.standard_normal((4, 8, d))
    got = oat.varlen_attention(q, kp, vp, tables, seq_ids, positions, bs, pool_lens=ctx, new_k=new_k,
                               new_v=new_v, new_rows=[[0, 1, 2, 3], [4, 5, 6, 7]])
    kw, vw = kp.copy(), vp.copy()
    slots = opg.varlen_write_index(tables, seq_ids, positions, bs)
    opg.kv_write(kw, slots, new_k)
    opg.kv_write(vw, slots, new_v)
    want = oat.varlen_attention(q, kw, vw, tables, seq_ids, positions, bs)
    np.testing.assert_allclose(got, want, rtol=0, atol=0)


def test_paged_operator_equals_sdpa_without_a_mask():
    rng = np.random.default_rng(5)
    kc = rng.standard_normal((6, 2, 16, 8))
    vc = rng.standard_normal((6, 2, 16, 8))
    q = rng.standard_normal((1, 2, 3, 8))
    got = oat.paged_operator(q, kc, vc, [4, 1], 20)
    keys = torch.from_numpy(np.concatenate([kc[4], kc[1, :, :4]], axis=1))[None]
    vals = torch.from_numpy(np.concatenate([vc[4], vc[1, :, :4]], axis=1))[None]
    ref = F.scaled_dot_product_attention(torch.from_numpy(q), keys, vals)[0]
    np.testing.assert_allclose(got, ref.permute(1, 0, 2).reshape(1, 3, 16).numpy(), atol=1e-13)


def test_cpu_baseline_port_equals_the_oracle():
    rng = np.random.default_rng(6)
    kp, vp = _pool(rng, 20, 16, 2, 32)
    tables = [[3, 9, 1], [4], [7, 8, 10, 11]]
    ctx = [40, 16, 61]
    q = rng.standard_normal((3, 8, 32))
    got = cpu_baseline.decode_attention_cpu(torch.from_numpy(q), torch.from_numpy(kp), torch.from_numpy(vp),
                                            tables, ctx, 16).numpy()
    want = oat.varlen_attention(q.transpose(1, 0, 2), kp, vp, tables, [0, 1, 2], [c - 1 for c in ctx], 16)
    np.testing.assert_allclose(got, want.transpose(1, 0, 2), atol=1e-12)


def test_cpu_baseline_operator_and_varlen_ports_equal_the_oracle():
    """The C1 operator port against the operator oracle (itself pinned by
    SDPA), and the C2/C3 materialised varlen port -- causal chunks on a prior
    context beside decode rows, GQA 3:1 -- against the varlen oracle."""
    rng = np.random.default_rng(8)
    kc = rng.standard_normal((10, 3, 16, 32))
    vc = rng.standard_normal((10, 3, 16, 32))
    q = rng.standard_normal((1, 3, 2, 32))
    got = cpu_baseline.operator_cpu(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc), [6, 2, 9], 37)
    # the softmax runs in float32 (paged_attention.py:133), whatever the input dtype
    np.testing.assert_allclose(got.numpy(), oat.paged_operator(q, kc, vc, [6, 2, 9], 37), atol=1e-6)

    kp, vp = _pool(rng, 30, 16, 2, 32)
    tables = [[3, 9, 1, 12], [4], [7, 8, 10, 11, 20, 21]]
    q_lens, starts = [20, 1, 7], [30, 9, 80]
    cu = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    positions = [s + i for s, n in zip(starts, q_lens) for i in range(n)]
    seq_ids = [e for e, n in enumerate(q_lens) for _ in range(n)]
    qr = rng.standard_normal((sum(q_lens), 6, 32))
    got = cpu_baseline.varlen_cpu(torch.from_numpy(qr).float(), torch.from_numpy(kp).float(),
                                  torch.from_numpy(vp).float(), tables, cu, positions, 16).double().numpy()
    want = oat.varlen_attention(qr.astype(np.float32).transpose(1, 0, 2), kp.astype(np.float32),
                                vp.astype(np.float32), tables, seq_ids, positions, 16)
    np.testing.assert_allclose(got, want.transpose(1, 0, 2), atol=1e-5)


def test_cpu_baseline_greedy_equals_transformers_generate():
    """The C4 CPU baseline's greedy loop against transformers' own generate
    on a tiny random Llama (CPU)."""
    from tests.tiny_models import tiny_llama

    model = tiny_llama(num_layers=2, seed=3, device="cpu")
    prompts = [[5, 9, 33, 2, 7], [100, 3]]
    got = cpu_baseline.greedy_cpu(model, prompts, 6)
    for p, toks in zip(prompts, got):
        ref = model.generate(torch.tensor([p]), max_new_tokens=6, do_sample=False, min_new_tokens=6,
                             pad_token_id=0)[0, len(p):].tolist()
        assert toks == ref


# --------------------------------------------------------------------- paging


def test_slot_indices_known_answers_from_the_reference_tests():
    phys, slots = opg.slot_indices([5, 2, 7], 0, 10, 4)
    assert phys.tolist() == [5, 5, 5, 5, 2, 2, 2, 2, 7, 7]
    assert slots.tolist() == [0, 1, 2, 3, 0, 1, 2, 3, 0, 1]
    phys, slots = opg.slot_indices([5, 2, 7], 6, 9, 4)
    assert phys.tolist() == [2, 2, 7] and slots.tolist() == [2, 3, 0]
    with pytest.raises(IndexError, match="outside a block table"):
        opg.slot_indices([5, 2], 0, 12, 4)


def test_kv_write_and_gather_follow_index_copy_and_index_select():
    rng = np.random.default_rng(7)
    pool = rng.standard_normal((6, 4, 2, 3))
    rows = rng.standard_normal((5, 2, 3))
    slots = np.array([17, 2, 9, 22, 0])
    got = pool.copy()
    opg.kv_write(got, slots, rows)
    ref = torch.from_numpy(pool.copy()).view(24, 2, 3)
    ref.index_copy_(0, torch.from_numpy(slots), torch.from_numpy(rows))
    assert np.array_equal(got.reshape(24, 2, 3), ref.numpy())
    assert np.array_equal(opg.kv_gather(got, slots), torch.index_select(ref, 0, torch.from_numpy(slots)).numpy())


def test_varlen_write_index_checks_and_messages():
    tables = [[3, 8], [0]]
    assert opg.varlen_write_index(tables, [1, 0, 0], [2, 4, 0], 4).tolist() == [2, 32, 12]
    with pytest.raises(ValueError, match="same pool slot"):
        opg.varlen_write_index(tables, [0, 0], [1, 1], 4)
    with pytest.raises(IndexError, match="logical block"):
        opg.varlen_write_index(tables, [1], [4], 4)
    with pytest.raises(IndexError, match="no block table"):
        opg.varlen_write_index(tables, [2], [0], 4)
    with pytest.raises(ValueError, match="negative position"):
        opg.varlen_write_index(tables, [0], [-1], 4)


def test_ragged_pack_agrees_with_the_write_index_and_reports_faults():
    entries = [(3, 4, 7, [9, 2], [11, 12, 13]), (1, 5, 6, [4, 6], [40]), (2, 0, 2, [1], [7, 8])]
    got = opg.ragged_pack(entries, 4, 3)
    assert got["token_ids"].tolist() == [11, 12, 13, 40, 7, 8]
    assert got["positions"].tolist() == [4, 5, 6, 5, 0, 1]
    assert got["cu_seqlens"].tolist() == [0, 3, 4, 6] and got["kv_lens"].tolist() == [7, 6, 2]
    want = opg.varlen_write_index([[9, 2], [4, 6], [1]], [0, 0, 0, 1, 2, 2], [4, 5, 6, 5, 0, 1], 4)
    assert got["slot_mapping"].tolist() == want.tolist()
    assert got["block_tables"].tolist() == [[9, 2, 0], [4, 6, 0], [1, 0, 0]]
    assert got["first_overflow_row"] == -1 and got["first_duplicate_row"] == -1
    bad = opg.ragged_pack([(2, 3, 5, [1], [1, 2]), (1, 1, 2, [1], [3])], 4, 1)
    assert bad["slot_mapping"].tolist() == [7, -1, 5] and bad["first_overflow_row"] == 1
    dup = opg.ragged_pack([(1, 1, 2, [1], [1]), (1, 1, 2, [1], [3])], 4, 1)
    assert dup["first_duplicate_row"] == 1


# ------------------------------------------------------------------ rejection


@pytest.mark.parametrize("seed", range(20))
def test_multinomial_is_argmax_of_p_over_exponential_noise(seed):
    """torch.multinomial(p, 1) consumes one Exp(1) draw per entry and returns
    argmax(p / E) -- the identity the explicit-noise oracle rests on."""
    g = torch.Generator().manual_seed(seed)
    p = torch.softmax(torch.randn(500, generator=g) * 3, dim=-1)
    p[::11] = 0.0
    torch.manual_seed(seed)
    a = int(torch.multinomial(p, 1).item())
    torch.manual_seed(seed)
    e = torch.empty_like(p).exponential_(1.0)
    assert a == int(torch.argmax(p / e))
    torch.manual_seed(seed)
    assert orj.sample_from_probs(p.numpy(), torch.empty_like(p).exponential_(1.0).numpy()) == a


@pytest.mark.parametrize("seed", range(30))
def test_explicit_randomness_oracle_equals_the_torch_rng_restatement(seed):
    """Drawing u and E in the reference's order and handing them to the
    explicit oracle gives what the torch-RNG restatement (torch.rand,
    torch.multinomial) gives under the same seed."""
    g = torch.Generator().manual_seed(500 + seed)
    k, v = 4, 64
    target = [torch.softmax(torch.randn(v, generator=g) * 2, -1) for _ in range(k + 1)]
    mix = (seed % 4) / 3.0
    draft = [mix * target[i] + (1 - mix) * torch.softmax(torch.randn(v, generator=g) * 2, -1) for i in range(k)]
    toks = [int(torch.multinomial(d, 1, generator=g)) for d in draft]
    torch.manual_seed(seed)
    want = orj.verify_tokens_global_rng(toks, draft, target)
    torch.manual_seed(seed)
    u = []
    for i in range(k):
        u.append(float(torch.rand(1).item()))
        q, p = float(draft[i][toks[i]]), float(target[i][toks[i]])
        if not u[-1] <= min(1.0, p / (q + 1e-9)):
            break
    noise = torch.empty(v).exponential_(1.0).numpy()
    u += [0.0] * (k - len(u))
    got = orj.verify_tokens(toks, [d.numpy() for d in draft], [t.numpy() for t in target], u, noise)
    assert got == want


def test_reference_known_answers():
    v = 100
    draft = [np.zeros(v, np.float32) for _ in range(4)]
    target = [np.zeros(v, np.float32) for _ in range(5)]
    for i, t in enumerate([10, 20, 30, 40]):
        draft[i][t] = target[i][t] = 1.0
    target[4][50] = 1.0
    noise = np.ones(v, np.float32)
    assert orj.verify_tokens([10, 20, 30, 40], draft, target, [0.99] * 4, noise) == (
        [10, 20, 30, 40, 50], [True, True, True, True, False], 4)
    draft = [np.zeros(50, np.float32)]
    target = [np.zeros(50, np.float32), np.zeros(50, np.float32)]
    draft[0][15] = 1.0
    target[0][25] = 1.0
    assert orj.verify_tokens([15], draft, target, [0.5], np.ones(50, np.float32)) == ([25], [False], 0)


def test_probs_from_logits_and_vocab_clipping():
    rng = np.random.default_rng(9)
    logits = rng.standard_normal(40).astype(np.float32) * 3
    np.testing.assert_allclose(orj.probs_from_logits(logits, 0.7),
                               torch.softmax(torch.from_numpy(logits) / 0.7, -1).numpy(), rtol=2e-6, atol=1e-8)
    one = orj.probs_from_logits(logits, 0.0)
    assert one.sum() == 1.0 and one[np.argmax(logits)] == 1.0
    # greedy verify: accept while the candidate is the target argmax, then the argmax
    t = [np.full(8, -5.0, np.float32) for _ in range(3)]
    t[0][3] = t[1][6] = t[2][1] = 5.0
    d = [np.eye(8, dtype=np.float32)[3], np.eye(8, dtype=np.float32)[2]]
    assert orj.resolve_round([3, 2], d, t, 0.0, [0.5, 0.5], np.ones(8, np.float32)) == ([3, 6], [True, False], 1)
    # a wider target vocabulary is clipped to the draft's before the softmax
    wide = [np.concatenate([x, np.full(4, 50.0, np.float32)]) for x in t]
    assert orj.resolve_round([3, 2], d, wide, 0.0, [0.5, 0.5], np.ones(8, np.float32)) == ([3, 6], [True, False], 1)


def test_speculative_sampling_preserves_the_target_distribution():
    """The first emitted token of a round is distributed as the target p,
    whatever the draft q (the theorem rejection sampling exists for)."""
    rng = np.random.default_rng(11)
    p = np.array([0.05, 0.4, 0.1, 0.25, 0.2], np.float32)
    q = np.array([0.3, 0.1, 0.3, 0.1, 0.2], np.float32)
    n = 40000
    counts = np.zeros(5)
    toks = rng.choice(5, size=n, p=q / q.sum())
    us = rng.random(n)
    noise = rng.exponential(size=(n, 5)).astype(np.float32)
    for i in range(n):
        acc, _, _ = orj.verify_tokens([int(toks[i])], [q], [p, p], [us[i]], noise[i])
        counts[acc[0]] += 1
    expected = p * n
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 20.5, (counts, expected)  # 4 dof, p ~ 4e-4


def test_accept_rule_zero_uniform_accepts_zero_target_mass():
    """Closed form of the accept test r <= min(1, p / (q + 1e-9))
    (rejection_sampler.py:55-57): a uniform of exactly 0.0 accepts a
    candidate whose target probability is 0 (ratio 0, and 0 <= 0), and any
    positive uniform rejects it. The explicit-noise oracle and the global-RNG
    restatement both follow it; the generator position that yields an exact
    0.0 draw is the one the GPU tests use."""
    V = 8
    q = np.full(V, 1.0 / V, dtype=np.float32)
    p = np.zeros(V, dtype=np.float32)
    p[3] = 1.0
    noise = np.ones(V, dtype=np.float32)
    acc, flags, n = orj.verify_tokens([5, 6], [q, q], [p, p, p], [0.0, 0.0], noise)
    assert acc == [5, 6, 3] and flags == [True, True, False] and n == 2
    acc, flags, n = orj.verify_tokens([5, 6], [q, q], [p, p, p], [0.0, 2.0 ** -24], noise)
    assert acc == [5, 3] and flags == [True, False] and n == 1
    # torch.rand's CPU stream at seed 0 holds an exact 0.0 at this position
    torch.manual_seed(0)
    torch.rand(41102971)
    assert torch.rand(1).item() == 0.0
    torch.manual_seed(0)
    torch.rand(41102971)
    acc, flags, n = orj.verify_tokens_global_rng([5], [torch.from_numpy(q)], [torch.from_numpy(p)] * 2)
    assert acc[0] == 5 and flags[0] is True
