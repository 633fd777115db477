"""GPU tests of ContinuousBatchingEngine: every step is one packed varlen pass
through the HIP kernels, and its greedy output must be exactly what plain
transformers decoding produces for each request on its own (the reference's
tests/python/test_continuous_engine.py, test_chunked_prefill.py,
test_prefix_sharing.py, test_fused_prefill.py and test_speculative_batching.py
cover the same behaviour)."""

import pytest
import torch

from tests.tiny_models import StubTokenizer, hf_greedy, tiny_llama

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(device):
    return tiny_llama(num_layers=2, seed=0)


@pytest.fixture(scope="module")
def draft(device):
    return tiny_llama(num_layers=1, seed=1)


@pytest.fixture(scope="module")
def tok():
    return StubTokenizer()


def greedy(n=8, **kw):
    from memforge_amd.runtime.sampling import SamplingParams

    return SamplingParams(max_new_tokens=n, temperature=0.0, top_p=1.0, **kw)


def make_engine(model, tok, **kw):
    from memforge_amd.runtime.continuous_engine import ContinuousBatchingEngine

    opts = dict(block_size=4, num_blocks=64, max_num_seqs=4, max_model_len=128)
    opts.update(kw)
    return ContinuousBatchingEngine(model, tok, **opts)


PROMPTS = ["alpha prompt", "a much longer beta prompt here", "gamma", "the fourth one, mid length"]


def expected(model, tok, prompts, n, stop_on_eos=True):
    return [hf_greedy(model, tok(p)["input_ids"], n, stop_on_eos=stop_on_eos) for p in prompts]


def test_batched_greedy_equals_plain_transformers(model, tok):
    engine = make_engine(model, tok)
    results = engine.generate(PROMPTS, greedy(10))
    for r, exp in zip(results, expected(model, tok, PROMPTS, 10)):
        assert r["token_ids"] == exp
    assert engine.total_forward_passes < sum(r["generated_tokens"] for r in results)
    assert engine.telemetry()["tokens_per_forward_pass"] > 1.0


@pytest.mark.parametrize("block_size", [4, 16])
def test_block_sizes_agree(model, tok, block_size):
    engine = make_engine(model, tok, block_size=block_size, num_blocks=256 // block_size)
    results = engine.generate(PROMPTS[:3], greedy(6))
    for r, exp in zip(results, expected(model, tok, PROMPTS[:3], 6)):
        assert r["token_ids"] == exp


def test_generates_the_requested_count_and_reclaims_every_block(model, tok):
    engine = make_engine(model, tok)
    total = engine.allocator.get_total_blocks()
    r = engine.generate("hello world", greedy(8, stop_on_eos=False))[0]
    assert r["generated_tokens"] == 8 and r["finish_reason"] == "length"
    assert r["time_to_first_token_ms"] is not None
    engine.step()
    assert engine.allocator.get_num_free_blocks() == total


def test_requests_can_join_while_others_are_running(model, tok):
    from memforge_amd.runtime.sampling import SamplingParams

    engine = make_engine(model, tok)
    first = engine.submit("early request", SamplingParams(max_new_tokens=12, temperature=0.0, stop_on_eos=False))
    for _ in range(3):
        engine.step()
    late = engine.submit("late request", SamplingParams(max_new_tokens=4, temperature=0.0, stop_on_eos=False))
    engine.step()
    engine.step()
    assert len(engine.runtimes[late].generated) >= 1 and not engine.runtimes[first].done
    engine.run_until_idle()
    assert engine.runtimes[first].generated == hf_greedy(model, tok("early request")["input_ids"], 12,
                                                         stop_on_eos=False)
    assert engine.runtimes[late].generated == hf_greedy(model, tok("late request")["input_ids"], 4,
                                                        stop_on_eos=False)
    assert engine.total_fused_steps > 0, "a prefill joined a step that also decoded"


def test_preempted_output_matches_an_unpressured_run(model, tok):
    prompts = ["prompt number one", "prompt number two", "prompt number three"]
    params = greedy(10, stop_on_eos=False)
    pressured = make_engine(model, tok, num_blocks=12, max_num_seqs=3)
    roomy = make_engine(model, tok, num_blocks=128, max_num_seqs=3)
    a = pressured.generate(prompts, params)
    b = roomy.generate(prompts, params)
    pressured.step()
    assert pressured.total_preemptions > 0 and roomy.total_preemptions == 0
    for x, y in zip(a, b):
        assert x["token_ids"] == y["token_ids"] and x["generated_tokens"] == 10
    assert pressured.allocator.get_num_free_blocks() == pressured.allocator.get_total_blocks()


def test_submit_validation(model, tok):
    engine = make_engine(model, tok, max_model_len=32)
    with pytest.raises(ValueError):
        engine.submit("x" * 40, greedy(4))
    with pytest.raises(ValueError):
        engine.submit([], greedy(4))
    seq = engine.submit("x" * 20, greedy(100))
    assert engine.runtimes[seq].params.max_new_tokens == 12


def test_abort_stops_a_sequence_and_frees_its_memory(model, tok):
    engine = make_engine(model, tok)
    seq = engine.submit("abort me please", greedy(50, stop_on_eos=False))
    engine.step()
    engine.step()
    assert engine.abort(seq)
    engine.run_until_idle()
    engine.step()
    assert engine.runtimes[seq].finish_reason == "aborted"
    assert engine.allocator.get_num_free_blocks() == engine.allocator.get_total_blocks()
    assert not engine.abort(seq)


def test_eos_stops_generation_early(model, tok):
    engine = make_engine(model, tok)
    engine.eos_token_ids = set(range(256))  # every token is EOS
    r = engine.generate("stop at once", greedy(8))[0]
    assert r["generated_tokens"] == 1 and r["finish_reason"] == "stop"


def test_seeded_sampling_is_reproducible(model, tok):
    from memforge_amd.runtime.sampling import SamplingParams

    p = SamplingParams(max_new_tokens=10, temperature=0.9, top_p=0.95, seed=123, stop_on_eos=False)
    a = make_engine(model, tok).generate("sample this", p)[0]["token_ids"]
    b = make_engine(model, tok).generate("sample this", p)[0]["token_ids"]
    assert a == b and len(a) == 10


def test_chunked_prefill_does_not_change_the_output(model, tok):
    long_prompt = "a long prompt that needs several chunks to prefill " * 2
    prompts = [long_prompt, "short one"]
    plain = make_engine(model, tok, num_blocks=128, max_model_len=256)
    chunked = make_engine(model, tok, num_blocks=128, max_model_len=256, max_prefill_tokens_per_step=16)
    a = plain.generate(prompts, greedy(8))
    b = chunked.generate(prompts, greedy(8))
    for x, y, exp in zip(a, b, expected(model, tok, prompts, 8)):
        assert x["token_ids"] == y["token_ids"] == exp
    assert chunked.total_prefill_chunks > plain.total_prefill_chunks
    t = chunked.telemetry()
    assert t["chunked_prefill_enabled"] and t["max_prefill_tokens_per_step"] == 16


def test_prefix_sharing_is_byte_identical_and_saves_blocks(model, tok):
    shared = "a shared system prompt that spans several blocks: "
    prompts = [shared + "first question", shared + "second question", shared + "third"]
    on = make_engine(model, tok, num_blocks=128, max_model_len=256, enable_prefix_sharing=True)
    off = make_engine(model, tok, num_blocks=128, max_model_len=256, enable_prefix_sharing=False)
    first = on.generate(prompts[:1], greedy(6))  # registers the prefix
    rest = on.generate(prompts[1:], greedy(6))
    ref = off.generate(prompts, greedy(6))
    assert [r["token_ids"] for r in first + rest] == [r["token_ids"] for r in ref]
    assert on.total_cached_prefix_tokens > 0 and off.total_cached_prefix_tokens == 0
    t = on.telemetry()
    assert t["prefix_sharing_enabled"] and t["prefix_cache_hits"] > 0
    assert off.telemetry()["memory_saved_mb"] == 0.0
    on.step()
    assert on.allocator.get_num_allocated_blocks() == 0
    assert on.allocator.get_num_free_blocks() == on.allocator.get_total_blocks()
    assert on.prefix_cache.num_cached_blocks() == 0 and on.allocator.get_num_shared_blocks() == 0


def test_concurrent_identical_prefixes_share_blocks(model, tok):
    prefix = [2 + ((i * 7) % 200) for i in range(40)]
    engine = make_engine(model, tok, block_size=16, num_blocks=64, max_model_len=256)
    first = engine.submit(prefix + [50], greedy(30, stop_on_eos=False))
    engine.step()  # prefill registers the two full blocks
    second = engine.submit(prefix + [51], greedy(4, stop_on_eos=False))
    engine.step()
    engine.step()
    assert engine.allocator.get_num_shared_blocks() >= 2
    owners = engine.telemetry()["block_owners"]
    assert any(sorted(v) == sorted([first, second]) for v in owners.values())
    engine.run_until_idle()
    want = hf_greedy(model, prefix + [51], 4, stop_on_eos=False)
    assert engine.runtimes[second].generated == want


def test_block_occupancy_and_owners(model, tok):
    engine = make_engine(model, tok)
    a = engine.submit("owner one", greedy(20, stop_on_eos=False))
    b = engine.submit("owner two", greedy(20, stop_on_eos=False))
    engine.step()
    engine.step()
    occ = engine.block_occupancy()
    assert {a, b} <= set(occ)
    owners = engine.block_owners()
    for block_id, seqs in owners.items():
        assert occ[int(block_id)] in seqs


def test_telemetry_and_describe(model, tok):
    engine = make_engine(model, tok)
    engine.generate(["one", "two"], greedy(4))
    t = engine.telemetry()
    for key in ("tokens_generated", "forward_passes", "free_blocks", "total_blocks", "block_size", "kv_pool_mb",
                "fused_steps", "speculation_enabled", "memory_utilization"):
        assert key in t
    assert t["total_blocks"] == 64 and t["block_size"] == 4
    d = engine.describe()
    assert d["kv_pool"]["num_blocks"] == 64 and d["block_attention"]
    with pytest.raises(NotImplementedError):
        make_engine(model, tok, decode_view_cache=True)


def test_model_routing_is_restored_after_each_step(model, tok):
    from memforge_amd.kernels import attention_backend

    before = model.config._attn_implementation
    make_engine(model, tok).generate("routing", greedy(3))
    assert model.config._attn_implementation == before
    assert not attention_backend.is_enabled_on(model)


def test_bf16_engine_runs_and_first_tokens_agree(tok, device):
    m = tiny_llama(num_layers=2, seed=0, dtype=torch.bfloat16, hidden=256, heads=4, kv_heads=2)
    engine = make_engine(m, tok, block_size=16, num_blocks=32)
    results = engine.generate(PROMPTS, greedy(4))
    exp = expected(m, tok, PROMPTS, 4)
    same_first = sum(r["token_ids"][0] == e[0] for r, e in zip(results, exp))
    assert same_first >= len(PROMPTS) - 1, "bf16 first tokens should agree with transformers"


# ------------------------------------------------------------------ speculation


def test_self_draft_accepts_everything_and_stays_greedy(model, tok):
    engine = make_engine(model, tok, draft_model=model, lookahead_k=3, num_blocks=128)
    results = engine.generate(PROMPTS[:3], greedy(12, stop_on_eos=False))
    for r, exp in zip(results, expected(model, tok, PROMPTS[:3], 12, stop_on_eos=False)):
        assert r["token_ids"] == exp
    t = engine.telemetry()
    assert t["speculation_enabled"] and t["draft_acceptance_rate"] == 1.0
    assert t["speculative_rounds"] > 0


def test_speculative_output_is_identical_to_plain_greedy(model, draft, tok):
    plain = make_engine(model, tok, num_blocks=128).generate(PROMPTS, greedy(12, stop_on_eos=False))
    spec = make_engine(model, tok, num_blocks=128, draft_model=draft, lookahead_k=2)
    results = spec.generate(PROMPTS, greedy(12, stop_on_eos=False))
    for a, b in zip(results, plain):
        assert a["token_ids"] == b["token_ids"]
    spec.step()
    assert spec.allocator.get_num_free_blocks() == spec.allocator.get_total_blocks()
    assert spec.total_speculative_sequence_rounds >= spec.total_speculative_rounds


# ------------------------------------------------------------- graphed decode


def test_graphed_decoder_step_equals_the_eager_packed_pass(model, device):
    """GraphedPagedDecoder.step against the same decode run eagerly through
    the varlen path, over many replays of two batch buckets with eager work
    (pool writes, other replays) in between."""
    from memforge_amd.kernels import attention_backend
    from memforge_amd.runtime.graphed_paged_decode import GraphedPagedDecoder
    from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool
    from memforge_amd.runtime.varlen_cache import VarlenPackedCache

    spec = ModelKVSpec.from_config(model.config, torch.float32, "cuda:0")
    pool = PagedKVPool(spec, num_blocks=96, block_size=16)
    gen = torch.Generator().manual_seed(5)
    pool.key_pool.copy_(torch.randn(pool.key_pool.shape, generator=gen).to(device))
    pool.value_pool.copy_(torch.randn(pool.value_pool.shape, generator=gen).to(device))
    dec = GraphedPagedDecoder(model, pool, max_batch=8, max_model_len=256)
    perm = torch.randperm(96, generator=gen).tolist()
    tables = [perm[i * 12:(i + 1) * 12] for i in range(6)]
    for step in range(6):
        n = 3 if step % 2 == 0 else 6
        ctx = [20 + 7 * i + step for i in range(n)]
        toks = [(11 * i + step) % 250 + 2 for i in range(n)]
        want_pool_k = pool.key_pool.clone()
        want_pool_v = pool.value_pool.clone()
        got = dec.step(toks, ctx, tables[:n])
        # eager reference on a copy of the pool as it was before the step
        got_pool_k, got_pool_v = pool.key_pool.clone(), pool.value_pool.clone()
        pool.key_pool.copy_(want_pool_k)
        pool.value_pool.copy_(want_pool_v)
        cache = VarlenPackedCache(pool, 2, [torch.tensor(t) for t in tables[:n]], list(range(n)), ctx)
        with attention_backend.backend_enabled_on(model):
            with attention_backend.varlen_attention_context(pool, [torch.tensor(t) for t in tables[:n]],
                                                            list(range(n)), ctx):
                with torch.no_grad():
                    ref = model(input_ids=torch.tensor([toks], device=device),
                                position_ids=torch.tensor([ctx], device=device), past_key_values=cache,
                                use_cache=True).logits[0]
        torch.testing.assert_close(got, ref, atol=2e-5, rtol=1e-4)
        assert torch.equal(got_pool_k, pool.key_pool) and torch.equal(got_pool_v, pool.value_pool)
    assert dec.captures == 2 and dec.replays == 6


@pytest.mark.parametrize("max_model_len", [6600, 9000])
def test_graphed_decoder_long_context(model, device, max_model_len):
    """A 6,400-token context next to short ones. Up to 8,192 reachable tokens
    the decoder plans merge-free steps (here the planner's own pick would
    split the long range, so the step is replanned with 128-tile waves) and
    captures no merge launch; beyond that the graph keeps the merge launch and
    the step runs split-K. Both against the eager varlen pass."""
    from memforge_amd import _native as nat
    from memforge_amd.kernels import attention_backend
    from memforge_amd.runtime.graphed_paged_decode import GraphedPagedDecoder
    from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool
    from memforge_amd.runtime.varlen_cache import VarlenPackedCache

    spec = ModelKVSpec.from_config(model.config, torch.float32, "cuda:0")
    pool = PagedKVPool(spec, num_blocks=440, block_size=16)
    gen = torch.Generator().manual_seed(9)
    pool.key_pool.copy_(torch.randn(pool.key_pool.shape, generator=gen).to(device))
    pool.value_pool.copy_(torch.randn(pool.value_pool.shape, generator=gen).to(device))
    dec = GraphedPagedDecoder(model, pool, max_batch=4, max_model_len=max_model_len)
    assert dec.merge_free == (max_model_len <= 8176)
    perm = torch.randperm(440, generator=gen).tolist()
    tables = [perm[:402], perm[402:412], perm[412:420]]
    ctx = [6400, 150, 99]
    toks = [5, 17, 33]
    hkv, d = spec.num_kv_heads, spec.head_dim
    kv = [c + 1 for c in ctx] + [0]
    auto_merges = int(nat.plan_attention_host(list(range(5)), kv, model.config.num_attention_heads, hkv, d,
                                              torch.float32)[2][2])
    assert auto_merges > 0, "want a step whose own plan splits the long range"
    want_k, want_v = pool.key_pool.clone(), pool.value_pool.clone()
    got = dec.step(toks, ctx, tables)
    assert (dec._buckets[4].plan.cap_merges == 0) == dec.merge_free
    pool.key_pool.copy_(want_k)
    pool.value_pool.copy_(want_v)
    cache = VarlenPackedCache(pool, 2, [torch.tensor(t) for t in tables], [0, 1, 2], ctx)
    with attention_backend.backend_enabled_on(model):
        with attention_backend.varlen_attention_context(pool, [torch.tensor(t) for t in tables], [0, 1, 2], ctx):
            with torch.no_grad():
                ref = model(input_ids=torch.tensor([toks], device=device),
                            position_ids=torch.tensor([ctx], device=device), past_key_values=cache,
                            use_cache=True).logits[0]
    torch.testing.assert_close(got, ref, atol=2e-5, rtol=1e-4)


def test_graphed_engine_output_equals_eager(model, tok):
    prompts = PROMPTS + ["five", "a sixth prompt that is rather long indeed, for padding"]
    eager = make_engine(model, tok, num_blocks=128, max_num_seqs=8)
    graphed = make_engine(model, tok, num_blocks=128, max_num_seqs=8, paged_cuda_graph=True)
    a = eager.generate(prompts, greedy(12, stop_on_eos=False))
    b = graphed.generate(prompts, greedy(12, stop_on_eos=False))
    for x, y, exp in zip(a, b, expected(model, tok, prompts, 12, stop_on_eos=False)):
        assert x["token_ids"] == y["token_ids"] == exp
    t = graphed.telemetry()
    assert t["paged_cuda_graph_enabled"] and t["graph_replays"] > 5 and t["graph_captures"] >= 1
    # staggered arrivals: graph replays interleave with eager prefill steps
    from memforge_amd.runtime.sampling import SamplingParams

    g2 = make_engine(model, tok, num_blocks=128, max_num_seqs=8, paged_cuda_graph="auto")
    ids = []
    for p in prompts:
        ids.append(g2.submit(p, SamplingParams(max_new_tokens=10, temperature=0.0, stop_on_eos=False)))
        g2.step()
        g2.step()
    g2.run_until_idle()
    for i, p in zip(ids, prompts):
        assert g2.runtimes[i].generated == hf_greedy(model, tok(p)["input_ids"], 10, stop_on_eos=False)
    g2.step()
    assert g2.allocator.get_num_free_blocks() == g2.allocator.get_total_blocks()


def test_copy_on_write_moves_the_shared_block(model, tok):
    """A block another sequence also holds is copied before a write
    (test_prefix_sharing.py:270-303): the sequence gets a private block with
    the same K/V in every layer, and the original keeps its contents."""
    from memforge_amd.runtime.prefix_sharing import copy_block

    engine = make_engine(model, tok)
    sid = engine.submit("a prompt to copy on write", greedy(30, stop_on_eos=False))
    engine.step()
    seq = engine.scheduler.get_sequence(sid)
    table = list(seq.get_block_table())
    target = table[0]
    assert engine.allocator.add_ref(target)
    before_k = engine.pool.key_pool[:, target].clone()
    before_v = engine.pool.value_pool[:, target].clone()
    cow = engine.allocator.prepare_write(seq, 0)
    assert cow is not None
    old_block, new_block = cow
    assert old_block == target and new_block != target
    assert seq.get_block_table()[0] == new_block
    copy_block(engine.pool, old_block, new_block)
    assert torch.equal(engine.pool.key_pool[:, new_block], before_k)
    assert torch.equal(engine.pool.value_pool[:, new_block], before_v)
    assert torch.equal(engine.pool.key_pool[:, old_block], before_k)
    engine.pool.key_pool[:, 3].fill_(1.5)
    copy_block(engine.pool, 3, 3)
    assert bool((engine.pool.key_pool[:, 3] == 1.5).all())


# ------------------------------------------------------------ batched draft


DRAFT_PROMPTS = ["alpha prompt", "a much longer beta prompt here, with more to say", "gamma",
                 "the fourth one, mid length"]


def _spec_run(model, tok, prompts, params=None, slots=4, **kw):
    eng = make_engine(model, tok, num_blocks=256, max_num_seqs=slots, max_model_len=256, **kw)
    res = eng.generate(prompts, params or greedy(16, stop_on_eos=False))
    return eng, [r["token_ids"] for r in res], [r["token_sources"] for r in res]


def test_batched_draft_matches_plain_and_the_eager_draft(model, draft, tok):
    """Batched graphed drafting changes speed only: tokens equal plain decoding
    and the eager draft, and the proposals (token sources) equal the eager
    draft's (test_batched_graphed_draft.py:44-53)."""
    _, plain, _ = _spec_run(model, tok, DRAFT_PROMPTS)
    _, eager, eager_src = _spec_run(model, tok, DRAFT_PROMPTS, draft_model=draft, lookahead_k=4)
    eng, got, src = _spec_run(model, tok, DRAFT_PROMPTS, draft_model=draft, lookahead_k=4,
                              draft_cuda_graph="batched")
    assert got == plain == eager
    assert src == eager_src, "batched draft proposes different tokens than the eager draft"
    eng_self, got_self, src_self = _spec_run(model, tok, DRAFT_PROMPTS, draft_model=model, lookahead_k=4,
                                             draft_cuda_graph="batched")
    assert got_self == plain
    assert any(x == "draft" for seq in src_self for x in seq), "nothing was ever accepted"
    assert eng_self.telemetry()["draft_acceptance_rate"] == 1.0
    pool = eng._draft_pool
    assert len(pool._free) == 4 and pool._graph
    t = eng.telemetry()
    assert t["draft_graph_enabled"] and t["draft_graph_replays"] > 0


@pytest.mark.parametrize("n_prompts,slots", [(1, 4), (2, 4), (3, 8), (7, 4)])
def test_batched_draft_any_batch_size(model, draft, tok, n_prompts, slots):
    prompts = (DRAFT_PROMPTS * 2)[:n_prompts]
    _, plain, _ = _spec_run(model, tok, prompts, slots=slots)
    eng, got, _ = _spec_run(model, tok, prompts, slots=slots, draft_model=draft, lookahead_k=3,
                            draft_cuda_graph="batched")
    assert got == plain
    assert len(eng._draft_pool._free) == slots


def test_batched_draft_replays_per_round_do_not_grow_with_the_batch(model, draft, tok):
    eng, _, _ = _spec_run(model, tok, DRAFT_PROMPTS, draft_model=draft, lookahead_k=3,
                          draft_cuda_graph="batched")
    before_replays, before_rounds = eng._draft_pool.replays, eng.total_speculative_rounds
    eng.generate(DRAFT_PROMPTS, greedy(16, stop_on_eos=False))
    replays = eng._draft_pool.replays - before_replays
    rounds = eng.total_speculative_rounds - before_rounds
    assert rounds > 0 and replays == rounds * (3 + 1)


def test_batched_draft_sampling_runs_and_frees_slots(model, draft, tok):
    from memforge_amd.runtime.sampling import SamplingParams

    params = SamplingParams(max_new_tokens=16, temperature=0.8, top_p=1.0, stop_on_eos=False)
    torch.manual_seed(0)
    eng, got, _ = _spec_run(model, tok, DRAFT_PROMPTS, params=params, draft_model=draft, lookahead_k=3,
                            draft_cuda_graph="batched")
    assert all(len(g) == 16 for g in got) and len(eng._draft_pool._free) == 4


def test_batched_draft_mixed_temperatures_keep_greedy_rows_exact(model, draft, tok):
    """Rows with different temperatures are drafted per temperature group; the
    greedy rows still equal plain decoding."""
    from memforge_amd.runtime.sampling import SamplingParams

    eng = make_engine(model, tok, num_blocks=256, max_num_seqs=4, max_model_len=256, draft_model=draft,
                      lookahead_k=3, draft_cuda_graph="batched")
    g = eng.submit(DRAFT_PROMPTS[1], greedy(16, stop_on_eos=False))
    s = eng.submit(DRAFT_PROMPTS[3], SamplingParams(max_new_tokens=16, temperature=0.9, stop_on_eos=False))
    eng.run_until_idle()
    want = hf_greedy(model, tok(DRAFT_PROMPTS[1])["input_ids"], 16, stop_on_eos=False)
    assert eng.runtimes[g].generated == want
    assert len(eng.runtimes[s].generated) == 16 and len(eng._draft_pool._free) == 4


@pytest.mark.parametrize("n_prompts,slots", [(1, 4), (3, 4), (4, 8), (7, 4)])
def test_unrolled_draft_one_replay_per_round_matches_eager(model, draft, tok, n_prompts, slots):
    prompts = (DRAFT_PROMPTS * 2)[:n_prompts]
    _, plain, _ = _spec_run(model, tok, prompts, slots=slots)
    _, eager, esrc = _spec_run(model, tok, prompts, slots=slots, draft_model=draft, lookahead_k=4)
    eng, got, src = _spec_run(model, tok, prompts, slots=slots, draft_model=draft, lookahead_k=4,
                              draft_cuda_graph="batched-unrolled")
    assert got == plain == eager
    assert src == esrc, "unrolled draft proposes different tokens than the eager draft"
    pool = eng._draft_pool
    assert pool._ugraph and len(pool._free) == slots
    assert pool.replays == eng.total_speculative_rounds


def test_unrolled_draft_steps_when_sampling(model, draft, tok):
    from memforge_amd.runtime.sampling import SamplingParams

    params = SamplingParams(max_new_tokens=12, temperature=0.8, top_p=1.0, stop_on_eos=False)
    eng, got, _ = _spec_run(model, tok, DRAFT_PROMPTS, params=params, draft_model=draft, lookahead_k=3,
                            draft_cuda_graph="batched-unrolled")
    assert all(len(g) == 12 for g in got) and not eng._draft_pool._ugraph


def test_draft_graph_auto_and_deprecated_true(model, draft, tok):
    from memforge_amd.runtime.batched_speculative import BatchedGraphedDraftPool

    _, plain, _ = _spec_run(model, tok, DRAFT_PROMPTS[:2], slots=2)
    eng, got, _ = _spec_run(model, tok, DRAFT_PROMPTS[:2], slots=2, draft_model=draft, lookahead_k=3,
                            paged_cuda_graph="auto", draft_cuda_graph="auto")
    assert eng._paged_graph is not None and isinstance(eng._draft_pool, BatchedGraphedDraftPool)
    assert got == plain
    with pytest.warns(DeprecationWarning, match="batched"):
        eng = make_engine(model, tok, max_num_seqs=2, draft_model=draft, lookahead_k=2, draft_cuda_graph=True)
    assert isinstance(eng._draft_pool, BatchedGraphedDraftPool)
    assert make_engine(model, tok, draft_model=draft, lookahead_k=2)._draft_pool is None


def test_batched_draft_survives_preemption(model, draft, tok):
    """A preempted sequence gives its draft slot back and re-feeds its draft
    when it runs again; the output still equals plain decoding."""
    prompts = ["first prompt that runs long", "second prompt, also long", "third"]
    plain = make_engine(model, tok, num_blocks=256, max_model_len=128).generate(
        prompts, greedy(24, stop_on_eos=False))
    eng = make_engine(model, tok, block_size=4, num_blocks=22, max_num_seqs=3, max_model_len=128,
                      draft_model=draft, lookahead_k=3, draft_cuda_graph="batched")
    res = eng.generate(prompts, greedy(24, stop_on_eos=False))
    assert [r["token_ids"] for r in res] == [p["token_ids"] for p in plain]
    assert eng.total_preemptions > 0
    assert len(eng._draft_pool._free) == 3


def test_draft_pool_api(draft, device):
    """acquire / release / prefill / rollback_to on the pool directly, and
    proposals from two rows at different positions against the eager draft."""
    from memforge_amd.runtime.batched_speculative import (BatchedGraphedDraftPool, DraftState,
                                                           propose_draft_tokens)

    pool = BatchedGraphedDraftPool(draft, max_len=64, num_slots=3, device="cuda:0")
    a, b = pool.acquire(), pool.acquire()
    assert (a.slot, b.slot) == (0, 1)
    ta = [5, 9, 14, 22, 31, 40, 41]
    tb = [7, 8]
    pool.prefill(a, ta[:3])
    assert a.position == 3
    out = pool.propose([a, b], [ta, tb], 3, 0.0)
    assert a.position == len(ta) + 3 and b.position == len(tb) + 3
    for (cand, probs), toks in zip(out, [ta, tb]):
        ref_cand, ref_probs = propose_draft_tokens(draft, DraftState(), toks, 3, 0.0, "cuda:0")
        assert cand == ref_cand
        assert len(probs) == 3 and all(int(p.argmax()) == c for p, c in zip(probs, cand))
    a.rollback_to(len(ta) + 1)
    with pytest.raises(ValueError):
        a.rollback_to(a.position + 1)
    with pytest.raises(ValueError):
        a.rollback_to(-1)
    # after a rollback the next round continues from the confirmed tokens
    ta2 = ta + [out[0][0][0], 17]
    out2 = pool.propose([a], [ta2], 2, 0.0)
    ref_cand, _ = propose_draft_tokens(draft, DraftState(), ta2, 2, 0.0, "cuda:0")
    assert out2[0][0] == ref_cand
    pool.release(a)
    pool.release(b)
    with pytest.raises(ValueError):
        pool.release(b)
    assert sorted(pool._free) == [0, 1, 2]
    with pytest.raises(ValueError):
        pool.propose([pool.acquire()], [list(range(2, 64))], 4, 0.0)


def test_graphed_decode_with_a_batch_limit_that_is_not_a_power_of_two(model, tok):
    """Buckets are powers of two capped at max_num_seqs, so three running
    sequences with max_num_seqs=3 replay a 3-row graph."""
    eng = make_engine(model, tok, num_blocks=128, max_num_seqs=3, paged_cuda_graph=True)
    res = eng.generate(PROMPTS[:3], greedy(10, stop_on_eos=False))
    for r, exp in zip(res, expected(model, tok, PROMPTS[:3], 10, stop_on_eos=False)):
        assert r["token_ids"] == exp
    assert 3 in eng._paged_graph._buckets and eng.telemetry()["graph_replays"] > 0


@pytest.mark.parametrize("draft_cuda_graph", [False, "batched"])
def test_batched_speculative_resolve_keeps_seeded_output(model, draft, tok, draft_cuda_graph):
    """The speculative step resolves every row with one rejection launch and
    writes every row's confirmed K/V with one launch per layer. From the same
    global seeds, sampled (temperature 0.8) and greedy requests produce the
    same tokens, sources and acceptance counts as resolving the rows one at a
    time with per-row writes."""
    from memforge_amd.runtime.sampling import SamplingParams

    runs = []
    for batched in (True, False):
        eng = make_engine(model, tok, num_blocks=256, max_num_seqs=4, max_model_len=256, draft_model=draft,
                          lookahead_k=3, draft_cuda_graph=draft_cuda_graph)
        eng._batched_resolve = batched
        torch.manual_seed(11)
        torch.cuda.manual_seed(11)
        ids = [eng.submit(p, SamplingParams(max_new_tokens=14, temperature=0.8 if i % 2 else 0.0, top_p=1.0,
                                            stop_on_eos=False))
               for i, p in enumerate(DRAFT_PROMPTS)]
        eng.run_until_idle()
        t = eng.telemetry()
        runs.append(([eng.runtimes[i].generated for i in ids], [eng.runtimes[i].sources for i in ids],
                     t["draft_tokens_proposed"], t["draft_tokens_accepted"], t["speculative_rounds"]))
    assert runs[0] == runs[1]
    assert runs[0][4] > 0 and runs[0][3] < runs[0][2]


@pytest.mark.parametrize("fused", [True, False])
def test_telemetry_reports_measured_data_path_bandwidth(model, tok, fused):
    """telemetry() carries the data path's measured figures (HIP events on
    sampled passes): attention and KV-write GB/s and fraction of the HBM peak
    on eager passes (one family for the launch doing both when the write rides
    in the attention launch), and the bytes-roofline fraction of
    graph-replayed decode steps; describe() names the pool layout."""
    engine = make_engine(model, tok, paged_cuda_graph=True, telemetry_sample_every=1, fused_kv_write=fused)
    engine.generate(PROMPTS, greedy(6, stop_on_eos=False))
    t = engine.telemetry()
    timed = ("attention_kv_write",) if fused else ("attention", "kv_write")
    idle = ("attention", "kv_write") if fused else ("attention_kv_write",)
    for family in idle:
        assert t[f"{family}_samples"] == 0 and t[f"{family}_gbps"] is None, family
    for family in (*timed, "decode_graph"):
        assert t[f"{family}_samples"] > 0, family
        assert t[f"{family}_gbps"] > 0 and 0 < t[f"{family}_hbm_frac"] < 1, (family, t[f"{family}_gbps"])
        assert t[f"{family}_us_per_launch"] > 0 and t[f"{family}_bytes_per_launch"] > 0
    assert t["hbm_peak_gbps"] == 8000.0 and t["data_path_sample_every"] == 1
    pool = engine.describe()["kv_pool"]
    assert pool["layout"] == "(layers, blocks, block_size, kv_heads, head_dim)" and pool["dtype"] == "torch.float32"
    off = make_engine(model, tok, telemetry_sample_every=0)
    off.generate(PROMPTS[:1], greedy(3))
    assert off.telemetry()["attention_kv_write_samples"] == 0 and off.telemetry()["attention_gbps"] is None


def test_streamed_text_adds_up_to_the_final_text(model, tok):
    engine = make_engine(model, tok)
    sid = engine.submit(PROMPTS[1], greedy(12, stop_on_eos=False))
    streamed = []
    while engine.has_work():
        engine.step()
        streamed.extend(ev.text for ev in engine.drain_events(sid))
    assert "".join(streamed) == engine.result_for(sid)["text"] and len(streamed) == 12
