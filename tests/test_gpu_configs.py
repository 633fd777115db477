"""Parity at the configs' own sizes and plans.

The attention tests elsewhere use reduced shapes. Here each benchmark config
runs at its full size through the plan the planner makes for it, and a
sample of rows (all of them where the oracle is cheap) is checked against the
float64 oracle:

* C5, the headline: 256 sequences at the 14B GQA shape, lognormal contexts up
  to 32,768 keys, through both plan forms: the decode slice plan the bench
  measures (one round of slices, sequences split across slices, merged) and
  the per-range plan (128-tile waves, 512-tile cooperative units, split-K
  merge records, the one-wave-per-record merge);
* the second block-table register of 65-128-tile waves, in fp32 at D 128;
* C2's mixed step through the engine's one-launch plan, after the KV scatter
  of its 2,076 new tokens;
* C3's 16 x 5 verify rows with their candidates attended in flight, through
  the cooperative plan with merges;
* C4's model shape end to end (test_c4_* below).

Bars: fp32 1e-5 max-abs; bf16 2e-2 max-abs and 1e-2 mean-rel.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from memforge_amd import _native as nat
from oracle import attention as oatt
from tests.gpu_helpers import assert_close_bf16, gpu_varlen, random_tables, to_np64

pytestmark = pytest.mark.gpu


def _compact(kpool, vpool, tables, rows):
    """The blocks the sampled rows read, as a small float32 host pool, and
    their tables renumbered into it."""
    used = sorted({int(x) for r in rows for x in tables[r]})
    remap = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, device=kpool.device)
    kp = kpool.index_select(0, idx).float().cpu().numpy()
    vp = vpool.index_select(0, idx).float().cpu().numpy()
    return kp, vp, [[remap[int(x)] for x in tables[r]] for r in rows]


@pytest.mark.parametrize("form", ["slices", "ranges"])
def test_c5_headline_plan_matches_the_oracle_on_sampled_rows(device, form):
    import bench

    ctx, tables, kpool, vpool, q = bench.make_workload(1.0, device)
    B = bench.B
    plan = nat.plan_attention(list(range(B + 1)), ctx.tolist(), bench.HQ, bench.HKV, bench.D,
                              torch.bfloat16, device, decode_slices=form == "slices")
    if form == "slices":
        # the plan the headline figure is measured on: one round of slices
        per_round = nat.device_cus(device) * nat.SLICE_WAVES_PER_CU // bench.HKV
        assert plan.sliced and plan.n_narrow <= per_round and plan.n_merges > 0
        assert int(plan.merges_host[:, 3].max()) > 4  # a merge of more than one batch
    else:
        assert not plan.sliced and plan.n_wide == 0 and plan.n_merges == 136, (plan.n_narrow, plan.n_merges)
        items = plan.items_host[: plan.n_narrow]
        assert (items[:, 11] == 1).any()                   # cooperative units
        assert int((items[:, 5] - items[:, 4]).max()) == 128  # 128-tile waves
    out = torch.full_like(q, float("nan"))
    pool = nat.PoolView.from_bshd(kpool, vpool)
    nat.paged_attention(q, out, pool, tables.to(device), torch.arange(B + 1, dtype=torch.int32, device=device),
                        ctx.to(torch.int32).to(device), (ctx - 1).to(device), plan, 1.0 / math.sqrt(bench.D),
                        bench.HKV)
    rows = bench.check_rows(ctx)  # the rows bench.py's own check samples
    c = ctx[rows].tolist()
    assert min(c) == int(ctx.min()) and max(c) == 32768 and any(1024 < x <= 2048 for x in c)
    assert any(2048 < x <= 8192 for x in c) and sum(x > 8192 for x in c) >= 2
    nblk = [(int(ctx[r]) + 15) // 16 for r in rows]
    kp, vp, tabs = _compact(kpool, vpool, [tables[r, :n].tolist() for r, n in zip(rows, nblk)],
                            range(len(rows)))
    want = oatt.varlen_attention(q[rows].permute(1, 0, 2).float().cpu().numpy(), kp, vp, tabs,
                                 list(range(len(rows))), (ctx[rows] - 1).tolist(), 16)
    got = to_np64(out[rows].permute(1, 0, 2))
    assert_close_bf16(got, want)
    print(f"C5 {form} rows {rows} (contexts {ctx[rows].tolist()}): max-abs {np.abs(got - want).max():.3e}")
    if form == "slices":
        # every row against the per-range plan: the two forms differ only in
        # where fp32 sums are split, so they agree to bf16 output rounding
        ranges = nat.plan_attention(list(range(B + 1)), ctx.tolist(), bench.HQ, bench.HKV, bench.D,
                                    torch.bfloat16, device)
        ref = torch.full_like(q, float("nan"))
        nat.paged_attention(q, ref, pool, tables.to(device), torch.arange(B + 1, dtype=torch.int32, device=device),
                            ctx.to(torch.int32).to(device), (ctx - 1).to(device), ranges,
                            1.0 / math.sqrt(bench.D), bench.HKV)
        assert_close_bf16(to_np64(out), to_np64(ref), max_abs=4e-3, mean_rel=1e-3)


def test_long_waves_use_both_table_registers_fp32_d128(device):
    """Single waves of 65-128 tiles read their second block-table entry from a
    second register per lane: forced 128-tile partitions in fp32 at D 128,
    contexts from 1,025 to 2,048 keys (and two that become cooperative
    units), against the oracle at 1e-5."""
    gen = torch.Generator().manual_seed(11)
    bs, hq, hkv, d = 16, 40, 8, 128
    ctx = torch.randint(1025, 2049, (6,), generator=gen).tolist() + [2048, 1025, 2049, 5000]
    need = sum((c + bs - 1) // bs for c in ctx)
    tables = random_tables(gen, need + 5, ctx, bs)
    kp = torch.randn((need + 5, bs, hkv, d), generator=gen).to(device)
    vp = torch.randn((need + 5, bs, hkv, d), generator=gen).to(device)
    q = torch.randn((hq, len(ctx), d), generator=gen).to(device)
    positions = [c - 1 for c in ctx]
    got = gpu_varlen(q, kp, vp, tables, list(range(len(ctx))), positions, partition_tiles=128)
    want = oatt.varlen_attention(to_np64(q), to_np64(kp), to_np64(vp), tables, list(range(len(ctx))),
                                 positions, bs)
    err = np.abs(to_np64(got) - want).max()
    assert err <= 1e-5, f"fp32 max-abs {err:.3e}"


@pytest.mark.parametrize("prefill_only", [False, True])
def test_c2_mixed_step_at_full_size(device, prefill_only):
    """C2: 4 chunks of 512 on priors U[0,2048] + 28 decodes of U[64,4096],
    bf16, 15q/5kv, D 64. The KV scatter of all 2,076 new tokens, then one
    attention call with the whole plan (decode and prefill items in one
    launch, split-K merge) -- the engine's form of the step. The scatter is
    checked bit-exactly; the attention of every decode row and of 48 rows per
    prefill chunk against the oracle. prefill_only: the same step planned with
    the decodes given no rows (a plan of wide items only, in the planner's
    XCD order), the prefill rows checked."""
    gen = torch.Generator().manual_seed(0)
    bs, hq, hkv, d = 16, 15, 5, 64
    prior = torch.randint(0, 2049, (4,), generator=gen).tolist()
    dctx = torch.randint(64, 4097, (28,), generator=gen).tolist()
    q_lens = [512] * 4 + [1] * 28
    kv = [p + 512 for p in prior] + dctx
    starts = prior + [c - 1 for c in dctx]
    need = sum((c + bs - 1) // bs for c in kv)
    tables = random_tables(gen, need, kv, bs)
    kp = torch.randn((need, bs, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    vp = torch.randn((need, bs, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    T = sum(q_lens)
    q = torch.randn((T, hq, d), generator=gen).to(torch.bfloat16).to(device)
    knew = torch.randn((T, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    vnew = torch.randn((T, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    positions = [s + i for s, n in zip(starts, q_lens) for i in range(n)]
    slots = [tables[e][p // bs] * bs + p % bs for e, (s0, n) in enumerate(zip(starts, q_lens))
             for p in range(s0, s0 + n)]
    pool = nat.PoolView.from_bshd(kp, vp)
    slot_t = torch.tensor(slots, dtype=torch.int64, device=device)
    nat.kv_write(knew, vnew, slot_t, pool)
    assert torch.equal(kp.view(-1, hkv, d)[slot_t], knew) and torch.equal(vp.view(-1, hkv, d)[slot_t], vnew)
    if prefill_only:
        cu = cu[:5] + [cu[4]] * 28
    plan = nat.plan_attention(cu, kv, hq, hkv, d, torch.bfloat16, device)
    if prefill_only:
        assert plan.n_narrow == 0 and plan.n_wide == 3600 and plan.n_merges
    else:
        assert plan.n_narrow and plan.n_wide and plan.n_merges  # one mixed launch, then the merge
    bt = torch.zeros((32, max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    out = torch.full_like(q, float("nan"))
    nat.paged_attention(q, out, pool, bt.to(device), torch.tensor(cu, dtype=torch.int32, device=device),
                        torch.tensor(kv, dtype=torch.int32, device=device),
                        torch.tensor(positions, dtype=torch.int64, device=device), plan, 1.0 / math.sqrt(d), hkv)
    rng = np.random.default_rng(2)
    rows = []
    for e in range(4):
        pick = {0, 511, 255} | set(rng.choice(512, 45, replace=False).tolist())
        rows += [cu[e] + i for i in sorted(pick)]
    if not prefill_only:
        rows += list(range(cu[4], T))
    seq_of = [e for e, n in enumerate(q_lens) for _ in range(n)]
    kp_h, vp_h = kp.float().cpu().numpy(), vp.float().cpu().numpy()
    want = oatt.varlen_attention(q[rows].permute(1, 0, 2).float().cpu().numpy(), kp_h, vp_h, tables,
                                 [seq_of[r] for r in rows], [positions[r] for r in rows], bs)
    assert_close_bf16(to_np64(out[rows].permute(1, 0, 2)), want)


def test_c3_verify_rows_at_full_size(device):
    """C3: 16 sequences of U[128,2048] context, 5 query rows each at
    positions ctx..ctx+4, the candidates' K/V attended in flight (nothing in
    the pool past ctx), through the auto plan (8-tile cooperative waves and
    merges); all 80 rows against the oracle."""
    gen = torch.Generator().manual_seed(0)
    bs, hq, hkv, d, B, K = 16, 15, 5, 64, 16, 4
    ctx = torch.randint(128, 2049, (B,), generator=gen).tolist()
    kvl = [c + K + 1 for c in ctx]
    need = sum((c + bs - 1) // bs for c in kvl)
    tables = random_tables(gen, need, kvl, bs)
    kp = torch.randn((need, bs, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    vp = torch.randn((need, bs, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    T = B * (K + 1)
    q = torch.randn((hq, T, d), generator=gen).to(torch.bfloat16).to(device)
    nk = torch.randn((T, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    nv = torch.randn((T, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    seq_ids = [b for b in range(B) for _ in range(K + 1)]
    positions = [c + j for c in ctx for j in range(K + 1)]
    plan = nat.plan_attention([b * (K + 1) for b in range(B + 1)], kvl, hq, hkv, d, torch.bfloat16, device)
    assert plan.n_merges > 0 and (plan.items_host[: plan.n_narrow, 11] == 1).any()
    got = gpu_varlen(q, kp, vp, tables, seq_ids, positions, pool_lens=ctx, new_k=nk, new_v=nv)
    new_rows = [[b * (K + 1) + j for j in range(K + 1)] for b in range(B)]
    want = oatt.varlen_attention(to_np64(q), kp.float().cpu().numpy(), vp.float().cpu().numpy(), tables,
                                 seq_ids, positions, bs, pool_lens=ctx, new_k=to_np64(nk), new_v=to_np64(nv),
                                 new_rows=new_rows)
    assert_close_bf16(to_np64(got), want)


# ------------------------------------------------------------------ C4 shape

C4_MODEL = dict(vocab_size=49152, hidden_size=960, intermediate_size=2560, num_hidden_layers=32,
                num_attention_heads=15, num_key_value_heads=5, head_dim=64)


def _c4_model(device, dtype):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(**C4_MODEL, max_position_embeddings=2048, tie_word_embeddings=True, bos_token_id=1,
                      eos_token_id=2, pad_token_id=0)
    torch.manual_seed(0)
    with torch.device(device):
        model = LlamaForCausalLM(cfg)
    return model.to(dtype).eval()


class _IdTokenizer:
    eos_token_id = 2
    pad_token_id = 0

    def __call__(self, text, return_tensors=None):
        return {"input_ids": [3 + (ord(c) % 1000) for c in text]}

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(int(i)) for i in ids)


def _c4_prompts(n, seed=0):
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(32, 1025, (n,), generator=gen)
    return [torch.randint(3, C4_MODEL["vocab_size"], (int(m),), generator=gen).tolist() for m in lens]


def test_c4_engine_at_the_smollm2_shape_fp32_equals_transformers_greedy(device):
    """C4's model (32 layers, hidden 960, 15q/5kv, D 64, vocab 49,152, random
    init) in fp32: 8 requests with prompts U[32,1024], chunked prefill (512
    tokens per step) and graph-replayed decode; every request's greedy tokens
    equal plain transformers greedy decoding with its own DynamicCache."""
    from memforge_amd.runtime import ContinuousBatchingEngine, SamplingParams
    from tests.tiny_models import hf_greedy

    model = _c4_model(device, torch.float32)
    prompts = _c4_prompts(8)
    engine = ContinuousBatchingEngine(model, _IdTokenizer(), block_size=16, kv_budget_mb=1024, max_num_seqs=8,
                                      max_model_len=2048, max_prefill_tokens_per_step=512,
                                      paged_cuda_graph=True)
    params = SamplingParams(max_new_tokens=12, temperature=0.0, stop_on_eos=False)
    results = engine.generate(prompts, params)
    assert engine._paged_graph is not None and engine._paged_graph.replays > 0
    for i, (r, p) in enumerate(zip(results, prompts)):
        want = hf_greedy(model, p, 12, stop_on_eos=False)
        assert r["token_ids"] == want, f"request {i} (prompt {len(p)} tokens)"
    engine.step()
    assert engine.allocator.get_num_free_blocks() == engine.allocator.get_total_blocks()


def test_c4_engine_at_the_smollm2_shape_bf16_first_tokens_and_blocks(device):
    """The same shape in bf16 with 16 requests: the first generated token of
    every request is transformers' greedy pick from the same prompt -- or,
    where bf16 logits tie or nearly tie, a token whose transformers logit is
    within two bf16 ulps of the maximum (later tokens may part ways at such
    near-ties) --, every request runs to its length, and every block returns
    to the free list."""
    from memforge_amd.runtime import ContinuousBatchingEngine, SamplingParams

    model = _c4_model(device, torch.bfloat16)
    prompts = _c4_prompts(16, seed=1)
    engine = ContinuousBatchingEngine(model, _IdTokenizer(), block_size=16, kv_budget_mb=1024, max_num_seqs=16,
                                      max_model_len=2048, max_prefill_tokens_per_step=1024,
                                      paged_cuda_graph=True, dtype=torch.bfloat16)
    total = engine.allocator.get_total_blocks()
    results = engine.generate(prompts, SamplingParams(max_new_tokens=8, temperature=0.0, stop_on_eos=False))
    agree = 0
    with torch.no_grad():
        for i, (r, p) in enumerate(zip(results, prompts)):
            assert r["generated_tokens"] == 8
            logits = model(input_ids=torch.tensor([p], device=device)).logits[0, -1].float()
            top = float(logits.max())
            ulp = 2.0 ** (math.floor(math.log2(abs(top))) - 7)
            first = r["token_ids"][0]
            agree += int(int(logits.argmax()) == first)
            assert float(logits[first]) >= top - 2 * ulp, (i, first, int(logits.argmax()))
    assert agree >= len(prompts) - 2, f"only {agree} of {len(prompts)} first tokens are the exact argmax"
    engine.step()
    assert engine.allocator.get_num_free_blocks() == total
