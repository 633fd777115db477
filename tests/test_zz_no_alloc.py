"""mf_paged_attention_noalloc against mf_paged_attention.

The no-allocation entry point runs the same kernels on the same plan, with
the split-K partials in the library's own per-GPU array instead of a buffer
the caller allocated, so its output must be bit-identical to the allocating
entry point's. Two calls in a row, the second smaller than the first (the
array keeps the first call's partials, which the second must not read), each
with a plan that splits ranges and merges them.
"""

from __future__ import annotations

import math

import pytest
import torch

from memforge_amd import _native as nat
from tests.gpu_helpers import random_tables

pytestmark = pytest.mark.gpu


def _case(device, gen, dtype, hq, hkv, d, contexts, chunk):
    """Decode rows for `contexts` plus one prefill chunk of `chunk` rows on a
    prior of 300 keys (a mixed plan), all on one shuffled pool."""
    bs = 16
    kv = list(contexts) + ([300 + chunk] if chunk else [])
    q_lens = [1] * len(contexts) + ([chunk] if chunk else [])
    need = sum((c + bs - 1) // bs for c in kv)
    tables = random_tables(gen, need, kv, bs)
    kp = torch.randn((need, bs, hkv, d), generator=gen).to(dtype).to(device)
    vp = torch.randn((need, bs, hkv, d), generator=gen).to(dtype).to(device)
    T = sum(q_lens)
    q = torch.randn((T, hq, d), generator=gen).to(dtype).to(device)
    cu = [0]
    for n in q_lens:
        cu.append(cu[-1] + n)
    positions = [c - 1 for c in contexts] + (list(range(300, 300 + chunk)) if chunk else [])
    bt = torch.zeros((len(kv), max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    plan = nat.plan_attention(cu, kv, hq, hkv, d, dtype, device)
    args = (q, nat.PoolView.from_bshd(kp, vp), bt.to(device), torch.tensor(cu, dtype=torch.int32, device=device),
            torch.tensor(kv, dtype=torch.int32, device=device),
            torch.tensor(positions, dtype=torch.int64, device=device), plan)
    return args


def _both(args, hkv):
    q, pool, bt, cu, kv, pos, plan = args
    scale = 1.0 / math.sqrt(q.shape[-1])
    want = torch.full_like(q, float("nan"))
    got = torch.full_like(q, float("nan"))
    nat.paged_attention(q, want, pool, bt, cu, kv, pos, plan, scale, hkv)
    nat.paged_attention_noalloc(q, got, pool, bt, cu, kv, pos, plan, scale, hkv)
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("dtype,hq,hkv,d", [(torch.bfloat16, 40, 8, 128), (torch.float32, 15, 5, 64),
                                            (torch.bfloat16, 15, 5, 64)])
def test_noalloc_equals_the_allocating_entry_point_on_two_calls(device, dtype, hq, hkv, d):
    gen = torch.Generator().manual_seed(31)
    first = _case(device, gen, dtype, hq, hkv, d, [20000, 9000, 300, 5000, 64, 12000], 200)
    second = _case(device, gen, dtype, hq, hkv, d, [9000, 2000, 77], 0)
    assert first[-1].n_merges > 0 and first[-1].partials_floats > 0
    assert second[-1].n_merges > 0 and second[-1].partials_floats < first[-1].partials_floats
    for args in (first, second):
        got, want = _both(args, hkv)
        assert not torch.isnan(want).any()
        assert torch.equal(got, want), float((got.float() - want.float()).abs().max())


def test_noalloc_refuses_a_plan_larger_than_its_array(device):
    gen = torch.Generator().manual_seed(5)
    q, pool, bt, cu, kv, pos, plan = _case(device, gen, torch.bfloat16, 40, 8, 128, [20000], 0)
    big = nat.AttentionPlan(plan.items, plan.merges, plan.n_narrow, plan.n_wide, plan.n_merges,
                            nat.NOALLOC_PARTIALS_FLOATS + 1, plan.items_host, plan.merges_host)
    out = torch.zeros_like(q)
    with pytest.raises(nat.MemforgeHipError, match="workspace"):
        nat.paged_attention_noalloc(q, out, pool, bt, cu, kv, pos, big, 0.1, 8)
    assert not out.any()
