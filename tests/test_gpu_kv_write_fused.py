"""The written-in-flight step (mf_paged_attention_kv_write): one launch that
writes a packed step's new K/V rows into the pool and attends with every
sequence's new keys read from those rows. It must leave the pool exactly as
mf_kv_write does and produce exactly the output of mf_kv_write followed by
mf_paged_attention, bit for bit, on every path of the kernel: decode items
(one in-flight key per row), cooperative units, wide items sharing each tile
through LDS (16-bit, block 16), wide items without sharing (fp32), the general
loads of other block sizes, split-K merges, and counted (graph) launches."""

from __future__ import annotations

from typing import List, Sequence, Tuple

import pytest
import torch

from memforge_amd import _native as nat
from tests.gpu_helpers import pad_tables, random_tables

pytestmark = pytest.mark.gpu


def _step(device, dtype, hq, hkv, d, bs, runs: Sequence[Tuple[int, int]], seed=0):
    """Pool, tables and one packed step: run i adds q_len new tokens after
    `prior` cached ones (a prefill chunk, or a decode when q_len is 1)."""
    gen = torch.Generator().manual_seed(seed)
    kv = [p + n for p, n in runs]
    nblocks = sum((k + bs - 1) // bs for k in kv) + 3
    tables = random_tables(gen, nblocks, kv, bs)
    kp = torch.randn((nblocks, bs, hkv, d), generator=gen).to(dtype).to(device)
    vp = torch.randn((nblocks, bs, hkv, d), generator=gen).to(dtype).to(device)
    T = sum(n for _, n in runs)
    q = torch.randn((T, hq, d), generator=gen).to(dtype).to(device)
    # new rows as a model hands them over: (1, Hkv, T, D) permuted to (T, Hkv, D)
    knew = torch.randn((hkv, T, d), generator=gen).to(dtype).to(device).permute(1, 0, 2)
    vnew = torch.randn((hkv, T, d), generator=gen).to(dtype).to(device).permute(1, 0, 2)
    cu, positions, slots = [0], [], []
    for (p, n), t in zip(runs, tables):
        cu.append(cu[-1] + n)
        for pos in range(p, p + n):
            positions.append(pos)
            slots.append(t[pos // bs] * bs + pos % bs)
    return dict(kp=kp, vp=vp, q=q, knew=knew, vnew=vnew, tables=tables, cu=cu, kv=kv,
                positions=positions, slots=slots, T=T, hq=hq, hkv=hkv, d=d)


def _device_meta(st, device):
    return (pad_tables(st["tables"], device), torch.tensor(st["cu"], dtype=torch.int32, device=device),
            torch.tensor(st["kv"], dtype=torch.int32, device=device),
            torch.tensor(st["positions"], dtype=torch.int64, device=device),
            torch.tensor(st["slots"], dtype=torch.int64, device=device))


def _two_calls(st, plan, device, scale):
    kp, vp = st["kp"].clone(), st["vp"].clone()
    pool = nat.PoolView.from_bshd(kp, vp)
    bt, cu, kv, pos, slots = _device_meta(st, device)
    out = torch.full_like(st["q"], float("nan"))
    nat.kv_write(st["knew"], st["vnew"], slots, pool)
    nat.paged_attention(st["q"], out, pool, bt, cu, kv, pos, plan, scale, st["hkv"])
    return out, kp, vp


def _one_call(st, plan, device, scale, slots=None):
    kp, vp = st["kp"].clone(), st["vp"].clone()
    pool = nat.PoolView.from_bshd(kp, vp)
    bt, cu, kv, pos, slot_t = _device_meta(st, device)
    if slots is not None:
        slot_t = torch.tensor(slots, dtype=torch.int64, device=device)
    out = torch.full_like(st["q"], float("nan"))
    nat.paged_attention_kv_write(st["q"], out, pool, bt, cu, kv, pos, plan, scale, st["hkv"],
                                 st["knew"], st["vnew"], slot_t)
    return out, kp, vp


def _check_same(st, device, partition_tiles=0, scale=None):
    scale = scale if scale is not None else st["d"] ** -0.5
    plan = nat.plan_attention(st["cu"], st["kv"], st["hq"], st["hkv"], st["d"], st["q"].dtype, device,
                              partition_tiles)
    want, wk, wv = _two_calls(st, plan, device, scale)
    got, gk, gv = _one_call(st, plan, device, scale)
    torch.cuda.synchronize()
    assert torch.equal(gk, wk) and torch.equal(gv, wv), "pool differs from mf_kv_write's"
    assert not torch.isnan(got).any()
    assert torch.equal(got, want), f"output differs: max-abs {(got.float() - want.float()).abs().max().item()}"
    return plan


C2_RUNS = [(1277, 512), (1017, 512), (1661, 512), (999, 512)] + [(c - 1, 1) for c in
                                                                   (64, 4096, 377, 1999, 2048, 17, 1025, 3000)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("partition_tiles", [0, 4])
def test_mixed_step_matches_write_then_attend(device, dtype, partition_tiles):
    """C2's shape: prefill chunks through LDS-shared wide workgroups (tiles of
    new rows read in flight) beside decodes in one mixed launch, with and
    without split-K merges."""
    st = _step(device, dtype, 15, 5, 64, 16, C2_RUNS)
    plan = _check_same(st, device, partition_tiles)
    assert plan.n_narrow and plan.n_wide


@pytest.mark.parametrize("runs", [
    [(0, 512)],                     # a first chunk: every key in flight
    [(16, 48), (32, 17), (5, 3)],   # priors on and off tile boundaries, short chunks
    [(0, 1), (15, 1), (16, 1), (31, 2)],
    [(700, 200), (0, 64), (123, 100), (2000, 1)],
])
@pytest.mark.parametrize("hq,hkv,d", [(15, 5, 64), (40, 8, 128), (16, 4, 32)])
def test_chunks_and_decodes_bf16(device, runs, hq, hkv, d):
    st = _step(device, torch.bfloat16, hq, hkv, d, 16, runs, seed=len(runs) + d)
    _check_same(st, device)


@pytest.mark.parametrize("bs,d", [(4, 16), (16, 64), (8, 32), (32, 16)])
def test_fp32_and_other_block_sizes(device, bs, d):
    """fp32 (wide items stream their own tiles) and blocks other than 16 (the
    general per-key loads read in-flight keys too)."""
    st = _step(device, torch.float32, 6, 2, d, bs, [(37, 20), (0, 9), (64, 1), (5, 1), (100, 33)], seed=bs)
    _check_same(st, device)
    _check_same(st, device, partition_tiles=4)


def test_decode_batch_cooperative_and_merged(device):
    """Decode rows whose ranges run as cooperative units and split-K merges:
    the last tile (the in-flight key) through the general loads."""
    runs = [(c - 1, 1) for c in (9000, 4097, 600, 33, 16, 17, 12000, 2500)]
    st = _step(device, torch.bfloat16, 40, 8, 128, 16, runs, seed=7)
    _check_same(st, device)
    _check_same(st, device, partition_tiles=8)


def test_skipped_slots_leave_the_pool_alone(device):
    """Slots -1 and past the pool are not written (as in mf_kv_write)."""
    st = _step(device, torch.bfloat16, 15, 5, 64, 16, [(40, 30), (10, 1)], seed=3)
    plan = nat.plan_attention(st["cu"], st["kv"], 15, 5, 64, torch.bfloat16, device)
    num_slots = st["kp"].shape[0] * 16
    slots = list(st["slots"])
    slots[0], slots[5], slots[-1] = -1, num_slots, num_slots + 100
    _, gk, gv = _one_call(st, plan, device, 0.125, slots=slots)
    kp, vp = st["kp"].clone(), st["vp"].clone()
    nat.kv_write(st["knew"], st["vnew"], torch.tensor(slots, dtype=torch.int64, device=device),
                 nat.PoolView.from_bshd(kp, vp))
    torch.cuda.synchronize()
    assert torch.equal(gk, kp) and torch.equal(gv, vp)
    assert torch.equal(gk.view(-1, 5, 64)[st["slots"][1]], st["knew"][1])


def test_counted_launch_with_padding_rows(device):
    """A graph-style launch: capacities, live counts on the device, and
    padding entries (no keys, slot -1) at the end of the batch."""
    runs = [(c, 1) for c in (100, 2000, 15, 700, 31)]
    st = _step(device, torch.bfloat16, 15, 5, 64, 16, runs, seed=11)
    pad = 3
    st["q"] = torch.cat([st["q"], torch.randn((pad, 15, 64), device=device).to(torch.bfloat16)])
    st["knew"] = torch.cat([st["knew"], torch.randn((pad, 5, 64), device=device).to(torch.bfloat16)])
    st["vnew"] = torch.cat([st["vnew"], torch.randn((pad, 5, 64), device=device).to(torch.bfloat16)])
    st["cu"] = st["cu"] + [st["cu"][-1] + i + 1 for i in range(pad)]
    st["kv"] = st["kv"] + [0] * pad
    st["positions"] = st["positions"] + [0] * pad
    st["slots"] = st["slots"] + [-1] * pad
    st["tables"] = st["tables"] + [[0]] * pad
    st["T"] += pad
    items, merges, counts = nat.plan_attention_host(st["cu"], st["kv"], 15, 5, 64, torch.bfloat16)
    plan = nat.CountedPlan(int(counts[0]) + 8, int(counts[1]) + 8, int(counts[2]) + 8,
                           int(counts[3]) + 64, device)
    plan.update(items, merges, counts)
    want, wk, wv = _two_calls(st, plan, device, 0.125)
    got, gk, gv = _one_call(st, plan, device, 0.125)
    torch.cuda.synchronize()
    n = st["T"] - pad
    assert torch.equal(gk, wk) and torch.equal(gv, wv)
    assert torch.equal(got[:n], want[:n])


def test_copy_only_call(device):
    """A step whose rows attend to nothing still writes them."""
    st = _step(device, torch.bfloat16, 15, 5, 64, 16, [(0, 3), (20, 2)], seed=5)
    empty = nat.plan_attention([0], [], 15, 5, 64, torch.bfloat16, device)
    kp, vp = st["kp"].clone(), st["vp"].clone()
    bt, cu, kv, pos, slots = _device_meta(st, device)
    out = torch.zeros_like(st["q"])
    nat.paged_attention_kv_write(st["q"], out, nat.PoolView.from_bshd(kp, vp), bt, cu, kv, pos, empty,
                                 0.125, 5, st["knew"], st["vnew"], slots)
    want_k, want_v = st["kp"].clone(), st["vp"].clone()
    nat.kv_write(st["knew"], st["vnew"], slots, nat.PoolView.from_bshd(want_k, want_v))
    torch.cuda.synchronize()
    assert torch.equal(kp, want_k) and torch.equal(vp, want_v)


def test_packed_pass_and_graphed_decode_fused_equal_unfused(device):
    """The engine's passes: an eager packed pass (a prefill chunk beside
    decodes) and graph-replayed decode steps give the same logits and leave
    the same pool with the write inside the attention launch as with a write
    launch of its own."""
    from memforge_amd.runtime.graphed_paged_decode import GraphedPagedDecoder
    from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool
    from memforge_amd.runtime.packed_pass import packed_forward
    from tests.tiny_models import tiny_llama

    model = tiny_llama(num_layers=2, seed=0)
    spec = ModelKVSpec.from_config(model.config, torch.float32, "cuda:0")
    gen = torch.Generator().manual_seed(1)
    tokens = [torch.randint(0, 200, (n,), generator=gen).tolist() for n in (37, 1, 1, 16)]
    starts = [11, 40, 5, 0]
    tables = [[3, 9, 1, 4], [7, 2, 8], [5, 6], [0, 10]]
    pools, logits = [], []
    for fuse in (False, True):
        pool = PagedKVPool(spec, num_blocks=16, block_size=16)
        torch.manual_seed(3)
        pool.key_pool.normal_()
        pool.value_pool.normal_()
        res = packed_forward(model, pool, tokens, starts, tables, keep_rows=[36, 37, 38, 54],
                             fuse_kv_write=fuse)
        dec = GraphedPagedDecoder(model, pool, max_batch=4, max_model_len=120, fuse_kv_write=fuse)
        steps = [dec.step([5, 6, 7], [48, 41, 6], tables[:3]), dec.step([8, 9, 10], [49, 42, 7], tables[:3])]
        torch.cuda.synchronize()
        pools.append((pool.key_pool.clone(), pool.value_pool.clone()))
        logits.append([res.logits.clone(), *steps])
        assert dec.fuse_kv_write == fuse
    assert torch.equal(pools[0][0], pools[1][0]) and torch.equal(pools[0][1], pools[1][1])
    for a, b in zip(*logits):
        assert torch.equal(a, b)
