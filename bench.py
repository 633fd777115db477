#!/usr/bin/env python3
"""Benchmark of MemForge's continuous-batching data path on one MI355X.

Workload (the HBM roofline case the headline
"paged decode attn HBM GB/s" is quoted on): 14B-class GQA decode attention,
40 query heads / 8 KV heads, head_dim 128, bf16 KV, batch 256, context
lengths lognormal (median 2048, sigma 1.0) clipped to [64, 32768], 16-token
blocks with seeded random placement in a pool sized to exactly fit. One
"step" is one decode attention pass over all 48 layers of that shape (the
single layer's pool re-read 48 times; it is 3.6 GB, far beyond every cache).

Prints one JSON line. ``value`` is the whole-job algorithmic HBM bandwidth
(bytes the attention must move / wall time of the timed steps);
``roofline.achieved`` is the same bytes over the attention kernel's own
average duration, measured with HIP events on the stream it runs on.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "paged decode attn HBM GB/s (% peak); output tok/s at 64 concurrent reqs"
HBM_PEAK_GBPS = 8000.0

B, HQ, HKV, D, BS, LAYERS = 256, 40, 8, 128, 16, 48

# HBM traffic of one attention launch on the default workload, from two
# rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), per
# plan form. Each is scaled by what the same counter reads for a plain copy of
# exactly 1 GiB on the MI355X: FETCH_SIZE reports half the bytes (x2.0),
# WRITE_SIZE all (x1.0). None: not measured for that kernel yet.
PMC_DEFAULT = {
    "ranges": {"fetch_kib": 1619051.2, "write_kib": 3210.7, "fetch_scale": 2.0, "write_scale": 1.0},
    "slices": {"fetch_kib": 1609298.0, "write_kib": 3934.5, "fetch_scale": 2.0, "write_scale": 1.0},
}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--sigma", type=float, default=1.0, help="lognormal sigma of context lengths")
    ap.add_argument("--partition-tiles", type=int, default=0,
                    help="split-K partition (16-key tiles) of a per-range plan; 0=auto")
    ap.add_argument("--ranges", action="store_true",
                    help="run C5 with the per-range plan (mf_attention_plan) instead of the decode slice plan")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline duration")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true",
                    help="skip the post-timing check of sampled output rows against a torch fp32 reference")
    ap.add_argument("--fused", action="store_true",
                    help="merge split-K partitions inside the attention kernel (last arrival) instead of a merge kernel")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy (scale factor for PMC byte counters)")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end continuous-batching run")
    ap.add_argument("--e2e-only", action="store_true", help="run only the end-to-end continuous-batching run")
    ap.add_argument("--e2e-requests", type=int, default=64)
    ap.add_argument("--e2e-tokens", type=int, default=128)
    ap.add_argument("--e2e-unfused", action="store_true",
                    help="engine with each layer's KV write as a launch of its own (fused_kv_write=False)")
    ap.add_argument("--e2e-eager", action="store_true",
                    help="run decode steps eagerly instead of replaying the captured decode graph")
    ap.add_argument("--no-mixed", action="store_true", help="skip the C2 mixed-step and C3 verify measurements")
    ap.add_argument("--only", choices=["c1", "c2", "c3", "kv-write", "draft", "c3-engine"],
                    help="run only one section (C2 mixed step, C3 verify, large KV write) and print its JSON")
    return ap.parse_args()


def make_workload(sigma: float, device):
    gen = torch.Generator().manual_seed(0)
    z = torch.randn(B, generator=gen, dtype=torch.float64)
    ctx = torch.clamp(torch.round(torch.exp(math.log(2048.0) + sigma * z)), 64, 32768).to(torch.int64)
    nblk = (ctx + BS - 1) // BS
    n_pool = int(nblk.sum())
    perm = torch.randperm(n_pool, generator=gen)
    max_blocks = int(nblk.max())
    tables = torch.zeros((B, max_blocks), dtype=torch.int32)
    k = 0
    for b in range(B):
        nb = int(nblk[b])
        tables[b, :nb] = perm[k:k + nb].to(torch.int32)
        k += nb
    gdev = torch.Generator(device=device).manual_seed(0)
    kpool = torch.randn((n_pool, BS, HKV, D), generator=gdev, device=device, dtype=torch.bfloat16)
    vpool = torch.randn((n_pool, BS, HKV, D), generator=gdev, device=device, dtype=torch.bfloat16)
    q = torch.randn((B, HQ, D), generator=gdev, device=device, dtype=torch.bfloat16)
    return ctx, tables, kpool, vpool, q


def attn_bytes(ctx: torch.Tensor) -> int:
    """Algorithmic HBM bytes of one decode-attention layer: every visible K and
    V row once (8 heads x 128 x 2 B each), the block-table entries, the query
    read and the output written."""
    kv = int(ctx.sum()) * HKV * D * 2 * 2
    tables = int(((ctx + BS - 1) // BS).sum()) * 4
    qo = B * HQ * D * 2 * 2
    return kv + tables + qo


def check_rows(ctx: torch.Tensor) -> list:
    """Rows of the C5 batch that cover every kind of work in either plan form:
    the shortest and the longest (32,768 keys, cut into several slice pieces
    or merged units), rows of 1,025-2,048 keys (per-range single waves whose
    lanes hold two block-table entries; slices hold several of them),
    2,049-8,192 keys (cooperative units; cut across slices) and more than
    8,192 keys (merged in both forms), the ends of the batch and three seeded
    others."""
    c = ctx.tolist()
    n = len(c)
    pick = [0, n - 1, int(np.argmin(c)), int(np.argmax(c))]
    for lo, hi, k in ((1025, 2048, 3), (2049, 8192, 2), (8193, 32767, 2)):
        pick += [i for i in range(n) if lo <= c[i] <= hi][:k]
    pick += np.random.default_rng(0).choice(n, 3, replace=False).tolist()
    return sorted(set(pick))


def check_output(ctx, tables, kpool, vpool, q, out) -> dict:
    """The kernel's output rows ``check_rows(ctx)`` against a plain torch
    float32 reference on the GPU (gather the context through the block
    table, repeat KV heads, softmax, value product)."""
    rows = check_rows(ctx)
    G = HQ // HKV
    scale = 1.0 / math.sqrt(D)
    kflat, vflat = kpool.view(-1, HKV, D), vpool.view(-1, HKV, D)
    errs, rels = [], []
    for r in rows:
        c = int(ctx[r])
        pos = torch.arange(c, device=q.device)
        table = tables[r, : (c + BS - 1) // BS].to(q.device).long()
        idx = table[pos // BS] * BS + pos % BS
        kk = kflat[idx].float().repeat_interleave(G, dim=1).permute(1, 2, 0).contiguous()  # (Hq, D, c)
        vv = vflat[idx].float().repeat_interleave(G, dim=1).permute(1, 0, 2).contiguous()  # (Hq, c, D)
        w = torch.softmax(torch.bmm(q[r].float().unsqueeze(1), kk) * scale, dim=-1)        # (Hq, 1, c)
        want = torch.bmm(w, vv)[:, 0]
        err = (out[r].float() - want).abs()
        errs.append(float(err.max()))
        rels.append(float(err.mean()) / max(float(want.abs().mean()), 1e-30))
    return {"rows": len(rows), "contexts": [int(ctx[r]) for r in rows], "max_abs_err": max(errs),
            "mean_rel_err": max(rels), "tolerance": "bf16: 2e-2 max-abs, 1e-2 mean-rel",
            "reference": "torch float32 gather + softmax on the GPU, per sampled row",
            "ok": max(errs) <= 2e-2 and max(rels) <= 1e-2}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_time(fn, seconds: float, max_reps: int = 200):
    """Mean wall seconds of fn() on all host cores over about ``seconds``
    (after one untimed call), and the number of timed calls."""
    torch.set_num_threads(os.cpu_count() or 1)
    fn()
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= seconds or reps >= max_reps:
            return dt / reps, reps


def _cpu_leg(value: float, unit: str, sample: str) -> dict:
    return {"value": value, "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "cpu_model": _cpu_model(), "sample": sample}


def cpu_baseline(ctx, tables, kpool, vpool, q, seconds: float):
    from oracle.cpu_baseline import decode_attention_cpu

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    # Bounded sample: the first sequences of the same workload whose contexts
    # add up to a few seconds of work per pass; passes repeat until `seconds`.
    order = list(range(B))
    sample, tok = [], 0
    for b in order:
        sample.append(b)
        tok += int(ctx[b])
        if tok >= 60000:
            break
    sel = torch.tensor(sample)
    used_blocks = sorted({int(x) for b in sample for x in tables[b, : (int(ctx[b]) + BS - 1) // BS]})
    remap = {blk: i for i, blk in enumerate(used_blocks)}
    idx = torch.tensor(used_blocks, device=kpool.device)
    kp = kpool.index_select(0, idx).float().cpu()
    vp = vpool.index_select(0, idx).float().cpu()
    tabs = [[remap[int(x)] for x in tables[b, : (int(ctx[b]) + BS - 1) // BS]] for b in sample]
    qs = q.index_select(0, sel.to(q.device)).float().cpu()
    cs = ctx[sel]
    t0 = time.perf_counter()
    passes = 0
    while True:
        decode_attention_cpu(qs, kp, vp, tabs, cs.tolist(), BS)
        passes += 1
        if time.perf_counter() - t0 >= seconds or passes >= 50:
            break
    dt = time.perf_counter() - t0
    nbytes = int(cs.sum()) * HKV * D * 2 * 2 * passes
    return _cpu_leg(round(nbytes / dt / 1e9, 3), "GB/s",
                    f"{len(sample)} of {B} sequences ({int(cs.sum())} context tokens), 1 layer, "
                    f"{passes} passes in {dt:.1f}s; reference gather+materialised attention ported "
                    f"to torch-CPU float32, bytes counted as the bf16 workload's")


# ------------------------------------------------------------- C2 / C3 steps

SM_HQ, SM_HKV, SM_D, SM_LAYERS = 15, 5, 64, 32  # SmolLM2-360M attention shape
BF16_PEAK_TFLOPS = 2500.0


def _tables_for(kv_lens, gen):
    nblk = [(int(n) + BS - 1) // BS for n in kv_lens]
    perm = torch.randperm(sum(nblk), generator=gen).tolist()
    tables, k = [], 0
    for nb in nblk:
        tables.append(perm[k:k + nb])
        k += nb
    return tables, sum(nblk)


def _graph_us(fn, layers, reps=10):
    """Per-layer GPU time of ``fn(i)`` for i < layers, captured once in a HIP
    graph and replayed: the launches run back to back, so the figure excludes
    the host's submission time that per-call events include at these sizes."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(layers):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(layers):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    evs = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        evs.append((a, b))
    torch.cuda.synchronize()
    return float(np.median([a.elapsed_time(b) for a, b in evs])) * 1e3 / layers


def _event_us(pairs):
    return float(np.mean([a.elapsed_time(b) for a, b in pairs])) * 1e3


def run_c1(dev, reps=50):
    """Config 1: one decode step at the SmolLM2 attention shape in fp32 -- 8
    sequences, contexts U[17, 512], a 1024 x 16 pool with random block
    placement, 15q/5kv heads, D 64, scale 1/8. Timed two ways: the standalone
    operator (PagedKVCache + PagedAttention, one call per sequence, KV heads
    repeated to 15 as that API needs) and one varlen launch for the batch
    (GQA in the kernel). The error is against a torch fp32 gather + softmax
    on the GPU."""
    from memforge_amd import _native as nat
    from memforge_amd.models.paged_attention import PagedAttention, PagedKVCache

    gen = torch.Generator().manual_seed(0)
    ctx = torch.randint(17, 513, (8,), generator=gen).tolist()
    nblk = [(c + BS - 1) // BS for c in ctx]
    perm = torch.randperm(1024, generator=gen).tolist()
    tables, k = [], 0
    for nb in nblk:
        tables.append(perm[k:k + nb])
        k += nb
    gdev = torch.Generator(device=dev).manual_seed(1)
    kp = torch.randn((1024, BS, SM_HKV, SM_D), generator=gdev, device=dev)
    vp = torch.randn_like(kp)
    q = torch.randn((8, SM_HQ, SM_D), generator=gdev, device=dev)
    scale = 1.0 / math.sqrt(SM_D)
    G = SM_HQ // SM_HKV

    # torch fp32 reference: gather each context, repeat KV heads, softmax
    ref = torch.empty_like(q)
    for i, (c, t) in enumerate(zip(ctx, tables)):
        idx = torch.tensor([t[p // BS] * BS + p % BS for p in range(c)], device=dev)
        kk = kp.view(-1, SM_HKV, SM_D)[idx].repeat_interleave(G, dim=1).transpose(0, 1)  # (Hq, c, D)
        vv = vp.view(-1, SM_HKV, SM_D)[idx].repeat_interleave(G, dim=1).transpose(0, 1)
        w = torch.softmax(torch.matmul(q[i][:, None, :], kk.transpose(1, 2).contiguous()) * scale, dim=-1)
        ref[i] = torch.matmul(w, vv)[:, 0]

    # one varlen launch
    out = torch.empty_like(q)
    view = nat.PoolView.from_bshd(kp, vp)
    bt = torch.zeros((8, max(nblk)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    bt = bt.to(dev)
    cu_t = torch.arange(9, dtype=torch.int32, device=dev)
    kv_t = torch.tensor(ctx, dtype=torch.int32, device=dev)
    pos_t = torch.tensor([c - 1 for c in ctx], dtype=torch.int64, device=dev)
    plan = nat.plan_attention(list(range(9)), ctx, SM_HQ, SM_HKV, SM_D, torch.float32, dev)
    partials = torch.empty(max(plan.partials_floats, 1), dtype=torch.float32, device=dev)

    def varlen():
        nat.paged_attention(q, out, view, bt, cu_t, kv_t, pos_t, plan, scale, SM_HKV, partials=partials)

    # the standalone operator over a (blocks, heads, slots, dim) cache with
    # the KV heads repeated
    cache = PagedKVCache(1024, BS, SM_HQ, SM_D, dtype=torch.float32, device=str(dev))
    cache.key_cache.copy_(kp.repeat_interleave(G, dim=2).permute(0, 2, 1, 3))
    cache.value_cache.copy_(vp.repeat_interleave(G, dim=2).permute(0, 2, 1, 3))
    op = PagedAttention(scale)
    qs = [q[i].view(1, SM_HQ, 1, SM_D) for i in range(8)]

    def operator():
        return [op(qs[i], cache, tables[i], ctx[i]) for i in range(8)]

    varlen()
    op_out = torch.stack([o.view(SM_HQ, SM_D) for o in operator()])
    torch.cuda.synchronize()
    err_varlen = float((out - ref).abs().max())
    err_op = float((op_out - ref).abs().max())
    times = {}
    for name, fn in (("varlen", varlen), ("operator", operator)):
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in ev:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        times[name] = _event_us(ev)
    kv_bytes = sum(ctx) * SM_HKV * SM_D * 4 * 2
    graph_us = _graph_us(lambda i: varlen(), 16)

    # CPU baseline: the reference operator (read_kv's per-block slices and
    # cat, fp32 softmax, value product), one call per sequence, on the host
    from oracle.cpu_baseline import operator_cpu

    kc, vc = cache.key_cache.cpu(), cache.value_cache.cpu()
    qs_cpu = [x.cpu() for x in qs]
    cpu_s, cpu_reps = _cpu_time(lambda: [operator_cpu(qs_cpu[i], kc, vc, tables[i], ctx[i]) for i in range(8)],
                                3.0)
    return {
        "workload": "C1: SmolLM2 decode, fp32, 8 sequences, ctx U[17,512], 15q/5kv, D 64, pool 1024x16 "
                    "random placement, scale 1/8",
        "varlen_launch_us": round(times["varlen"], 2),
        "graph_varlen_launch_us": round(graph_us, 2),
        "operator_8_calls_us": round(times["operator"], 2),
        "max_abs_err_varlen": err_varlen,
        "max_abs_err_operator": err_op,
        "tolerance": 1e-5,
        "kv_bytes": kv_bytes,
        "context_tokens": sum(ctx),
        "cpu_baseline": _cpu_leg(round(cpu_s * 1e6, 1), "us per 8 operator calls",
                                 f"the whole C1 step (8 PagedAttention.forward calls, fp32), {cpu_reps} timed "
                                 "repetitions; beside operator_8_calls_us"),
    }


def run_c2(dev, layers=SM_LAYERS, reps=3, fused_leg=True, cpu_leg=True):
    """Mixed ragged step: 4 prefill chunks of 512 on priors U[0,2048] + 28
    decodes with contexts U[64,4096]; per layer the KV scatter of all 2076
    new tokens, then one varlen attention launch pair (decode items, prefill
    items) and the split-K merge. A real per-layer pool (32 layers) so no
    layer's reads come from a cache another layer filled."""
    from memforge_amd import _native as nat

    gen = torch.Generator().manual_seed(0)
    prior = torch.randint(0, 2049, (4,), generator=gen).tolist()
    dctx = torch.randint(64, 4097, (28,), generator=gen).tolist()
    q_lens = [512] * 4 + [1] * 28
    kv = [p + 512 for p in prior] + dctx
    starts = prior + [c - 1 for c in dctx]
    tables, nblocks = _tables_for(kv, gen)
    T = sum(q_lens)
    gdev = torch.Generator(device=dev).manual_seed(0)
    kp = torch.randn((layers, nblocks, BS, SM_HKV, SM_D), generator=gdev, device=dev, dtype=torch.bfloat16)
    vp = torch.randn_like(kp)
    q = torch.randn((T, SM_HQ, SM_D), generator=gdev, device=dev, dtype=torch.bfloat16)
    knew = torch.randn((layers, T, SM_HKV, SM_D), generator=gdev, device=dev, dtype=torch.bfloat16)
    vnew = torch.randn_like(knew)
    out = torch.empty_like(q)
    cu = [0]
    for n in q_lens:
        cu.append(cu[-1] + n)
    positions = [s + i for s, n in zip(starts, q_lens) for i in range(n)]
    slots = [tables[e][p // BS] * BS + p % BS for e, (s0, n) in enumerate(zip(starts, q_lens))
             for p in range(s0, s0 + n)]
    slot_t = torch.tensor(slots, dtype=torch.int64, device=dev)
    bt = torch.zeros((len(kv), max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    bt = bt.to(dev)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    kv_t = torch.tensor(kv, dtype=torch.int32, device=dev)
    pos_t = torch.tensor(positions, dtype=torch.int64, device=dev)
    plan = nat.plan_attention(cu, kv, SM_HQ, SM_HKV, SM_D, torch.bfloat16, dev)
    partials = torch.empty(max(plan.partials_floats, 1), dtype=torch.float32, device=dev)
    # The mixed plan's three parts, each launched alone: its decode items,
    # its prefill items (the same items, partial slots and order as in the
    # mixed launch) and its merge, so the parts read and write the same
    # partials as the engine's launch.
    nn = plan.n_narrow
    narrow = nat.AttentionPlan(plan.items, plan.merges, nn, 0, 0, plan.partials_floats,
                               plan.items_host, plan.merges_host)
    wide = nat.AttentionPlan(plan.items[nn:], plan.merges, 0, plan.n_wide, 0, plan.partials_floats,
                             plan.items_host[nn:], plan.merges_host)
    merges = nat.AttentionPlan(plan.items, plan.merges, 0, 0, plan.n_merges, plan.partials_floats,
                               plan.items_host, plan.merges_host)
    # A prefill-only step (the decodes given no rows) plans the same chunks
    # as wide items only: the planner's XCD order and the single-class
    # partition. Its items are timed as a side figure.
    plan_pre = nat.plan_attention(cu[:5] + [cu[4]] * 28, kv, SM_HQ, SM_HKV, SM_D, torch.bfloat16, dev)
    assert plan_pre.n_narrow == 0 and plan_pre.n_wide > 0, "prefill-only plan holds decode items"
    wide_pre = nat.AttentionPlan(plan_pre.items, plan_pre.merges, 0, plan_pre.n_wide, 0, plan_pre.partials_floats,
                                 plan_pre.items_host, plan_pre.merges_host)
    partials_pre = torch.empty(max(plan_pre.partials_floats, 1), dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(SM_D)
    views = [nat.PoolView.from_bshd(kp[i], vp[i]) for i in range(layers)]

    def layer(i, ev=None):
        if ev:
            ev[0].record()
        nat.kv_write(knew[i], vnew[i], slot_t, views[i])
        if ev:
            ev[1].record()
        for part, e in ((narrow, 2), (wide, 3), (merges, 4)):
            if part.n_narrow + part.n_wide + part.n_merges:
                nat.paged_attention(q, out, views[i], bt, cu_t, kv_t, pos_t, part, scale, SM_HKV, partials=partials)
            if ev:
                ev[e].record()

    for i in range(layers):
        layer(i)
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(layers * reps)]
    for r in range(reps):
        for i in range(layers):
            layer(i, evs[r * layers + i])
    torch.cuda.synchronize()
    write_us = _event_us([(e[0], e[1]) for e in evs])
    dec_us = _event_us([(e[1], e[2]) for e in evs])
    pre_us = _event_us([(e[2], e[3]) for e in evs])
    mrg_us = _event_us([(e[3], e[4]) for e in evs])
    graph_layer_us = _graph_us(layer, layers)
    pre_evs = []
    for r in range(reps):
        for i in range(layers):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            nat.paged_attention(q, out, views[i], bt, cu_t, kv_t, pos_t, wide_pre, scale, SM_HKV,
                                partials=partials_pre)
            b.record()
            pre_evs.append((a, b))
    torch.cuda.synchronize()
    pre_only_us = _event_us(pre_evs)

    def layer_whole(i):
        # the engine's form: one call with the whole plan (decode and prefill
        # items in one launch, then the merge)
        nat.kv_write(knew[i], vnew[i], slot_t, views[i])
        nat.paged_attention(q, out, views[i], bt, cu_t, kv_t, pos_t, plan, scale, SM_HKV, partials=partials)

    graph_whole_us = _graph_us(layer_whole, layers)

    def layer_fused(i):
        # the engine's default form: the KV write rides in the attention launch
        # (new keys read from the new rows), then the merge
        nat.paged_attention_kv_write(q, out, views[i], bt, cu_t, kv_t, pos_t, plan, scale, SM_HKV,
                                     knew[i], vnew[i], slot_t)

    graph_fused_us = _graph_us(layer_fused, layers) if fused_leg else float("nan")
    kvb = SM_HKV * SM_D * 2 * 2  # K+V bytes per token per layer
    write_bytes = T * kvb * 2 + T * 8  # read new rows, write pool rows, read slots
    # The engine's layer (one launch for the KV write and every item, then the
    # merge): every attended K/V row read once (a chunk's own new rows among
    # them), the new rows written to the pool once, their slots, Q read and
    # the output written once, one block-table entry per key tile; FLOPs
    # 4 Hq D per (row, visible key), decode rows included.
    eng_bytes = (sum(kv) * kvb + T * kvb + T * 8 + T * SM_HQ * SM_D * 2 * 2
                 + sum((c + BS - 1) // BS for c in kv) * 4)
    eng_flops = (sum(4 * SM_HQ * SM_D * (p + i + 1) for p in prior for i in range(512))
                 + sum(4 * SM_HQ * SM_D * c for c in dctx))
    t_hbm = eng_bytes / (HBM_PEAK_GBPS * 1e3)
    t_mfma = eng_flops / (BF16_PEAK_TFLOPS * 1e6)
    dec_bytes = sum(dctx) * kvb + 28 * SM_HQ * SM_D * 2 * 2
    pre_bytes = sum(p + 512 for p in prior) * kvb + 4 * 512 * SM_HQ * SM_D * 2 * 2
    pre_flops = sum(4 * SM_HQ * SM_D * (p + i + 1) for p in prior for i in range(512))
    return {
        "workload": "C2: 4 prefill chunks x 512 (prior U[0,2048]) + 28 decodes (ctx U[64,4096]), 15q/5kv, "
                    "D 64, bf16, block 16, KV scatter of 2076 tokens, 32 layers x 3 reps",
        "kv_write_us": round(write_us, 2),
        "kv_write_gbps": round(write_bytes / write_us / 1e3, 1),
        "kv_write_frac": round(write_bytes / write_us / 1e3 / HBM_PEAK_GBPS, 4),
        "decode_attn_us": round(dec_us, 2),
        "decode_attn_gbps": round(dec_bytes / dec_us / 1e3, 1),
        "prefill_attn_us": round(pre_us, 2),
        "prefill_attn_tflops": round(pre_flops / pre_us / 1e6, 1),
        "prefill_mfma_frac": round(pre_flops / pre_us / 1e6 / BF16_PEAK_TFLOPS, 4),
        "prefill_attn_gbps": round(pre_bytes / pre_us / 1e3, 1),
        "merge_us": round(mrg_us, 2),
        "prefill_only_plan": {
            "us": round(pre_only_us, 2),
            "tflops": round(pre_flops / pre_only_us / 1e6, 1),
            "mfma_frac": round(pre_flops / pre_only_us / 1e6 / BF16_PEAK_TFLOPS, 4),
            "wide_items": plan_pre.n_wide,
            "note": "side figure: the same chunks planned as a prefill-only step (no decodes), its prefill "
                    "items alone between events",
        },
        "timing_note": "kv_write/decode/prefill/merge figures are the mixed plan's parts timed apart between "
                       "events (side figures: the engine runs decode and prefill items in one launch, see "
                       "engine_layer)",
        "plan": {"narrow": plan.n_narrow, "wide": plan.n_wide, "merges": plan.n_merges},
        "engine_layer": {
            "us": round(graph_fused_us, 2),
            "form": "graph_step_fused_layer_us: one launch for the KV write, decode and prefill items, "
                    "then the merge",
            "bytes": eng_bytes,
            "flops": eng_flops,
            "gbps": round(eng_bytes / graph_fused_us / 1e3, 1),
            "tflops": round(eng_flops / graph_fused_us / 1e6, 1),
            "hbm_us_at_peak": round(t_hbm, 2),
            "mfma_us_at_peak": round(t_mfma, 2),
            "bound": "hbm" if t_hbm >= t_mfma else "mfma",
            "bound_us": round(max(t_hbm, t_mfma), 2),
            "frac": round(max(t_hbm, t_mfma) / graph_fused_us, 4),
            "serial_bound_us": round(t_hbm + t_mfma, 2),
            "serial_frac": round((t_hbm + t_mfma) / graph_fused_us, 4),
            "note": "bound: the larger of the bytes at 8 TB/s and the FLOPs at the 2.5 PFLOP/s bf16 dense "
                    "peak (both overlapped); serial: their sum",
        } if fused_leg else None,
        "step_attn_us": round(dec_us + pre_us + mrg_us, 2),
        "graph_layer_us": round(graph_layer_us, 2),
        "graph_note": "one layer's KV write + decode items + prefill items + merge, replayed as a captured "
                      "graph of all layers (no host submission time)",
        "graph_step_layer_us": round(graph_whole_us, 2),
        "graph_step_note": "KV write, then one attention call with the whole plan (decode and prefill items "
                           "in one launch, then the merge)",
        "graph_step_fused_layer_us": round(graph_fused_us, 2),
        "graph_step_fused_note": "the layer as the engine runs it: one launch for the KV write and the decode "
                                 "and prefill items (new keys read from the new rows), then the merge",
        "cpu_baseline": _c2_c3_cpu_leg(kp[0], vp[0], knew[0], vnew[0], slot_t, q, tables, cu, positions,
                                       "C2 layer: KV scatter of 2076 rows + the materialised varlen attention "
                                       "of 2076 rows (4 causal chunks of 512 + 28 decodes); beside "
                                       "graph_step_fused_layer_us") if cpu_leg else None,
    }


def _c2_c3_cpu_leg(kp, vp, knew, vnew, slots, q, tables, cu, positions, what: str) -> dict:
    """CPU baseline of one C2/C3 layer: the reference's KV scatter
    (index_copy_ through slot_mapping) and its materialised varlen attention,
    in fp32 on the host cores, on the same data as the GPU leg."""
    from oracle.cpu_baseline import varlen_cpu

    kpc, vpc = kp.float().cpu(), vp.float().cpu()
    kn, vn, sl = knew.float().cpu(), vnew.float().cpu(), slots.cpu()
    qc = q.float().cpu()
    H, D = kpc.shape[2], kpc.shape[3]

    def layer():
        kpc.view(-1, H, D).index_copy_(0, sl, kn)
        vpc.view(-1, H, D).index_copy_(0, sl, vn)
        varlen_cpu(qc, kpc, vpc, tables, cu, positions, BS)

    secs, reps = _cpu_time(layer, 4.0)
    return _cpu_leg(round(secs * 1e6, 1), "us per layer", f"{what}; fp32, {reps} timed layers")


def run_kv_write_large(dev, tokens=33792, sets=6, reps=10):
    """KV write of a C4-sized prefill step (33,792 tokens of the SmolLM2
    shape, bf16) into a shuffled pool: the streaming case of the same kernel.
    Timed as graph replays of back-to-back launches (a single ~15 us launch
    between two events carries several us of submission gap), cycling through
    ``sets`` independent sources and pools (6 x 130 MB, more than the 256 MB
    Infinity Cache holds) so no launch reads what the previous one left in a
    cache."""
    from memforge_amd import _native as nat

    gen = torch.Generator().manual_seed(1)
    nblocks = (tokens + BS - 1) // BS + 64
    bufs = []
    for _ in range(sets):
        perm = torch.randperm(nblocks * BS, generator=gen)[:tokens].to(dev)
        kp = torch.zeros((nblocks, BS, SM_HKV, SM_D), device=dev, dtype=torch.bfloat16)
        vp = torch.zeros_like(kp)
        k = torch.randn((tokens, SM_HKV, SM_D), device=dev, dtype=torch.bfloat16)
        bufs.append((k, torch.randn_like(k), perm, nat.PoolView.from_bshd(kp, vp),
                     torch.empty_like(k), torch.empty_like(k)))
    us = _graph_us(lambda i: nat.kv_write(bufs[i][0], bufs[i][1], bufs[i][2], bufs[i][3]), sets, reps)
    gus = _graph_us(lambda i: nat.kv_gather(bufs[i][3], bufs[i][2], bufs[i][4], bufs[i][5]), sets, reps)
    nbytes = tokens * SM_HKV * SM_D * 2 * 2 * 2 + tokens * 8
    return {"tokens": tokens, "us": round(us, 2), "gbps": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4),
            "gather_us": round(gus, 2), "gather_gbps": round(nbytes / gus / 1e3, 1),
            "timing": f"graph replays of back-to-back launches over {sets} rotating buffer sets"}


def run_c3(dev, layers=SM_LAYERS, reps=3, cpu_leg=True):
    """Speculative verify step: 16 sequences, ctx U[128,2048], lookahead 4,
    so 5 query rows per sequence attend to the pool plus their own in-flight
    candidates; then rejection sampling over (16,5,49152) target and
    (16,4,49152) draft logits, N(0, variance 2), with seeded uniforms/noise."""
    from memforge_amd import _native as nat

    gen = torch.Generator().manual_seed(0)
    B, K, V = 16, 4, 49152
    ctx = torch.randint(128, 2049, (B,), generator=gen).tolist()
    tables, nblocks = _tables_for([c + K + 1 for c in ctx], gen)
    tl = torch.randn((B, K + 1, V), generator=gen) * math.sqrt(2.0)
    dl = torch.randn((B, K, V), generator=gen) * math.sqrt(2.0)
    dprobs = torch.softmax(dl, dim=-1)
    dtok = torch.stack([torch.multinomial(dprobs[b], 1, generator=gen).view(-1) for b in range(B)])
    u = torch.rand((B, K), generator=gen)
    noise = torch.empty((B, V)).exponential_(1.0, generator=gen)
    gdev = torch.Generator(device=dev).manual_seed(0)
    kp = torch.randn((layers, nblocks, BS, SM_HKV, SM_D), generator=gdev, device=dev, dtype=torch.bfloat16)
    vp = torch.randn_like(kp)
    T = B * (K + 1)
    q = torch.randn((T, SM_HQ, SM_D), generator=gdev, device=dev, dtype=torch.bfloat16)
    nk = torch.randn((layers, T, SM_HKV, SM_D), generator=gdev, device=dev, dtype=torch.bfloat16)
    nv = torch.randn_like(nk)
    out = torch.empty_like(q)
    cu = [b * (K + 1) for b in range(B + 1)]
    kvl = [c + K + 1 for c in ctx]
    positions = [c + j for c in ctx for j in range(K + 1)]
    bt = torch.zeros((B, max(len(t) for t in tables)), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    bt = bt.to(dev)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    kv_t = torch.tensor(kvl, dtype=torch.int32, device=dev)
    pl_t = torch.tensor(ctx, dtype=torch.int32, device=dev)
    pos_t = torch.tensor(positions, dtype=torch.int64, device=dev)
    plan = nat.plan_attention(cu, kvl, SM_HQ, SM_HKV, SM_D, torch.bfloat16, dev)
    partials = torch.empty(max(plan.partials_floats, 1), dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(SM_D)
    views = [nat.PoolView.from_bshd(kp[i], vp[i]) for i in range(layers)]

    def layer(i):
        nat.paged_attention(q, out, views[i], bt, cu_t, kv_t, pos_t, plan, scale, SM_HKV, pool_lens=pl_t,
                            new_k_rows=nk[i], new_v_rows=nv[i], partials=partials)

    for i in range(layers):
        layer(i)
    torch.cuda.synchronize()
    evs = []
    for _ in range(reps):
        for i in range(layers):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            layer(i)
            b.record()
            evs.append((a, b))
    torch.cuda.synchronize()
    attn_us = _event_us(evs)
    graph_attn_us = _graph_us(layer, layers)
    kvb = SM_HKV * SM_D * 2 * 2
    attn_bytes = sum(c + K + 1 for c in ctx) * kvb + T * SM_HQ * SM_D * 2 * 2
    attn_flops = sum(4 * SM_HQ * SM_D * (c + j + 1) for c in ctx for j in range(K + 1))

    tl_d, dp_d, dt_d = tl.to(dev), dprobs.to(dev), dtok.to(torch.int32).to(dev)
    u_d, n_d = u.to(dev), noise.to(dev)
    res = nat.spec_verify(dt_d, dp_d, tl_d, 1.0, u_d, n_d)
    torch.cuda.synchronize()
    vevs = []
    for _ in range(10):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        nat.spec_verify(dt_d, dp_d, tl_d, 1.0, u_d, n_d)
        b.record()
        vevs.append((a, b))
    torch.cuda.synchronize()
    ver_us = _event_us(vevs)
    graph_ver_us = _graph_us(lambda i: nat.spec_verify(dt_d, dp_d, tl_d, 1.0, u_d, n_d), 10)
    ver_bytes = (B * (K + 1) * V + B * K * V) * 4
    return {
        "workload": "C3: 16 sequences, ctx U[128,2048], lookahead 4 (5 query rows each, candidates attended "
                    "in flight), 15q/5kv, D 64, bf16, 32 layers x 3 reps; rejection over (16,5,49152) target "
                    "and (16,4,49152) draft fp32 logits N(0, var 2), temperature 1",
        "verify_attn_us": round(attn_us, 2),
        "verify_attn_gbps": round(attn_bytes / attn_us / 1e3, 1),
        "verify_attn_frac": round(attn_bytes / attn_us / 1e3 / HBM_PEAK_GBPS, 4),
        "verify_attn_tflops": round(attn_flops / attn_us / 1e6, 2),
        "graph_verify_attn_us": round(graph_attn_us, 2),
        "graph_verify_attn_gbps": round(attn_bytes / graph_attn_us / 1e3, 1),
        "rejection_us": round(ver_us, 2),
        "rejection_gbps": round(ver_bytes / ver_us / 1e3, 1),
        "graph_rejection_us": round(graph_ver_us, 2),
        "graph_rejection_note": "per call, ten calls captured in one graph and replayed (kernels only, no host submission)",
        "accepted_per_row": res.num_accepted.cpu().tolist(),
        # the candidates' K/V go through the same scatter the CPU path would
        # do before attending them (the reference writes them to the pool)
        "cpu_baseline": _c2_c3_cpu_leg(kp[0], vp[0], nk[0], nv[0], torch.tensor(
            [tables[b][p // BS] * BS + p % BS for b, c in enumerate(ctx) for p in range(c, c + K + 1)]),
            q, tables, cu, positions, "C3 layer: scatter of the 80 verify rows + the materialised varlen "
            "attention of 16 x 5 rows; beside graph_verify_attn_us") if cpu_leg else None,
        "rejection_cpu_baseline": _rejection_cpu_leg(dtok, dprobs, tl, u, noise) if cpu_leg else None,
    }


def _rejection_cpu_leg(dtok, dprobs, tl, u, noise) -> dict:
    """CPU baseline of the C3 rejection step: the reference's per-row
    resolve (vocabulary clip, fp32 softmax of the target, the accept walk in
    double and the final multinomial draw as argmax(p / E)), restated in
    numpy, on the same logits, uniforms and noise."""
    from oracle import rejection as orj

    dp, tlog, un, nz = dprobs.numpy(), tl.numpy(), u.numpy(), noise.numpy()
    cand = dtok.tolist()

    def rows():
        for b in range(len(cand)):
            orj.resolve_round(cand[b], list(dp[b]), list(tlog[b]), 1.0, list(un[b]), nz[b])

    secs, reps = _cpu_time(rows, 3.0, max_reps=20)
    return _cpu_leg(round(secs * 1e6, 1), "us per verify step",
                    f"16 rows x 4 candidates, vocab 49152, temperature 1; {reps} timed steps; beside rejection_us")


# --------------------------------------------------------------------- C4 E2E

E2E_MODEL = dict(vocab_size=49152, hidden_size=960, intermediate_size=2560, num_hidden_layers=32,
                 num_attention_heads=15, num_key_value_heads=5, head_dim=64)
E2E_RATE = 20.0  # requests per second
E2E_KV_MB = 4096


class _NullTokenizer:
    """Token ids in, short text out: the engine detokenizes every emitted token,
    and a real tokenizer (none is available offline) would only add host time."""

    eos_token_id = None
    pad_token_id = 0

    def __call__(self, text, return_tensors=None):
        return {"input_ids": [2 + (ord(c) % 1000) for c in text]}

    def decode(self, ids, skip_special_tokens=True):
        return "x" * len(ids)


def e2e_workload(n: int, seed: int = 0):
    """Arrival times (Exp(rate 20) gaps), prompts with lengths U[32, 1024] and
    ids U[0, 49152), drawn in that order from one seeded CPU generator."""
    gen = torch.Generator().manual_seed(seed)
    gaps = torch.empty(n, dtype=torch.float64).exponential_(E2E_RATE, generator=gen)
    arrivals = torch.cumsum(gaps, 0).tolist()
    lens = torch.randint(32, 1025, (n,), generator=gen)
    prompts = [torch.randint(0, E2E_MODEL["vocab_size"], (int(m),), generator=gen).tolist() for m in lens]
    return arrivals, prompts


def _drive(engine, prompts, arrivals, params):
    """Run requests to completion. With ``arrivals`` the clock is virtual: it
    advances by each step's measured wall time and jumps to the next arrival
    when the engine is idle; request i is submitted before the first step
    that starts at or after arrivals[i]. Without, all are submitted at 0."""
    n = len(prompts)
    i, clock, steps, ids = 0, 0.0, 0, []
    if arrivals is None:
        ids = [engine.submit(p, params) for p in prompts]
        i = n
    t0 = time.perf_counter()
    while i < n or engine.has_work():
        if arrivals is not None:
            if i < n and not engine.has_work():
                clock = max(clock, arrivals[i])
            while i < n and arrivals[i] <= clock:
                ids.append(engine.submit(prompts[i], params))
                i += 1
        s0 = time.perf_counter()
        engine.step()
        clock += time.perf_counter() - s0
        steps += 1
    wall = time.perf_counter() - t0
    tokens = sum(len(engine.runtimes[x].generated) for x in ids)
    return ids, tokens, steps, wall, clock


def run_e2e(args, dev):
    from transformers import LlamaConfig, LlamaForCausalLM

    from memforge_amd.runtime import ContinuousBatchingEngine, SamplingParams

    cfg = LlamaConfig(**E2E_MODEL, max_position_embeddings=2048, tie_word_embeddings=True,
                      bos_token_id=1, eos_token_id=2, pad_token_id=0)
    torch.manual_seed(0)
    with torch.device(dev):
        model = LlamaForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    n_params = sum(p.numel() for p in model.parameters())
    engine = ContinuousBatchingEngine(model, _NullTokenizer(), block_size=BS, kv_budget_mb=E2E_KV_MB,
                                      max_num_seqs=64, max_model_len=2048, dtype=torch.bfloat16,
                                      paged_cuda_graph=not args.e2e_eager,
                                      fused_kv_write=not args.e2e_unfused)
    params = SamplingParams(max_new_tokens=args.e2e_tokens, temperature=0.0, top_p=1.0, stop_on_eos=False)
    arrivals, prompts = e2e_workload(args.e2e_requests)

    _drive(engine, prompts[:4], None, SamplingParams(max_new_tokens=4, temperature=0.0, stop_on_eos=False))
    torch.cuda.synchronize()

    ids, tok_p, steps_p, wall_p, clock_p = _drive(engine, prompts, arrivals, params)
    kv0, rows0, passes0 = (engine.total_attended_kv_tokens, engine.total_packed_rows,
                           engine.total_forward_passes)
    ids_s, tok_s, steps_s, wall_s, _ = _drive(engine, prompts, None, params)
    kv_tokens = engine.total_attended_kv_tokens - kv0
    rows = engine.total_packed_rows - rows0
    passes = engine.total_forward_passes - passes0
    spec = engine.spec
    kv_bytes_per_token = spec.bytes_per_token  # K and V, every layer
    # bytes a step cannot avoid: every weight once per pass, every visible K/V
    # row once, every new K/V row written once
    bytes_s = passes * 2 * n_params + kv_tokens * kv_bytes_per_token + rows * kv_bytes_per_token
    ideal_s = bytes_s / (HBM_PEAK_GBPS * 1e9)
    return {
        "workload": (f"C4: {args.e2e_requests} requests, Poisson {E2E_RATE:g} req/s (virtual time), prompts "
                     f"U[32,1024], {args.e2e_tokens} greedy tokens, SmolLM2-360M-shaped Llama bf16 random "
                     f"init, KV {E2E_KV_MB} MB in 16-token blocks, max_num_seqs 64"),
        "decode_steps": "eager" if args.e2e_eager else "HIP graph replay (paged_cuda_graph)",
        "kv_write": "separate launch" if args.e2e_unfused else "inside each layer's attention launch",
        "poisson_tok_s": round(tok_p / max(clock_p - arrivals[0], 1e-9), 1),
        "poisson_steps": steps_p,
        "poisson_virtual_s": round(clock_p - arrivals[0], 3),
        "saturated_tok_s": round(tok_s / wall_s, 1),
        "saturated_steps": steps_s,
        "saturated_wall_s": round(wall_s, 3),
        "saturated_ms_per_step": round(wall_s / steps_s * 1e3, 3),
        "output_tokens": tok_s,
        "params": n_params,
        "kv_pool_blocks": engine.pool.num_blocks,
        "roofline": {
            "bound": "hbm",
            "bytes": bytes_s,
            "ideal_s": round(ideal_s, 4),
            "frac": round(ideal_s / wall_s, 4),
            "note": "algorithmic bytes of the saturated run (weights once per pass + visible K/V + K/V "
                    "writes) at 8 TB/s over its wall time",
        },
        "telemetry": {k: v for k, v in engine.telemetry().items()
                      if k.startswith(("attention_", "kv_write_", "decode_graph_", "data_path_"))},
        "cpu_baseline": None if args.no_cpu_baseline else _e2e_cpu_leg(cfg, prompts),
    }


def _e2e_cpu_leg(cfg, prompts, n_requests: int = 8, new_tokens: int = 64) -> dict:
    """CPU baseline of C4: the reference engine's CPU path (the host
    scheduler, a forward per prefill, one left-padded batched forward per
    decode step over contexts gathered from the pool; oracle.cpu_engine) with
    the same model shape in fp32 on the host cores, the first requests of the
    same workload all submitted at once."""
    from transformers import LlamaForCausalLM

    from oracle.cpu_engine import CpuBatchedEngine

    torch.set_num_threads(os.cpu_count() or 1)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).float().eval()
    sample = prompts[:n_requests]
    need = sum((len(p) + new_tokens + BS - 1) // BS for p in sample)
    eng = CpuBatchedEngine(model, num_blocks=need + n_requests, block_size=BS, max_num_seqs=n_requests)
    t0 = time.perf_counter()
    out = eng.generate(sample, new_tokens)
    dt = time.perf_counter() - t0
    assert all(len(o) == new_tokens for o in out)
    return _cpu_leg(round(n_requests * new_tokens / dt, 2), "output tok/s",
                    f"{n_requests} concurrent requests (prompts of {[len(p) for p in sample]} tokens) x "
                    f"{new_tokens} greedy tokens through the reference's batched CPU path (host scheduler, "
                    f"{eng.forward_passes} forward passes, left-padded batched decode), SmolLM2-360M shape, "
                    f"fp32, {dt:.1f} s incl. prefill; beside saturated_tok_s")


# --------------------------------------------------- draft proposals (C3 shape)

DRAFT_MODEL = dict(vocab_size=49152, hidden_size=576, intermediate_size=1536, num_hidden_layers=30,
                   num_attention_heads=9, num_key_value_heads=3, head_dim=64)


def run_draft(dev, rounds=8, warm=2, batch=16, k=4):
    """One speculative round's draft proposals for the C3 batch (16 sequences,
    contexts U[128, 2048], lookahead 4, greedy) with a SmolLM2-135M-shaped
    draft, bf16, random init. Three forms: the eager per-sequence draft
    (DynamicCache, one forward per token, a host read per candidate), the
    batched graphed pool (K+1 replays for the whole batch, argmax fed back on
    the device) and its unrolled form (one replay per round). Each timed round
    is the engine's steady state: one new confirmed token per sequence."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from memforge_amd.runtime.batched_speculative import (BatchedGraphedDraftPool, DraftState,
                                                           propose_draft_tokens)

    cfg = LlamaConfig(**DRAFT_MODEL, max_position_embeddings=4096, tie_word_embeddings=True,
                      bos_token_id=1, eos_token_id=2, pad_token_id=0)
    torch.manual_seed(0)
    with torch.device(dev):
        model = LlamaForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    gen = torch.Generator().manual_seed(3)
    lens = torch.randint(128, 2049, (batch,), generator=gen).tolist()
    base = [torch.randint(2, DRAFT_MODEL["vocab_size"], (n,), generator=gen).tolist() for n in lens]
    max_len = max(lens) + (warm + rounds) * 1 + k + 8

    def drive(propose, states):
        toks = [list(t) for t in base]
        times, cands = [], []
        for r in range(warm + rounds):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = propose(states, toks)
            torch.cuda.synchronize()
            if r >= warm:
                times.append(time.perf_counter() - t0)
            cands.append([c for c, _ in out])
            for st, t, (c, _) in zip(states, toks, out):
                st.rollback_to(len(t))
                t.append(c[0])
        return float(np.mean(times)) * 1e3, cands

    res = {"workload": f"C3 draft side: {batch} sequences, ctx U[128,2048], lookahead {k}, greedy, "
                       "SmolLM2-135M-shaped draft (30 layers, 9q/3kv, D 64, vocab 49152) bf16 random init; "
                       "one new confirmed token per sequence per round"}
    eager_states = [DraftState() for _ in range(batch)]
    ms, eager_c = drive(lambda sts, toks: [propose_draft_tokens(model, st, t, k, 0.0, dev)
                                            for st, t in zip(sts, toks)], eager_states)
    res["eager_ms_per_round"] = round(ms, 3)
    del eager_states
    torch.cuda.empty_cache()
    for name, unroll in (("batched", False), ("unrolled", True)):
        pool = BatchedGraphedDraftPool(model, max_len=max_len, num_slots=batch, device=str(dev), unroll=unroll)
        states = [pool.acquire() for _ in range(batch)]
        ms, c = drive(lambda sts, toks: pool.propose(sts, toks, k, 0.0), states)
        res[f"{name}_ms_per_round"] = round(ms, 3)
        res[f"{name}_replays_per_round"] = pool.replays / (warm + rounds)
        res[f"{name}_same_candidates_as_eager"] = sum(a == b for x, y in zip(c, eager_c) for a, b in zip(x, y))
        del pool, states
        torch.cuda.empty_cache()
    res["candidate_lists"] = batch * (warm + rounds)
    res["speedup_batched"] = round(res["eager_ms_per_round"] / res["batched_ms_per_round"], 2)
    res["speedup_unrolled"] = round(res["eager_ms_per_round"] / res["unrolled_ms_per_round"], 2)
    return res


def run_c3_engine(dev, batch=16, k=4, rounds=8):
    """Engine-level C3 round: a SmolLM2-360M-shaped target with a
    SmolLM2-135M-shaped draft (bf16, random init), 16 requests with contexts
    U[128, 2048], lookahead 4. One timed step is one speculative round for all
    16 rows: batched graphed draft proposals, one verify pass with the
    candidates attended in flight, the rejection step and the confirmed-prefix
    KV write. Timed with the rows resolved by one rejection launch and one
    KV write per layer, then (same seeds) one row at a time."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from memforge_amd.runtime import ContinuousBatchingEngine, SamplingParams

    def build(shape, seed):
        cfg = LlamaConfig(**shape, max_position_embeddings=4096, tie_word_embeddings=True, bos_token_id=1,
                          eos_token_id=2, pad_token_id=0)
        torch.manual_seed(seed)
        with torch.device(dev):
            m = LlamaForCausalLM(cfg)
        return m.to(torch.bfloat16).eval()

    target, draft = build(E2E_MODEL, 0), build(DRAFT_MODEL, 1)
    gen = torch.Generator().manual_seed(5)
    lens = torch.randint(128, 2049, (batch,), generator=gen).tolist()
    prompts = [torch.randint(3, E2E_MODEL["vocab_size"], (n,), generator=gen).tolist() for n in lens]
    out = {"workload": f"C3 engine round: {batch} requests, ctx U[128,2048], lookahead {k}, SmolLM2-360M-shaped "
                       "target + SmolLM2-135M-shaped draft, bf16 random init, greedy and T=0.8 rows alternating"}
    for name, batched in (("batched", True), ("per_row", False)):
        eng = ContinuousBatchingEngine(target, _NullTokenizer(), block_size=BS, kv_budget_mb=2048,
                                       max_num_seqs=batch, max_model_len=2048 + 64, dtype=torch.bfloat16,
                                       draft_model=draft, lookahead_k=k, draft_cuda_graph="batched",
                                       paged_cuda_graph=True)
        eng._batched_resolve = batched
        torch.manual_seed(7)
        torch.cuda.manual_seed(7)
        for i, p in enumerate(prompts):
            eng.submit(p, SamplingParams(max_new_tokens=60, temperature=0.8 if i % 2 else 0.0, top_p=1.0,
                                         stop_on_eos=False))
        while eng.total_speculative_rounds < 2:  # prefill, then two warm rounds
            eng.step()
        times, toks = [], 0
        for _ in range(rounds):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            rep = eng.step()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
            toks += rep.tokens_emitted
        t = eng.telemetry()
        out[f"{name}_round_ms"] = round(float(np.median(times)) * 1e3, 3)
        out[f"{name}_tokens_per_round"] = round(toks / rounds, 2)
        out[f"{name}_acceptance_rate"] = t["draft_acceptance_rate"]
        del eng
        torch.cuda.empty_cache()
    out["speedup"] = round(out["per_row_round_ms"] / out["batched_round_ms"], 3)
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU: every box in this run has a single "
                                   "MI355X, and the data path is per GPU (across GPUs it shards by "
                                   "request, each GPU with its own pool)"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device"}))
        sys.exit(1)
    from memforge_amd import _native as nat

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = 256 << 20
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "copies": 3}))
        return
    if args.e2e_only:
        print(json.dumps({"e2e": run_e2e(args, dev)}))
        return
    if args.only:
        section = {"c1": run_c1, "c2": run_c2, "c3": run_c3, "kv-write": run_kv_write_large, "draft": run_draft,
                   "c3-engine": run_c3_engine}[args.only]
        print(json.dumps({args.only: section(dev)}))
        return
    ctx, tables, kpool, vpool, q = make_workload(args.sigma, dev)
    out = torch.empty_like(q)
    bt = tables.to(dev)
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev)
    kv_lens = ctx.to(torch.int32).to(dev)
    positions = (ctx - 1).to(dev)
    # The decode slice plan unless a per-range plan is asked for (a forced
    # partition or the fused merge are per-range features).
    slices = not (args.ranges or args.partition_tiles or args.fused)
    plan = nat.plan_attention(list(range(B + 1)), ctx.tolist(), HQ, HKV, D, torch.bfloat16, dev,
                              args.partition_tiles, decode_slices=slices)
    form = "slices" if plan.sliced else "ranges"
    pool = nat.PoolView.from_bshd(kpool, vpool)
    partials = torch.empty(max(plan.partials_floats, 1), dtype=torch.float32, device=dev)
    counters = torch.zeros(max(plan.n_merges, 1), dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(D)
    merges_only = dataclasses.replace(plan, n_narrow=0, n_wide=0)
    items_only = dataclasses.replace(plan, n_merges=0)

    def run(p, fused):
        nat.paged_attention(q, out, pool, bt, cu, kv_lens, positions, p, scale, HKV, partials=partials,
                            counters=counters if fused else None, fused_merge=fused)

    def layer(events=None):
        if events is None:
            run(plan, args.fused)
            return
        e0, e1, e2 = events
        e0.record()
        if not args.fused:
            run(items_only, False)
            e1.record()
            run(merges_only, False)
        else:
            run(plan, True)
            e1.record()
        e2.record()

    for _ in range(args.warmup):
        for _ in range(args.layers):
            layer()
    torch.cuda.synchronize()

    # Timed region: wall clock over K steps, plus per-launch HIP events on the
    # stream the kernels run on.
    stream = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.layers * args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    i = 0
    for _ in range(args.steps):
        for _ in range(args.layers):
            layer(ev[i])
            i += 1
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    attn_ms = [a.elapsed_time(b) for a, b, _ in ev]
    merge_ms = [b.elapsed_time(c) for _, b, c in ev]

    per_layer = attn_bytes(ctx)
    total = per_layer * args.layers * args.steps
    traffic = None
    pmc = PMC_DEFAULT[form]
    if args.sigma == 1.0 and args.partition_tiles == 0 and not args.fused and pmc is not None:
        traffic = int(pmc["fetch_kib"] * 1024 * pmc["fetch_scale"] + pmc["write_kib"] * 1024 * pmc["write_scale"])
    value = total / wall / 1e9
    attn_avg_s = float(np.mean(attn_ms)) / 1e3
    achieved = per_layer / attn_avg_s / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/Q, seeded lognormal contexts, random block placement)",
        "config": {
            "workload": "C5: 14B-class paged decode attention, 40q/8kv heads, head_dim 128, bf16 KV, "
                        f"batch {B}, ctx lognormal(median 2048, sigma {args.sigma}) clip [64,32768], "
                        f"block 16, {args.layers} layers per step",
            "batch": B,
            "layers": args.layers,
            "context_tokens": int(ctx.sum()),
            "max_context": int(ctx.max()),
            "pool_blocks": int(kpool.shape[0]),
            "plan": form,
            "partition_tiles": args.partition_tiles,
            "plan_items": plan.n_narrow + plan.n_wide,
            "plan_merges": plan.n_merges,
        },
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBPS, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": ("PMC FETCH_SIZE x2.0 + WRITE_SIZE x1.0 of this plan form's launch, from "
                               + ("profiles/attn_slice_kernel_c5_decode_14b.md" if plan.sliced else
                                  "profiles/attn_kernel_c5_decode_14b.md")
                               + " (rocprofv3 --pmc; bench.py cannot read counters itself)") if traffic else None,
            "kernel": ("attn_slice_kernel<bf16,128>" if plan.sliced else
                       "attn_kernel<bf16,128,1,fast>" + (" (split-K merge fused)" if args.fused else "")),
            "kernel_avg_us": round(attn_avg_s * 1e6, 2),
            "merge_avg_us": round(float(np.mean(merge_ms)) * 1e3, 2),
            "bytes_per_launch": per_layer,
        },
    }
    if not args.no_check:
        # after the timed region: the output of the last timed launch
        result["check"] = check_output(ctx, tables, kpool, vpool, q, out)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(ctx, tables, kpool, vpool, q, args.cpu_seconds)
    if not args.no_mixed:
        del kpool, vpool, partials
        torch.cuda.empty_cache()
        result["c1"] = run_c1(dev)
        result["c2"] = run_c2(dev)
        result["c2"]["kv_write_c4_prefill"] = run_kv_write_large(dev)
        result["c3"] = run_c3(dev)
        torch.cuda.empty_cache()
        result["c3"]["draft"] = run_draft(dev)
        torch.cuda.empty_cache()
        result["c3"]["engine_round"] = run_c3_engine(dev)
        torch.cuda.empty_cache()
    if not args.no_e2e:
        kpool = vpool = partials = None
        torch.cuda.empty_cache()
        result["e2e"] = run_e2e(args, dev)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
