"""Scripted engine workloads shared by the host-engine tests and the fixture
generator (test infrastructure only).

``drive`` runs one seeded engine loop -- arrivals, oversized requests that
must be aborted, explicit aborts, chunked prefill, prefix registration,
copy-on-write probes, lookahead token bursts, memory pressure -- against a
``memforge_c``-compatible module and returns every step result. Every choice
comes from the seed and from the engine's own answers, so two engines that
agree take identical paths and produce identical traces.
"""

import json
import random
from pathlib import Path

TRACES = Path(__file__).resolve().with_name("engine_traces.json")

CONFIGS = {
    "plain": dict(num_blocks=40, bs=4, max_seqs=6, sharing=False, chunk=0, lookahead=0),
    "sharing": dict(num_blocks=64, bs=16, max_seqs=8, sharing=True, chunk=0, lookahead=0),
    "chunked+sharing": dict(num_blocks=48, bs=8, max_seqs=8, sharing=True, chunk=24, lookahead=0),
    "chunked+lookahead": dict(num_blocks=30, bs=4, max_seqs=5, sharing=False, chunk=10, lookahead=3),
    "pressure+all": dict(num_blocks=24, bs=16, max_seqs=16, sharing=True, chunk=32, lookahead=4),
}


def load_traces():
    return json.loads(TRACES.read_text())


def snapshot(r):
    return (
        [(i.seq_id, list(i.block_table), i.prompt_length, i.output_length, i.total_length, int(i.status),
          bool(i.is_prefill), i.num_cached_tokens, i.prefill_chunk_end) for i in r.running_sequences],
        list(r.finished_sequence_ids), list(r.preempted_sequence_ids), list(r.aborted_sequence_ids),
        r.num_waiting, r.num_free_blocks, r.total_blocks, round(r.memory_utilization_ratio, 9),
    )


def drive(mod, seed, num_blocks, bs, max_seqs, sharing, chunk, lookahead, steps=160):
    """A scripted engine loop; every choice comes from ``seed`` and the
    engine's own answers, so two engines that agree take identical paths."""
    rng = random.Random(seed)
    a = mod.BlockAllocator(num_blocks, bs)
    pc = mod.PrefixCache(a, bs) if sharing else None
    s = mod.Scheduler(a, max_seqs, pc, chunk, lookahead)
    prefixes = [[rng.randrange(2, 500) for _ in range(rng.randrange(1, 3 * bs))] for _ in range(3)]
    trace, next_id, live = [], 1, set()
    for _ in range(steps):
        if rng.random() < 0.5:
            prompt = list(rng.choice(prefixes)) + [rng.randrange(2, 500) for _ in range(rng.randrange(1, 2 * bs))]
            if rng.random() < 0.03:  # larger than the whole pool: aborted as unschedulable
                prompt = prompt * (num_blocks * bs // len(prompt) + 2)
            s.add_sequence(next_id, prompt, rng.randrange(1, 64))
            live.add(next_id)
            next_id += 1
        if live and rng.random() < 0.05:
            victim = rng.choice(sorted(live))
            trace.append(("abort", victim, s.abort_sequence(victim)))
        r = s.step()
        trace.append(snapshot(r))
        for sid in list(r.finished_sequence_ids) + list(r.aborted_sequence_ids):
            live.discard(sid)
        for info in r.running_sequences:
            if info.is_prefill:
                end = info.prefill_chunk_end or info.total_length
                if end < info.total_length:
                    continue
                if pc is not None:
                    seq = s.get_sequence(info.seq_id)
                    pc.register_full_blocks(list(seq.get_all_tokens()), list(info.block_table))
            else:
                seq = s.get_sequence(info.seq_id)
                if pc is not None and seq is not None:
                    cow = a.prepare_write(seq, (info.total_length - 1) // bs)
                    trace.append(("cow", info.seq_id, None if cow is None else tuple(cow)))
            n = rng.randrange(1, lookahead + 1) if lookahead and not info.is_prefill else 1
            for _ in range(n):
                s.update_sequence(info.seq_id, rng.randrange(2, 500), rng.random() < 0.02)
        trace.append((a.get_num_free_blocks(), a.get_num_shared_blocks(), a.get_num_blocks_saved(),
                      pc.num_cached_blocks() if pc else -1, pc.num_hits() if pc else -1))
    return trace
