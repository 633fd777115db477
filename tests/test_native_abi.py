"""CPU tests of the C ABI library: it loads, exports every entry point the
header declares, and its host-only routines (status strings, the attention
work planner, workspace sizing) behave as documented. Nothing here launches a
kernel."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from memforge_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "memforge_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mf_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(nat.LIB_PATH))
    names = declared_functions()
    assert len(names) >= 9, names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # every declared function also has a ctypes signature in the binding
    assert set(names) <= set(nat._SIGNATURES), set(names) - set(nat._SIGNATURES)


def test_version_and_status_strings():
    L = nat.lib()
    assert L.mf_version().decode().startswith("memforge_hip")
    for code in (0, -1, -2, -3, -4):
        s = L.mf_status_string(code).decode()
        assert s and s != L.mf_status_string(12345).decode()


def _plan(cu, kv, hq=8, hkv=2, d=128, dtype=torch.bfloat16, pt=0):
    return nat.plan_attention(cu, kv, hq, hkv, d, dtype, "cpu", partition_tiles=pt)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 64), (torch.float16, 256),
                                     (torch.float32, 128)])
@pytest.mark.parametrize("pt", [0, 1, 3, 64])
def test_plan_covers_every_tile_exactly_once_and_merges_line_up(dtype, d, pt):
    rng = np.random.default_rng(pt + d)
    q_lens = [1, 1, 7, 40, 0, 3, 130, 1]
    kv = [int(x) for x in rng.integers(1, 3000, len(q_lens))]
    kv[4] = 0
    kv[2] = 7
    _check_plan_cover(q_lens, kv, 8, 2, d, dtype, pt)


def _check_plan_cover(q_lens, kv, hq, hkv, d, dtype, pt):
    cu = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    G = hq // hkv
    p = _plan(cu, kv, hq, hkv, d, dtype, pt)
    items = p.items_host
    merges = p.merges_host
    assert items.shape[0] == p.n_narrow + p.n_wide
    cover = {}
    slots = {}
    # wide items come in workgroups of four: either one (sequence, head, key
    # range) with distinct column groups (shared K/V tiles), or four
    # independent items; padding items carry no columns and no partial slot
    assert p.n_wide % 4 == 0
    for u in range(p.n_narrow, p.n_narrow + p.n_wide, 4):
        unit = [tuple(int(x) for x in it[:11]) for it in items[u:u + 4]]
        if len({(it[0], it[1], it[4], it[5]) for it in unit}) == 1:
            real = [it[2] for it in unit if it[3] > 0]
            assert len(real) == len(set(real)), "shared workgroup repeats a column group"
    # narrow items come in workgroups of four too: four single items, or one
    # cooperative unit (flag in the last int) whose waves take consecutive
    # key ranges of one (sequence, head, column tile) and share its slot
    assert p.n_narrow % 4 == 0
    for u in range(0, p.n_narrow, 4):
        unit = items[u:u + 4]
        flags = {int(it[11]) for it in unit}
        assert len(flags) == 1, "a workgroup mixes cooperative and single items"
        if flags == {1}:
            assert len({(int(it[0]), int(it[1]), int(it[2]), int(it[6]), int(it[7])) for it in unit}) == 1
            assert all(int(unit[w][5]) == int(unit[w + 1][4]) for w in range(3)), "quarters not consecutive"
            assert int(unit[0][3]) == 1
    for i in range(p.n_narrow, p.n_narrow + p.n_wide):
        assert int(items[i][11]) == 0
    for i, it in enumerate(items):
        s, h, c0, nct, kt0, kt1, slot, merge, row0, nrows, kvl = (int(x) for x in it[:11])
        coop = int(it[11]) == 1
        if nct == 0:
            assert slot == -1 and merge == -1, "padding item owns a partial slot"
            continue
        assert (row0, nrows, kvl) == (cu[s], q_lens[s], kv[s]), "item carries its sequence's bounds"
        assert kt1 >= kt0 and kt1 - kt0 <= 128
        assert kt1 > kt0 or coop, "an empty key range outside a cooperative unit"
        for c in range(c0, c0 + nct):
            for kt in range(kt0, kt1):
                key = (s, h, c, kt)
                assert key not in cover, f"tile {key} planned twice"
                cover[key] = True
            if slot >= 0:
                sl = slot + (c - c0)
                if coop and i % 4:
                    assert slots[sl] == (s, h, c)  # the unit's first wave claimed it
                    continue
                assert sl not in slots
                slots[sl] = (s, h, c)
    # every key tile a column tile's last column can see is planned (once,
    # above); a plan may also cover tiles past that, which the kernel masks
    for s, (q, n) in enumerate(zip(q_lens, kv)):
        if q == 0 or n == 0:
            continue
        nct = (q * G + 15) // 16
        for h in range(hkv):
            for c in range(nct):
                last_row = (min((c + 1) * 16, q * G) - 1) // G
                for kt in range(min((n + 15) // 16, (n - q + last_row) // 16 + 1)):
                    assert (s, h, c, kt) in cover, f"visible tile {(s, h, c, kt)} not planned"
    for s, h, c, kt in cover:
        assert kt < (kv[s] + 15) // 16, "a tile past the sequence's keys"
    # each merge record reads exactly the partial slots of its (s, h, column)
    seen = set()
    for m in merges:
        s, h, c, nparts, slot0, stride, row0, nrows = (int(x) for x in m[:8])
        assert (row0, nrows) == (cu[s], q_lens[s])
        want = sorted(sl for sl, owner in slots.items() if owner == (s, h, c))
        got = sorted(slot0 + j * stride for j in range(nparts))
        assert got == want and nparts > 1
        seen.add((s, h, c))
    assert len(seen) == merges.shape[0]
    assert p.partials_floats >= len(slots) * 16 * (max(d, 32) + 2)
    return p


def _wide_work(it, G):
    """Key tiles a wide item runs: up to the last one its last column sees."""
    s, h, c0, nct, kt0, kt1 = (int(x) for x in it[:6])
    nrows, kvl = int(it[9]), int(it[10])
    last_col = min((c0 + nct) * 16, nrows * G) - 1
    if nct <= 0 or last_col < 0:
        return 0
    last_pos = kvl - nrows + last_col // G
    return max(0, min(kt1, last_pos // 16 + 1) - kt0)


@pytest.mark.parametrize("seed", range(6))
def test_mixed_plans_of_random_shapes_cover_every_visible_tile_once(seed):
    """Decode rows beside prefill chunks (one mixed launch, quad partitions
    for the chunks): every key tile a column can see planned exactly once,
    partial slots owned once and every merge record reading exactly its
    column's slots, across GQA ratios, head sizes, dtypes, chunk lengths
    (one column group up to many quads) and contexts up to 40,000 keys."""
    rng = np.random.default_rng(100 + seed)
    for hq, hkv, d, dtype in ((15, 5, 64, torch.bfloat16), (8, 2, 128, torch.bfloat16), (16, 4, 32, torch.float16),
                              (8, 8, 64, torch.bfloat16), (32, 2, 64, torch.float16)):
        chunks = [int(x) for x in rng.integers(2, 900, int(rng.integers(1, 6)))]
        decodes = int(rng.integers(1, 40))
        q_lens = chunks + [1] * decodes
        kv = [q + int(x) for q, x in zip(chunks, rng.integers(0, 4000, len(chunks)))]
        kv += [int(x) for x in rng.integers(1, 40000 if seed % 2 else 3000, decodes)]
        order = rng.permutation(len(q_lens))
        p = _check_plan_cover([q_lens[i] for i in order], [kv[i] for i in order], hq, hkv, d, dtype, 0)
        assert p.n_narrow > 0


@pytest.mark.parametrize("q_lens,kv", [
    ([40], [40]),                      # one short run: fewer workgroups than XCDs
    ([20, 33, 70], [20, 900, 3000]),   # pooled (loose) wide items beside shared runs
    ([512, 7, 300], [700, 2000, 300]),
    ([2048], [4096]),                  # one long sequence, many partitions
])
def test_prefill_only_plans_of_any_shape_cover_every_tile_once(q_lens, kv):
    """The XCD order of plans without single-tile items only permutes
    workgroups: every tile is still planned once and every partial slot and
    merge record lines up, down to plans smaller than one round of XCDs."""
    for hq, hkv, d in ((8, 2, 128), (15, 5, 64)):
        p = _check_plan_cover(q_lens, kv, hq, hkv, d, torch.bfloat16, 0)
        assert p.n_narrow == 0


@pytest.mark.parametrize("decodes", [0, 12])
@pytest.mark.parametrize("hq,hkv,d", [(15, 5, 64), (8, 2, 128), (16, 4, 32)])
def test_plan_keeps_each_key_range_on_one_xcd(hq, hkv, d, decodes):
    """The wide workgroups of one key range (in a mixed plan, of one
    sequence and kv head) sit at wide positions of one residue mod 8 (the
    XCD the dispatcher sends them to; in a mixed launch the single-tile
    workgroups before them only rotate the residues), the
    eight residue classes carry near-equal causal work, and each class runs
    its workgroups most work first. With and without decode rows."""
    rng = np.random.default_rng(d)
    q_lens = [512, 512, 384, 512, 200] + [1] * decodes
    kv = [q + int(x) for q, x in zip(q_lens, rng.integers(0, 2049, len(q_lens)))]
    p = _check_plan_cover(q_lens, kv, hq, hkv, d, torch.bfloat16, 0)
    assert (p.n_narrow > 0) == (decodes > 0) and p.n_wide >= 64
    G = hq // hkv
    wide = p.items_host[p.n_narrow:p.n_narrow + p.n_wide]
    units = [wide[u:u + 4] for u in range(0, p.n_wide, 4)]
    work = [max(_wide_work(it, G) for it in u) for u in units]
    ranges, run_work = {}, {}
    for w, u in enumerate(units):
        keys = {(int(it[0]), int(it[1]), int(it[4]), int(it[5])) for it in u}
        if len(keys) == 1:
            key = keys.pop()
            if decodes:  # a mixed plan's quads of one (sequence, kv head) read overlapping ranges
                key = key[:2]
            ranges.setdefault(key, set()).add(w % 8)
            run_work[key] = run_work.get(key, 0) + work[w]
    # a run split between two queues (at most one per queue but the last)
    spilled = sum(len(r) > 1 for r in ranges.values())
    assert spilled <= 7, f"{spilled} of {len(ranges)} key ranges span XCDs"
    load = [sum(work[w] for w in range(c, len(units), 8)) for c in range(8)]
    # runs dealt most work first to the least-loaded queue: the queues differ
    # by at most one run (the mixed plans' longer partitions make fewer, larger runs)
    assert max(load) - min(load) <= max(run_work.values()), (load, max(run_work.values()))
    if not decodes:
        assert max(load) <= 1.1 * min(load), load
    full = (len(units) // 8) * 8  # whole rounds of the interleave
    for c in range(8):
        seq = [work[w] for w in range(c, full, 8)]
        assert seq == sorted(seq, reverse=True)


def test_plan_capacity_and_argument_errors():
    L = nat.lib()
    cu = np.array([0, 1, 2], dtype=np.int32)
    kv = np.array([100, 5000], dtype=np.int32)
    counts = np.zeros(4, dtype=np.int64)
    st = L.mf_attention_plan(2, cu.ctypes.data, kv.ctypes.data, 8, 2, 128, 2, 4, None, 0, None, 0,
                             counts.ctypes.data)
    assert st == -3 and counts[0] > 0  # sizes reported even when the buffers are too small
    assert L.mf_attention_plan(2, cu.ctypes.data, kv.ctypes.data, 8, 3, 128, 2, 4, None, 0, None, 0,
                               counts.ctypes.data) == -1  # heads not a multiple
    assert L.mf_attention_plan(2, cu.ctypes.data, kv.ctypes.data, 8, 2, 512, 2, 4, None, 0, None, 0,
                               counts.ctypes.data) == -2  # head_dim beyond the kernels
    with pytest.raises(ValueError):
        nat.plan_attention([0, 1], [5, 6], 8, 2, 128, torch.bfloat16, "cpu")


def test_plan_orders_longest_items_first():
    p = _plan([0, 1, 2, 3], [40, 4000, 900], pt=64)
    narrow = p.items_host[: p.n_narrow]
    # workgroups ordered by their longest wave
    lengths = [int((narrow[u:u + 4, 5] - narrow[u:u + 4, 4]).max()) for u in range(0, p.n_narrow, 4)]
    assert lengths == sorted(lengths, reverse=True)


def test_plan_cooperative_units_replace_split_k_up_to_four_partitions():
    """A narrow range of more than P tiles runs as one cooperative workgroup
    (four waves on consecutive quarters, combined in LDS) up to 4P tiles; only
    longer ranges leave split-K partials for the merge kernel."""
    P = 8
    # one decode row each: 8 tiles (single), 9 and 32 tiles (one unit), 33 tiles (two units)
    kv = [8 * 16, 9 * 16, 32 * 16, 33 * 16]
    p = _plan([0, 1, 2, 3, 4], kv, hq=8, hkv=2, pt=P)
    items = p.items_host[: p.n_narrow]
    per_seq = {}
    for it in items:
        if int(it[3]) == 0:
            continue
        per_seq.setdefault(int(it[0]), []).append(it)
    assert all(int(it[11]) == 0 for it in per_seq[0]) and len(per_seq[0]) == 2  # one per head
    for s in (1, 2):
        assert len(per_seq[s]) == 8 and all(int(it[11]) == 1 and int(it[6]) == -1 for it in per_seq[s])
        assert max(int(it[5] - it[4]) for it in per_seq[s]) == -(-kv[s] // 16 // 4)
    assert len(per_seq[3]) == 16 and all(int(it[6]) >= 0 for it in per_seq[3])
    assert p.n_merges == 2  # sequence 3, both heads
    assert all(int(m[3]) == 2 for m in p.merges_host)


def test_verify_workspace_size_grows_with_the_batch():
    L = nat.lib()
    a = L.mf_spec_verify_workspace_size(4, 3)
    b = L.mf_spec_verify_workspace_size(64, 3)
    assert 0 <= a <= b


def test_product_path_has_no_cpu_fallback(monkeypatch):
    """The HIP entry points refuse CPU tensors instead of computing elsewhere."""
    k = torch.zeros((4, 16, 2, 64))
    with pytest.raises(Exception):
        nat.kv_write(torch.zeros((3, 2, 64)), torch.zeros((3, 2, 64)), torch.zeros(3, dtype=torch.int64),
                     nat.PoolView.from_bshd(k, k.clone()))


@pytest.mark.parametrize("scale", [float("nan"), float("inf"), float("-inf")])
def test_attention_rejects_a_non_finite_scale(scale):
    """A NaN or infinite scale is an argument error, returned before any launch
    (so this runs without a GPU). Finite scales -- negative and zero included --
    are checked against the oracle on the GPU."""
    L = nat.lib()
    # the scale is the first thing checked: no pointer is needed to see it refused
    st = L.mf_paged_attention(None, 64, 64, None, 64, 64, 2, None, None, 16 * 64, 64, 64, 16,
                              None, 4, None, None, None, None, None, None, None, 0, 0,
                              1, 1, 64, scale, None, 1, 0, None, 0, None, 0, None, None)
    assert st == -1, st


@pytest.mark.parametrize("pairs", [
    [(0, 8)],            # destination outside 8 blocks
    [(-1, 2)],           # negative source
    [(1, 2), (3, 2)],    # a block written twice
    [(1, 2), (2, 3)],    # a written block is also read: order-dependent
])
def test_block_copy_rejects_bad_pairs_before_any_launch(pairs):
    """mf_kv_copy_blocks checks every pair on the host first (the pool
    pointers are never touched, so this runs without a GPU)."""
    L = nat.lib()
    flat = np.asarray(pairs, dtype=np.int64).reshape(-1)
    dummy = 1 << 20  # never dereferenced: the call fails before any launch
    st = L.mf_kv_copy_blocks(dummy, dummy, 2, 3, 8 * 16 * 4 * 64, 16 * 4 * 64, 16 * 4 * 64, 8,
                             flat.ctypes.data, len(pairs), None)
    assert st == -1, st


def test_block_copy_pairs_on_themselves_are_a_no_op():
    L = nat.lib()
    flat = np.asarray([(3, 3), (5, 5)], dtype=np.int64).reshape(-1)
    st = L.mf_kv_copy_blocks(1 << 20, 1 << 20, 2, 3, 8 * 1024, 1024, 1024, 8, flat.ctypes.data, 2, None)
    assert st == 0, st


def test_block_copy_rejects_a_bad_geometry():
    L = nat.lib()
    flat = np.asarray([(1, 2)], dtype=np.int64)
    # the block stride is shorter than one block
    assert L.mf_kv_copy_blocks(1 << 20, 1 << 20, 2, 3, 8 * 1024, 512, 1024, 8, flat.ctypes.data, 1, None) == -1
    # layers overlap
    assert L.mf_kv_copy_blocks(1 << 20, 1 << 20, 2, 3, 1024, 1024, 1024, 8, flat.ctypes.data, 1, None) == -1
    # unknown dtype
    assert L.mf_kv_copy_blocks(1 << 20, 1 << 20, 7, 3, 8 * 1024, 1024, 1024, 8, flat.ctypes.data, 1, None) == -1


def test_upload_packs_parts_with_their_dtypes_and_shapes():
    """nat.upload's packing (shared by the pinned GPU path): int64 parts land
    on 8-byte boundaries and every part comes back intact."""
    rng = np.random.default_rng(0)
    parts = [rng.integers(-2**31, 2**31, 5, dtype=np.int64).astype(np.int32),
             rng.integers(-2**62, 2**62, (3, 2), dtype=np.int64),
             np.zeros((0, 12), np.int32),
             rng.integers(0, 100, (2, 3), dtype=np.int64).astype(np.int32),
             np.array([7], np.int64)]
    out = nat.upload(parts, "cpu")
    for p, t in zip(parts, out):
        assert t.dtype == (torch.int64 if p.dtype == np.int64 else torch.int32)
        assert tuple(t.shape) == p.shape
        assert np.array_equal(t.numpy(), p)
    _, offs, n = nat._layout(parts)
    assert all(o % 2 == 0 for o in offs) and n >= offs[-1] + 2
    with pytest.raises(TypeError):
        nat.upload([np.zeros(3, np.float32)], "cpu")


def _partition_of(items):
    """Tiles per wave the plan used: the longest single-wave item, or a
    cooperative unit's range / 4, rounded up to the planner's powers of two."""
    longest = 0
    for u in range(0, items.shape[0], 4):
        unit = items[u:u + 4]
        if int(unit[0][11]) == 1:
            longest = max(longest, -(-int(unit[3][5] - unit[0][4]) // 4))
        else:
            longest = max(longest, int((unit[:, 5] - unit[:, 4]).max()))
    return longest


def test_planner_partition_picks_on_the_config_shapes():
    """The narrow-partition estimate (bandwidth time or longest chain, plus a
    merge when a range is split) on the configs' decode shapes: merge-free
    on a 64-sequence decode step at C4's contexts, 8-tile waves on C3's verify
    rows, 128-tile waves (and only the longest sequences split) on C5."""
    import math

    g = torch.Generator().manual_seed(5)
    c4 = torch.randint(96, 1153, (64,), generator=g).tolist()
    p = _plan(list(range(65)), c4, hq=15, hkv=5, d=64)
    assert p.n_merges == 0 and 16 < _partition_of(p.items_host[: p.n_narrow]) <= 32
    g = torch.Generator().manual_seed(0)
    ctx = [c + 5 for c in torch.randint(128, 2049, (16,), generator=g).tolist()]
    p = _plan([5 * i for i in range(17)], ctx, hq=15, hkv=5, d=64)
    assert p.n_merges > 0 and _partition_of(p.items_host[: p.n_narrow]) <= 8
    gen = torch.Generator().manual_seed(0)
    z = torch.randn(256, generator=gen, dtype=torch.float64)
    c5 = torch.clamp(torch.round(torch.exp(math.log(2048.0) + z)), 64, 32768).to(torch.int64).tolist()
    p = _plan(list(range(257)), c5, hq=40, hkv=8, d=128)
    long_seqs = sum(1 for c in c5 if (c + 15) // 16 > 512)
    assert p.n_merges == 8 * long_seqs and _partition_of(p.items_host[: p.n_narrow]) == 128


def test_planner_mixed_step_partitions_on_the_c2_shape():
    """The C2 mixed step (4 chunks of 512 on priors U[0,2048] + 28 decodes of
    U[64,4096], bf16 D 64): the narrow partition is raised to the smallest
    power of two that keeps wide items within the target (32 tiles), because
    both classes share one launch. Each column quad (the four column groups
    of one wide workgroup) cuts the tiles its last column sees into
    round(visible / W) equal ranges, W = the visible work over 2 x 256 compute
    units, and partitions are merged until at most 512 wide workgroups (two
    per compute unit) remain: every wide workgroup holds about the same
    work."""
    g = torch.Generator().manual_seed(0)
    prior = torch.randint(0, 2049, (4,), generator=g).tolist()
    dctx = torch.randint(64, 4097, (28,), generator=g).tolist()
    q_lens = [512] * 4 + [1] * 28
    kv = [p + 512 for p in prior] + dctx
    cu = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    p = _check_plan_cover(q_lens, kv, 15, 5, 64, torch.bfloat16, 0)
    G, hkv = 3, 5
    wide = p.items_host[p.n_narrow:]
    units = [wide[u:u + 4] for u in range(0, p.n_wide, 4)]
    visible = {}
    for e in range(4):
        for qd in range(12):  # 96 column tiles, 8 per quad
            last_row = (min((qd + 1) * 128, 512 * G) - 1) // G
            visible[(e, qd)] = min((kv[e] + 15) // 16, (kv[e] - 512 + last_row) // 16 + 1)
    W = hkv * sum(visible.values()) / 512
    parts = {}
    for u in units:
        s, h, c0, _, k0, k1 = (int(x) for x in u[0][:6])
        assert {(int(x[0]), int(x[1]), int(x[4]), int(x[5])) for x in u} == {(s, h, k0, k1)}
        parts.setdefault((s, h, c0 // 8), []).append((k0, k1))
    counts = {}
    for (s, h, qd), ranges in parts.items():
        ranges.sort()
        v = visible[(s, qd)]
        n = len(ranges)
        # equal ranges; round(visible / W) of them, or fewer where the cap
        # below merged partitions
        assert ranges == [(i * v // n, (i + 1) * v // n) for i in range(n)], (s, h, qd, ranges)
        assert 1 <= n <= max(1, round(v / W)), (s, qd, n, v / W)
        counts[(s, qd)] = n
    # every kv head of a quad is cut alike; at most two wide workgroups per CU
    assert len(parts) == hkv * len(counts)
    assert len(units) <= 512 and len(units) == hkv * sum(counts.values())
    merged = sum(max(1, round(v / W)) for v in visible.values()) - sum(counts.values())
    assert 0 < merged <= 5 and len(units) > 512 - hkv, (merged, len(units))
    assert _partition_of(p.items_host[: p.n_narrow]) == 32
    # decode rows alone keep the estimate's own pick
    alone = _plan(list(range(29)), dctx, hq=15, hkv=5, d=64)
    assert _partition_of(alone.items_host[: alone.n_narrow]) == 16
    # the same chunks with no decodes: one class, 32-tile partitions in equal strides
    pre = _plan(cu[:5], kv[:4], hq=15, hkv=5, d=64)
    live = pre.items_host[pre.items_host[:, 3] > 0]
    assert pre.n_narrow == 0 and int((live[:, 5] - live[:, 4]).max()) <= 32
    assert len({(int(r[0]), int(r[4])) for r in live}) == sum(-(-((c + 15) // 16) // 32) for c in kv[:4])


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_graphed_split_capacity_holds_the_longest_context_plans(bs):
    """The capacity a graphed decode bucket reserves when plans may need a
    merge counts 16-key tiles, not pool blocks: every plan of a full bucket at
    the longest context fits it, at the planner's own pick and at the smallest
    partition it uses."""
    from memforge_amd.runtime.graphed_paged_decode import _MIN_PARTITION_TILES, split_plan_capacity

    max_model_len = 12000
    mb = (max_model_len + bs - 1) // bs + 1
    for b, hkv, hq, d in ((1, 5, 15, 64), (8, 8, 40, 128), (4, 2, 16, 64)):
        cap_items, _, cap_merges, floats = split_plan_capacity(b, hkv, mb, bs, d)
        kv = [mb * bs] * b
        for pt in (0, _MIN_PARTITION_TILES, 8):
            items, merges, counts = nat.plan_attention_host(list(range(b + 1)), kv, hq, hkv, d,
                                                            torch.bfloat16, pt)
            assert counts[0] <= cap_items and counts[1] == 0, (bs, b, pt, counts, cap_items)
            assert counts[2] <= cap_merges and counts[3] <= floats, (bs, b, pt, counts)


def test_pack_host_check_names_the_malformed_entry():
    ent = np.array([[2, 0, 2, 0, 1, 0], [1, 5, 6, 1, 1, 2]], dtype=np.int32)
    tables = np.array([3, 4], dtype=np.int32)
    nat.check_pack_entries(ent, tables, 3, 3, num_blocks=8)
    for bad, what in (((1, 3), -1), ((1, 4), 2), ((1, 5), 3), ((0, 0), 4)):
        e = ent.copy()
        e[bad] = what
        with pytest.raises(ValueError, match="entry"):
            nat.check_pack_entries(e, tables, 3, int(max(e[:, 0].sum(), 0)), num_blocks=8)
    with pytest.raises(ValueError, match="rows"):
        nat.check_pack_entries(ent, tables, 3, 4)
    with pytest.raises(IndexError, match="outside a pool"):
        nat.check_pack_entries(ent, tables, 3, 3, num_blocks=4)
    with pytest.raises(ValueError, match="no entries"):
        nat.check_pack_entries(np.zeros((0, 6), np.int32), tables, 3, 2)


def test_pack_rejects_rows_without_entries_and_bad_lengths_before_any_launch():
    """mf_ragged_pack's argument checks run before any launch (no GPU needed):
    packed rows with no entry to take them from, negative array lengths and
    missing arrays are MF_ERR_ARG."""
    L = nat.lib()
    dummy = 1 << 20  # never dereferenced
    base = dict(entries=dummy, n=1, tables=dummy, tl=4, tokens=dummy, kl=4, bs=16, mb=1, T=2)

    def call(**kw):
        a = {**base, **kw}
        return L.mf_ragged_pack(a["entries"], a["n"], a["tables"], a["tl"], a["tokens"], a["kl"], a["bs"],
                                a["mb"], a["T"], dummy, dummy, dummy, dummy, dummy, dummy, dummy, None, 0,
                                dummy, None)

    assert call(n=0) == -1            # two rows, no entry
    assert call(tl=-1) == -1
    assert call(kl=-1) == -1
    assert call(tables=None) == -1    # a table length without a table
    assert call(tokens=None) == -1
    assert call(bs=0) == -1


def test_noalloc_attention_refuses_oversized_plans_before_touching_the_device():
    """mf_paged_attention_noalloc checks the plan's partials against its fixed
    array (MF_NOALLOC_PARTIALS_FLOATS) first: too large is MF_ERR_WORKSPACE,
    negative MF_ERR_ARG, with no device call (so this runs without a GPU)."""
    L = nat.lib()

    def call(floats):
        return L.mf_paged_attention_noalloc(None, 64, 64, None, 64, 64, 2, None, None, 16 * 64, 64, 64, 16,
                                            None, 4, None, None, None, None, None, None, None, 0, 0,
                                            1, 1, 64, 0.125, None, 1, 0, None, 1, floats, None)

    assert call(nat.NOALLOC_PARTIALS_FLOATS + 1) == -3
    assert call(-1) == -1
    m = re.search(r"#define MF_NOALLOC_PARTIALS_FLOATS \((\d+) \* 1024 \* 1024\)", HEADER.read_text())
    assert m and nat.NOALLOC_PARTIALS_FLOATS == int(m.group(1)) << 20


@pytest.mark.parametrize("dtype,hq,hkv,d", [(torch.bfloat16, 40, 8, 128), (torch.float32, 15, 5, 64),
                                            (torch.bfloat16, 15, 5, 64), (torch.float16, 8, 8, 16)])
def test_plan_partials_reach_is_what_the_planner_counts(dtype, hq, hkv, d):
    """The highest partial slot a planner-made plan names ends exactly at the
    partials the planner reports: every slot it counts is used, no more."""
    rng = np.random.default_rng(d + hq)
    q_lens = [1, 512, 1, 5, 1, 300, 1]
    kv = [int(x) for x in rng.integers(600, 9000, len(q_lens))]
    cu = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    for pt in (0, 4, 16):
        plan = nat.plan_attention(cu, kv, hq, hkv, d, dtype, "cpu", partition_tiles=pt)
        assert plan.n_merges > 0
        assert nat.plan_partials_reach(plan, d) == plan.partials_floats


def test_noalloc_refuses_a_plan_whose_slots_reach_past_its_array():
    """A plan whose items or merge records name partial slots past the
    library's array is refused before any device call, even when its declared
    partials_floats is small (the slots, not the declaration, are what the
    kernels write)."""
    cu, kv = [0, 1, 2], [30000, 20000]
    plan = nat.plan_attention(cu, kv, 40, 8, 128, torch.bfloat16, "cpu", partition_tiles=4)
    assert plan.n_merges > 0 and 0 < plan.partials_floats <= nat.NOALLOC_PARTIALS_FLOATS
    stride = 16 * (128 + 2)
    far = nat.NOALLOC_PARTIALS_FLOATS // stride + 1
    for field in ("item", "merge"):
        items, merges = plan.items_host.copy(), plan.merges_host.copy()
        if field == "item":
            k = int(np.nonzero(items[:plan.n_narrow + plan.n_wide, 6] >= 0)[0][0])
            items[k, 6] = far
        else:
            merges[0, 4] = far
        bad = nat.AttentionPlan(plan.items, plan.merges, plan.n_narrow, plan.n_wide, plan.n_merges,
                                plan.partials_floats, items, merges)
        assert nat.plan_partials_reach(bad, 128) > nat.NOALLOC_PARTIALS_FLOATS
        q = torch.zeros((2, 40, 128), dtype=torch.bfloat16)
        with pytest.raises(nat.MemforgeHipError, match="workspace"):
            nat.paged_attention_noalloc(q, q.clone(), None, None, None, None, None, bad, 0.1, 8)


def test_plan_host_cache_returns_read_only_plans_and_stays_bounded():
    """plan_host hands back the same read-only arrays for the same inputs
    (the planners are pure functions of them), a different plan for any
    changed input, and keeps at most PLAN_CACHE_SIZE plans."""
    a = nat.plan_host([0, 1, 2], [300, 40], 15, 5, 64, torch.float32, "cpu")
    b = nat.plan_host([0, 1, 2], [300, 40], 15, 5, 64, torch.float32, "cpu")
    assert a[0] is b[0] and a[1] is b[1] and a[2] is b[2] and a[3] is False and b[3] is False
    for arr in a[:3]:
        assert not arr.flags.writeable
        with pytest.raises(ValueError):
            arr[...] = 0
    fresh = nat.plan_attention_host([0, 1, 2], [300, 40], 15, 5, 64, torch.float32)
    assert all(np.array_equal(x, y) for x, y in zip(a[:3], fresh))
    for other in (([0, 1, 2], [300, 41], 15, 5, 64, torch.float32), ([0, 1, 2], [300, 40], 15, 5, 64, torch.bfloat16),
                  ([0, 2, 3], [300, 40], 15, 5, 64, torch.float32), ([0, 1, 2], [300, 40], 16, 4, 64, torch.float32)):
        c = nat.plan_host(*other, "cpu")
        want = nat.plan_attention_host(*other)
        assert c[0] is not a[0] and all(np.array_equal(x, y) for x, y in zip(c[:3], want))
    for n in range(nat.PLAN_CACHE_SIZE + 10):
        nat.plan_host([0, 1], [17 + n], 8, 2, 64, torch.float32, "cpu")
    assert len(nat._PLAN_CACHE) == nat.PLAN_CACHE_SIZE


def test_uploads_refuse_graph_capture(monkeypatch):
    """Host-array uploads stage through a temporary pinned buffer, which a
    captured copy would read again on every replay: under capture they raise
    before any allocation (captured steps stage through buffers of their own)."""
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    parts = [np.arange(4, dtype=np.int32)]
    for call in (lambda: nat.upload(parts, "cuda"), lambda: nat.upload_packed(parts, "cuda"),
                 lambda: nat.upload_packed_cached(parts, "cuda")):
        with pytest.raises(nat.MemforgeHipError, match="graph capture"):
            call()
    # a CPU destination is never captured
    assert nat.upload(parts, "cpu")[0].tolist() == [0, 1, 2, 3]


def test_plan_verify_units_give_the_last_wave_fewer_tiles():
    """In the cooperative unit that holds a multi-row sequence's last tile (a
    verify pass: boundary and in-flight tiles), the last wave's quarter is
    shorter than the others'; the quarters still tile the unit's range. Single
    rows (decodes) keep even quarters."""
    P = 8
    kv = [32 * 16, 32 * 16]
    verify = _plan([0, 5, 6], kv, hq=8, hkv=2, pt=P)     # 5 rows, then 1 row
    items = verify.items_host[: verify.n_narrow]
    units = {}
    for u in range(0, items.shape[0], 4):
        unit = items[u:u + 4]
        if int(unit[0][11]) == 1:
            units.setdefault(int(unit[0][0]), []).append(unit)
    for s, us in units.items():
        for unit in us:
            assert all(int(unit[w][5]) == int(unit[w + 1][4]) for w in range(3))
            lens = [int(unit[w][5] - unit[w][4]) for w in range(4)]
            assert int(unit[0][4]) == 0 and int(unit[3][5]) == 32 and sum(lens) == 32
            if s == 0:
                assert lens[3] < min(lens[:3]), lens
            else:
                assert max(lens) - min(lens) <= 1, lens
