"""CPU tests of the decode slice planner (mf_attention_plan_slices): the plan
covers every tile of every sequence exactly once, in order, slices stay within
the kernel's limits and carry equal shares, split sequences line up with their
merge records and partial slots, and the planner declines what the slice
kernel does not serve. Nothing here launches a kernel."""

import math
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from memforge_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "memforge_hip.h"
RING = 3  # MF_NARROW_DEPTH: segments are padded to whole rounds of the register ring


def _define(name):
    m = re.search(rf"#define {name} (\d+)", HEADER.read_text())
    return int(m.group(1))


def test_python_constants_match_the_header():
    assert nat.SLICE_INTS == _define("MF_SLICE_INTS")
    assert nat.SLICE_MAX_TILES == _define("MF_SLICE_MAX_TILES")
    assert nat.SLICE_MAX_SEGMENTS == _define("MF_SLICE_MAX_SEGMENTS")
    assert nat.SLICE_MIN_TILES == _define("MF_SLICE_MIN_TILES")
    assert nat.SLICE_WAVES_PER_CU == _define("MF_SLICE_WAVES_PER_CU")


def _lognormal(n=256, seed=0):
    gen = torch.Generator().manual_seed(seed)
    z = torch.randn(n, generator=gen, dtype=torch.float64)
    return torch.clamp(torch.round(torch.exp(math.log(2048.0) + z)), 64, 32768).to(torch.int64).tolist()


def _check_plan(kv, hkv, d, cus, made):
    slices, merges, counts = made
    ns, nseg, nm, floats = (int(x) for x in counts)
    assert slices.shape == (ns + nseg, nat.SLICE_INTS)
    hdr, segs = slices[:ns], slices[ns:]
    # slices partition the segment list, within the kernel's limits
    assert hdr[0, 0] == 0 and (hdr[1:, 0] == hdr[:-1, 0] + hdr[:-1, 1]).all()
    assert int(hdr[-1, 0] + hdr[-1, 1]) == nseg
    assert (hdr[:, 1] >= 1).all() and (hdr[:, 1] <= nat.SLICE_MAX_SEGMENTS).all()
    lens = segs[:, 2] - segs[:, 1]
    assert (lens >= 1).all()
    padded = -(-lens // RING) * RING
    for b, n, tiles in hdr[:, :3]:
        assert tiles == padded[b:b + n].sum() <= nat.SLICE_MAX_TILES
    # every sequence's tiles, once each, in order, with consistent pieces
    T = [(k + 15) // 16 for k in kv]
    seen = {}
    for s, k0, k1, row, kvl, slot0, parts, part in segs:
        assert row == s and kvl == kv[s]  # one decode row per sequence: row s
        got = seen.setdefault(int(s), [])
        assert k0 == (got[-1][1] if got else 0) and part == len(got)
        got.append((int(k0), int(k1), int(slot0), int(parts)))
    for s, t in enumerate(T):
        pieces = seen[s]
        assert pieces[-1][1] == t
        assert all(p[3] == len(pieces) for p in pieces)
        assert len({p[2] for p in pieces}) == 1
        assert (pieces[0][2] < 0) == (len(pieces) == 1)
    # split sequences: one merge record per kv head over disjoint slot runs
    split = [s for s in range(len(kv)) if len(seen[s]) > 1]
    assert nm == len(split) * hkv and merges.shape == (nm, nat.PLAN_MERGE_INTS)
    slots = []
    for s, h, ct, parts, slot0, stride, row0, rows in merges:
        assert parts == len(seen[s]) and stride == 1 and ct == 0 and rows == 1 and row0 == s
        assert slot0 == seen[s][0][2] + h * parts
        slots += range(slot0, slot0 + parts)
    assert sorted(slots) == list(range(len(slots)))
    assert floats == len(slots) * 16 * (max(d, 32) + 2)
    # equal shares: slice i carries total // n or one tile more (the first
    # total % n of them), unless the segment cap closed it earlier
    real = np.add.reduceat(lens, hdr[:, 0]) if ns else np.zeros(0)
    base = max(1, cus * nat.SLICE_WAVES_PER_CU // hkv)
    cap = nat.SLICE_MAX_TILES - 16 * (RING - 1)
    total = sum(T)
    n = base * -(-total // (base * cap))
    share = total // n
    assert (real <= share + 1).all()
    capped = hdr[:, 1] == nat.SLICE_MAX_SEGMENTS
    if not capped.any():
        assert len(hdr) == min(n, len(hdr)) and (real >= share).all()
    return hdr, segs


@pytest.mark.parametrize("hkv,d,cus", [(8, 128, 256), (5, 64, 256), (8, 128, 32), (2, 256, 10)])
def test_lognormal_batches(hkv, d, cus):
    kv = _lognormal()
    made = nat.plan_slices_host(list(range(len(kv) + 1)), kv, 5 * hkv, hkv, d, torch.bfloat16, cus,
                                min_tiles=0)
    hdr, _ = _check_plan(kv, hkv, d, cus, made)
    base = max(1, cus * nat.SLICE_WAVES_PER_CU // hkv)
    assert len(hdr) <= base * -(-sum((k + 15) // 16 for k in kv) // (base * (nat.SLICE_MAX_TILES - 32)))


def test_the_c5_workload_runs_in_one_round():
    """The bench's C5 batch on MI355X (256 CUs, one workgroup of four waves
    each): 128 slices of 8 kv heads, all in a single round."""
    kv = _lognormal()
    made = nat.plan_slices_host(list(range(257)), kv, 40, 8, 128, torch.bfloat16, 256)
    assert made is not None
    hdr, segs = _check_plan(kv, 8, 128, 256, made)
    assert len(hdr) == 128 and int(hdr[:, 1].max()) <= 10


def test_many_short_sequences_hit_the_segment_cap():
    kv = [1 + (i * 7) % 30 for i in range(500)]
    made = nat.plan_slices_host(list(range(501)), kv, 40, 8, 128, torch.bfloat16, 4, min_tiles=0)
    hdr, _ = _check_plan(kv, 8, 128, 4, made)
    assert int(hdr[:, 1].max()) == nat.SLICE_MAX_SEGMENTS


def test_whole_rounds_when_a_share_exceeds_one_slice():
    """1,024 sequences of 2,048 keys on 128 slices per round: three rounds of
    equal slices, never a short extra round."""
    kv = [2048] * 1024
    made = nat.plan_slices_host(list(range(1025)), kv, 40, 8, 128, torch.bfloat16, 256)
    hdr, segs = _check_plan(kv, 8, 128, 256, made)
    real = np.add.reduceat(segs[:, 2] - segs[:, 1], hdr[:, 0])
    assert len(hdr) == 3 * 128 and real.max() - real.min() == 1 and real.sum() == 1024 * 128


def test_small_launches_and_non_decode_steps_get_no_slice_plan():
    cu = list(range(65))
    assert nat.plan_slices_host(cu, [300] * 64, 40, 8, 128, torch.bfloat16, 256) is None  # fits one round
    assert nat.plan_slices_host([0, 1, 5], [900, 900], 40, 8, 128, torch.bfloat16, 16, 0) is None  # prefill rows
    assert nat.plan_slices_host([0, 1], [900], 40, 8, 80, torch.bfloat16, 16, 0) is None  # head_dim 80
    assert nat.plan_slices_host([0, 1], [900], 68, 4, 128, torch.bfloat16, 16, 0) is None  # 17 heads per group
    assert nat.plan_slices_host([0, 1], [900], 8, 8, 16, torch.bfloat16, 16, 0) is None  # bf16 pads D 16
    # sequences without rows or keys take no tiles and no segment
    made = nat.plan_slices_host([0, 1, 1, 2], [700, 500, 0], 8, 8, 64, torch.float32, 16, 0)
    segs = made[0][int(made[2][0]):]
    assert set(segs[:, 0].tolist()) == {0}


def test_capacity_and_argument_errors():
    L = nat.lib()
    cu = np.arange(5, dtype=np.int32)
    kv = np.array([900, 40, 3, 5000], dtype=np.int32)
    counts = np.zeros(4, dtype=np.int64)

    def call(cus=16, min_tiles=0, cap=0, mcap=0, buf=None, mbuf=None, hq=40, hkv=8):
        return L.mf_attention_plan_slices(4, cu.ctypes.data, kv.ctypes.data, hq, hkv, 128, nat.MF_BF16,
                                          cus, min_tiles, buf, cap, mbuf, mcap, counts.ctypes.data)

    assert call() == -3  # sizes only: counts filled, capacities too small
    need, nm = int(counts[0] + counts[1]), int(counts[2])
    assert need > 0 and nm > 0
    sl = np.zeros((need, nat.SLICE_INTS), np.int32)
    mg = np.zeros((nm, nat.PLAN_MERGE_INTS), np.int32)
    assert call(cap=need - 1, mcap=nm, buf=sl.ctypes.data, mbuf=mg.ctypes.data) == -3
    assert call(cap=need, mcap=nm, buf=sl.ctypes.data, mbuf=mg.ctypes.data) == 0
    assert call(cus=0) == -1 and call(min_tiles=-1) == -1 and call(hq=41) == -1
