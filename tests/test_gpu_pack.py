"""Ragged-pack kernel: token ids, positions, sequence slots, slot_mapping,
cu_seqlens, kv_lens and padded block tables bit-exact against the oracle's
brute-force restatement of the engine's packing, plus its error reporting."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from memforge_amd import _native as nat
from oracle import paging

pytestmark = pytest.mark.gpu


def _upload(entries, device):
    """entries: (q_len, start, kv_len, table, tokens) -> device descriptor tensors."""
    desc, tables, tokens = [], [], []
    for q_len, start, kv_len, table, toks in entries:
        desc.append([q_len, start, kv_len, len(tables), len(table), len(tokens)])
        tables.extend(table)
        tokens.extend(toks)
    d = torch.tensor(desc, dtype=torch.int32, device=device).reshape(-1, nat.ENTRY_INTS)
    t = torch.tensor(tables or [0], dtype=torch.int32, device=device)
    k = torch.tensor(tokens or [0], dtype=torch.int32, device=device)
    total = sum(e[0] for e in entries)
    return d, t, k, total


def _random_step(gen, n_prefill, n_decode, bs, num_blocks, vocab=49152):
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    entries, k = [], 0
    for i in range(n_prefill + n_decode):
        if i < n_prefill:
            prior = int(torch.randint(0, 300, (1,), generator=gen))
            q_len = int(torch.randint(1, 120, (1,), generator=gen))
        else:
            prior = int(torch.randint(1, 500, (1,), generator=gen))
            q_len = 1
        n = prior + q_len
        nb = (n + bs - 1) // bs
        table = perm[k:k + nb]
        k += nb
        toks = torch.randint(0, vocab, (q_len,), generator=gen).tolist()
        entries.append((q_len, prior, n, table, toks))
    return entries


@pytest.mark.parametrize("bs", [16, 4])
def test_pack_matches_oracle(device, bs):
    gen = torch.Generator().manual_seed(bs)
    entries = _random_step(gen, 4, 28, bs, 4000)
    max_blocks = max(len(e[3]) for e in entries)
    d, t, k, total = _upload(entries, device)
    bitmap = torch.zeros((4000 * bs + 31) // 32, dtype=torch.int32, device=device)
    out = nat.ragged_pack(d, t, k, total, bs, max_blocks, bitmap, 4000 * bs)
    want = paging.ragged_pack(entries, bs, max_blocks)
    for name in ("token_ids", "positions", "seq_slot", "slot_mapping", "cu_seqlens", "kv_lens", "block_tables"):
        np.testing.assert_array_equal(getattr(out, name).cpu().numpy(), want[name], err_msg=name)
    assert out.status.cpu().tolist() == [0, -1, -1, -1]
    assert int(bitmap.abs().sum()) == 0, "bitmap not returned to zero"


def test_pack_reports_table_overflow_and_duplicates(device):
    bs = 16
    # entry 1 shares entry 0's block 7 at the same offset -> duplicate slots;
    # entry 2 runs past its one-block table -> overflow from its row 3 on.
    entries = [
        (4, 0, 4, [7], [1, 2, 3, 4]),
        (2, 2, 4, [7], [5, 6]),
        (5, 14, 19, [9], [7, 8, 9, 10, 11]),
    ]
    d, t, k, total = _upload(entries, device)
    bitmap = torch.zeros(64, dtype=torch.int32, device=device)
    out = nat.ragged_pack(d, t, k, total, bs, 1, bitmap, 64 * 32)
    want = paging.ragged_pack(entries, bs, 1)
    st = out.status.cpu().tolist()
    assert st[0] & nat.PACK_TABLE_OVERFLOW and st[0] & nat.PACK_DUPLICATE_SLOT
    assert st[1] == want["first_overflow_row"] == 8
    # which of two colliding rows sees the other's bit first is up to the atomics
    assert want["first_duplicate_row"] == 4 and st[2] in (2, 3, 4, 5)
    np.testing.assert_array_equal(out.slot_mapping.cpu().numpy(), want["slot_mapping"])
    assert int(bitmap.abs().sum()) == 0


def test_pack_verify_rows(device):
    """Verify rows: [last token] + k candidates at positions ctx..ctx+k
    (batched_speculative.py:696-701)."""
    gen = torch.Generator().manual_seed(3)
    bs, kk = 16, 4
    entries = []
    perm = torch.randperm(200, generator=gen).tolist()
    off = 0
    for ctx in (130, 512, 2047):
        nb = (ctx + kk + 1 + bs - 1) // bs
        toks = torch.randint(0, 1000, (kk + 1,), generator=gen).tolist()
        entries.append((kk + 1, ctx, ctx + kk + 1, perm[off:off + nb], toks))
        off += nb
    max_blocks = max(len(e[3]) for e in entries)
    d, t, k, total = _upload(entries, device)
    out = nat.ragged_pack(d, t, k, total, bs, max_blocks)
    want = paging.ragged_pack(entries, bs, max_blocks)
    for name in ("token_ids", "positions", "slot_mapping", "cu_seqlens", "kv_lens"):
        np.testing.assert_array_equal(getattr(out, name).cpu().numpy(), want[name], err_msg=name)


def test_pack_skips_malformed_entries_and_reports_them(device):
    """Malformed descriptors through the C ABI are reported, not followed:
    an entry whose table run or token run leaves the arrays, or with a
    negative field, loads nothing (token 0, slot -1, an all-zero table row),
    a block id outside the pool gives slot -1, and well-formed entries in the
    same step pack exactly as the oracle packs them."""
    bs = 16
    good = [(3, 5, 8, [2], [11, 12, 13]), (1, 40, 41, [4, 1, 6], [14])]
    d, t, k, total = _upload(good, device)
    want = paging.ragged_pack(good, bs, 3)
    desc = d.cpu()
    rows = desc.tolist()
    # entry 2: its table run leaves `tables`; entry 3: its token run leaves
    # `tokens`; entry 4: a negative table length
    rows.append([2, 0, 2, t.numel() - 1, 5, 0])
    rows.append([2, 0, 2, 0, 1, k.numel() + 100])
    rows.append([1, 0, 1, 0, -3, 0])
    bad = torch.tensor(rows, dtype=torch.int32, device=device)
    out = nat.ragged_pack(bad, t, k, total + 5, bs, 3, num_slots=8 * bs)
    st = out.status.cpu().tolist()
    assert st[0] & nat.PACK_BAD_ENTRY and st[3] == 2, st
    assert not st[0] & nat.PACK_ROW_COUNT
    slots = out.slot_mapping.cpu().numpy()
    toks = out.token_ids.cpu().numpy()
    np.testing.assert_array_equal(slots[:total], want["slot_mapping"])
    np.testing.assert_array_equal(toks[:total], want["token_ids"])
    assert (slots[total:] == -1).all() and (toks[total:] == 0).all()
    bt = out.block_tables.cpu().numpy()
    np.testing.assert_array_equal(bt[:2], want["block_tables"])
    assert (bt[2:] == 0).all()
    # a block id past a pool of 5 blocks: its row gets slot -1, its table entry 0
    out = nat.ragged_pack(d, t, k, total, bs, 3, num_slots=5 * bs)
    st = out.status.cpu().tolist()
    assert st[0] & nat.PACK_BLOCK_OUT_OF_POOL and st[1] == 3, st
    assert out.slot_mapping.cpu().tolist() == want["slot_mapping"][:3].tolist() + [-1]
    assert out.block_tables.cpu().numpy()[1].tolist() == [4, 1, 0]
    # more rows declared than the entries hold: the surplus rows load nothing
    out = nat.ragged_pack(d, t, k, total + 2, bs, 3)
    st = out.status.cpu().tolist()
    assert st[0] & nat.PACK_ROW_COUNT, st
    assert out.slot_mapping.cpu().tolist()[total:] == [-1, -1]
    assert out.seq_slot.cpu().tolist()[total:] == [-1, -1]
    assert out.cu_seqlens.cpu().tolist() == [0, 3, 4]
