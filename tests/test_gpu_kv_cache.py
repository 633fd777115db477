"""KV write (slot_mapping scatter) and gather kernels: bit-exact against the
oracle, including the dtype conversion of a write into a narrower pool."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from memforge_amd import _native as nat
from oracle import bf16 as obf16
from oracle import paging

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def expected_bits(src: torch.Tensor, pool_dtype: torch.dtype) -> np.ndarray:
    """Source values converted to the pool dtype by the oracle's own rounding."""
    if src.dtype == pool_dtype:
        return bits(src)
    f32 = src.detach().cpu().to(torch.float32).numpy()
    if pool_dtype == torch.float32:
        return f32.view(np.uint32).copy()
    if pool_dtype == torch.bfloat16:
        return obf16.f32_to_bf16_bits(f32)
    return f32.astype(np.float16).view(np.uint16)  # numpy rounds to nearest even


@pytest.mark.parametrize("src,dst", [("fp32", "fp32"), ("fp32", "bf16"), ("bf16", "bf16"),
                                     ("fp16", "fp16"), ("fp32", "fp16"), ("bf16", "fp32")])
@pytest.mark.parametrize("bs,d", [(16, 128), (4, 8), (16, 64), (8, 12)])
def test_kv_write_bit_exact(device, src, dst, bs, d):
    gen = torch.Generator().manual_seed(bs * 1000 + d)
    L, N, H, T = 3, 20, 5, 37
    pool_k = torch.randn((L, N, bs, H, d), generator=gen).to(DT[dst]).to(device)
    pool_v = torch.randn((L, N, bs, H, d), generator=gen).to(DT[dst]).to(device)
    before_k, before_v = bits(pool_k), bits(pool_v)
    # HF's (1, H, T, D) projection output as a transposed view
    keys = torch.randn((1, T, H, d), generator=gen).to(DT[src]).transpose(1, 2).to(device)
    vals = torch.randn((1, T, H, d), generator=gen).to(DT[src]).transpose(1, 2).to(device)
    slots = torch.randperm(N * bs, generator=gen)[:T]
    slots[5] = -1  # skipped row
    layer = 1
    nat.kv_write(keys[0].permute(1, 0, 2), vals[0].permute(1, 0, 2), slots.to(device),
                 nat.PoolView.from_bshd(pool_k[layer], pool_v[layer]))
    torch.cuda.synchronize()
    for pool, before, src_t in ((pool_k, before_k, keys), (pool_v, before_v, vals)):
        want = before.copy()
        rows = expected_bits(src_t[0].permute(1, 0, 2).contiguous(), DT[dst])
        paging.kv_write(want[layer], slots.numpy(), rows)
        np.testing.assert_array_equal(bits(pool), want)


def test_kv_write_operator_layout(device):
    """PagedKVCache (blocks, heads, slots, dim) through the same kernel
    (PagedKVCache.write_kv, paged_attention.py:45-67)."""
    gen = torch.Generator().manual_seed(2)
    N, H, bs, d, T = 8, 4, 16, 32, 25
    kc = torch.zeros((N, H, bs, d), device=device)
    vc = torch.zeros((N, H, bs, d), device=device)
    table = [2, 5]
    keys = torch.randn((T, H, d), generator=gen)
    vals = torch.randn((T, H, d), generator=gen)
    slots = torch.from_numpy(paging.slot_mapping(table, 0, T, bs))
    nat.kv_write(keys.to(device), vals.to(device), slots.to(device), nat.PoolView.from_bhsd(kc, vc))
    for i in range(T):
        blk, off = table[i // bs], i % bs
        assert torch.equal(kc[blk, :, off, :].cpu(), keys[i])
        assert torch.equal(vc[blk, :, off, :].cpu(), vals[i])


@pytest.mark.parametrize("pool_dt,dst_dt", [("bf16", "bf16"), ("fp32", "fp32"), ("bf16", "fp32")])
def test_kv_gather_bit_exact(device, pool_dt, dst_dt):
    gen = torch.Generator().manual_seed(4)
    N, bs, H, d, T = 16, 16, 3, 64, 50
    pk = torch.randn((N, bs, H, d), generator=gen).to(DT[pool_dt]).to(device)
    pv = torch.randn((N, bs, H, d), generator=gen).to(DT[pool_dt]).to(device)
    slots = torch.randint(0, N * bs, (T,), generator=gen)  # duplicates allowed when reading
    out_k = torch.empty((1, H, T, d), dtype=DT[dst_dt], device=device)
    out_v = torch.empty((1, H, T, d), dtype=DT[dst_dt], device=device)
    nat.kv_gather(nat.PoolView.from_bshd(pk, pv), slots.to(device), out_k[0].permute(1, 0, 2),
                  out_v[0].permute(1, 0, 2))
    for pool, out in ((pk, out_k), (pv, out_v)):
        want = paging.kv_gather(pool.cpu().to(DT[dst_dt]).float().numpy(), slots.numpy())
        np.testing.assert_array_equal(out[0].permute(1, 0, 2).cpu().float().numpy(), want)


def test_gather_inverts_write(device):
    """Write then gather through the same slots returns the rows
    (test_kernels.py:270-295)."""
    gen = torch.Generator().manual_seed(6)
    N, bs, H, d, T = 10, 16, 2, 64, 40
    pk = torch.zeros((N, bs, H, d), dtype=torch.bfloat16, device=device)
    pv = torch.zeros_like(pk)
    rows_k = torch.randn((T, H, d), generator=gen).to(torch.bfloat16).to(device)
    rows_v = torch.randn((T, H, d), generator=gen).to(torch.bfloat16).to(device)
    slots = torch.randperm(N * bs, generator=gen)[:T].to(device)
    view = nat.PoolView.from_bshd(pk, pv)
    nat.kv_write(rows_k, rows_v, slots, view)
    gk = torch.empty_like(rows_k)
    gv = torch.empty_like(rows_v)
    nat.kv_gather(view, slots, gk, gv)
    assert torch.equal(gk, rows_k) and torch.equal(gv, rows_v)


# ------------------------------------------------------------------ block copy

@pytest.mark.parametrize("dt", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("geom", [(3, 24, 16, 5, 64), (2, 80, 4, 2, 32), (2, 12, 2, 1, 3), (4, 9, 1, 1, 2)])
def test_block_copy_moves_whole_blocks_in_every_layer(dt, geom):
    """mf_kv_copy_blocks against a host copy: destination blocks take the
    source blocks' bits in every layer of K and V, nothing else changes. The
    geometries cover 16-byte and 4-byte vector paths and more than 32 pairs
    (two launches)."""
    L, N, bs, H, D = geom
    g = torch.Generator().manual_seed(sum(geom))
    k = torch.randn((L, N, bs, H, D), generator=g).to(DT[dt])
    v = torch.randn((L, N, bs, H, D), generator=g).to(DT[dt])
    perm = torch.randperm(N, generator=g).tolist()
    half = N // 2
    pairs = list(zip(perm[:half], perm[half:2 * half]))
    pairs.append((perm[0], perm[0]))  # on itself: skipped
    want_k, want_v = bits(k).copy(), bits(v).copy()
    for s, d in pairs:
        want_k[:, d] = bits(k)[:, s]
        want_v[:, d] = bits(v)[:, s]
    kd, vd = k.cuda(), v.cuda()
    nat.kv_copy_blocks(kd, vd, pairs)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kd), want_k)
    assert np.array_equal(bits(vd), want_v)


def test_block_copy_errors_surface_as_exceptions():
    k = torch.zeros((2, 8, 1, 1, 1), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(nat.MemforgeHipError):  # 2-byte blocks: below the 4-byte unit
        nat.kv_copy_blocks(k, k.clone(), [(0, 1)])
    k = torch.zeros((2, 8, 4, 2, 16), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(nat.MemforgeHipError):
        nat.kv_copy_blocks(k, k.clone(), [(0, 8)])
    with pytest.raises(ValueError):
        nat.kv_copy_blocks(k[:, :, :, :, :8], k.clone()[:, :, :, :, :8], [(0, 1)])
