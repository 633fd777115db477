"""CPU tests of the host-side argument checks that keep malformed block ids
away from the kernels: they raise the reference's exception types before
anything is uploaded or launched, so they run without a GPU."""

import pytest
import torch

from memforge_amd import _native as nat
from memforge_amd.kernels._varlen import run_varlen
from memforge_amd.models.paged_attention import PagedKVCache


def _cache(num_blocks=6, block_size=4):
    c = PagedKVCache.__new__(PagedKVCache)  # geometry only: no device memory
    c.num_blocks, c.block_size = num_blocks, block_size
    return c


def test_operator_block_ids_follow_torch_indexing():
    """A negative id counts from the end, as ``key_cache[id]`` does, and an id
    outside [-N, N) raises torch's own IndexError message."""
    c = _cache()
    assert c._blocks([5, -1, -6, 0], 4).tolist() == [5, 5, 0, 0]
    assert c._blocks([1, 2, 99], 2).tolist() == [1, 2]  # entries past `needed` are never read
    ref = torch.zeros(6, 2)
    for bad in (6, -7):
        with pytest.raises(IndexError) as theirs:
            ref[bad]
        with pytest.raises(IndexError) as ours:
            c._blocks([0, bad], 2)
        assert str(ours.value) == str(theirs.value)


def _pool(num_blocks=4, bs=16, hkv=2, d=64):
    k = torch.zeros((num_blocks, bs, hkv, d))
    return nat.PoolView.from_bshd(k, k.clone())


@pytest.mark.parametrize("table,msg", [([0, 4], "outside the pool"), ([-1, 1], "outside the pool"),
                                       ([2], "block table has")])
def test_varlen_launcher_refuses_tables_that_leave_the_pool(table, msg):
    pool = _pool()
    q = torch.zeros((1, 4, 64))
    with pytest.raises(IndexError, match=msg):
        run_varlen(q, q.clone(), pool, [table], [0], [20], None, 2)


def test_varlen_launcher_reads_only_the_pool_part_of_a_verify_table():
    """With pool_lens, only the blocks below pool_lens are read from the pool:
    a table sized for them passes the check (the launch itself then needs a
    GPU, which the CPU suite does not have)."""
    pool = _pool()
    q = torch.zeros((1, 4, 64))
    with pytest.raises(ValueError, match="GPU"):
        run_varlen(q, q.clone(), pool, [[3]], [0], [20], None, 2, pool_lens=[16],
                   new_k_rows=torch.zeros((1, 2, 64)), new_v_rows=torch.zeros((1, 2, 64)))


def test_pool_view_bounds():
    pool = _pool(num_blocks=5, bs=16)
    assert pool.num_blocks == 5 and pool.num_slots == 80
