"""GPU tests of the drop-in runtime layer: PagedKVPool, PagedCache,
VarlenPackedCache, the attention backend and the operator mirrors, each
against transformers' own cache/attention or the CPU oracle (the reference's
tests/python/test_kv_pool.py, test_paged_cache.py, test_varlen_cache.py,
test_attention_backend.py and test_kernels.py cover the same behaviour)."""

import numpy as np
import pytest
import torch

from oracle import paging as opg
from tests.tiny_models import StubTokenizer, tiny_llama

pytestmark = pytest.mark.gpu


def _pool(model, num_blocks=64, block_size=4, dtype=None):
    from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool

    spec = ModelKVSpec.from_config(model.config, dtype or next(model.parameters()).dtype, "cuda:0")
    return PagedKVPool(spec, num_blocks=num_blocks, block_size=block_size)


@pytest.fixture(scope="module")
def model(device):
    return tiny_llama(num_layers=2, seed=0)


# ------------------------------------------------------------------ PagedKVPool


def test_slot_indices_translate_through_a_scattered_table(model):
    pool = _pool(model)
    table = torch.tensor([7, 2, 9], device="cuda:0")
    phys, slots = pool.slot_indices(table, 3, 10)
    ph, sl = opg.slot_indices([7, 2, 9], 3, 10, 4)
    assert phys.cpu().tolist() == list(ph) and slots.cpu().tolist() == list(sl)
    with pytest.raises(IndexError, match="outside a block table"):
        pool.slot_indices(table, 0, 13)


def test_pool_write_then_gather_round_trips_and_layers_are_isolated(model):
    pool = _pool(model)
    pool.zero_()
    g = torch.Generator(device="cuda:0").manual_seed(1)
    table = torch.tensor([5, 1, 12, 3], device="cuda:0")
    k = torch.randn((1, 2, 13, 16), generator=g, device="cuda:0")
    v = torch.randn((1, 2, 13, 16), generator=g, device="cuda:0")
    phys, slots = pool.slot_indices(table, 0, 13)
    pool.write(1, phys, slots, k, v)
    k2, v2 = pool.gather(1, phys, slots)
    assert torch.equal(k2, k) and torch.equal(v2, v)
    assert int(pool.key_pool[0].count_nonzero()) == 0, "layer 0 must be untouched"
    flat = pool.flat_indices(table, 0, 13)
    expected = opg.flat_slot_index(phys.cpu().numpy(), slots.cpu().numpy(), 4)
    assert flat.cpu().numpy().tolist() == expected.tolist()


def test_pool_geometry(model):
    from memforge_amd.runtime.kv_pool import PagedKVPool

    pool = _pool(model, num_blocks=10, block_size=4)
    spec = pool.spec
    assert spec.bytes_per_token == 2 * spec.num_layers * spec.num_kv_heads * spec.head_dim * 4
    assert pool.capacity_tokens == 40
    n = PagedKVPool.blocks_for_budget(spec, 16, 1.0)
    assert n * spec.bytes_per_token * 16 <= 1024 * 1024 < (n + 1) * spec.bytes_per_token * 16


def test_sequences_sharing_a_pool_do_not_corrupt_each_other(model):
    pool = _pool(model)
    pool.zero_()
    a, b = torch.tensor([0, 1], device="cuda:0"), torch.tensor([2, 3], device="cuda:0")
    ka = torch.full((1, 2, 8, 16), 1.0, device="cuda:0")
    kb = torch.full((1, 2, 8, 16), 2.0, device="cuda:0")
    pool.write_flat(0, pool.flat_indices(a, 0, 8), ka, ka)
    pool.write_flat(0, pool.flat_indices(b, 0, 8), kb, kb)
    assert torch.equal(pool.gather_flat(0, pool.flat_indices(a, 0, 8))[0], ka)
    assert torch.equal(pool.gather_flat(0, pool.flat_indices(b, 0, 8))[1], kb)


# ------------------------------------------------------------------ PagedCache


def _dynamic_logits(model, ids_chunks):
    from transformers.cache_utils import DynamicCache

    cache = DynamicCache()
    outs = []
    with torch.no_grad():
        for ids in ids_chunks:
            outs.append(model(input_ids=torch.tensor([ids], device="cuda:0"), past_key_values=cache,
                              use_cache=True).logits[0])
    return outs


@pytest.mark.parametrize("lazy", [False, True])
def test_paged_cache_matches_dynamic_cache(model, lazy):
    from memforge_amd.kernels import attention_backend
    from memforge_amd.runtime.paged_cache import PagedCache

    pool = _pool(model)
    chunks = [[5, 9, 11, 40, 41, 77, 3], [12], [19], [200], [31]]
    expected = _dynamic_logits(model, chunks)
    cache = PagedCache(pool, [9, 3, 30, 1], lazy_read=lazy)
    with torch.no_grad():
        for ids, exp in zip(chunks, expected):
            with attention_backend.backend_enabled_on(model):
                with attention_backend.paged_attention_context(pool, cache) as bound:
                    got = model(input_ids=torch.tensor([ids], device="cuda:0"), past_key_values=cache,
                                use_cache=True).logits[0]
            if lazy and len(ids) == 1:
                assert bound.used == model.config.num_hidden_layers, "every decode layer takes the kernel"
            torch.testing.assert_close(got, exp, atol=2e-5, rtol=1e-4)
    assert cache.position == sum(len(c) for c in chunks)
    assert all(layer.position == cache.position for layer in cache.layers)


def test_paged_cache_rollback_then_replay_matches_a_clean_run(model):
    from memforge_amd.runtime.paged_cache import PagedCache

    pool = _pool(model)
    cache = PagedCache(pool, [4, 8, 15])
    table_before = cache.block_table
    with torch.no_grad():
        model(input_ids=torch.tensor([[3, 4, 5, 6, 7]], device="cuda:0"), past_key_values=cache, use_cache=True)
        model(input_ids=torch.tensor([[90, 91, 92]], device="cuda:0"), past_key_values=cache, use_cache=True)
        cache.rollback(3)
        assert cache.position == 5 and cache.block_table == table_before
        got = model(input_ids=torch.tensor([[8]], device="cuda:0"), past_key_values=cache, use_cache=True).logits[0]
    exp = _dynamic_logits(model, [[3, 4, 5, 6, 7], [8]])[1]
    torch.testing.assert_close(got, exp, atol=2e-5, rtol=1e-4)


def test_paged_cache_growing_table_and_batch_rejection(model):
    from memforge_amd.runtime.paged_cache import PagedCache

    pool = _pool(model)
    cache = PagedCache(pool, [0])
    with torch.no_grad():
        model(input_ids=torch.tensor([[3, 4, 5, 6]], device="cuda:0"), past_key_values=cache, use_cache=True)
        cache.set_block_table([0, 6])
        got = model(input_ids=torch.tensor([[7]], device="cuda:0"), past_key_values=cache, use_cache=True).logits[0]
    exp = _dynamic_logits(model, [[3, 4, 5, 6], [7]])[1]
    torch.testing.assert_close(got, exp, atol=2e-5, rtol=1e-4)
    with pytest.raises(ValueError, match="single-sequence"):
        cache.layers[0].update(torch.zeros((2, 2, 1, 16), device="cuda:0"), torch.zeros((2, 2, 1, 16), device="cuda:0"))
    with pytest.raises(NotImplementedError):
        PagedCache(pool, [0], view_capacity=64)


# ----------------------------------------------------------- VarlenPackedCache


def test_varlen_write_index_matches_oracle_in_any_packing_order(model):
    from memforge_amd.runtime.varlen_cache import build_write_index

    pool = _pool(model)
    tables = [[3, 8, 1], [0, 5], [11]]
    seq_ids = [1, 0, 0, 2, 1, 1, 0]
    positions = [4, 0, 1, 2, 5, 6, 2]
    got = build_write_index(pool, [torch.tensor(t) for t in tables], seq_ids, positions).cpu().numpy()
    assert got.tolist() == opg.varlen_write_index(tables, seq_ids, positions, 4).tolist()


def test_varlen_cache_rejects_what_the_reference_rejects(model):
    from memforge_amd.runtime.varlen_cache import VarlenPackedCache

    pool = _pool(model)
    t = [torch.tensor([3, 8]), torch.tensor([0])]
    with pytest.raises(ValueError, match="same pool slot"):
        VarlenPackedCache(pool, 2, t, [0, 0], [1, 1])
    with pytest.raises(ValueError, match="same pool slot"):
        VarlenPackedCache(pool, 2, [torch.tensor([3]), torch.tensor([3])], [0, 1], [2, 2])
    with pytest.raises(IndexError, match="logical block"):
        VarlenPackedCache(pool, 2, t, [1], [4])
    with pytest.raises(IndexError, match="no block table"):
        VarlenPackedCache(pool, 2, t, [2], [0])
    with pytest.raises(ValueError, match="negative position"):
        VarlenPackedCache(pool, 2, t, [0], [-1])
    with pytest.raises(ValueError):
        VarlenPackedCache(pool, 2, t, [0, 1], [0])
    with pytest.raises(ValueError):
        VarlenPackedCache(pool, 2, t, [], [])
    cache = VarlenPackedCache(pool, 2, t, [0, 1], [0, 0])
    with pytest.raises(NotImplementedError):
        cache.crop(1)
    assert cache.get_seq_length() == 0
    with pytest.raises(ValueError):
        cache.layers[0].update(torch.zeros((1, 2, 3, 16), device="cuda:0"), torch.zeros((1, 2, 3, 16), device="cuda:0"))
    # a rejected pass leaves the duplicate bitmap clear for the next one
    VarlenPackedCache(pool, 2, t, [0, 0, 1], [0, 1, 0])


def test_packed_pass_equals_per_sequence_passes(model):
    """A prefill chunk, a fresh prefill and a decode in one packed forward give
    each sequence the logits of its own DynamicCache run."""
    from memforge_amd.kernels import attention_backend
    from memforge_amd.runtime.paged_cache import PagedCache
    from memforge_amd.runtime.varlen_cache import VarlenPackedCache

    pool = _pool(model, num_blocks=64, block_size=4)
    a_prompt, b_prompt, c_prompt = [5, 6, 7, 8, 9, 10, 11], [40, 41, 42, 43, 44], [90, 91, 92, 93, 94, 95]
    tables = [[10, 2, 33], [7, 8], [20, 21]]
    # A: 4 tokens resident, next 3 in this pass; C: all 6 resident, decodes one
    with torch.no_grad():
        for s, ids in ((0, a_prompt[:4]), (2, c_prompt)):
            cache = PagedCache(pool, tables[s])
            model(input_ids=torch.tensor([ids], device="cuda:0"), past_key_values=cache, use_cache=True)
    seq_ids = [0] * 3 + [1] * 5 + [2]
    positions = [4, 5, 6] + list(range(5)) + [6]
    tokens = a_prompt[4:] + b_prompt + [17]
    cache = VarlenPackedCache(pool, 2, [torch.tensor(t) for t in tables], seq_ids, positions)
    with attention_backend.backend_enabled_on(model):
        with attention_backend.varlen_attention_context(pool, [torch.tensor(t) for t in tables], seq_ids,
                                                        positions) as bound:
            with torch.no_grad():
                got = model(input_ids=torch.tensor([tokens], device="cuda:0"),
                            position_ids=torch.tensor([positions], device="cuda:0"), past_key_values=cache,
                            use_cache=True).logits[0]
    assert bound.used == 2
    exp_a = _dynamic_logits(model, [a_prompt[:4], a_prompt[4:]])[1]
    exp_b = _dynamic_logits(model, [b_prompt])[0]
    exp_c = _dynamic_logits(model, [c_prompt, [17]])[1]
    torch.testing.assert_close(got[:3], exp_a, atol=2e-5, rtol=1e-4)
    torch.testing.assert_close(got[3:8], exp_b, atol=2e-5, rtol=1e-4)
    torch.testing.assert_close(got[8:], exp_c, atol=2e-5, rtol=1e-4)
    assert not attention_backend.is_enabled_on(model), "routing is restored after the pass"


# ------------------------------------------------------------ attention backend


def test_register_is_idempotent_and_enable_on_routes(device):
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    from memforge_amd.kernels import attention_backend as ab

    assert ab.register() and ab.register()
    assert ALL_ATTENTION_FUNCTIONS[ab.BACKEND_NAME] is ab.paged_attention_forward
    assert ab.BACKEND_NAME in ALL_MASK_ATTENTION_FUNCTIONS
    m = tiny_llama(num_layers=1, seed=3)
    assert not ab.is_enabled_on(m)
    assert ab.enable_on(m) and ab.is_enabled_on(m)


def test_unbound_backend_prefill_matches_the_default_attention(model):
    from memforge_amd.kernels import attention_backend as ab

    ids = torch.tensor([[4, 8, 15, 16, 23, 42]], device="cuda:0")
    with torch.no_grad():
        exp = model(input_ids=ids).logits
        with ab.backend_enabled_on(model):
            got = model(input_ids=ids).logits
    torch.testing.assert_close(got, exp, atol=2e-5, rtol=1e-4)


def test_implicit_causal_mask_matches_an_explicit_one(device):
    from memforge_amd.kernels import attention_backend as ab

    s = torch.randn((1, 2, 3, 5), device="cuda:0")
    got = ab._apply_implicit_causal_mask(s)
    keep = torch.ones(3, 5, dtype=torch.bool, device="cuda:0").tril(diagonal=2)
    assert torch.equal(got[..., keep], s[..., keep])
    assert bool((got[..., ~keep] == torch.finfo(s.dtype).min).all())


# ------------------------------------------------------------- operator mirror


def test_paged_kv_cache_and_paged_attention_operator(device):
    """PagedKVCache + PagedAttention (models/paged_attention.py) against a
    dense softmax of the same K/V."""
    from memforge_amd.models.paged_attention import PagedAttention, PagedKVCache

    torch.manual_seed(0)
    kv = PagedKVCache(num_blocks=16, block_size=16, num_heads=4, head_dim=64, dtype=torch.float32, device="cuda:0")
    table = [3, 9, 1]
    k = torch.randn((1, 4, 40, 64), device="cuda:0")
    v = torch.randn((1, 4, 40, 64), device="cuda:0")
    kv.write_kv(k, v, table, 0)
    k2, v2 = kv.read_kv(table, 40)
    assert torch.equal(k2, k[0]) and torch.equal(v2, v[0])
    q = torch.randn((1, 4, 1, 64), device="cuda:0")
    out = PagedAttention()(q, kv, table, 40)
    w = torch.softmax(torch.matmul(q, k.transpose(2, 3).contiguous()) / 8.0, dim=-1)
    exp = torch.matmul(w, v).transpose(1, 2).reshape(1, 1, 256)
    torch.testing.assert_close(out, exp, atol=1e-5, rtol=1e-5)
    with pytest.raises(IndexError):
        kv.write_kv(torch.randn((1, 4, 60, 64), device="cuda:0"), torch.randn((1, 4, 60, 64), device="cuda:0"),
                    table, 0)


def test_blockwise_and_varlen_operators_match_their_torch_references(device):
    from memforge_amd.kernels.block_attention import paged_attention_blockwise, reference_attention
    from memforge_amd.kernels.varlen_attention import paged_attention_varlen, reference_varlen_attention

    torch.manual_seed(1)
    L, N, bs, hkv, d = 2, 24, 16, 2, 64
    kp = torch.randn((L, N, bs, hkv, d), device="cuda:0")
    vp = torch.randn((L, N, bs, hkv, d), device="cuda:0")
    table = torch.tensor([5, 17, 2, 9], device="cuda:0")
    q = torch.randn((1, 8, 1, d), device="cuda:0")
    out = paged_attention_blockwise(q, kp, vp, 1, table, 53, bs)
    flat = (table.repeat_interleave(bs)[:53] * bs + torch.arange(53, device="cuda:0") % bs)
    keys = kp[1].reshape(-1, hkv, d)[flat].permute(1, 0, 2).unsqueeze(0)
    vals = vp[1].reshape(-1, hkv, d)[flat].permute(1, 0, 2).unsqueeze(0)
    torch.testing.assert_close(out, reference_attention(q, keys, vals), atol=1e-5, rtol=1e-5)

    tables = [table, torch.tensor([1, 3], device="cuda:0")]
    seq_ids = [1, 0, 1, 0]
    positions = [17, 52, 18, 40]
    qv = torch.randn((1, 8, 4, d), device="cuda:0")
    got = paged_attention_varlen(qv, kp, vp, 0, tables, seq_ids, positions, bs)
    exp = reference_varlen_attention(qv, kp, vp, 0, tables, seq_ids, positions, bs)
    torch.testing.assert_close(got, exp, atol=1e-5, rtol=1e-5)
    with pytest.raises(IndexError):
        paged_attention_varlen(qv, kp, vp, 0, tables, seq_ids, [17, 52, 40, 40], bs)
    with pytest.raises(ValueError):
        paged_attention_varlen(qv, kp, vp, 0, tables, seq_ids, [17, -1, 18, 40], bs)


def test_batched_decode_assembly_is_left_padded_and_scatter_is_its_inverse(model):
    from memforge_amd.kernels.batched_decode import BatchedDecodeBuffers, assemble_batch, scatter_new_tokens

    pool = _pool(model, block_size=4)
    torch.manual_seed(2)
    pool.key_pool.normal_()
    pool.value_pool.normal_()
    tables = [torch.tensor([3, 7, 1], device="cuda:0"), torch.tensor([9], device="cuda:0")]
    lens = [10, 3]
    bufs = BatchedDecodeBuffers(num_layers=2, block_size=4)
    layers, mask, padded = assemble_batch(pool, bufs, tables, lens)
    assert padded == 16 and mask.sum(1).tolist() == lens
    for li in range(2):
        for row, (t, n) in enumerate(zip(tables, lens)):
            k, v = pool.gather_flat(li, pool.flat_indices(t, 0, n))
            assert torch.equal(layers[li][0][row, :, padded - n:], k[0])
            assert torch.equal(layers[li][1][row, :, padded - n:], v[0])
            assert int(layers[li][0][row, :, : padded - n].count_nonzero()) == 0
    nk = [torch.randn((2, 2, 1, 16), device="cuda:0") for _ in range(2)]
    nv = [torch.randn((2, 2, 1, 16), device="cuda:0") for _ in range(2)]
    tables[1] = torch.tensor([9, 0], device="cuda:0")
    scatter_new_tokens(pool, tables, lens, nk, nv)
    for li in range(2):
        for row, (t, n) in enumerate(zip(tables, lens)):
            k, v = pool.gather_flat(li, pool.flat_indices(t, n, n + 1))
            assert torch.equal(k[0, :, 0], nk[li][row, :, 0]) and torch.equal(v[0, :, 0], nv[li][row, :, 0])
