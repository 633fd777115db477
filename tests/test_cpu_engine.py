"""The C4 CPU leg (oracle.cpu_engine: the reference engine's batched CPU path
on the host scheduler) against plain transformers greedy decoding, one
request at a time (oracle.cpu_baseline.greedy_cpu). A wrong position id, a
mask over the wrong columns of the left-padded batch or a K/V row scattered to
the wrong slot changes the tokens."""

import pytest
import torch

from oracle.cpu_baseline import greedy_cpu
from oracle.cpu_engine import CpuBatchedEngine
from tests.tiny_models import tiny_llama


@pytest.fixture(scope="module")
def model():
    return tiny_llama(num_layers=2, seed=0, device="cpu")


def _prompts(n, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(2, 256, (int(m),), generator=g).tolist() for m in torch.randint(3, 90, (n,), generator=g)]


@pytest.mark.parametrize("num_blocks,max_seqs,chunk", [
    (200, 4, 0),    # queueing: more requests than batch slots
    (200, 8, 24),   # chunked prefill: later chunks attend to the pooled prefix
    (14, 4, 0),     # a small pool: the scheduler preempts and recomputes
])
def test_cpu_engine_equals_plain_greedy(model, num_blocks, max_seqs, chunk):
    prompts = _prompts(7, seed=num_blocks + chunk)
    eng = CpuBatchedEngine(model, num_blocks=num_blocks, block_size=16, max_num_seqs=max_seqs,
                           max_prefill_tokens_per_step=chunk)
    got = eng.generate(prompts, 20)
    assert got == greedy_cpu(model, prompts, 20)
    assert eng.allocator.get_num_free_blocks() == eng.allocator.get_total_blocks()
    # batched decode: fewer forward passes than tokens
    assert eng.forward_passes < 7 * 20
