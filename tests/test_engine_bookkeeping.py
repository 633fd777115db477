"""CPU tests of the engine's per-request bookkeeping helpers: the deferred
abort queue, the throughput window, incremental detokenisation and the
block-owner maps (no model and no GPU needed)."""

import threading

import pytest

from memforge_amd.runtime.continuous_engine import (ContinuousBatchingEngine, SequenceRuntime, _AbortRequests,
                                                    _ThroughputWindow)
from memforge_amd.runtime.prefix_sharing import block_owners
from memforge_amd.runtime.sampling import SamplingParams


def test_abort_requests_are_taken_once_from_any_thread():
    q = _AbortRequests()
    threads = [threading.Thread(target=q.add, args=(i,)) for i in range(50)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert q and q.take() == list(range(50))
    assert not q and q.take() == []


def test_throughput_window_counts_tokens_over_the_span_of_the_window():
    w = _ThroughputWindow(5.0)
    assert w.rate(0.0) == 0.0
    w.mark(10.0, 10.0, 1)
    assert w.rate(10.0) == 0.0            # fewer than two tokens
    w.mark(10.0, 10.0, 3)
    assert w.rate(10.0) == 0.0            # no span yet
    w.mark(12.0, 12.0, 4)
    assert w.rate(12.0) == 4.0            # 8 tokens over 2 s
    w.mark(13.0, 13.0, 0)                 # empty commits leave no mark
    # at 16.5 the marks at 10.0 have left the window: the 4 tokens at 12.0
    # remain, with no span to divide by
    assert w.rate(16.5) == 0.0 and w._count == 4
    w.mark(17.0, 17.0, 6)
    assert w.rate(17.0) == 2.0            # 10 tokens over 5 s


def test_throughput_window_one_multi_token_commit_has_a_span():
    """A window holding a single commit of several tokens spans from its first
    token to its last, as per-token timestamps would (the reference stamps
    each token, memforge_ml/runtime/continuous_engine.py:1342-1352, 1422-1430)."""
    w = _ThroughputWindow(5.0)
    w.mark(20.0, 20.5, 5)
    assert w.rate(20.5) == 10.0           # 5 tokens over 0.5 s
    # a mark stays while its last token is inside the window
    w.mark(24.0, 26.0, 3)
    assert w.rate(25.2) == round(8 / 6.0, 2)
    assert w.rate(25.6) == 1.5 and w._count == 3   # the 20.0-20.5 mark left: 3 over 2 s


class _SpaceTokenizer:
    """Pieces with a leading-space marker that decode drops at the start of
    the text (as SentencePiece does), plus two tokens that each carry half of
    a two-byte character (an incomplete character decodes to U+FFFD)."""

    pieces = {1: "_hello", 2: "_world", 3: "!", 4: "\xc3", 5: "\xa9", 6: "_again"}

    def decode(self, ids, skip_special_tokens=True):
        raw = "".join(self.pieces[i] for i in ids).replace("_", " ")
        if raw.startswith(" "):
            raw = raw[1:]
        data = raw.encode("latin-1")
        return data.decode("utf-8", errors="replace")


def _stream(ids):
    eng = ContinuousBatchingEngine.__new__(ContinuousBatchingEngine)
    eng.tokenizer = _SpaceTokenizer()
    rt = SequenceRuntime(seq_id=1, prompt_ids=[0], params=SamplingParams(), tokens=[0])
    out = []
    for i in ids:
        rt.generated.append(i)
        out.append(eng._text_delta(rt))
    return out, rt


def test_incremental_text_adds_up_to_the_full_decode():
    ids = [1, 2, 4, 5, 3, 6, 1]
    deltas, rt = _stream(ids)
    full = _SpaceTokenizer().decode(ids)
    assert "".join(deltas) == full == "hello world\xe9! again hello"
    assert deltas[0] == "hello" and deltas[1] == " world"
    assert deltas[2] == "" and deltas[3] == "\xe9"   # the character appears once complete
    assert rt.decoded_chars == len(full)
    # the decode window stays short however long the output grows
    assert len(rt.generated) - rt.text_from <= 2


def test_block_owners_lists_every_holder_sorted():
    owners = block_owners([(7, [3, 1, 9]), (2, [3, 4]), (5, [1, 1, 12])], total_blocks=10)
    assert owners == {"1": [5, 5, 7], "3": [2, 7], "4": [2], "9": [7]}
