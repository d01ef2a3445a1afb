"""The oracle against the reference's own known answers for the speculative step.

Traces follow the reference's scheduler tests (Tests/MLXCatTests/SchedulerSpeculativeDecodingTests.swift):
prompt [1,2,3,1,2,3,1,2], K=4, minContext 8, maxTokens 10, fake models with logits +20 at
next(token) and -20 elsewhere (:174-261).  Expected values were derived by hand from
Sources/MLXCat/TrackB/BatchGenerator.swift:875-1010 and Scheduler.swift:599-668.
"""
import pytest

from tests._common import FAKE_MISMATCHING, FAKE_REPEATING, spec

PROMPT = [1, 2, 3, 1, 2, 3, 1, 2]


def run_oracle(O, model_cfg, spec_cfg, prompt=PROMPT, max_tokens=10, sampling=None):
    m = O.Model(model_cfg, 1, 64, 1)
    g = O.Generator(m, spec_cfg, 1, 64)
    tok, fin = g.insert(0, prompt, max_tokens, sampling or O.make_sampling())
    toks = [tok]
    while g.active(0):
        t, c, f = g.step()
        toks += t[0, :c[0]].tolist()
    return toks, g.stats(), g.call_widths()


@pytest.mark.parametrize("acceptance", [0, 1])
def test_repeating_model_trace(oracle, acceptance):
    toks, stats, widths = run_oracle(oracle, FAKE_REPEATING, spec(k=4, min_ctx=8, acceptance=acceptance))
    assert toks == [3, 1, 2, 3, 1, 2, 3, 1, 2, 3]
    assert stats == dict(proposed=7, accepted=7, proposal_batches=2, rejected_batches=0)
    assert widths == [1, 4, 5]


@pytest.mark.parametrize("acceptance", [0, 1])
def test_mismatching_model_trace(oracle, acceptance):
    toks, stats, widths = run_oracle(oracle, FAKE_MISMATCHING, spec(k=4, min_ctx=8, acceptance=acceptance))
    assert toks == [3, 4, 1, 2, 3, 4, 1, 2, 3, 4]
    # proposals [1,2,3] (rejected at position 0), none, [2,3,4,1], [3]
    assert stats == dict(proposed=8, accepted=5, proposal_batches=3, rejected_batches=1)


@pytest.mark.parametrize("model", [FAKE_REPEATING, FAKE_MISMATCHING])
def test_speculation_matches_plain_decode(oracle, model):
    """testNgramSpeculationProducesIdenticalTokensWithFewerDecodeCalls (:9-37) and
    testRejectedNgramProposalFallsBackWithoutChangingOutput (:39-61)."""
    base, bstats, bw = run_oracle(oracle, model, spec(enabled=False))
    sp, sstats, sw = run_oracle(oracle, model, spec(k=4, min_ctx=8))
    assert sp == base
    assert len(sp) == 10
    assert bstats == dict(proposed=0, accepted=0, proposal_batches=0, rejected_batches=0)
    if model is FAKE_REPEATING:
        assert sstats["accepted"] > 0 and sstats["proposal_batches"] > 0
        assert len(sw) < len(bw)
        assert sum(sw) / len(sw) > sum(bw) / len(bw)
    else:
        assert sstats["rejected_batches"] > 0


def test_tool_trigger_rejects_verify_block(oracle):
    """A verify position that samples the tool-call trigger rejects the block
    (BatchGenerator.swift:916-923); the output still equals plain decoding."""
    sp = oracle.make_sampling(reject_token=1)
    toks, stats, _ = run_oracle(oracle, FAKE_REPEATING, spec(k=4, min_ctx=8), sampling=sp)
    base, _, _ = run_oracle(oracle, FAKE_REPEATING, spec(enabled=False), sampling=sp)
    assert toks == base
    assert stats["rejected_batches"] > 0


def test_eos_stops_acceptance(oracle):
    """EOS inside an accepted block ends the row there (:932-934, Scheduler.swift:1215-1227)."""
    sp = oracle.make_sampling(eos=(2,))
    toks, stats, _ = run_oracle(oracle, FAKE_REPEATING, spec(k=4, min_ctx=8), sampling=sp)
    assert toks == [3, 1, 2]


def test_single_row_and_greedy_gates(oracle):
    """canSpeculate (:957-975): no speculation for seeded / sampled rows in the reference mode."""
    sp = oracle.make_sampling(temperature=0.0, seed=5)
    _, stats, _ = run_oracle(oracle, FAKE_REPEATING, spec(k=4, min_ctx=8), sampling=sp)
    assert stats["proposal_batches"] == 0


def test_max_tokens_caps_proposal(oracle):
    """proposalLimit = min(K, remaining - 1) (:876-884): the step never overshoots maxTokens."""
    for mt in range(1, 9):
        toks, _, _ = run_oracle(oracle, FAKE_REPEATING, spec(k=4, min_ctx=8), max_tokens=mt)
        assert toks == [3, 1, 2, 3, 1, 2, 3, 1, 2, 3][:mt]


def test_trim_known_answer(oracle):
    """BatchCacheShapeTests.testTrimKeepsMixedLengthSequenceRowsConsistent (:170-195): rows of
    length 2 and 5 merged left-padded, trim(4) -> 4, row lengths [0, 1], offsets [0, 1]."""
    import ctypes as C
    import numpy as np
    idx = C.c_int(5)
    lp = np.array([3, 0], dtype=np.int32)
    off = np.array([2, 5], dtype=np.int32)
    n = oracle.lib().or_batch_trim(C.byref(idx), 2, lp.ctypes.data_as(C.c_void_p), off.ctypes.data_as(C.c_void_p), 4)
    assert n == 4
    assert [idx.value - int(lp[0]), idx.value - int(lp[1])] == [0, 1]
    assert off.tolist() == [0, 1]
    # nothing left to trim past the longest row
    n2 = oracle.lib().or_batch_trim(C.byref(idx), 2, lp.ctypes.data_as(C.c_void_p), off.ctypes.data_as(C.c_void_p), 9)
    assert n2 == 1 and idx.value == 0
