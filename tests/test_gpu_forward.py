"""The verify forward on the GPU against the oracle (bf16 logits within 2e-2 abs + 1e-2 rel),
and the M-invariance the acceptance relies on (bit for bit)."""
import numpy as np
import pytest

from tests._common import (LLAMA3_8B_1L, QWEN3_4B_2L, TINY, TINY_LLAMA, assert_close_bf16, assert_close_bf16_kv,
                           assert_close_bf16_wide)

pytestmark = pytest.mark.gpu
SEED = 1234


def pair(hip, oracle, cfg, rows=1, ctx=256, k=8):
    gm = hip.Model(cfg)
    gm.init_synthetic(SEED)
    gb = hip.Batch(gm, rows, ctx, dict(enabled=1, max_proposal_tokens=k, max_suffix_tokens=3, min_context_tokens=8,
                                       acceptance=1, single_row_only=0, greedy_only=0))
    om = oracle.Model(cfg, SEED, ctx, rows)
    return gm, gb, om


@pytest.mark.parametrize("cfg", [TINY, TINY_LLAMA], ids=["qwen3", "llama"])
def test_forward_matches_oracle(hip, oracle, cfg):
    gm, gb, om = pair(hip, oracle, cfg, rows=3)
    rng = np.random.default_rng(0)
    V = cfg["vocab"]
    # prefill of uneven lengths (one call, at most 64 tokens), then verify blocks of mixed widths
    lens = [34, 7, 23]
    toks = rng.integers(0, V, sum(lens)).tolist()
    assert_close_bf16(gb.forward([0, 1, 2], lens, toks), om.forward([0, 1, 2], lens, toks), what="prefill")
    for widths in ([6, 1, 3], [1, 6, 6]):
        toks = rng.integers(0, V, sum(widths)).tolist()
        assert_close_bf16(gb.forward([0, 1, 2], widths, toks), om.forward([0, 1, 2], widths, toks), what="verify")
    for r in range(3):
        assert gb.kv_len(r) == om.kv_len(r)
        for layer in range(cfg["n_layers"]):
            for w in (0, 1):
                assert_close_bf16_kv(gb.read_kv(layer, r, w), om.kv(layer, r, w), what=f"kv {layer} {r} {w}")


@pytest.mark.parametrize("cfg", [QWEN3_4B_2L, LLAMA3_8B_1L], ids=["qwen3-4b-2layers", "llama3-8b-1layer"])
def test_forward_full_shapes_match_oracle(hip, oracle, cfg):
    """Every GEMV shape of the Qwen3-4B / Llama-3-8B verify step (incl. the vocab-sized head)."""
    gm, gb, om = pair(hip, oracle, cfg, rows=2, ctx=160)
    om_rev = oracle.Model(cfg, SEED, 160, 2)  # every reduction reordered: the rounding-noise floor
    rng = np.random.default_rng(1)
    V = cfg["vocab"]
    toks = rng.integers(0, V, 60).tolist()
    gb.forward([0, 1], [40, 20], toks, want_logits=False)
    om.forward([0, 1], [40, 20], toks, want_logits=False)
    with oracle.reversed_reduction_order():
        om_rev.forward([0, 1], [40, 20], toks, want_logits=False)
    toks = rng.integers(0, V, 11).tolist()
    with oracle.reversed_reduction_order():
        alt = om_rev.forward([0, 1], [6, 5], toks)
    assert_close_bf16_wide(gb.forward([0, 1], [6, 5], toks), om.forward([0, 1], [6, 5], toks), what="verify",
                           floor_u16=alt)


def test_forward_long_context_split_kv(hip, oracle):
    """Attention across many 64-key chunks (contiguous KV of 1500 positions)."""
    gm, gb, om = pair(hip, oracle, TINY, rows=1, ctx=1600)
    rng = np.random.default_rng(2)
    for _ in range(24):  # 24 x 62 tokens of prefill
        toks = rng.integers(0, 4096, 62).tolist()
        gb.forward([0], [62], toks, want_logits=False)
        om.forward([0], [62], toks, want_logits=False)
    toks = rng.integers(0, 4096, 6).tolist()
    assert_close_bf16(gb.forward([0], [6], toks), om.forward([0], [6], toks), what="long verify")


def test_verify_logits_are_m_invariant(hip):
    """Position j of a verify block is bit-identical to decoding the same tokens one at a
    time, so the reject path's one-token decode can reuse position 0."""
    gm = hip.Model(TINY)
    gm.init_synthetic(SEED)
    spec = dict(enabled=1, max_proposal_tokens=8, max_suffix_tokens=3, min_context_tokens=8, acceptance=1,
                single_row_only=0, greedy_only=0)
    a, b = hip.Batch(gm, 2, 128, spec), hip.Batch(gm, 2, 128, spec)
    rng = np.random.default_rng(3)
    p = rng.integers(0, 4096, 30).tolist()
    a.forward([0], [30], p, want_logits=False)
    b.forward([0], [30], p, want_logits=False)
    blk = rng.integers(0, 4096, 7).tolist()
    # a: the block alongside another row's tokens; b: one token at a time
    other = rng.integers(0, 4096, 5).tolist()
    la = a.forward([1, 0], [5, 7], other + blk)[5:]
    lb = np.concatenate([b.forward([0], [1], [t]) for t in blk])
    np.testing.assert_array_equal(la, lb)
    for layer in range(2):
        np.testing.assert_array_equal(a.read_kv(layer, 0, 0), b.read_kv(layer, 0, 0))
