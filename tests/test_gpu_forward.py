"""The verify forward on the GPU against the oracle (bf16 logits within 2e-2 abs + 1e-2 rel),
and the M-invariance the acceptance relies on (bit for bit)."""
import numpy as np
import pytest

from tests._common import (LLAMA3_8B_1L, QWEN3_30B_A3B_1L, QWEN3_4B_2L, QWEN3_8B_1L_V4K, TINY, TINY_LLAMA, TINY_MOE,
                           assert_close_bf16,
                           assert_close_bf16_kv, assert_close_bf16_wide, inside_fraction)

pytestmark = pytest.mark.gpu
SEED = 1234


def pair(hip, oracle, cfg, rows=1, ctx=256, k=8):
    gm = hip.Model(cfg)
    gm.init_synthetic(SEED)
    gb = hip.Batch(gm, rows, ctx, dict(enabled=1, max_proposal_tokens=k, max_suffix_tokens=3, min_context_tokens=8,
                                       acceptance=1, single_row_only=0, greedy_only=0))
    om = oracle.Model(cfg, SEED, ctx, rows)
    return gm, gb, om


@pytest.mark.parametrize("cfg", [TINY, TINY_LLAMA, TINY_MOE], ids=["qwen3", "llama", "qwen3-moe"])
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


def _rows_block_vs_oracle(hip, oracle, cfg, rows, ctx, prefill, width, seed):
    """Uneven prefills of `rows` rows, then one verify block of `width` tokens per row,
    against the oracle with the reordered-oracle floor."""
    gm, gb, om = pair(hip, oracle, cfg, rows=rows, ctx=ctx, k=width - 1)
    om_rev = oracle.Model(cfg, SEED, ctx, rows)
    rng = np.random.default_rng(seed)
    V = cfg["vocab"]
    lens = [int(x) for x in rng.integers(prefill // 2, prefill + 1, rows)]
    toks = rng.integers(0, V, sum(lens)).tolist()
    # prefill in calls of at most 64 tokens
    done = [0] * rows
    while any(d < n for d, n in zip(done, lens)):
        rs, cs, ts, budget = [], [], [], 64
        for r in range(rows):
            k = min(lens[r] - done[r], budget)
            if k > 0:
                off = sum(lens[:r]) + done[r]
                rs.append(r); cs.append(k); ts += toks[off:off + k]
                done[r] += k
                budget -= k
            if budget == 0:
                break
        gb.forward(rs, cs, ts, want_logits=False)
        om.forward(rs, cs, ts, want_logits=False)
        with oracle.reversed_reduction_order():
            om_rev.forward(rs, cs, ts, want_logits=False)
    vt = rng.integers(0, V, width * rows).tolist()
    with oracle.reversed_reduction_order():
        alt = om_rev.forward(list(range(rows)), [width] * rows, vt)
    assert_close_bf16_wide(gb.forward(list(range(rows)), [width] * rows, vt), om.forward(list(range(rows)), [width] * rows, vt),
                           what=f"verify of {rows} x {width}", floor_u16=alt)
    for r in range(rows):
        assert gb.kv_len(r) == om.kv_len(r)


def test_batch8_llama3_8b_shape_matches_oracle(hip, oracle):
    """8 rows x K+1 = 5 tokens (M = 40): the multi-row GEMV at the Llama-3-8B shapes."""
    _rows_block_vs_oracle(hip, oracle, LLAMA3_8B_1L, rows=8, ctx=96, prefill=40, width=5, seed=4)


def test_m288_qwen3_8b_shape_matches_oracle(hip, oracle):
    """32 rows x K+1 = 9 tokens (M = 288, five launches of at most 64 rows) at the Qwen3-8B
    layer shapes."""
    _rows_block_vs_oracle(hip, oracle, QWEN3_8B_1L_V4K, rows=32, ctx=48, prefill=16, width=9, seed=5)


def test_moe_full_shape_matches_oracle(hip, oracle):
    """The Qwen3-30B-A3B-shape verify block of 4 rows x 5 tokens (M = 20): the grouped
    expert GEMVs over 128 experts, top-8, and the GQA-8 attention, after uneven prefills."""
    cfg = QWEN3_30B_A3B_1L
    rows = 4
    gm, gb, om = pair(hip, oracle, cfg, rows=rows, ctx=160)
    om_rev = oracle.Model(cfg, SEED, 160, rows)
    rng = np.random.default_rng(3)
    V = cfg["vocab"]
    lens = [30, 12, 17, 5]
    toks = rng.integers(0, V, sum(lens)).tolist()
    gb.forward(list(range(rows)), lens, toks, want_logits=False)
    om.forward(list(range(rows)), lens, toks, want_logits=False)
    with oracle.reversed_reduction_order():
        om_rev.forward(list(range(rows)), lens, toks, want_logits=False)
    toks = rng.integers(0, V, 5 * rows).tolist()
    with oracle.reversed_reduction_order():
        alt = om_rev.forward(list(range(rows)), [5] * rows, toks)
    got = gb.forward(list(range(rows)), [5] * rows, toks)
    want = om.forward(list(range(rows)), [5] * rows, toks)
    # Routing near-ties: bf16 router logits of 128 experts often tie within an ulp at the
    # top-8 boundary, so any change of summation order (the reordered oracle included)
    # flips some token's expert set, and that token's logits diverge as a whole.  Tokens
    # are classified by the fraction of their logits within the bound; the agreeing ones
    # are held to the full-width criterion, the diverging ones counted against the
    # reordered oracle's own count.
    frac_got = [inside_fraction(got[t], want[t]) for t in range(len(toks))]
    frac_alt = [inside_fraction(alt[t], want[t]) for t in range(len(toks))]
    div_got = [t for t, f in enumerate(frac_got) if f < 0.99]
    div_alt = [t for t, f in enumerate(frac_alt) if f < 0.99]
    assert len(div_got) <= len(div_alt) + 3, (div_got, div_alt, [round(f, 3) for f in frac_got])
    keep = [t for t in range(len(toks)) if t not in div_got and t not in div_alt]
    assert len(keep) >= len(toks) // 2
    assert_close_bf16_wide(got[keep], want[keep], what="moe verify (agreeing tokens)", floor_u16=alt[keep])
    for r in range(rows):
        assert gb.kv_len(r) == om.kv_len(r)


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


def test_fused_attention_many_new_keys(hip, oracle):
    """A 30-token call of the tiny model (GQA 2: 60 queries per kv head) takes the fused
    attention path, whose blocks append more new keys than one batch of their waves (16)
    covers; its logits and every appended key and value against the oracle."""
    gm, gb, om = pair(hip, oracle, TINY, rows=1, ctx=256)
    rng = np.random.default_rng(7)
    for n in (30, 6, 29):
        toks = rng.integers(0, 4096, n).tolist()
        assert_close_bf16(gb.forward([0], [n], toks), om.forward([0], [n], toks), what=f"call of {n}")
    assert gb.kv_len(0) == om.kv_len(0) == 65
    for layer in range(TINY["n_layers"]):
        for w in (0, 1):
            assert_close_bf16_kv(gb.read_kv(layer, 0, w), om.kv(layer, 0, w), what=f"kv {layer} {w}")
