"""The verify forward on the GPU against the oracle (bf16 logits within 2e-2 abs + 1e-2 rel),
and the M-invariance the acceptance relies on (bit for bit)."""
import numpy as np
import pytest

from tests._common import (LLAMA3_8B_1L, QWEN3_30B_A3B_1L, QWEN3_4B_2L, QWEN3_8B_1L_V4K, TINY, TINY_LLAMA, TINY_MOE,
                           assert_close_bf16, assert_close_bf16_kv, assert_close_bf16_wide, bf16_to_f32,
                           inside_fraction)

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
    """32 rows x K+1 = 9 tokens (M = 288: the large-M GEMM, split K) at the Qwen3-8B layer
    shapes."""
    _rows_block_vs_oracle(hip, oracle, QWEN3_8B_1L_V4K, rows=32, ctx=48, prefill=16, width=9, seed=5)


def _topk_set(logits_u16, k):
    """Top-k experts of bf16 router logits: value descending, lower index first on ties."""
    v = bf16_to_f32(logits_u16).astype(np.float64)
    return frozenset(np.lexsort((np.arange(len(v)), -v))[:k].tolist())


def _margin_ulps(logits_u16, k):
    """(k-th largest - (k+1)-th largest) router logit, in bf16 ulps of the k-th."""
    v = np.sort(bf16_to_f32(logits_u16).astype(np.float64))[::-1]
    ulp = 2.0 ** (np.floor(np.log2(max(abs(v[k - 1]), 1e-30))) - 7)
    return (v[k - 1] - v[k]) / ulp


def test_moe_full_shape_matches_oracle(hip, oracle):
    """The Qwen3-30B-A3B-shape verify block of 4 rows x 5 tokens (M = 20): the grouped
    expert GEMVs over 128 experts, top-8, and the GQA-8 attention, after uneven prefills.

    Router-margin gate: a token whose GPU top-8 expert set differs from the oracle's is
    excused only if the oracle's 8th/9th router-logit margin is at most one bf16 ulp (a tie
    that any change of summation order may flip); every token routed to the same experts is
    held to the full-width bound."""
    cfg = QWEN3_30B_A3B_1L
    rows, TK = 4, cfg["n_experts_per_tok"]
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
    M = len(toks)
    with oracle.reversed_reduction_order():
        alt, alt_rl = om_rev.forward(list(range(rows)), [5] * rows, toks, router=True)
    got = gb.forward(list(range(rows)), [5] * rows, toks)
    got_rl = gb.read_router(M)
    want, want_rl = om.forward(list(range(rows)), [5] * rows, toks, router=True)
    want_rl, alt_rl = want_rl[-1], alt_rl[-1]
    same, excused = [], []
    for t in range(M):
        ws = _topk_set(want_rl[t], TK)
        if _topk_set(got_rl[t], TK) == ws:
            same.append(t)
            continue
        m = _margin_ulps(want_rl[t], TK)
        assert m <= 1.0, f"token {t}: GPU routes to other experts with an oracle top-{TK} margin of {m:.2f} ulp"
        excused.append(t)
    # the reordering's floor only from tokens the reordered oracle routes like the oracle
    floor = alt.copy()
    for t in range(M):
        if _topk_set(alt_rl[t], TK) != _topk_set(want_rl[t], TK):
            floor[t] = want[t]
    print(f"moe verify: {M} tokens, {len(same)} routed as the oracle, {len(excused)} excused "
          f"(margins {[round(float(_margin_ulps(want_rl[t], TK)), 2) for t in excused]} ulp); "
          f"{inside_fraction(got[same], want[same]):.5f} of their logits inside the bound")
    assert len(same) >= M // 2  # the gate excuses exact ties only; most tokens are compared
    assert_close_bf16_wide(got[same], want[same], what="moe verify (same experts)", floor_u16=floor[same])
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
