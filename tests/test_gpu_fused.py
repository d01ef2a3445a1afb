"""The persistent (single-kernel) verify forward on the GPU against the oracle: logits within
2e-2 abs + 1e-2 rel, the KV it appends, long contexts (many attention blocks), several rows
in one call, and whole speculative steps against the multi-kernel forward."""
import numpy as np
import pytest

from tests._common import (ARCH_QWEN3, LLAMA3_8B_1L, QWEN3_4B_2L, assert_close_bf16, assert_close_bf16_kv,
                           assert_close_bf16_wide, cfg, top2_margin)

pytestmark = pytest.mark.gpu
SEED = 1234
# smallest shape the persistent forward serves: head_dim 128, widths multiples of 256
SMALL_D128 = cfg(ARCH_QWEN3, 2, 256, 4, 2, 128, 512, 4096, 1, 1e6)
SPEC = dict(enabled=1, max_proposal_tokens=5, max_suffix_tokens=3, min_context_tokens=8, acceptance=1,
            single_row_only=0, greedy_only=0)


def pair(hip, oracle, c, rows=1, ctx=256):
    gm = hip.Model(c)
    gm.init_synthetic(SEED)
    gb = hip.Batch(gm, rows, ctx, SPEC)
    om = oracle.Model(c, SEED, ctx, rows)
    return gm, gb, om


@pytest.mark.parametrize("c", [SMALL_D128, QWEN3_4B_2L], ids=["small-d128", "qwen3-4b-2layers"])
def test_fused_verify_matches_oracle(hip, oracle, c):
    gm, gb, om = pair(hip, oracle, c, rows=1, ctx=256)
    assert gb.fused_available()
    wide = c is not SMALL_D128
    om_rev = oracle.Model(c, SEED, 256, 1) if wide else None  # the reordered-oracle floor
    rng = np.random.default_rng(5)
    V = c["vocab"]
    toks = rng.integers(0, V, 40).tolist()
    gb.forward([0], [40], toks, want_logits=False)  # 40 tokens: the multi-kernel forward
    om.forward([0], [40], toks, want_logits=False)
    if wide:
        with oracle.reversed_reduction_order():
            om_rev.forward([0], [40], toks, want_logits=False)
    gb.set_fused(2)
    for width in (6, 1, 8):
        toks = rng.integers(0, V, width).tolist()
        got, want = gb.forward([0], [width], toks), om.forward([0], [width], toks)
        if wide:
            with oracle.reversed_reduction_order():
                alt = om_rev.forward([0], [width], toks)
            assert_close_bf16_wide(got, want, what=f"verify {width}", floor_u16=alt)
        else:
            assert_close_bf16(got, want, what=f"verify {width}")
    assert gb.kv_len(0) == om.kv_len(0) == 40 + 15
    for layer in range(c["n_layers"]):
        for w in (0, 1):
            assert_close_bf16_kv(gb.read_kv(layer, 0, w), om.kv(layer, 0, w), what=f"kv {layer} {w}")


def test_fused_equals_multi_kernel_forward(hip):
    """Both forwards on identical state: same logits to the tolerance, same argmax where clear."""
    gm = hip.Model(QWEN3_4B_2L)
    gm.init_synthetic(SEED)
    a, b = hip.Batch(gm, 1, 256, SPEC), hip.Batch(gm, 1, 256, SPEC)
    rng = np.random.default_rng(6)
    p = rng.integers(0, 151936, 50).tolist()
    a.forward([0], [50], p, want_logits=False)
    b.forward([0], [50], p, want_logits=False)
    a.set_fused(2)
    b.set_fused(0)
    blk = rng.integers(0, 151936, 6).tolist()
    la, lb = a.forward([0], [6], blk), b.forward([0], [6], blk)
    assert_close_bf16_wide(la, lb, what="fused vs multi-kernel")
    for j in range(6):
        if top2_margin(lb[j]) > 0.05:
            fa = (la[j].astype(np.uint32) << 16).view(np.float32)
            fb = (lb[j].astype(np.uint32) << 16).view(np.float32)
            assert int(np.argmax(fa)) == int(np.argmax(fb))


def test_fused_long_context_many_blocks(hip, oracle):
    """~1000 cached positions: 16 key chunks over several blocks and partials per (row, kv head)."""
    gm, gb, om = pair(hip, oracle, SMALL_D128, rows=1, ctx=1200)
    gb.fill_synthetic_kv(0, 1000, 77)
    om.fill_kv(0, 1000, 77)
    gb.set_fused(2)
    rng = np.random.default_rng(7)
    for width in (6, 3):
        toks = rng.integers(0, 4096, width).tolist()
        assert_close_bf16(gb.forward([0], [width], toks), om.forward([0], [width], toks), what=f"long verify {width}")
    for layer in range(2):
        for w in (0, 1):
            assert_close_bf16_kv(gb.read_kv(layer, 0, w), om.kv(layer, 0, w), what=f"kv {layer} {w}")


def test_fused_several_rows(hip, oracle):
    """Three rows of different lengths and widths in one persistent launch (7 tokens)."""
    gm, gb, om = pair(hip, oracle, SMALL_D128, rows=3, ctx=400)
    rng = np.random.default_rng(8)
    lens = [30, 9, 21]
    toks = rng.integers(0, 4096, sum(lens)).tolist()
    gb.forward([0, 1, 2], lens, toks, want_logits=False)
    om.forward([0, 1, 2], lens, toks, want_logits=False)
    gb.fill_synthetic_kv(2, 300, 5)  # row 2: a longer cached context
    om.fill_kv(2, 300, 5)
    gb.set_fused(2)
    for rows, widths in (([0, 1, 2], [3, 1, 3]), ([2, 0], [4, 4])):
        toks = rng.integers(0, 4096, sum(widths)).tolist()
        assert_close_bf16(gb.forward(rows, widths, toks), om.forward(rows, widths, toks), what=f"rows {rows}")
    for r in range(3):
        assert gb.kv_len(r) == om.kv_len(r)


def test_fused_steps_match_multi_kernel_steps(hip):
    """Greedy speculative steps (drafts from copied spans) with either forward, replayed from
    the captured step graph: same tokens.  The prompt's prefill (300 tokens) takes the
    multi-kernel forward in both; the last step runs with profiling on to show which
    forward served the verify blocks."""
    from mlxcat_amd.workloads import copy_span_prompt

    gm = hip.Model(QWEN3_4B_2L)
    gm.init_synthetic(SEED)
    prompt = copy_span_prompt(9, 300, 151936)
    outs, fused_launches = [], []
    for mode in (1, 0):
        b = hip.Batch(gm, 1, 512, SPEC)
        b.set_fused(mode)
        b.insert(0, prompt, 200, hip.make_sampling())  # 12 steps emit at most 72 tokens
        toks = []
        for i in range(12):
            b.set_profiling(i == 11)
            t, n, _f = b.step()
            toks += t[0][: n[0]].tolist()
        fused_launches.append(b.profile(3)[2])
        outs.append(toks)
    assert outs[0] == outs[1]
    assert fused_launches[0] >= 1 and fused_launches[1] == 0


def test_fused_unavailable_shapes_fall_back(hip):
    """hidden 4096 exceeds one work unit's K-range: the multi-kernel forward serves it and
    requiring the persistent forward is refused."""
    gm = hip.Model(LLAMA3_8B_1L)
    gm.init_synthetic(SEED)
    b = hip.Batch(gm, 1, 128, SPEC)
    assert not b.fused_available()
    with pytest.raises(hip.HipError):
        b.set_fused(2)
