"""The oracle's building blocks against closed forms, library routines and brute force."""
import math

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from tests._common import bf16_to_f32, f32_to_bf16


# ---------------------------------------------------------------------------
# numeric helpers
# ---------------------------------------------------------------------------
def test_exp_neg_matches_libm(oracle):
    L = oracle.lib()
    xs = np.concatenate([-np.logspace(-8, math.log10(80), 4000), np.linspace(-30, 0, 3001)])
    for x in xs:
        got = L.or_exp_neg(float(np.float32(x)))
        want = math.exp(float(np.float32(x)))
        if want < 2.0 ** -40:  # flushed to zero: such masses round to 0 in 2^32 units anyway
            assert got == 0.0 or abs(got - want) <= 2e-5 * want
            continue
        # float range reduction y = x log2(e) carries ~|y| 2^-24 absolute error into the result
        assert abs(got - want) <= (3.0 + 1.5 * abs(x)) * 1.2e-7 * want + 1e-38, (x, got, want)
    assert L.or_exp_neg(0.0) == 1.0
    assert L.or_exp_neg(-100.0) == 0.0
    assert L.or_exp_neg(float("-inf")) == 0.0


def test_exp_neg_monotone(oracle):
    L = oracle.lib()
    xs = np.float32(np.linspace(-25, 0, 200001))
    ys = np.array([L.or_exp_neg(float(x)) for x in xs[::7]])
    assert np.all(np.diff(ys) >= 0)


def test_bf16_round_to_nearest_even(oracle):
    L = oracle.lib()
    cases = {1.0: 0x3F80, -2.0: 0xC000, 1.00390625: 0x3F80, 1.01171875: 0x3F82, 3.0e38: 0x7F62,
             float("inf"): 0x7F80}
    for v, h in cases.items():
        assert L.or_f32_to_bf16(v) == h, v
    rng = np.random.default_rng(0)
    x = rng.standard_normal(10000).astype(np.float32) * 10
    got = np.array([L.or_f32_to_bf16(float(v)) for v in x[:500]], dtype=np.uint16)
    np.testing.assert_array_equal(got, f32_to_bf16(x[:500]))
    # torch's bf16 cast rounds to nearest even as well
    import torch
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
    np.testing.assert_array_equal(f32_to_bf16(x), t)


# ---------------------------------------------------------------------------
# MLX 4-bit affine g64 format
# ---------------------------------------------------------------------------
def numpy_dequant(wq, s, b):
    N, KW = wq.shape
    q = np.zeros((N, KW * 8), dtype=np.float64)
    for j in range(8):
        q[:, j::8] = (wq >> np.uint32(4 * j)) & np.uint32(0xF)
    sc = np.repeat(bf16_to_f32(s).astype(np.float64), 64, axis=1)
    bi = np.repeat(bf16_to_f32(b).astype(np.float64), 64, axis=1)
    return sc * q + bi


def test_packing_known_answer(oracle):
    """Element j of a word sits at bits 4j: 0x76543210 dequantises to 0..7 with s=1, b=0."""
    wq = np.full((1, 8), 0x76543210, dtype=np.uint32)
    s = np.full((1, 1), 0x3F80, dtype=np.uint16)
    b = np.zeros((1, 1), dtype=np.uint16)
    x = np.eye(64, dtype=np.float32)
    y = oracle.qmatmul(wq, s, b, x)
    np.testing.assert_array_equal(y[:, 0], np.tile(np.arange(8, dtype=np.float32), 8))


@pytest.mark.parametrize("N,K,M", [(48, 128, 1), (130, 256, 6), (64, 704, 5)])
def test_qmatmul_vs_numpy(oracle, N, K, M):
    wq, s, b = oracle.gen_linear(11, 3, N, K)
    W = numpy_dequant(wq, s, b)
    rng = np.random.default_rng(N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    got = oracle.qmatmul(wq, s, b, x)
    want = x.astype(np.float64) @ W.T
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_synthetic_weight_statistics(oracle):
    """Random-init weights: mean ~0, std ~0.02 (N(0, 0.02) in 4-bit affine g64)."""
    wq, s, b = oracle.gen_linear(1, 7, 512, 1024)
    W = numpy_dequant(wq, s, b)
    assert abs(W.mean()) < 2e-3
    assert 0.015 < W.std() < 0.025


# ---------------------------------------------------------------------------
# n-gram proposer (BatchGenerator.swift:982-1010)
# ---------------------------------------------------------------------------
def literal_propose(ctx, max_suffix, min_ctx, limit):
    """The reference's nested loop, line for line in Python."""
    if len(ctx) < min_ctx or limit <= 0:
        return None
    n = len(ctx)
    max_len = min(max_suffix, n - 1)
    if max_len <= 0:
        return None
    for L in range(max_len, 0, -1):
        s0 = n - L
        suffix = ctx[s0:]
        if s0 <= 0:
            continue
        for c in range(s0 - 1, -1, -1):
            e = c + L
            if e > s0:
                continue
            if ctx[c:e] == suffix:
                pe = min(n, e + limit)
                if e >= pe:
                    continue
                return ctx[e:pe]
    return None


def lexmax_propose(ctx, max_suffix, min_ctx, limit):
    """Closed form: the proposal starts at the end e maximising (l(e), e), where l(e) is the
    backward match length at e capped by max_suffix, e and n - e."""
    n = len(ctx)
    if n < min_ctx or limit <= 0 or min(max_suffix, n - 1) <= 0:
        return None
    best = None
    for e in range(1, n):
        cap = min(max_suffix, n - 1, e, n - e)
        l = 0
        while l < cap and ctx[e - 1 - l] == ctx[n - 1 - l]:
            l += 1
        if l > 0 and (best is None or (l, e) > best):
            best = (l, e)
    return None if best is None else ctx[best[1]:best[1] + limit]


@settings(max_examples=400, deadline=None)
@given(ctx=st.lists(st.integers(0, 3), min_size=0, max_size=40), max_suffix=st.integers(1, 6),
       min_ctx=st.integers(2, 10), limit=st.integers(0, 6))
def test_ngram_brute_force(oracle, ctx, max_suffix, min_ctx, limit):
    want = literal_propose(ctx, max_suffix, min_ctx, limit)
    assert (lexmax_propose(ctx, max_suffix, min_ctx, limit) or None) == want
    got = oracle.ngram_propose(ctx, max_suffix, min_ctx, limit)
    assert got == (want or [])


def test_ngram_known_answers(oracle):
    # longest suffix wins over a more recent shorter one; the latest occurrence wins among equals
    assert oracle.ngram_propose([5, 6, 7, 9, 6, 7, 1, 5, 6, 7], 3, 2, 4) == [9, 6, 7, 1]
    assert oracle.ngram_propose([1, 2, 3, 1, 2, 3, 1, 2, 3], 16, 8, 4) == [1, 2, 3]
    # below minContext: nil
    assert oracle.ngram_propose([1, 1, 1], 3, 4, 4) == []
    # the proposal may run into the suffix region and be shorter than the limit
    assert oracle.ngram_propose([4, 4, 4, 4], 1, 2, 5) == [4]


# ---------------------------------------------------------------------------
# top-p (Sampling.swift:847-858) known answers, TopPSamplingTests.swift:10-53
# ---------------------------------------------------------------------------
def kept(oracle, probs, top_p):
    lg = f32_to_bf16(np.log(np.asarray(probs, dtype=np.float64)).astype(np.float32))
    d = oracle.dist_build(lg, 1.0, top_p)
    L = oracle.lib()
    import ctypes as C
    return [L.or_dist_mass(C.byref(d), lg.ctypes.data_as(C.c_void_p), 1.0, i) > 0 for i in range(len(probs))]


def test_top_p_keeps_top_token_at_tiny_thresholds(oracle):
    with np.errstate(divide="ignore"):
        for tp in [1e-8, 1e-6, 1e-4, 1e-3]:
            assert kept(oracle, [0.9, 0, 0, 0.1], tp) == [True, False, False, False]


def test_top_p_keeps_nucleus(oracle):
    assert kept(oracle, [0.5, 0.3, 0.15, 0.05], 0.7) == [True, True, False, False]


def test_top_p_never_masks_every_token(oracle):
    rng = np.random.default_rng(0)
    for row in range(2):
        lg = f32_to_bf16((rng.standard_normal(4096) * 3).astype(np.float32))
        for tp in [1e-8, 1e-6, 1e-4, 1e-3]:
            d = oracle.dist_build(lg, 1.0, tp)
            assert d.total > 0 and d.tau == bf16_to_f32(lg).max()


# ---------------------------------------------------------------------------
# speculative sampling (Leviathan et al. 2023; one-hot n-gram draft)
# ---------------------------------------------------------------------------
def target_probs(lg_u16, T, top_p):
    v = bf16_to_f32(lg_u16).astype(np.float64)
    p1 = np.exp(v - v.max())
    p1 /= p1.sum()
    keep = np.ones_like(v, dtype=bool)
    if 0 < top_p < 1:
        order = np.argsort(-v, kind="stable")
        keep[:] = False
        above = 0.0
        for i in order:
            if above >= top_p:
                # ties of the last kept value are kept
                if v[i] < v[order[0]] and not np.isclose(v[i], thr):
                    break
            thr = v[i]
            keep[i] = True
            above += p1[i]
    pt = np.where(keep, np.exp((v - v.max()) / T), 0.0)
    return pt / pt.sum()


@pytest.mark.parametrize("T,top_p,draft", [(1.0, 0.0, 3), (0.7, 0.0, 0), (0.7, 0.95, 5), (1.3, 0.8, 2)])
def test_speculative_sampling_preserves_target_distribution(oracle, T, top_p, draft):
    """The first emitted token (accepted draft or residual sample) is distributed as p;
    a residual that did not exclude the draft, or a missing accept test, fails this."""
    from scipy.stats import chisquare
    V = 12
    rng = np.random.default_rng(int(T * 10) + draft)
    lg = f32_to_bf16((rng.standard_normal((2, V)) * 1.5).astype(np.float32))
    p = target_probs(lg[0], T, top_p)
    sp = oracle.make_sampling(temperature=T, top_p=top_p, seed=0)
    n = 20000
    counts = np.zeros(V)
    for c in range(n):
        out, keep, nacc, rej = oracle.accept_row(lg, [draft], sp, 1234, c, 1)
        counts[out[0]] += 1
    nz = p > 0
    assert counts[~nz].sum() == 0
    stat, pv = chisquare(counts[nz], p[nz] * n)
    assert pv > 1e-4, (pv, counts, p * n)


def test_accept_rules_known_answers(oracle):
    V = 8

    def onehot(toks):
        lg = np.full((len(toks), V), int(f32_to_bf16(np.float32(-20.0))), dtype=np.uint16)
        for i, t in enumerate(toks):
            lg[i, t] = int(f32_to_bf16(np.float32(20.0)))
        return lg

    g = oracle.make_sampling()
    # all agree: P drafts + bonus, keep P + 1
    assert oracle.accept_row(onehot([1, 2, 3, 4]), [1, 2, 3], g, 0, 0, 0) == ([1, 2, 3, 4], 4, 3, 0)
    # reference rule: mismatch at position 1 -> discard the block, one-token decode of position 0
    assert oracle.accept_row(onehot([1, 5, 3, 4]), [1, 2, 3], g, 0, 0, 0) == ([1], 1, 0, 1)
    # prefix rule: keep the agreeing prefix and emit the correction
    assert oracle.accept_row(onehot([1, 5, 3, 4]), [1, 2, 3], g, 0, 0, 1) == ([1, 5], 2, 1, 1)
    # forced cap of 1 accepted draft
    assert oracle.accept_row(onehot([1, 2, 3, 4]), [1, 2, 3], g, 0, 0, 1, 1) == ([1, 2], 2, 1, 1)
    # EOS inside the block
    e = oracle.make_sampling(eos=(2,))
    assert oracle.accept_row(onehot([1, 2, 3, 4]), [1, 2, 3], e, 0, 0, 0) == ([1, 2], 4, 1, 0)
    assert oracle.accept_row(onehot([1, 2, 3, 4]), [1, 2, 3], e, 0, 0, 1) == ([1, 2], 3, 2, 1)
    # ties: lowest index wins
    tie = np.zeros((1, V), dtype=np.uint16)
    assert oracle.accept_row(tie, [], g, 0, 0, 0) == ([0], 1, 0, 0)
