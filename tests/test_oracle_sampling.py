"""The oracle's sampler options (logit bias, min_tokens, repetition / presence / frequency
penalties, top-k, min-p, with top-p and temperature) against the reference's known answers
(Tests/MLXCatTests/BatchSamplingTests.swift:6-47 and :49-70), closed forms, brute force
over small vocabularies, and the sampled distribution."""
import math

import numpy as np
import pytest

from tests._common import bf16_to_f32, f32_to_bf16

# BatchSamplingTests.swift:17-22: four rows of six logits
KA_LOGITS = np.array([[0, 4, 5, 1, -1, 3], [2, 1, 0, 6, 4, 3], [1, 3, 2, 0, 5, 4], [5, 0, 1, 2, 3, 4]], dtype=np.float32)
KA_HISTORIES = [[2, 2, 5], [3, 4], [4, 4, 4], [0, 5]]  # :23-28


def bf(x):
    return f32_to_bf16(np.asarray(x, dtype=np.float32))


def sample(oracle, logits, sp, generated=(), counter=0, seed=99):
    out, _, _, _ = oracle.accept_row(bf(logits)[None, :], [], sp, seed, counter, 1, generated=generated)
    return out[0]


def test_known_answer_penalties_and_logit_bias(oracle):
    """BatchSamplingTests.swift:6-47: greedy with repetition 1.2, presence 0.4, frequency 0.3
    and bias {2: 1.5}; the reference asserts batch == scalar, whose values are [2, 3, 5, 0]:
    row 0 is [0, 4, 6.5 / 1.2 - 0.4 - 2 * 0.3, 1, -1, 3 / 1.2 - 0.4 - 0.3]."""
    sp = oracle.make_sampling(temperature=0.0, repetition_penalty=1.2, presence_penalty=0.4, frequency_penalty=0.3,
                              logit_bias={2: 1.5}, eos=[5])
    got = [sample(oracle, KA_LOGITS[r], sp, KA_HISTORIES[r]) for r in range(4)]
    assert got == [2, 3, 5, 0]
    # without the penalties the bias alone decides row 0 and 3 differently
    plain = oracle.make_sampling(temperature=0.0, logit_bias={2: 1.5}, eos=[5])
    assert [sample(oracle, KA_LOGITS[r], plain, KA_HISTORIES[r]) for r in range(4)] == [2, 3, 4, 0]


def test_known_answer_top_k_one(oracle):
    """BatchSamplingTests.swift:49-70: temperature 1 with top-k 1 is the argmax, whatever the draws."""
    sp = oracle.make_sampling(temperature=1.0, top_k=1)
    for counter in range(64):
        assert [sample(oracle, KA_LOGITS[r], sp, counter=counter) for r in range(4)] == [2, 3, 4, 0]


def test_processed_values_closed_form(oracle):
    """Each processor on its own, with the arithmetic of Sampling.swift:592-636 in fp32."""
    lg = bf([2.0, -3.0, 0.5, 4.0, -1.0, 1.0])
    f = np.float32
    v = oracle.process_logits(lg, oracle.make_sampling(repetition_penalty=2.0), [0, 1, 1])
    assert v.tolist() == [1.0, -6.0, 0.5, 4.0, -1.0, 1.0]  # v < 0: v * rp, else v / rp; once per token
    v = oracle.process_logits(lg, oracle.make_sampling(presence_penalty=0.5, frequency_penalty=0.25), [3, 3, 3, 5])
    assert v[3] == f(f(4.0) - f(0.5)) - f(3) * f(0.25) and v[5] == f(1.0) - f(0.5) - f(0.25)
    assert v[[0, 1, 2, 4]].tolist() == [2.0, -3.0, 0.5, -1.0]
    v = oracle.process_logits(lg, oracle.make_sampling(logit_bias={1: 10.0, 9: 5.0, -1: 5.0}))
    assert v.tolist() == [2.0, 7.0, 0.5, 4.0, -1.0, 1.0]  # out-of-vocabulary ids ignored
    # no generated tokens: penalties change nothing (Sampling.swift:597)
    v = oracle.process_logits(lg, oracle.make_sampling(repetition_penalty=3.0, presence_penalty=1.0), [])
    assert v.tolist() == bf16_to_f32(lg).tolist()


@pytest.mark.parametrize("n_gen,blocked", [(0, True), (2, True), (3, False), (7, False)])
def test_min_tokens_blocks_eos(oracle, n_gen, blocked):
    """EOS is masked while fewer than min_tokens tokens were generated (:677-684)."""
    lg = [0.0, 1.0, 5.0, 3.0]  # EOS id 2 is the argmax, id 3 the runner-up
    sp = oracle.make_sampling(min_tokens=3, eos=[2])
    assert sample(oracle, lg, sp, [1] * n_gen) == (3 if blocked else 2)
    # without EOS ids there is nothing to mask
    assert sample(oracle, lg, oracle.make_sampling(min_tokens=3), [1] * n_gen) == 2


def test_min_tokens_inside_a_verify_block(oracle):
    """Position j of a verify block has n_gen + j generated tokens: with one generated token and
    min_tokens 3, positions 0 and 1 mask EOS and position 2 does not."""
    lg = np.tile(bf([0.0, 1.0, 5.0, 3.0]), (3, 1))
    sp = oracle.make_sampling(min_tokens=3, eos=[2])
    out, keep, nacc, rej = oracle.accept_row(lg, [3, 3], sp, 0, 0, 1, generated=[1])
    assert out == [3, 3, 2] and keep == 3 and nacc == 2 and rej == 0
    out, _, _, _ = oracle.accept_row(lg, [3, 3], sp, 0, 0, 1, generated=[1, 1])
    assert out == [3, 2]  # the draft at position 1 disagrees with the now-unmasked EOS


def test_penalties_see_accepted_drafts(oracle):
    """generatedHistory grows by each accepted token (BatchGenerator.swift:930): a draft accepted
    at position 0 is penalised at position 1."""
    lg = np.tile(bf([0.0, 3.0, 2.9, 0.0]), (2, 1))
    sp = oracle.make_sampling(presence_penalty=0.5)
    out, keep, nacc, _ = oracle.accept_row(lg, [1], sp, 0, 0, 1, generated=[0])
    assert out == [1, 2] and nacc == 1  # 3.0 - 0.5 < 2.9 at position 1
    out, _, _, _ = oracle.accept_row(lg, [1], oracle.make_sampling(), 0, 0, 1, generated=[0])
    assert out == [1, 1]


def test_top_k_keeps_lowest_ids_among_ties(oracle):
    v = np.array([1.0, 3.0, 3.0, 3.0, 0.0], dtype=np.float32)
    d = oracle.dist_build_f(v, 1.0, top_k=2)
    assert oracle.kept_mask(d, v).tolist() == [False, True, True, False, False]
    d = oracle.dist_build_f(v, 1.0, top_k=4)
    assert oracle.kept_mask(d, v).tolist() == [True, True, True, True, False]
    d = oracle.dist_build_f(v, 1.0, top_k=5)  # k >= V: off (Sampling.swift:895)
    assert oracle.kept_mask(d, v).all()


def test_min_p_closed_form(oracle):
    """min-p keeps v - max >= log(min_p) (Sampling.swift:860-863)."""
    v = np.array([0.0, -1.0, -2.0, -3.0, -10.0], dtype=np.float32)
    for min_p, want in [(0.3, [1, 1, 0, 0, 0]), (math.exp(-2.5), [1, 1, 1, 0, 0]), (1.0, [1, 0, 0, 0, 0]),
                        (1e-4, [1, 1, 1, 1, 0]), (1e-6, [1, 1, 1, 1, 1])]:
        d = oracle.dist_build_f(v, 1.0, min_p=min_p)
        assert oracle.kept_mask(d, v).astype(int).tolist() == want, min_p


def top_p_boundary(v, top_p):
    """Distance of the reference's top-p comparison from its boundary, relative to the total."""
    s = np.sort(v)
    p = np.exp(s - v.max())
    above = np.concatenate([np.cumsum(p[::-1])[::-1][1:], [0.0]])
    return float(np.min(np.abs(above - top_p * p.sum())) / p.sum())


def brute_force_kept(v, top_p, top_k, min_p):
    """The reference's filter chain (Sampling.swift:500-522) in float64: top-p exactly as
    :847-858 (ascending sort, reverse exclusive cumulative mass, drop the positions whose mass
    above reaches top_p of the total, keep values >= the first kept one), min-p on logprobs,
    top-k by value then index."""
    V = len(v)
    keep = np.ones(V, dtype=bool)
    lp = v - (v.max() + np.log(np.exp(v - v.max()).sum()))
    if 0 < top_p < 1:
        s = np.sort(v)
        p = np.exp(s - v.max())
        above = np.concatenate([np.cumsum(p[::-1])[::-1][1:], [0.0]])
        dropped = int((above >= top_p * p.sum()).sum())
        keep &= v >= s[dropped]
    if min_p > 0:
        keep &= lp >= lp.max() + np.log(min_p)
    if 0 < top_k < V:
        order = sorted(range(V), key=lambda i: (-v[i], i))
        topk = np.zeros(V, dtype=bool)
        topk[order[:top_k]] = True
        keep &= topk
    return keep


def test_filters_against_brute_force(oracle):
    rng = np.random.default_rng(3)
    checked = 0
    for trial in range(300):
        V = int(rng.integers(2, 40))
        v = np.round(rng.normal(0, 2, V) * 4) / 4  # quarter steps: ties
        v = bf16_to_f32(bf(v))
        top_p = float(rng.choice([0.0, 0.3, 0.6, 0.9]))
        top_k = int(rng.choice([0, 1, 3, 10]))
        min_p = float(rng.choice([0.0, 0.02, 0.2]))
        want = brute_force_kept(v.astype(np.float64), top_p, top_k, min_p)
        # skip vectors that sit within rounding of a top-p or min-p boundary
        lp = v - v.max()
        if min_p and np.min(np.abs(lp - np.log(min_p))) < 1e-4:
            continue
        if 0 < top_p < 1 and top_p_boundary(v.astype(np.float64), top_p) < 1e-6:
            continue
        d = oracle.dist_build_f(v, 1.0, top_p=top_p, top_k=top_k, min_p=min_p)
        got = oracle.kept_mask(d, v) | (np.exp(lp) < 2 ** -33)  # zero-mass tokens are never drawn
        assert got.tolist() == (want | (np.exp(lp) < 2 ** -33)).tolist(), (v, top_p, top_k, min_p)
        checked += 1
    assert checked > 250


def test_top_k_distribution(oracle):
    """Temperature 0.7, top-k 3: the draws follow softmax(v / T) over the three largest values."""
    v = np.array([1.0, 0.0, 2.0, -1.0, 1.5, 0.5], dtype=np.float32)
    sp = oracle.make_sampling(temperature=0.7, top_k=3)
    n = 6000
    counts = np.bincount([sample(oracle, v, sp, counter=c) for c in range(n)], minlength=6)
    kept = [2, 4, 0]
    p = np.exp(v[kept] / 0.7)
    p /= p.sum()
    assert counts[[1, 3, 5]].sum() == 0
    exp = p * n
    chi2 = float((((counts[kept] - exp) ** 2) / exp).sum())
    assert chi2 < 13.8, (counts, exp)  # 2 dof, p = 0.001


def test_caller_uniforms_replace_derived_ones(oracle):
    """Supplying the derived uniforms explicitly changes nothing; other uniforms change draws."""
    rng = np.random.default_rng(5)
    V, P = 64, 4
    lg = bf(rng.normal(0, 1.5, (P + 1, V)))
    drafts = rng.integers(0, V, P).tolist()
    sp = oracle.make_sampling(temperature=0.9, top_p=0.95, seed=77)
    L = oracle.lib()
    for counter in range(20):
        u = np.array([[L.or_uniform_u32(77, counter, j, k) for k in (0, 1)] for j in range(P + 1)], dtype=np.uint32)
        a = oracle.accept_row(lg, drafts, sp, 77, counter, 1)
        b = oracle.accept_row(lg, drafts, sp, 77, counter, 1, uniforms=u)
        assert a == b
    # u = 0 accepts every draft with mass; u = 2^32 - 1 rejects at the first draft below certainty
    zero = np.zeros((P + 1, 2), dtype=np.uint32)
    out, keep, nacc, _ = oracle.accept_row(lg, drafts, oracle.make_sampling(temperature=1.0), 0, 0, 1, uniforms=zero)
    assert nacc == P and keep == P + 1
    full = np.full((P + 1, 2), 0xFFFFFFFF, dtype=np.uint32)
    out, keep, nacc, _ = oracle.accept_row(lg, drafts, oracle.make_sampling(temperature=1.0), 0, 0, 1, uniforms=full)
    assert nacc == 0 and keep == 1
