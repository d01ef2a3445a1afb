"""The sampler options on the GPU (logit bias, min_tokens, repetition / presence / frequency
penalties, top-k, min-p with top-p and temperature) and caller-supplied uniforms, through
mc_accept and mc_step, against the reference's known answers and the oracle bit for bit."""
import numpy as np
import pytest

from tests._common import FAKE_REPEATING, TINY, f32_to_bf16, spec
from tests.test_gpu_step import PROMPT, _oracle_run, gen_gpu

pytestmark = pytest.mark.gpu
KA_LOGITS = np.array([[0, 4, 5, 1, -1, 3], [2, 1, 0, 6, 4, 3], [1, 3, 2, 0, 5, 4], [5, 0, 1, 2, 3, 4]], dtype=np.float32)
KA_HISTORIES = [[2, 2, 5], [3, 4], [4, 4, 4], [0, 5]]


def test_known_answers_through_mc_accept(hip):
    """BatchSamplingTests.swift:6-47 ([2, 3, 5, 0]) and :49-70 ([2, 3, 4, 0])."""
    rows = [f32_to_bf16(KA_LOGITS[r])[None, :] for r in range(4)]
    sp = hip.make_sampling(temperature=0.0, repetition_penalty=1.2, presence_penalty=0.4, frequency_penalty=0.3,
                           logit_bias={2: 1.5}, eos=[5])
    got, _, _ = hip.accept(rows, [[]] * 4, [sp] * 4, [0] * 4, 1, generated=KA_HISTORIES)
    assert [g[0] for g in got] == [2, 3, 5, 0]
    for counter in (0, 1, 17, 123456):
        sp = hip.make_sampling(temperature=1.0, top_k=1, seed=counter)
        got, _, _ = hip.accept(rows, [[]] * 4, [sp] * 4, [counter] * 4, 1)
        assert [g[0] for g in got] == [2, 3, 4, 0]


def _random_case(rng, V, hip, oracle, r):
    P = int(rng.integers(0, 6))
    lg = f32_to_bf16((np.round(rng.standard_normal((P + 1, V)) * 4) / 4).astype(np.float32))  # ties
    lg[:, :12] = f32_to_bf16((rng.integers(8, 20, (P + 1, 12)) * 0.5).astype(np.float32))  # a strong head
    drafts = [int(rng.integers(0, 12 if rng.integers(0, 2) else 40)) for _ in range(P)]
    gen = rng.integers(0, 12, int(rng.integers(0, 16))).tolist()
    kw = dict(temperature=float(rng.choice([0.0, 0.7, 1.0, 1.5])), top_p=float(rng.choice([0.0, 0.9, 0.5])),
              top_k=int(rng.choice([0, 1, 5, 50])), min_p=float(rng.choice([0.0, 0.05, 0.3])),
              repetition_penalty=float(rng.choice([1.0, 1.3, 0.8])),
              presence_penalty=float(rng.choice([0.0, 0.5])), frequency_penalty=float(rng.choice([0.0, 0.25])),
              eos=tuple(int(x) for x in rng.integers(0, 12, int(rng.integers(0, 3)))),
              logit_bias={int(t): float(rng.choice([2.5, -1.75])) for t in rng.integers(0, 40, int(rng.integers(0, 4)))},
              seed=5000 + r)
    if rng.integers(0, 2):
        kw["min_tokens"] = len(gen) + int(rng.integers(0, 4))
    return lg, drafts, gen, kw


@pytest.mark.parametrize("V", [4096, 151936])
def test_sampler_options_match_oracle(hip, oracle, V):
    """Random sampler options, generated histories and drafts: mc_accept against or_accept_row,
    with derived and with caller uniforms, under both greedy acceptance rules."""
    rng = np.random.default_rng(V + 1)
    n = 24
    cases = [_random_case(rng, V, hip, oracle, r) for r in range(n)]
    rows = [c[0] for c in cases]
    drafts = [c[1] for c in cases]
    gens = [c[2] for c in cases]
    ctrs = [int(rng.integers(0, 1000)) for _ in range(n)]
    uni = [rng.integers(0, 2 ** 32, (len(c[1]) + 1, 2), dtype=np.uint64).astype(np.uint32) for c in cases]
    for acceptance in (0, 1):
        for use_u in (False, True):
            sps = [hip.make_sampling(**c[3]) for c in cases]
            got, keep, nacc = hip.accept(rows, drafts, sps, ctrs, acceptance, generated=gens,
                                         uniforms=uni if use_u else None)
            for r in range(n):
                osp = oracle.make_sampling(**cases[r][3])
                want, wkeep, wnacc, _ = oracle.accept_row(rows[r], drafts[r], osp, cases[r][3]["seed"], ctrs[r],
                                                          acceptance, generated=gens[r],
                                                          uniforms=uni[r] if use_u else None)
                assert (got[r], keep[r], nacc[r]) == (want, wkeep, wnacc), (r, acceptance, use_u, cases[r][3])


def test_caller_uniforms_equal_to_derived_change_nothing(hip, oracle):
    rng = np.random.default_rng(9)
    V, n = 4096, 8
    rows, drafts, sps, ctrs, uni = [], [], [], [], []
    L = oracle.lib()
    for r in range(n):
        P = int(rng.integers(1, 6))
        rows.append(f32_to_bf16(rng.standard_normal((P + 1, V)).astype(np.float32)))
        drafts.append(rng.integers(0, V, P).tolist())
        sps.append(hip.make_sampling(temperature=0.9, top_p=0.95, seed=40 + r))
        ctrs.append(r * 3)
        uni.append(np.array([[L.or_uniform_u32(40 + r, r * 3, j, k) for k in (0, 1)] for j in range(P + 1)],
                            dtype=np.uint32))
    assert hip.accept(rows, drafts, sps, ctrs, 1) == hip.accept(rows, drafts, sps, ctrs, 1, uniforms=uni)


def test_step_uniforms(hip, oracle):
    """mc_step with caller uniforms: the derived ones reproduce the default step; all-zero
    uniforms accept every draft that has mass."""
    from mlxcat_amd.workloads import motif_prompt
    sp_cfg = spec(k=4, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=0)
    prompts = [motif_prompt(3 + r, 96, 4096).tolist() for r in range(3)]
    L = oracle.lib()

    def run(mode):
        m = hip.Model(TINY)
        m.init_synthetic(1234)
        b = hip.Batch(m, 3, 256, sp_cfg)
        for r, p in enumerate(prompts):
            b.insert(r, p, 40, hip.make_sampling(temperature=0.8, seed=11 + r))
        outs = []
        for step in range(6):
            counter = step + 1  # the first token at admission drew with counter 0
            if mode == "derived":
                u = np.array([[[L.or_uniform_u32(11 + r, counter, j, k) for k in (0, 1)] for j in range(5)]
                              for r in range(3)], dtype=np.uint32)
            elif mode == "zero":
                u = np.zeros((3, 5, 2), dtype=np.uint32)
            else:
                u = None
            t, c, f = b.step(uniforms=u)
            outs.append([t[r, :c[r]].tolist() for r in range(3)])
        return outs, b.stats()

    base, st0 = run("none")
    same, st1 = run("derived")
    assert same == base and st0 == st1
    _, stz = run("zero")
    assert stz["proposed"] > 0 and stz["accepted"] == stz["proposed"]


def test_step_sampler_options_match_oracle(hip, oracle):
    """mc_step rows with logit bias, min_tokens, penalties and sampled ties on the reference's
    fake model (exact logits), against the oracle generator token for token."""
    sp_cfg = spec(k=4, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=0)
    kinds = [
        dict(logit_bias={3: 45.0}),                                        # token 3 always wins
        dict(min_tokens=5, eos=(3,)),                                      # EOS 3 masked for 5 tokens
        dict(presence_penalty=45.0),                                       # generated tokens lose
        dict(temperature=1.0, presence_penalty=40.0, top_k=2, seed=21),    # sampled among ties
        dict(temperature=0.7, presence_penalty=40.0, min_p=0.5, seed=22),
        dict(repetition_penalty=3.0, frequency_penalty=7.0, eos=(2,), min_tokens=2),
    ]
    mt = [14] * len(kinds)
    sps = [hip.make_sampling(**k) for k in kinds]
    osps = [oracle.make_sampling(**k) for k in kinds]
    prompts = [PROMPT] * len(kinds)
    got, st, _, _, _ = gen_gpu(hip, FAKE_REPEATING, sp_cfg, prompts, mt, samplings=sps)
    want, ost = _oracle_run(oracle, FAKE_REPEATING, sp_cfg, prompts, mt, osps)
    assert got == want
    assert st == ost
    assert got[0] == [3] * 14
    assert 3 not in got[1][:5]
