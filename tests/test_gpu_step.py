"""The fused speculative step (mc_step: propose, verify forward, accept, rollback, history,
finish) on the GPU, against the reference's known answers, the oracle, and invariants."""
import numpy as np
import pytest

from tests._common import FAKE_MISMATCHING, FAKE_REPEATING, TINY, spec, top2_margin

pytestmark = pytest.mark.gpu
SEED = 1234
PROMPT = [1, 2, 3, 1, 2, 3, 1, 2]


def gen_gpu(hip, model_cfg, spec_cfg, prompts, max_tokens, samplings=None, rows=None, ctx=256, forced=None,
            model=None):
    m = model or hip.Model(model_cfg)
    if model is None:
        m.init_synthetic(SEED)
    R = rows or len(prompts)
    b = hip.Batch(m, R, ctx, spec_cfg)
    out = {r: [] for r in range(len(prompts))}
    for r, p in enumerate(prompts):
        sp = samplings[r] if samplings else hip.make_sampling()
        tok, fin = b.insert(r, p, max_tokens[r] if isinstance(max_tokens, list) else max_tokens, sp)
        out[r].append(tok)
        if fin:
            b.remove(r)
    step = 0
    active = {r for r in range(len(prompts)) if out[r]}
    fins = {}
    while True:
        fa = None if forced is None else forced(step, R)
        t, c, f = b.step(fa)
        step += 1
        if c.sum() == 0:
            break
        for r in range(len(prompts)):
            out[r] += t[r, :c[r]].tolist()
            if f[r]:
                fins[r] = int(f[r])
        if step > 10000:
            raise RuntimeError("runaway")
    return out, b.stats(), b.call_widths(), b, m


@pytest.mark.parametrize("acceptance", [0, 1])
def test_reference_traces(hip, acceptance):
    out, stats, widths, _, _ = gen_gpu(hip, FAKE_REPEATING, spec(k=4, min_ctx=8, acceptance=acceptance), [PROMPT], 10)
    assert out[0] == [3, 1, 2, 3, 1, 2, 3, 1, 2, 3]
    assert stats == dict(proposed=7, accepted=7, proposal_batches=2, rejected_batches=0)
    assert widths == [1, 4, 5]
    out, stats, widths, _, _ = gen_gpu(hip, FAKE_MISMATCHING, spec(k=4, min_ctx=8, acceptance=acceptance), [PROMPT], 10)
    assert out[0] == [3, 4, 1, 2, 3, 4, 1, 2, 3, 4]
    assert stats == dict(proposed=8, accepted=5, proposal_batches=3, rejected_batches=1)


def test_fake_models_match_plain_decode(hip):
    for cfg in (FAKE_REPEATING, FAKE_MISMATCHING):
        base, bst, bw, _, _ = gen_gpu(hip, cfg, spec(enabled=False), [PROMPT], 10)
        sp, sst, sw, _, _ = gen_gpu(hip, cfg, spec(k=4, min_ctx=8), [PROMPT], 10)
        assert sp == base and len(sp[0]) == 10
        assert bst["proposal_batches"] == 0


def test_generator_api_mirrors_reference(hip):
    """Scheduler.submit / step / isIdle and SpeculativeDecodingStats through the host mirror."""
    from mlxcat_amd import generator as G
    m = hip.Model(FAKE_REPEATING)
    sched = G.Scheduler(m, 1, 64, G.SpeculativeDecodingConfiguration(enabled=True, max_proposal_tokens=4,
                                                                      min_context_tokens=8))
    toks = G.generate(sched, [G.Request("repeat", PROMPT, 10)])
    assert toks["repeat"] == [3, 1, 2, 3, 1, 2, 3, 1, 2, 3]
    st = sched.speculative_decoding_stats
    assert st.accepted_token_count == 7 and st.proposal_batch_count == 2


@pytest.mark.parametrize("acceptance", [0, 1])
def test_tiny_speculation_equals_plain_greedy(hip, acceptance):
    """Greedy speculative output is token-identical to plain decoding on the same device path."""
    from mlxcat_amd.workloads import motif_prompt
    prompt = motif_prompt(11, 128, 4096).tolist()
    base, _, _, _, m = gen_gpu(hip, TINY, spec(enabled=False), [prompt], 64)
    sp, st, _, _, _ = gen_gpu(hip, TINY, spec(k=4, max_suffix=3, min_ctx=8, acceptance=acceptance), [prompt], 64,
                              model=m)
    assert sp[0] == base[0]
    assert st["proposal_batches"] > 0


def test_tiny_generation_matches_oracle(hip, oracle):
    """GPU tokens equal the oracle's until the first position where the oracle's top-2 logit
    margin is within bf16 rounding (BatchInvarianceTests.swift:248-253 method)."""
    from mlxcat_amd.workloads import motif_prompt
    prompt = motif_prompt(11, 128, 4096).tolist()
    sp_cfg = spec(k=4, max_suffix=3, min_ctx=8, acceptance=1, single_row_only=0)
    g, _, _, _, _ = gen_gpu(hip, TINY, sp_cfg, [prompt], 64)
    om = oracle.Model(TINY, SEED, 256, 1)
    og = oracle.Generator(om, sp_cfg, 1, 256)
    tok, _ = og.insert(0, prompt, 64, oracle.make_sampling())
    o = [tok]
    while og.active(0):
        t, c, f = og.step()
        o += t[0, :c[0]].tolist()
    if g[0] == o:
        return
    i = next(i for i in range(min(len(g[0]), len(o))) if g[0][i] != o[i])
    # replay the oracle's greedy logits at the divergence: it must be a near-tie
    om2 = oracle.Model(TINY, SEED, 256, 1)
    seq = prompt + o[:i]
    lg = om2.forward([0], [len(seq)], seq)[-1]
    assert top2_margin(lg) <= 0.05, (i, top2_margin(lg))
    assert i >= 8, f"diverged at token {i}"


def test_batched_rows_are_independent(hip):
    """Each row of a mixed batch (greedy and seeded-sampled) emits exactly what it emits alone
    (PerRequestRNGTests.swift:8-41: seeded rows independent of batch composition)."""
    from mlxcat_amd.workloads import copy_span_prompt, motif_prompt
    prompts = [motif_prompt(21, 100, 4096).tolist(), copy_span_prompt(22, 90, 4096).tolist(),
               motif_prompt(23, 60, 4096).tolist(), copy_span_prompt(24, 120, 4096).tolist()]
    sps = [hip.make_sampling(), hip.make_sampling(temperature=0.7, top_p=0.95, seed=5),
           hip.make_sampling(temperature=1.0, seed=6), hip.make_sampling(eos=(17,))]
    sp_cfg = spec(k=3, max_suffix=3, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=0)
    mt = [40, 33, 48, 20]
    m = hip.Model(TINY)
    m.init_synthetic(SEED)
    both, st, _, _, _ = gen_gpu(hip, TINY, sp_cfg, prompts, mt, samplings=sps, model=m)
    assert st["proposal_batches"] > 0
    for r in range(4):
        alone, _, _, _, _ = gen_gpu(hip, TINY, sp_cfg, [prompts[r]], [mt[r]], samplings=[sps[r]], rows=4, model=m)
        assert both[r] == alone[0], r
        assert 1 <= len(both[r]) <= mt[r]


def test_forced_rollback_leaves_no_phantom_kv(hip):
    """A forced accept-length schedule rolls back rejected drafts by length; the surviving
    KV equals the KV of decoding the emitted tokens one at a time."""
    from mlxcat_amd.workloads import motif_prompt
    prompt = motif_prompt(31, 80, 4096).tolist()
    rng = np.random.default_rng(9)
    sched = {}

    def forced(step, R):
        if step not in sched:
            sched[step] = rng.integers(0, 5, R).astype(np.int32)
        return sched[step]

    m = hip.Model(TINY)
    m.init_synthetic(SEED)
    sp_cfg = spec(k=4, max_suffix=3, min_ctx=8, acceptance=1, single_row_only=0)
    out, st, _, b, _ = gen_gpu(hip, TINY, sp_cfg, [prompt], 60, model=m, forced=forced, ctx=256)
    assert st["accepted"] > 0 and st["rejected_batches"] > 0
    hist = b.history(0)
    assert hist == prompt + out[0]
    L = b.kv_len(0)
    # reference: same prompt prefill, then the emitted tokens one at a time
    ref = hip.Batch(m, 1, 256, spec(enabled=False))
    ref.insert(0, prompt, 60, hip.make_sampling())
    for t in hist[len(prompt):L]:
        ref.forward([0], [1], [t], want_logits=False)
    assert ref.kv_len(0) == L
    for layer in range(TINY["n_layers"]):
        for w in (0, 1):
            np.testing.assert_array_equal(b.read_kv(layer, 0, w), ref.read_kv(layer, 0, w))


def test_trim_and_rollback_api(hip):
    """BatchKVCache.trim known answer (BatchCacheShapeTests.swift:170-195) on device rows of
    length 2 and 5, and the per-row rollback."""
    m = hip.Model(TINY)
    m.init_synthetic(SEED)
    b = hip.Batch(m, 2, 64, spec(enabled=False))
    b.forward([0, 1], [2, 5], [1, 2, 3, 4, 5, 6, 7], want_logits=False)
    assert b.trim(4) == 4
    assert [b.kv_len(0), b.kv_len(1)] == [0, 1]
    assert b.trim(9) == 1
    b.forward([0], [3], [1, 2, 3], want_logits=False)
    b.rollback(0, 2)
    assert b.kv_len(0) == 1
    b.rollback(0, 5)
    assert b.kv_len(0) == 0


def test_capacity_errors_are_loud(hip):
    m = hip.Model(TINY)
    m.init_synthetic(SEED)
    b = hip.Batch(m, 1, 32, spec(k=4))
    with pytest.raises(hip.HipError):
        b.insert(0, list(range(1, 30)), 10, hip.make_sampling())
    with pytest.raises(hip.HipError):
        b.forward([0], [40], list(range(40)))


def _oracle_run(oracle, cfg, spec_cfg, prompts, max_tokens, samplings):
    om = oracle.Model(cfg, SEED, 256, len(prompts))
    og = oracle.Generator(om, spec_cfg, len(prompts), 256)
    out = {}
    for r, p in enumerate(prompts):
        tok, _ = og.insert(r, p, max_tokens[r], samplings[r])
        out[r] = [tok]
    while any(og.active(r) for r in range(len(prompts))):
        t, c, f = og.step()
        for r in range(len(prompts)):
            out[r] += t[r, :c[r]].tolist()
    return out, og.stats()


def test_single_row_gate_matches_oracle(hip, oracle):
    """The reference speculates only while exactly one row runs (rowUIDs.count == 1,
    BatchGenerator.swift:959): two active rows make no proposals; once the short row
    finishes, the remaining row speculates.  Tokens and stats equal the oracle's."""
    sp_cfg = spec(k=4, min_ctx=8, acceptance=0, single_row_only=1, greedy_only=1)
    mt = [4, 12]
    got, st, _, _, _ = gen_gpu(hip, FAKE_REPEATING, sp_cfg, [PROMPT, PROMPT], mt)
    want, ost = _oracle_run(oracle, FAKE_REPEATING, sp_cfg, [PROMPT, PROMPT], mt,
                            [oracle.make_sampling(), oracle.make_sampling()])
    assert got == want
    assert st == ost
    assert 0 < st["proposal_batches"]
    # while both rows ran (the first 3 steps) nothing was proposed: every token of the short
    # row came from plain decodes, one per step
    assert len(got[0]) == 4
    both = dict(st)
    alone, st2, _, _, _ = gen_gpu(hip, FAKE_REPEATING, sp_cfg, [PROMPT], [12])
    assert alone[0] == got[1]
    assert both["proposed"] < st2["proposed"]


def test_greedy_gate_matches_oracle(hip, oracle):
    """Rows with temperature > 0 or a seed do not speculate under the reference gate
    (BatchGenerator.swift:963,970); greedy rows beside them do.  Against the oracle."""
    sp_cfg = spec(k=4, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=1)
    mt = [12, 12, 12]
    sps = [hip.make_sampling(), hip.make_sampling(temperature=0.8, seed=3), hip.make_sampling(seed=4)]
    osps = [oracle.make_sampling(), oracle.make_sampling(temperature=0.8, seed=3), oracle.make_sampling(seed=4)]
    got, st, _, _, _ = gen_gpu(hip, FAKE_REPEATING, sp_cfg, [PROMPT] * 3, mt, samplings=sps)
    want, ost = _oracle_run(oracle, FAKE_REPEATING, sp_cfg, [PROMPT] * 3, mt, osps)
    assert got == want
    assert st == ost
    # only the greedy, unseeded row proposes: its two batches, as when it runs alone
    alone, st1, _, _, _ = gen_gpu(hip, FAKE_REPEATING, sp_cfg, [PROMPT], [12])
    assert st["proposal_batches"] == st1["proposal_batches"] > 0
