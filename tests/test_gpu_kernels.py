"""HIP kernels through the C ABI against the oracle: weight layout, n-gram proposer,
acceptance.  Integer and index results are compared bit for bit."""
import numpy as np
import pytest

from tests._common import TINY, TINY_MOE, f32_to_bf16

pytestmark = pytest.mark.gpu
SEED = 1234


def _model(hip, cfg, seed=SEED):
    m = hip.Model(cfg)
    m.init_synthetic(seed)
    return m


def test_synthetic_weights_match_oracle(hip, oracle):
    """The device generator writes exactly the oracle's MLX tensors (checked through the
    lossless export of the tile layout)."""
    gm = _model(hip, TINY)
    om = oracle.Model(TINY, SEED, 16, 1)
    for layer in range(TINY["n_layers"]):
        for which in range(7):
            got = gm.get_linear(layer, which)
            want = om.linear(layer, which)
            for g, w in zip(got, want):
                np.testing.assert_array_equal(g, w, err_msg=f"layer {layer} slot {which}")
    for g, w in zip(gm.get_linear(-1, hip.W_EMBED), om.linear(-1, 0)):
        np.testing.assert_array_equal(g, w)


def test_synthetic_expert_weights_match_oracle(hip, oracle):
    """Qwen3-MoE: the router and every expert's gate / up / down, as the oracle generates them."""
    gm = _model(hip, TINY_MOE)
    om = oracle.Model(TINY_MOE, SEED, 16, 1)
    for layer in range(TINY_MOE["n_layers"]):
        for g, w in zip(gm.get_linear(layer, hip.W_ROUTER), om.linear(layer, 11)):
            np.testing.assert_array_equal(g, w, err_msg=f"router {layer}")
        for e in (0, 5, TINY_MOE["n_experts"] - 1):
            for which in (hip.W_GATE, hip.W_UP, hip.W_DOWN):
                for g, w in zip(gm.get_linear(layer, which, e), om.linear(layer, which, e)):
                    np.testing.assert_array_equal(g, w, err_msg=f"layer {layer} expert {e} slot {which}")
    rng = np.random.default_rng(6)
    N, K = gm._lshape(hip.W_DOWN, 3)
    wq = rng.integers(0, 2**32, (N, K // 8), dtype=np.uint32)
    sc = rng.integers(0, 2**16, (N, K // 64), dtype=np.uint16)
    bi = rng.integers(0, 2**16, (N, K // 64), dtype=np.uint16)
    gm.set_linear(1, hip.W_DOWN, wq, sc, bi, expert=3)
    for g, w in zip(gm.get_linear(1, hip.W_DOWN, 3), (wq, sc, bi)):
        np.testing.assert_array_equal(g, w)
    for g, w in zip(gm.get_linear(1, hip.W_DOWN, 4), om.linear(1, 6, 4)):  # the neighbour is untouched
        np.testing.assert_array_equal(g, w)


def test_set_get_linear_roundtrip(hip):
    gm = _model(hip, TINY)
    rng = np.random.default_rng(5)
    for which in (hip.W_Q, hip.W_K, hip.W_GATE, hip.W_UP, hip.W_DOWN):
        N, K = gm._lshape(which)
        wq = rng.integers(0, 2**32, (N, K // 8), dtype=np.uint32)
        s = rng.integers(0, 2**16, (N, K // 64), dtype=np.uint16)
        b = rng.integers(0, 2**16, (N, K // 64), dtype=np.uint16)
        gm.set_linear(1, which, wq, s, b)
        for g, w in zip(gm.get_linear(1, which), (wq, s, b)):
            np.testing.assert_array_equal(g, w)


def test_ngram_matches_oracle(hip, oracle):
    rng = np.random.default_rng(7)
    hists, limits, cfgs = [], [], []
    for i in range(300):
        n = int(rng.choice([0, 1, 2, 3, 8, 9, 17, 64, 200, 1000]))
        alpha = int(rng.choice([2, 3, 5, 50]))
        hists.append(rng.integers(0, alpha, n).astype(np.int32))
        limits.append(int(rng.integers(0, 9)))
    # long histories: 16K copy-span context and a 2K motif prompt
    from mlxcat_amd.workloads import copy_span_prompt, motif_prompt
    hists.append(copy_span_prompt(3, 16384, 151936))
    limits.append(8)
    hists.append(motif_prompt(4, 2048, 151936))
    limits.append(5)
    for ms, mc in [(16, 8), (3, 2), (1, 2), (5, 40)]:
        got = hip.ngram_propose(hists, ms, mc, limits)
        for h, lim, g in zip(hists, limits, got):
            want = oracle.ngram_propose(h, ms, mc, lim)
            assert g == want, (len(h), lim, ms, mc)


def _random_block(rng, V, P, agree):
    """P+1 logits rows whose argmax agrees with the first `agree` drafts."""
    lg = f32_to_bf16((rng.standard_normal((P + 1, V)) * 2).astype(np.float32))
    am = np.argmax((lg.astype(np.uint32) << 16).view(np.float32), axis=1)
    drafts = []
    for j in range(P):
        if j < agree:
            drafts.append(int(am[j]))
        else:
            drafts.append(int(rng.integers(0, V)))
    return lg, drafts


@pytest.mark.parametrize("V", [8, 4096, 151936])
def test_accept_matches_oracle(hip, oracle, V):
    rng = np.random.default_rng(V)
    rows, drafts, sps, ctrs, ospec = [], [], [], [], []
    kinds = [dict(), dict(eos=(3,)), dict(temperature=0.7, top_p=0.95), dict(temperature=1.0),
             dict(temperature=0.7, top_p=0.95, eos=(5,)), dict(temperature=1.3, top_p=0.5), dict(reject_token=2)]
    for i in range(28):
        P = int(rng.integers(0, 6))
        agree = int(rng.integers(0, P + 1))
        lg, dr = _random_block(rng, V, P, agree)
        if i % 5 == 0:  # sharpen: make sampled drafts likely to be accepted
            for j, t in enumerate(dr):
                lg[j, t] = int(f32_to_bf16(np.float32(12.0)))
        if i % 7 == 3:  # exact ties across the row
            lg[0, :] = lg[0, 0]
        kw = kinds[i % len(kinds)]
        sps.append(kw)
        rows.append(lg)
        drafts.append(dr)
        ctrs.append(int(rng.integers(0, 1000)))
    for acceptance in (0, 1):
        samplings = [hip.make_sampling(seed=1000 + r, **kw) for r, kw in enumerate(sps)]
        got, keep, nacc = hip.accept(rows, drafts, samplings, ctrs, acceptance)
        for r in range(len(rows)):
            osp = oracle.make_sampling(seed=1000 + r, **sps[r])
            want, wkeep, wnacc, _ = oracle.accept_row(rows[r], drafts[r], osp, 1000 + r, ctrs[r], acceptance)
            assert got[r] == want, (r, acceptance, sps[r])
            assert keep[r] == wkeep and nacc[r] == wnacc, r


def test_accept_rejects_bad_drafts(hip):
    lg = np.zeros((2, 8), dtype=np.uint16)
    with pytest.raises(hip.HipError):
        hip.accept([lg], [[9]], [hip.make_sampling()], [0], 0)
