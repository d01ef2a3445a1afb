"""The default verify forward at long context on the GPU against the oracle: head_dim 128 at
the Qwen3-8B / Llama-3-8B layer shapes, 2K, 4K and 16K cached keys written by the same seeded
generator on both sides (fill_synthetic_kv), split-KV attention with 2 to 65 sub-chunks of 64
keys per block; the attention output itself, the logits and the appended K/V.

The synthetic keys make the softmax nearly uniform over thousands of keys, so the logits
alone barely see the attention; the attention output (before o_proj) is compared elementwise,
relative to each head vector's RMS: an attention block that skipped one 64-key sub-chunk of
16K keys moves the output by about 6% of that RMS."""
import math

import numpy as np
import pytest

from tests._common import LLAMA3_8B_1L, QWEN3_8B_1L_V4K, assert_close_bf16_kv, assert_close_bf16_wide, bf16_to_f32

pytestmark = pytest.mark.gpu
SEED = 1234
KV_SEED = 77
CHUNK = 64


def attn_split(R, nkv, nchunk):
    """Sub-chunks per attention block as the library chooses them (mc_kernels.hip attn_split)."""
    return max(8 if R * nkv >= 64 else 3, (R * nkv * nchunk + 1023) // 1024)


def assert_attention_close(got_u16, want_u16, nq, d, what, rel=2e-2, rtol=1e-2, frac=0.999):
    """Each (token, head) vector within rel x its RMS + rtol x |value|, elementwise."""
    g = bf16_to_f32(got_u16).astype(np.float64).reshape(-1, nq, d)
    w = bf16_to_f32(want_u16).astype(np.float64).reshape(-1, nq, d)
    rms = np.sqrt((w ** 2).mean(axis=2, keepdims=True)) + 1e-30
    ratio = np.abs(g - w) / (rel * rms + rtol * np.abs(w))
    inside = float((ratio <= 1).mean())
    print(f"{what}: attention inside {inside:.5f}, worst {ratio.max():.3f} x the bound")
    assert ratio.max() <= 2.0 and inside >= frac, (what, inside, float(ratio.max()))


def run_case(hip, oracle, cfg, rows, n_keys, width, seed):
    nkv, nq, d, V = cfg["n_kv_heads"], cfg["n_q_heads"], cfg["head_dim"], cfg["vocab"]
    ctx = n_keys + width + CHUNK
    gm = hip.Model(cfg)
    gm.init_synthetic(SEED)
    gb = hip.Batch(gm, rows, ctx, dict(enabled=1, max_proposal_tokens=width - 1, max_suffix_tokens=3,
                                       min_context_tokens=8, acceptance=1, single_row_only=0, greedy_only=0))
    om = oracle.Model(cfg, SEED, ctx, rows)
    om_rev = oracle.Model(cfg, SEED, ctx, rows)
    rng = np.random.default_rng(seed)
    lens = [n_keys - int(rng.integers(0, 3 * CHUNK)) if r else n_keys for r in range(rows)]  # ragged rows
    for r in range(rows):
        gb.fill_synthetic_kv(r, lens[r], KV_SEED + r)
        om.fill_kv(r, lens[r], KV_SEED + r)
        om_rev.fill_kv(r, lens[r], KV_SEED + r)
    nchunk = (ctx + CHUNK - 1) // CHUNK
    S = attn_split(rows, nkv, nchunk)
    print(f"{rows} rows x {width} queries, {n_keys} keys: {S} sub-chunks of 64 keys per attention block")
    toks = rng.integers(0, V, rows * width).tolist()
    rr, ww = list(range(rows)), [width] * rows
    got = gb.forward(rr, ww, toks)
    got_att = gb.read_attention(rows * width)
    want, want_att = om.forward(rr, ww, toks, attention=True)
    with oracle.reversed_reduction_order():
        alt = om_rev.forward(rr, ww, toks)
    assert_attention_close(got_att, want_att[-1], nq, d, f"{rows}x{width} at {n_keys} keys")
    assert_close_bf16_wide(got, want, what=f"{rows}x{width} logits at {n_keys} keys", floor_u16=alt)
    for r in range(rows):
        assert gb.kv_len(r) == om.kv_len(r) == lens[r] + width
        for w in (0, 1):  # the appended positions
            g = gb.read_kv(0, r, w).reshape(nkv, -1, d)[:, lens[r]:]
            o = om.kv(0, r, w).reshape(nkv, -1, d)[:, lens[r]:]
            assert_close_bf16_kv(g, o, what=f"row {r} {'V' if w else 'K'} appended")
    return S


@pytest.mark.parametrize("rows,n_keys,width", [(1, 2048, 6), (8, 4096, 5), (4, 16384, 9), (16, 16384, 9)],
                         ids=["1x6-2K", "8x5-4K", "4x9-16K", "16x9-16K"])
def test_long_context_qwen3_8b(hip, oracle, rows, n_keys, width):
    S = run_case(hip, oracle, QWEN3_8B_1L_V4K, rows, n_keys, width, seed=rows + n_keys)
    assert 2 <= S <= 65


def test_many_subchunks_llama3_8b(hip, oracle):
    """Llama-3-8B layer (no q/k norm), 8 rows of about 1100 keys, 5-token verify: 8 sub-chunks
    per block, the 8-way split merged by the last-arriving block."""
    S = run_case(hip, oracle, LLAMA3_8B_1L, 8, 1100, 5, seed=3)
    assert S == 8


def test_cfg5_shaped_step(hip, oracle):
    """32 rows x (K = 8) + 1 = 288 verify slots at the Qwen3-8B layer shapes (one layer, a
    4096-token vocabulary), even rows greedy, odd rows seeded (T 0.8, top-p 0.95), a forced
    accept-length schedule (exactly L drafts accepted, then the history's next token),
    through mc_step on synthetic 1K-token contexts.
    - Every row's emitted tokens equal or_accept_row on the step's own verify logits, bit for
      bit, and mc_accept's speculative sampling on those logits equals or_accept_row's.
    - The step's logits are within the full-width bound of the oracle's forward of the same
      verify blocks, and greedy rows whose every used position has a clear top-2 margin emit
      what the oracle's acceptance emits on the oracle's logits."""
    from mlxcat_amd.workloads import copy_span_prompt
    from tests._common import ATOL, RTOL, top2_margin
    cfg = QWEN3_8B_1L_V4K
    R, K, L, V = 32, 8, 1024, cfg["vocab"]
    spec = dict(enabled=1, max_proposal_tokens=K, max_suffix_tokens=3, min_context_tokens=8, acceptance=1,
                single_row_only=0, greedy_only=0)
    ctx_cap = L + 2 * CHUNK
    gm = hip.Model(cfg)
    gm.init_synthetic(SEED)
    gb = hip.Batch(gm, R, ctx_cap, spec)
    om = oracle.Model(cfg, SEED, ctx_cap, R)
    rng = np.random.default_rng(5)
    prompts, sps, osps = [], [], []
    for r in range(R):
        p = copy_span_prompt(100 + r, L, V).tolist()
        p = p[:L - 12] + p[100 + r:112 + r]  # the tail repeats an earlier span: a full proposal
        prompts.append(p)
        kw = dict() if r % 2 == 0 else dict(temperature=0.8, top_p=0.95, seed=700 + r)
        sps.append(hip.make_sampling(**kw))
        osps.append(oracle.make_sampling(**kw))
        gb.fill_synthetic_kv(r, L - 1, KV_SEED + r)
        om.fill_kv(r, L - 1, KV_SEED + r)
        gb.insert_prefilled(r, p, 64, sps[r])
    forced = rng.integers(0, K + 1, R).tolist()
    toks, counts, fins = gb.step(forced)
    blocks, drafts, exts = [], [], []
    for r in range(R):
        d = oracle.ngram_propose(prompts[r], 3, 8, K + 1)  # + the history's next token
        drafts.append(d[:K])
        exts.append(d[K] if len(d) > K else None)
        blocks.append([prompts[r][-1]] + d[:K])
    assert sum(len(d) for d in drafts) > 4 * R  # the repeated tails give proposals
    gpu_lg = [gb.read_logits(r * (K + 1), len(blocks[r])) for r in range(R)]
    # the step's acceptance on its own logits
    for r in range(R):
        want, keep, nacc, _ = oracle.accept_row(gpu_lg[r], drafts[r], osps[r], 700 + r, 0, 1, forced_cap=forced[r],
                                                generated=[prompts[r][-1]], ext=exts[r])
        assert toks[r, :counts[r]].tolist() == want, r
    # the sampled rows' speculative sampling on the same logits (no forced schedule) through
    # mc_accept, against or_accept_row
    odd = list(range(1, R, 2))
    got, keep, nacc = hip.accept([gpu_lg[r] for r in odd], [drafts[r] for r in odd], [sps[r] for r in odd],
                                 [0] * len(odd), 1)
    for i, r in enumerate(odd):
        want, wkeep, wnacc, _ = oracle.accept_row(gpu_lg[r], drafts[r], osps[r], 700 + r, 0, 1)
        assert (got[i], keep[i], nacc[i]) == (want, wkeep, wnacc), r
    # the forward against the oracle's
    want_lg = om.forward(list(range(R)), [len(b) for b in blocks], [t for b in blocks for t in b])
    assert_close_bf16_wide(np.concatenate(gpu_lg), want_lg, what="cfg5-shaped verify logits")
    off = np.cumsum([0] + [len(b) for b in blocks])
    compared = 0
    for r in range(0, R, 2):
        w = want_lg[off[r]:off[r + 1]]
        want, _, _, _ = oracle.accept_row(w, drafts[r], osps[r], 0, 0, 1, forced_cap=forced[r], ext=exts[r])
        used = max(len(want), int(counts[r]))  # verify positions either side's decision read
        vals = bf16_to_f32(w[:used]).astype(np.float64)
        if any(top2_margin(w[j]) <= 2 * (ATOL + RTOL * abs(vals[j].max())) for j in range(used)):
            continue  # a near-tie within the tolerance at a position the decision read
        assert toks[r, :counts[r]].tolist() == want, r
        compared += 1
    print(f"greedy rows compared against the oracle's logits: {compared} of {R // 2}")
    assert compared >= 3
