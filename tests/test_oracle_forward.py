"""The oracle's decoder forward against a PyTorch fp32 restatement built from library
routines (torch.nn.functional.rms_norm, scaled_dot_product_attention with GQA, silu),
plus the invariants the verify step relies on (M-invariance, per-row positions, rollback)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests._common import TINY, TINY_LLAMA, TINY_MOE, assert_close_bf16, bf16_to_f32

SEED = 1234


def dequant(O, m, layer, which, expert=-1):
    wq, s, b = m.linear(layer, which, expert)
    N, KW = wq.shape
    q = np.zeros((N, KW * 8), dtype=np.float32)
    for j in range(8):
        q[:, j::8] = (wq >> np.uint32(4 * j)) & np.uint32(0xF)
    sc = np.repeat(bf16_to_f32(s), 64, axis=1)
    bi = np.repeat(bf16_to_f32(b), 64, axis=1)
    return torch.from_numpy(sc * q + bi)


def bf(t):
    return t.to(torch.bfloat16).to(torch.float32)


def norm_w(O, seed, tid, n):
    w = np.zeros(n, dtype=np.uint16)
    O.lib().or_gen_norm(seed, tid, n, w.ctypes.data_as(__import__("ctypes").c_void_p))
    return torch.from_numpy(bf16_to_f32(w))


def torch_moe(O, m, cfg, l, h):
    """Qwen3-MoE sparse block (Qwen3MoeSparseMoeBlock: router softmax in fp32, top-k,
    norm_topk_prob renormalisation, SwiGLU experts) over the normalised rows h.  The router
    logits are bf16 like every linear output of the model."""
    E, TK = cfg["n_experts"], cfg["n_experts_per_tok"]
    probs = torch.softmax(bf(h @ dequant(O, m, l, 11).T), dim=-1)
    w, sel = torch.topk(probs, TK, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    out = torch.zeros_like(h)
    for t in range(h.shape[0]):
        for kk in range(TK):
            e = int(sel[t, kk])
            g = h[t] @ dequant(O, m, l, 4, e).T
            u = h[t] @ dequant(O, m, l, 5, e).T
            out[t] += w[t, kk] * (bf(F.silu(g) * u) @ dequant(O, m, l, 6, e).T)
    return out


def torch_forward(O, m, cfg, tokens, positions):
    """Single-row forward of `tokens` at absolute `positions` with an empty cache before
    positions[0] == 0 (prefill from scratch)."""
    H, d, nq, nkv = cfg["hidden"], cfg["head_dim"], cfg["n_q_heads"], cfg["n_kv_heads"]
    eps = cfg["rms_eps"]
    T = len(tokens)
    E = dequant(O, m, -1, 0)
    x = bf(E[torch.tensor(tokens)])
    pos = torch.tensor(positions, dtype=torch.float64)
    inv = torch.tensor(cfg["rope_theta"], dtype=torch.float64) ** (-2.0 * torch.arange(d // 2, dtype=torch.float64) / d)
    ang = pos[:, None] * inv[None, :]
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()

    def rope(v):  # v [T, heads, d], rotate-half
        a, b2 = v[..., : d // 2], v[..., d // 2:]
        c, s = cos[:, None, :], sin[:, None, :]
        return bf(torch.cat([a * c - b2 * s, a * s + b2 * c], dim=-1))

    mask = torch.tensor(positions)[:, None] >= torch.tensor(positions)[None, :]
    for l in range(cfg["n_layers"]):
        tid = lambda w: O.lib().or_tensor_id(l, w)
        h = bf(F.rms_norm(x, (H,), norm_w(O, SEED, tid(7), H), eps))
        q = bf(h @ dequant(O, m, l, 0).T).view(T, nq, d)
        k = bf(h @ dequant(O, m, l, 1).T).view(T, nkv, d)
        v = bf(h @ dequant(O, m, l, 2).T).view(T, nkv, d)
        if cfg["arch"] in (0, 2):
            q = bf(F.rms_norm(q, (d,), norm_w(O, SEED, tid(9), d), eps))
            k = bf(F.rms_norm(k, (d,), norm_w(O, SEED, tid(10), d), eps))
        q, k = rope(q), rope(k)
        a = F.scaled_dot_product_attention(q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None],
                                           attn_mask=mask, enable_gqa=True)
        a = bf(a[0].transpose(0, 1).reshape(T, nq * d))
        x = bf(x + a @ dequant(O, m, l, 3).T)
        h = bf(F.rms_norm(x, (H,), norm_w(O, SEED, tid(8), H), eps))
        if cfg["arch"] == 2:
            x = bf(x + torch_moe(O, m, cfg, l, h))
            continue
        g = h @ dequant(O, m, l, 4).T
        u = h @ dequant(O, m, l, 5).T
        x = bf(x + bf(F.silu(g) * u) @ dequant(O, m, l, 6).T)
    h = bf(F.rms_norm(x, (H,), norm_w(O, SEED, 0xE0000003, H), eps))
    head = dequant(O, m, -1, 0 if cfg["tied_embeddings"] else 1)
    return (h @ head.T).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)


@pytest.mark.parametrize("cfg", [TINY, TINY_LLAMA, TINY_MOE], ids=["qwen3", "llama", "qwen3-moe"])
def test_forward_vs_torch(oracle, cfg):
    m = oracle.Model(cfg, SEED, 64, 1)
    rng = np.random.default_rng(0)
    toks = rng.integers(0, cfg["vocab"], 24).tolist()
    got = m.forward([0], [24], toks)
    want = torch_forward(oracle, m, cfg, toks, list(range(24)))
    assert_close_bf16(got, want, what="oracle vs torch fp32")


def test_verify_block_is_m_invariant(oracle):
    """Logits of a token do not depend on how many tokens share the forward: the verify
    block's position 0 equals the one-token decode, which the reference's reject path
    (BatchGenerator.swift:937-940) recomputes."""
    m1 = oracle.Model(TINY, SEED, 64, 1)
    m2 = oracle.Model(TINY, SEED, 64, 1)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, 4096, 20).tolist()
    m1.forward([0], [20], prompt, want_logits=False)
    m2.forward([0], [20], prompt, want_logits=False)
    block = rng.integers(0, 4096, 6).tolist()
    a = m1.forward([0], [6], block)
    seq = np.concatenate([m2.forward([0], [1], [t]) for t in block])
    np.testing.assert_array_equal(a, seq)


def test_rows_are_independent(oracle):
    """Per-row positions (the per-row RoPE offsets of BatchCache.swift:123-139): each row of a
    mixed-length batch equals its solo forward (RoPEBatchGridProbeTests.swift:62-64)."""
    rng = np.random.default_rng(2)
    pa, pb = rng.integers(0, 4096, 9).tolist(), rng.integers(0, 4096, 17).tolist()
    mb = oracle.Model(TINY, SEED, 64, 2)
    mb.forward([0, 1], [9, 17], pa + pb, want_logits=False)
    nxt = rng.integers(0, 4096, 5).tolist()
    both = mb.forward([0, 1], [2, 3], nxt)
    ma = oracle.Model(TINY, SEED, 64, 1)
    ma.forward([0], [9], pa, want_logits=False)
    sa = ma.forward([0], [2], nxt[:2])
    mc = oracle.Model(TINY, SEED, 64, 1)
    mc.forward([0], [17], pb, want_logits=False)
    sb = mc.forward([0], [3], nxt[2:])
    np.testing.assert_array_equal(both[:2], sa)
    np.testing.assert_array_equal(both[2:], sb)


def test_rollback_equals_never_verified(oracle):
    """Dropping rejected positions by length leaves no phantom KV: decode after a rollback
    equals decode on a cache that never saw the rejected drafts."""
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, 4096, 12).tolist()
    a = oracle.Model(TINY, SEED, 64, 1)
    b = oracle.Model(TINY, SEED, 64, 1)
    a.forward([0], [12], prompt, want_logits=False)
    b.forward([0], [12], prompt, want_logits=False)
    a.forward([0], [5], rng.integers(0, 4096, 5).tolist(), want_logits=False)
    a.set_kv_len(0, 12)
    t = [7, 8]
    np.testing.assert_array_equal(a.forward([0], [2], t), b.forward([0], [2], t))


def test_reversed_reduction_order_is_a_reordering(oracle):
    """The reordered reductions (the GPU tests' rounding-noise floor) compute the same sums:
    fp32 results agree to reordering error, bf16 logits to the elementwise bound."""
    rng = np.random.default_rng(11)
    wq, s, b = oracle.gen_linear(SEED, 77, 96, 512)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    y0 = oracle.qmatmul(wq, s, b, x)
    with oracle.reversed_reduction_order():
        y1 = oracle.qmatmul(wq, s, b, x)
    np.testing.assert_allclose(y1, y0, rtol=1e-5, atol=1e-5 * float(np.abs(y0).max()))
    a, r = oracle.Model(TINY, SEED, 64, 1), oracle.Model(TINY, SEED, 64, 1)
    toks = rng.integers(0, TINY["vocab"], 12).tolist()
    la = a.forward([0], [12], toks)
    with oracle.reversed_reduction_order():
        lr = r.forward([0], [12], toks)
    assert_close_bf16(lr, la, what="reversed order")
