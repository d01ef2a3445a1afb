"""Shared shapes, tolerances and helpers of the parity tests."""
from __future__ import annotations

import numpy as np

# bf16 verify-logit tolerance (absolute, relative)
ATOL, RTOL = 2e-2, 1e-2

ARCH_QWEN3, ARCH_LLAMA, ARCH_QWEN3_MOE = 0, 1, 2
ARCH_FAKE_REPEATING, ARCH_FAKE_MISMATCHING = 100, 101


def cfg(arch, n_layers, hidden, nq, nkv, d, inter, vocab, tied, theta, eps=1e-6):
    return dict(arch=arch, n_layers=n_layers, hidden=hidden, n_q_heads=nq, n_kv_heads=nkv, head_dim=d,
                intermediate=inter, vocab=vocab, tied_embeddings=tied, rms_eps=eps, rope_theta=theta,
                n_experts=0, n_experts_per_tok=0, moe_intermediate=0)


# the tiny Qwen3-style decoder (2 layers, hidden 256, 4 q / 2 kv heads, head_dim 64)
TINY = cfg(ARCH_QWEN3, 2, 256, 4, 2, 64, 704, 4096, 1, 1e6)
# Llama-style tiny decoder (no q/k norm, untied head)
TINY_LLAMA = cfg(ARCH_LLAMA, 2, 256, 4, 2, 64, 704, 4096, 0, 5e5)
# the reference's scheduler test doubles (vocab 8)
FAKE_REPEATING = cfg(ARCH_FAKE_REPEATING, 1, 64, 1, 1, 64, 64, 8, 1, 1e6)
FAKE_MISMATCHING = cfg(ARCH_FAKE_MISMATCHING, 1, 64, 1, 1, 64, 64, 8, 1, 1e6)
# Qwen3-4B layer shapes with 2 layers (every GEMV shape of the full model incl. the 151936-row head)
QWEN3_4B_2L = cfg(ARCH_QWEN3, 2, 2560, 32, 8, 128, 9728, 151936, 1, 1e6)
# Llama-3-8B layer shapes with 1 layer
LLAMA3_8B_1L = cfg(ARCH_LLAMA, 1, 4096, 32, 8, 128, 14336, 128256, 0, 5e5)


def moe(base, n_experts, top_k, moe_inter):
    return dict(base, n_experts=n_experts, n_experts_per_tok=top_k, moe_intermediate=moe_inter)


# Qwen3-8B layer shapes with 1 layer and a 4096-token vocab (the M = 288 verify of 32 rows x 9)
QWEN3_8B_1L_V4K = cfg(ARCH_QWEN3, 1, 4096, 32, 8, 128, 12288, 4096, 0, 1e6)
# a small Qwen3-MoE decoder: 16 experts of width 128, top-4
TINY_MOE = moe(cfg(ARCH_QWEN3_MOE, 2, 256, 4, 2, 64, 512, 4096, 1, 1e6), 16, 4, 128)
# Qwen3-30B-A3B layer shapes with 1 layer: 128 experts of width 768, top-8, GQA group 8, untied head
QWEN3_30B_A3B_1L = moe(cfg(ARCH_QWEN3_MOE, 1, 2048, 32, 4, 128, 6144, 151936, 0, 1e6), 128, 8, 768)


def spec(enabled=True, k=4, max_suffix=16, min_ctx=8, acceptance=0, single_row_only=1, greedy_only=1):
    return dict(enabled=int(enabled), max_proposal_tokens=k, max_suffix_tokens=max_suffix, min_context_tokens=min_ctx,
                acceptance=acceptance, single_row_only=single_row_only, greedy_only=greedy_only)


def bf16_to_f32(a) -> np.ndarray:
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a) -> np.ndarray:
    u = np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def assert_close_bf16(got_u16, want_u16, atol=ATOL, rtol=RTOL, what=""):
    g = bf16_to_f32(got_u16).astype(np.float64)
    w = bf16_to_f32(want_u16).astype(np.float64)
    err = np.abs(g - w)
    bad = err > atol + rtol * np.abs(w)
    if bad.any():
        i = np.unravel_index(int(np.argmax(np.where(bad, err, -1.0))), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside {atol} abs + {rtol} rel; "
                             f"max err {err.max():.4g}; worst outlier at {tuple(int(x) for x in i)}: "
                             f"got {g[i]:.6g} want {w[i]:.6g}")


def assert_close_bf16_kv(got_u16, want_u16, atol=ATOL, rtol=RTOL, frac=0.999, what=""):
    """Cached K/V against the oracle.  K is RMS-normalised and then rotated (k0 cos - k1 sin):
    a one-ulp bf16 rounding flip of a large component on either side lands on a small
    rotated value as several of its ulps.  Every element must be within twice the logit
    bound and at least `frac` of them within it."""
    g = bf16_to_f32(got_u16).astype(np.float64)
    w = bf16_to_f32(want_u16).astype(np.float64)
    err = np.abs(g - w)
    bound = atol + rtol * np.abs(w)
    if not (err <= 2 * bound).all():
        i = np.unravel_index(int(np.argmax(err - 2 * bound)), err.shape)
        raise AssertionError(f"{what}: element {tuple(int(x) for x in i)} got {g[i]:.6g} want {w[i]:.6g}, "
                             f"beyond twice the bound")
    inside = float((err <= bound).mean())
    assert inside >= frac, f"{what}: only {inside:.5f} within {atol} abs + {rtol} rel"


def inside_fraction(got_u16, want_u16, atol=ATOL, rtol=RTOL) -> float:
    g = bf16_to_f32(got_u16).astype(np.float64)
    w = bf16_to_f32(want_u16).astype(np.float64)
    return float((np.abs(g - w) <= atol + rtol * np.abs(w)).mean())


def assert_close_bf16_wide(got_u16, want_u16, atol=ATOL, rtol=RTOL, frac=0.999, what="", floor_u16=None):
    """Full-width decoders: bf16 rounding of the hidden state (2^-8 relative) flips in a
    different place on each side and drifts through the layers, so a few logits land just
    outside the elementwise bound.  Every logit must be within twice the bound, at least
    `frac` of them within it, and greedy argmax must agree wherever the top-2 margin is clear.

    floor_u16: the oracle's own logits for the same inputs with every fp32 reduction in
    another order (oracle.reversed_reduction_order), an equally exact forward.  A one-ulp
    change of an RMSNorm scale flips an element sitting on a bf16 rounding boundary, which
    moves every projection of that token, so two exact summation orders already disagree on
    some logits.  The HIP path then has to be as close to the oracle as that reordering:
    within the bound for at least the lower of `frac` and the floor's fraction less 0.001,
    and no logit further out than the larger of twice the bound and 1.25 x the floor's
    worst ratio."""
    g = bf16_to_f32(got_u16).astype(np.float64)
    w = bf16_to_f32(want_u16).astype(np.float64)
    err = np.abs(g - w)
    bound = atol + rtol * np.abs(w)
    need, cap, fl = frac, 2.0, None
    if floor_u16 is not None:
        fe = np.abs(bf16_to_f32(floor_u16).astype(np.float64) - w) / bound
        fl = (float((fe <= 1).mean()), float(fe.max()))
        need, cap = min(frac, fl[0] - 0.001), max(2.0, 1.25 * fl[1])
    ratio = err / bound
    inside = float((ratio <= 1).mean())
    print(f"[wide] {what}: inside {inside:.5f} (required {need:.5f}), worst {ratio.max():.3f} x the bound "
          f"(cap {cap:.3f}); reordered oracle (inside, worst) {fl}")
    assert ratio.max() <= cap, f"{what}: max err {ratio.max():.3f} x the bound (cap {cap:.3f}; reordered oracle {fl})"
    assert inside >= need, (f"{what}: only {inside:.5f} within {atol} abs + {rtol} rel (required {need:.5f}; "
                            f"reordered oracle (inside, max ratio) {fl})")
    ws = np.sort(w, axis=-1)
    clear = (ws[..., -1] - ws[..., -2]) > 4 * 2 * (atol + rtol * np.abs(ws[..., -1]))
    am_g, am_w = np.argmax(g, axis=-1), np.argmax(w, axis=-1)
    assert (am_g[clear] == am_w[clear]).all(), f"{what}: argmax differs on a clear row"


def top2_margin(logits_u16_row) -> float:
    v = np.sort(bf16_to_f32(logits_u16_row).astype(np.float64))
    return float(v[-1] - v[-2])
