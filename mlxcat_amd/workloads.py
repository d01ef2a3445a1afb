"""Model shapes and seeded synthetic prompts of the speculative-decode workloads.

Shapes are the decoders the verify step is measured on (random-init weights in MLX
4-bit affine g64 format); prompts are built so that the n-gram proposer finds hits.
"""
from __future__ import annotations

import numpy as np

from . import _lib as L


def _cfg(arch, n_layers, hidden, nq, nkv, d, inter, vocab, tied, theta, eps=1e-6, ne=0, ntok=0, moe_i=0):
    return dict(arch=arch, n_layers=n_layers, hidden=hidden, n_q_heads=nq, n_kv_heads=nkv, head_dim=d,
                intermediate=inter, vocab=vocab, tied_embeddings=tied, rms_eps=eps, rope_theta=theta,
                n_experts=ne, n_experts_per_tok=ntok, moe_intermediate=moe_i)


MODELS = {
    # tiny Qwen3-style decoder (plumbing)
    "tiny-qwen3": _cfg(L.ARCH_QWEN3, 2, 256, 4, 2, 64, 704, 4096, 1, 1e6),
    # Qwen3-4B shape (tied embeddings)
    "qwen3-4b": _cfg(L.ARCH_QWEN3, 36, 2560, 32, 8, 128, 9728, 151936, 1, 1e6),
    # Llama-3-8B shape
    "llama3-8b": _cfg(L.ARCH_LLAMA, 32, 4096, 32, 8, 128, 14336, 128256, 0, 5e5),
    # Qwen3-8B shape
    "qwen3-8b": _cfg(L.ARCH_QWEN3, 36, 4096, 32, 8, 128, 12288, 151936, 0, 1e6),
    # Qwen3-30B-A3B shape (MoE)
    "qwen3-30b-a3b": _cfg(L.ARCH_QWEN3_MOE, 48, 2048, 32, 4, 128, 6144, 151936, 0, 1e6, ne=128, ntok=8, moe_i=768),
}


def motif_prompt(seed: int, n: int, vocab: int, motif_len: int = 16, sub_rate: float = 0.10) -> np.ndarray:
    """A random motif repeated to length n with a fraction of uniform substitutions."""
    rng = np.random.Generator(np.random.PCG64(seed))
    motif = rng.integers(0, vocab, motif_len)
    p = np.resize(motif, n).astype(np.int64)
    mask = rng.random(n) < sub_rate
    p[mask] = rng.integers(0, vocab, int(mask.sum()))
    return p.astype(np.int32)


def copy_span_prompt(seed: int, n: int, vocab: int, copy_frac: float = 0.40, span=(8, 32)) -> np.ndarray:
    """Uniform tokens with ~copy_frac of positions covered by spans copied from earlier."""
    rng = np.random.Generator(np.random.PCG64(seed))
    p = rng.integers(0, vocab, n).astype(np.int64)
    covered = 0
    target = int(copy_frac * n)
    tries = 0
    while covered < target and tries < 100 * n:
        tries += 1
        ln = int(rng.integers(span[0], span[1] + 1))
        pos = int(rng.integers(ln + 1, n - ln)) if n > 2 * ln + 2 else -1
        if pos < 0:
            break
        src = int(rng.integers(0, pos - ln + 1))
        p[pos:pos + ln] = p[src:src + ln]
        covered += ln
    return p.astype(np.int32)
