"""ctypes binding of libmlxcat_hip.so (the C ABI in include/mlxcat_hip.h).

The HIP library is the only compute path: if it is missing this module raises,
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libmlxcat_hip.so")

ARCH_QWEN3, ARCH_LLAMA, ARCH_QWEN3_MOE = 0, 1, 2
ARCH_FAKE_REPEATING, ARCH_FAKE_MISMATCHING = 100, 101
W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN, W_ROUTER = 0, 1, 2, 3, 4, 5, 6, 11
W_EMBED, W_LM_HEAD = 100, 101
N_INPUT, N_POST, N_Q, N_K, N_FINAL = 7, 8, 9, 10, 102
ACCEPT_ALL_OR_NOTHING, ACCEPT_PREFIX = 0, 1

# every symbol the header declares (checked by the CPU tests)
EXPORTS = [
    "mc_last_error", "mc_set_device", "mc_model_create", "mc_model_destroy", "mc_model_init_synthetic",
    "mc_model_set_linear", "mc_model_get_linear", "mc_model_set_norm", "mc_batch_create", "mc_batch_destroy",
    "mc_batch_insert", "mc_batch_insert_prefilled", "mc_batch_fill_synthetic_kv", "mc_batch_remove",
    "mc_batch_trim", "mc_batch_rollback", "mc_batch_kv_len", "mc_batch_read_kv", "mc_batch_read_attention",
    "mc_batch_read_logits",
    "mc_batch_history", "mc_batch_filter", "mc_batch_extract_kv", "mc_batch_read_router",
    "mc_batch_insert_cached", "mc_batch_export_kv_block", "mc_batch_import_kv_block",
    "mc_forward", "mc_ngram_propose", "mc_accept", "mc_accept_noalloc", "mc_step", "mc_batch_stats", "mc_batch_call_widths",
    "mc_batch_set_profiling", "mc_batch_profile", "mc_probe_hbm_read",
]


class ModelConfig(C.Structure):
    _fields_ = [
        ("arch", C.c_int32), ("n_layers", C.c_int32), ("hidden", C.c_int32), ("n_q_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("intermediate", C.c_int32), ("vocab", C.c_int32),
        ("tied_embeddings", C.c_int32), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("n_experts", C.c_int32), ("n_experts_per_tok", C.c_int32), ("moe_intermediate", C.c_int32),
    ]


class SpecConfig(C.Structure):
    _fields_ = [
        ("enabled", C.c_int32), ("max_proposal_tokens", C.c_int32), ("max_suffix_tokens", C.c_int32),
        ("min_context_tokens", C.c_int32), ("acceptance", C.c_int32), ("single_row_only", C.c_int32),
        ("greedy_only", C.c_int32),
    ]


class Sampling(C.Structure):
    _fields_ = [
        ("temperature", C.c_float), ("top_p", C.c_float), ("has_seed", C.c_int32), ("seed", C.c_uint64),
        ("n_eos", C.c_int32), ("eos", C.c_int32 * 8), ("reject_token", C.c_int32), ("top_k", C.c_int32),
        ("min_p", C.c_float), ("repetition_penalty", C.c_float), ("presence_penalty", C.c_float),
        ("frequency_penalty", C.c_float), ("min_tokens", C.c_int32), ("n_bias", C.c_int32),
        ("bias_token", C.c_int32 * 16), ("bias_value", C.c_float * 16),
    ]


class SpecStats(C.Structure):
    _fields_ = [("proposed", C.c_int64), ("accepted", C.c_int64), ("proposal_batches", C.c_int64),
                ("rejected_batches", C.c_int64)]


class HipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def load(path: str = LIB_PATH):
    """Loads the library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -m mlxcat_amd.build` "
                          "(there is no CPU fallback)")
    L = C.CDLL(path)
    P, I32, U64 = C.c_void_p, C.c_int32, C.c_uint64
    sig = {
        "mc_last_error": (C.c_char_p, []),
        "mc_set_device": (C.c_int, [C.c_int]),
        "mc_model_create": (C.c_int, [P, P]),
        "mc_model_destroy": (None, [P]),
        "mc_model_init_synthetic": (C.c_int, [P, U64]),
        "mc_model_set_linear": (C.c_int, [P, I32, I32, I32, P, P, P]),
        "mc_model_get_linear": (C.c_int, [P, I32, I32, I32, P, P, P]),
        "mc_model_set_norm": (C.c_int, [P, I32, I32, P]),
        "mc_batch_create": (C.c_int, [P, I32, I32, I32, P, P]),
        "mc_batch_destroy": (None, [P]),
        "mc_batch_insert": (C.c_int, [P, I32, P, I32, I32, P, P, P]),
        "mc_batch_insert_prefilled": (C.c_int, [P, I32, P, I32, I32, P]),
        "mc_batch_insert_cached": (C.c_int, [P, I32, P, I32, I32, I32, P, P, P]),
        "mc_batch_export_kv_block": (C.c_int, [P, I32, I32, I32, P, P]),
        "mc_batch_import_kv_block": (C.c_int, [P, I32, I32, I32, P, P]),
        "mc_batch_fill_synthetic_kv": (C.c_int, [P, I32, I32, U64]),
        "mc_batch_remove": (C.c_int, [P, I32]),
        "mc_batch_trim": (C.c_int, [P, I32]),
        "mc_batch_rollback": (C.c_int, [P, I32, I32]),
        "mc_batch_filter": (C.c_int, [P, P, I32]),
        "mc_probe_hbm_read": (C.c_int, [C.c_int64, I32, P, P]),
        "mc_batch_extract_kv": (C.c_int, [P, I32, P, I32]),
        "mc_batch_kv_len": (C.c_int, [P, I32, P]),
        "mc_batch_read_kv": (C.c_int, [P, I32, I32, I32, P]),
        "mc_batch_history": (C.c_int, [P, I32, P, I32, P]),
        "mc_batch_read_attention": (C.c_int, [P, I32, P]),
        "mc_batch_read_logits": (C.c_int, [P, I32, I32, P]),
        "mc_batch_read_router": (C.c_int, [P, I32, P]),
        "mc_forward": (C.c_int, [P, I32, P, P, P, P]),
        "mc_ngram_propose": (C.c_int, [P, P, I32, I32, I32, P, I32, P, P]),
        "mc_accept": (C.c_int, [P, I32, I32, P, P, I32, P, P, P, P, P, P, I32, P, P, P, P]),
        "mc_accept_noalloc": (C.c_int, [P, I32, I32, I32, P, P, P, P, P, I32, P, P, P, P]),
        "mc_step": (C.c_int, [P, P, P, P, P, P]),
        "mc_batch_stats": (C.c_int, [P, P]),
        "mc_batch_call_widths": (C.c_int, [P, P, I32]),
        "mc_batch_set_profiling": (C.c_int, [P, I32]),
        "mc_batch_profile": (C.c_int, [P, I32, P, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int) -> int:
    if rc < 0:
        raise HipError(rc, load().mc_last_error().decode(errors="replace"))
    return rc


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _i32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


def make_sampling(temperature=0.0, top_p=0.0, seed=None, eos=(), reject_token=-1, top_k=0, min_p=0.0,
                  repetition_penalty=1.0, presence_penalty=0.0, frequency_penalty=0.0, min_tokens=0,
                  logit_bias=None) -> Sampling:
    """SamplingParameters (Sampling.swift:163-194) as the C ABI's mc_sampling."""
    sp = Sampling()
    sp.temperature = float(temperature)
    sp.top_p = float(top_p)
    sp.has_seed = 0 if seed is None else 1
    sp.seed = 0 if seed is None else int(seed)
    if len(eos) > 8:
        raise ValueError("at most 8 EOS ids")
    sp.n_eos = len(eos)
    for i, e in enumerate(eos):
        sp.eos[i] = int(e)
    sp.reject_token = int(reject_token)
    sp.top_k = int(top_k)
    sp.min_p = float(min_p)
    sp.repetition_penalty = float(repetition_penalty)
    sp.presence_penalty = float(presence_penalty)
    sp.frequency_penalty = float(frequency_penalty)
    sp.min_tokens = max(0, int(min_tokens))
    bias = sorted((logit_bias or {}).items())
    if len(bias) > 16:
        raise ValueError("at most 16 logit bias entries")
    sp.n_bias = len(bias)
    for i, (t, b) in enumerate(bias):
        sp.bias_token[i] = int(t)
        sp.bias_value[i] = float(b)
    return sp


class Model:
    """Device-resident 4-bit decoder (the LanguageModel the verify forward runs)."""

    def __init__(self, cfg: dict):
        L = load()
        self.cfg = ModelConfig(**cfg)
        h = C.c_void_p()
        _check(L.mc_model_create(C.byref(self.cfg), C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            load().mc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def init_synthetic(self, seed: int) -> None:
        _check(load().mc_model_init_synthetic(self.h, seed))

    def _lshape(self, which: int, expert: int = -1):
        c = self.cfg
        H, d, nq, nkv, I = c.hidden, c.head_dim, c.n_q_heads, c.n_kv_heads, c.intermediate
        if expert >= 0:  # a Qwen3-MoE expert's gate / up / down
            I = c.moe_intermediate
        return {W_Q: (nq * d, H), W_K: (nkv * d, H), W_V: (nkv * d, H), W_O: (H, nq * d), W_GATE: (I, H),
                W_UP: (I, H), W_DOWN: (H, I), W_ROUTER: (c.n_experts, H), W_EMBED: (c.vocab, H),
                W_LM_HEAD: (c.vocab, H)}[which]

    def set_linear(self, layer: int, which: int, wq, scales, biases, expert: int = -1) -> None:
        N, K = self._lshape(which, expert)
        wq = np.ascontiguousarray(wq, dtype=np.uint32).reshape(N, K // 8)
        s = np.ascontiguousarray(scales, dtype=np.uint16).reshape(N, K // 64)
        b = np.ascontiguousarray(biases, dtype=np.uint16).reshape(N, K // 64)
        _check(load().mc_model_set_linear(self.h, layer, which, expert, _p(wq), _p(s), _p(b)))

    def get_linear(self, layer: int, which: int, expert: int = -1):
        N, K = self._lshape(which, expert)
        wq = np.zeros((N, K // 8), dtype=np.uint32)
        s = np.zeros((N, K // 64), dtype=np.uint16)
        b = np.zeros((N, K // 64), dtype=np.uint16)
        _check(load().mc_model_get_linear(self.h, layer, which, expert, _p(wq), _p(s), _p(b)))
        return wq, s, b

    def set_norm(self, layer: int, which: int, w) -> None:
        w = np.ascontiguousarray(w, dtype=np.uint16)
        _check(load().mc_model_set_norm(self.h, layer, which, _p(w)))


class Batch:
    """Device state of a continuous batch: per-row KV, token histories, sampling."""

    def __init__(self, model: Model, max_rows: int, max_ctx: int, spec: dict, max_draft: int | None = None):
        L = load()
        self.model = model
        self.spec = SpecConfig(**spec)
        self.R = max_rows
        self.K = self.spec.max_proposal_tokens if self.spec.enabled else 0
        self.K1 = self.K + 1
        h = C.c_void_p()
        _check(L.mc_batch_create(model.h, max_rows, max_ctx, self.K if max_draft is None else max_draft,
                                 C.byref(self.spec), C.byref(h)))
        self.h = h
        self._tok = np.zeros((self.R, self.K1), dtype=np.int32)
        self._cnt = np.zeros(self.R, dtype=np.int32)
        self._fin = np.zeros(self.R, dtype=np.int32)

    def close(self):
        if getattr(self, "h", None):
            load().mc_batch_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def insert(self, row: int, prompt, max_tokens: int, sampling: Sampling):
        p = _i32(prompt)
        tok, fin = C.c_int32(), C.c_int32()
        _check(load().mc_batch_insert(self.h, row, _p(p), len(p), max_tokens, C.byref(sampling), C.byref(tok),
                                      C.byref(fin)))
        return tok.value, fin.value

    def insert_cached(self, row: int, prompt, n_cached: int, max_tokens: int, sampling: Sampling):
        """insert() after a prefix hit: the row's K/V holds prompt[:n_cached] already
        (import_kv_block) and prefill resumes at n_cached."""
        p = _i32(prompt)
        tok, fin = C.c_int32(), C.c_int32()
        _check(load().mc_batch_insert_cached(self.h, row, _p(p), len(p), n_cached, max_tokens, C.byref(sampling),
                                             C.byref(tok), C.byref(fin)))
        return tok.value, fin.value

    def export_kv_block(self, row: int, t0: int, n: int):
        """Positions [t0, t0 + n) of the row's K/V as (keys, values), each
        [n_layers][n_kv][n][d] uint16 (bf16 bits): the per-layer cache-state slices a prefix
        block holds."""
        c = self.model.cfg
        keys = np.zeros((c.n_layers, c.n_kv_heads, n, c.head_dim), dtype=np.uint16)
        values = np.zeros_like(keys)
        _check(load().mc_batch_export_kv_block(self.h, row, t0, n, _p(keys), _p(values)))
        return keys, values

    def import_kv_block(self, row: int, t0: int, keys, values) -> None:
        """Writes positions [t0, t0 + n) of the row from (keys, values) of export_kv_block's
        shape; the row becomes inactive with K/V length t0 + n."""
        c = self.model.cfg
        k = np.ascontiguousarray(keys, dtype=np.uint16)
        v = np.ascontiguousarray(values, dtype=np.uint16)
        n = k.shape[2] if k.ndim == 4 else -1
        want = (c.n_layers, c.n_kv_heads, n, c.head_dim)
        if k.shape != want or v.shape != want:
            raise ValueError(f"import_kv_block: keys / values must be {want}, got {k.shape} / {v.shape}")
        _check(load().mc_batch_import_kv_block(self.h, row, t0, n, _p(k), _p(v)))

    def fill_synthetic_kv(self, row: int, n: int, seed: int) -> None:
        _check(load().mc_batch_fill_synthetic_kv(self.h, row, n, seed))

    def insert_prefilled(self, row: int, ctx, max_tokens: int, sampling: Sampling) -> None:
        c = _i32(ctx)
        _check(load().mc_batch_insert_prefilled(self.h, row, _p(c), len(c), max_tokens, C.byref(sampling)))

    def remove(self, row: int) -> None:
        _check(load().mc_batch_remove(self.h, row))

    def trim(self, n: int) -> int:
        return _check(load().mc_batch_trim(self.h, n))

    def rollback(self, row: int, n: int) -> None:
        _check(load().mc_batch_rollback(self.h, row, n))

    def filter(self, rows) -> None:
        """Keep rows[i] as row i (BatchKVCache.filter(keeping:)); the other rows become empty."""
        r = _i32(rows)
        _check(load().mc_batch_filter(self.h, _p(r) if len(r) else None, len(r)))

    def extract_kv(self, row: int, dst: "Batch", dst_row: int) -> None:
        """Copy this row's K/V into dst's row dst_row (BatchKVCache.extract)."""
        _check(load().mc_batch_extract_kv(self.h, row, dst.h, dst_row))

    def kv_len(self, row: int) -> int:
        v = C.c_int32()
        _check(load().mc_batch_kv_len(self.h, row, C.byref(v)))
        return v.value

    def read_kv(self, layer: int, row: int, which_v: int) -> np.ndarray:
        c = self.model.cfg
        out = np.zeros((c.n_kv_heads, self.kv_len(row), c.head_dim), dtype=np.uint16)
        _check(load().mc_batch_read_kv(self.h, layer, row, which_v, _p(out)))
        return out

    def read_attention(self, M: int) -> np.ndarray:
        """The last layer's attention output of the last forward's first M slots [M][nq * d]."""
        c = self.model.cfg
        out = np.zeros((M, c.n_q_heads * c.head_dim), dtype=np.uint16)
        _check(load().mc_batch_read_attention(self.h, M, _p(out)))
        return out

    def read_logits(self, slot0: int, n: int) -> np.ndarray:
        """Logits [n][V] of token slots slot0.. of the last forward (after step(): row r's
        position j is slot r * (K + 1) + j)."""
        out = np.zeros((n, self.model.cfg.vocab), dtype=np.uint16)
        _check(load().mc_batch_read_logits(self.h, slot0, n, _p(out)))
        return out

    def read_router(self, M: int) -> np.ndarray:
        """Qwen3-MoE: the last layer's router logits of the last forward's slots [M][E]."""
        out = np.zeros((M, self.model.cfg.n_experts), dtype=np.uint16)
        _check(load().mc_batch_read_router(self.h, M, _p(out)))
        return out

    def history(self, row: int) -> list[int]:
        n = C.c_int32()
        _check(load().mc_batch_history(self.h, row, None, 0, C.byref(n)))
        out = np.zeros(max(n.value, 1), dtype=np.int32)
        _check(load().mc_batch_history(self.h, row, _p(out), n.value, C.byref(n)))
        return out[: n.value].tolist()

    def forward(self, rows, counts, tokens, want_logits: bool = True):
        rows, counts, tokens = _i32(rows), _i32(counts), _i32(tokens)
        M = int(counts.sum())
        lg = np.zeros((M, self.model.cfg.vocab), dtype=np.uint16) if want_logits else None
        _check(load().mc_forward(self.h, len(rows), _p(rows), _p(counts), _p(tokens), _p(lg)))
        return lg

    def step(self, forced_accept=None, uniforms=None):
        """One speculative step; uniforms [rows][K + 1][2] uint32 replaces the derived draws."""
        fa = _i32(forced_accept) if forced_accept is not None else None
        u = None
        if uniforms is not None:
            u = np.ascontiguousarray(uniforms, dtype=np.uint32)
            if u.size != self._tok.size * 2:
                raise ValueError("uniforms must hold rows * (K + 1) * 2 draws")
        _check(load().mc_step(self.h, _p(fa), _p(u), _p(self._tok), _p(self._cnt), _p(self._fin)))
        return self._tok.copy(), self._cnt.copy(), self._fin.copy()

    def stats(self) -> dict:
        s = SpecStats()
        _check(load().mc_batch_stats(self.h, C.byref(s)))
        return {"proposed": s.proposed, "accepted": s.accepted, "proposal_batches": s.proposal_batches,
                "rejected_batches": s.rejected_batches}

    def call_widths(self) -> list[int]:
        n = _check(load().mc_batch_call_widths(self.h, None, 0))
        out = np.zeros(max(n, 1), dtype=np.int32)
        load().mc_batch_call_widths(self.h, _p(out), n)
        return out[:n].tolist()

    def set_profiling(self, enabled: bool) -> None:
        _check(load().mc_batch_set_profiling(self.h, 1 if enabled else 0))

    def profile(self, kind: int):
        ms, by, n = C.c_double(), C.c_double(), C.c_int32()
        _check(load().mc_batch_profile(self.h, kind, C.byref(ms), C.byref(by), C.byref(n)))
        return ms.value, by.value, n.value


def ngram_propose(histories, max_suffix: int, min_context: int, limits) -> list[list[int]]:
    """GPU n-gram proposer over host histories (one proposal per history)."""
    B = len(histories)
    off = np.zeros(B + 1, dtype=np.int64)
    for i, h in enumerate(histories):
        off[i + 1] = off[i] + len(h)
    flat = _i32(np.concatenate([np.asarray(h, dtype=np.int32) for h in histories]) if B else np.zeros(0))
    lim = _i32(limits)
    stride = max(1, int(lim.max()) if B else 1)
    out = np.zeros((B, stride), dtype=np.int32)
    n = np.zeros(B, dtype=np.int32)
    _check(load().mc_ngram_propose(_p(flat) if flat.size else None, _p(off), B, max_suffix, min_context, _p(lim),
                                   stride, _p(out), _p(n)))
    return [out[i, : n[i]].tolist() for i in range(B)]


def accept(logits_rows: list[np.ndarray], drafts: list[list[int]], samplings: list[Sampling], counters,
           acceptance: int, generated=None, uniforms=None):
    """GPU acceptance over host logits: row r has len(drafts[r]) + 1 logits rows;
    generated[r] the row's generated tokens so far (penalties, min_tokens); uniforms[r] a
    [len(drafts[r]) + 1][2] array of caller draws (None = derived from seed and counter)."""
    B = len(drafts)
    V = logits_rows[0].shape[1]
    stride = max(1, max(len(d) for d in drafts))
    off = np.zeros(B + 1, dtype=np.int64)
    for r in range(B):
        off[r + 1] = off[r] + len(drafts[r]) + 1
    lg = np.ascontiguousarray(np.concatenate(logits_rows, axis=0), dtype=np.uint16)
    dr = np.zeros((B, stride), dtype=np.int32)
    nd = np.zeros(B, dtype=np.int32)
    for r, d in enumerate(drafts):
        dr[r, : len(d)] = d
        nd[r] = len(d)
    sp = (Sampling * B)(*samplings)
    ctr = np.ascontiguousarray(counters, dtype=np.uint64)
    gen = goff = None
    if generated is not None:
        goff = np.zeros(B + 1, dtype=np.int64)
        for r in range(B):
            goff[r + 1] = goff[r] + len(generated[r])
        gen = _i32(np.concatenate([np.asarray(g, dtype=np.int32) for g in generated]) if goff[-1] else np.zeros(1))
    u = None
    if uniforms is not None:
        u = np.zeros((B, stride + 1, 2), dtype=np.uint32)
        for r in range(B):
            ur = np.asarray(uniforms[r], dtype=np.uint32).reshape(-1, 2)
            u[r, : len(ur)] = ur
    out = np.zeros((B, stride + 1), dtype=np.int32)
    n_emit = np.zeros(B, dtype=np.int32)
    keep = np.zeros(B, dtype=np.int32)
    nacc = np.zeros(B, dtype=np.int32)
    _check(load().mc_accept(_p(lg), V, B, _p(off), _p(dr), stride, _p(nd), C.cast(sp, C.c_void_p), _p(gen), _p(goff),
                            _p(ctr), _p(u), acceptance, _p(out), _p(n_emit), _p(keep), _p(nacc)))
    return [out[r, : n_emit[r]].tolist() for r in range(B)], keep.tolist(), nacc.tolist()


def accept_noalloc(logits_ptr: int, vocab: int, B: int, K: int, drafts_ptr: int, n_draft_ptr: int,
                   samplings: list[Sampling], counters, uniforms_ptr: int | None, acceptance: int, out_ptr: int,
                   n_emit_ptr: int, keep_ptr: int, nacc_ptr: int) -> None:
    """mc_accept_noalloc over device buffers given as raw addresses (logits [B][K+1][V] bf16,
    drafts [B][K], n_draft [B], uniforms [B][K+1][2] or None; outputs out [B][K+1], n_emit,
    kv_keep, n_accepted [B], all int32)."""
    sp = (Sampling * B)(*samplings)
    ctr = np.ascontiguousarray(counters, dtype=np.uint64)
    _check(load().mc_accept_noalloc(C.c_void_p(logits_ptr), vocab, B, K, C.c_void_p(drafts_ptr),
                                    C.c_void_p(n_draft_ptr), C.cast(sp, C.c_void_p), _p(ctr),
                                    C.c_void_p(uniforms_ptr) if uniforms_ptr else None, acceptance,
                                    C.c_void_p(out_ptr), C.c_void_p(n_emit_ptr), C.c_void_p(keep_ptr),
                                    C.c_void_p(nacc_ptr)))


def probe_hbm_read(nbytes: int, launches: int) -> tuple[float, float]:
    """(us per launch, GB/s) of a streaming read of nbytes per launch, each launch from its
    own slice of a pool larger than the Infinity Cache (mc_probe_hbm_read)."""
    us, gbs = C.c_double(), C.c_double()
    _check(load().mc_probe_hbm_read(nbytes, launches, C.byref(us), C.byref(gbs)))
    return us.value, gbs.value
