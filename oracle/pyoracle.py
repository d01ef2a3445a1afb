"""ctypes binding of the CPU oracle (oracle/build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the mlxcat_amd product package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")

ARCH_QWEN3, ARCH_LLAMA, ARCH_QWEN3_MOE = 0, 1, 2
ARCH_FAKE_REPEATING, ARCH_FAKE_MISMATCHING = 100, 101
ACCEPT_ALL_OR_NOTHING, ACCEPT_PREFIX = 0, 1
T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN = 0, 1, 2, 3, 4, 5, 6
T_IN_NORM, T_POST_NORM, T_Q_NORM, T_K_NORM, T_ROUTER = 7, 8, 9, 10, 11


def build(force: bool = False) -> None:
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-s"] + (["-B"] if force else []), check=True)


class Config(C.Structure):
    _fields_ = [
        ("arch", C.c_int), ("n_layers", C.c_int), ("hidden", C.c_int), ("n_q_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("intermediate", C.c_int), ("vocab", C.c_int),
        ("tied_embeddings", C.c_int), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("n_experts", C.c_int), ("n_experts_per_tok", C.c_int), ("moe_intermediate", C.c_int),
    ]


class SpecConfig(C.Structure):
    _fields_ = [
        ("enabled", C.c_int), ("max_proposal_tokens", C.c_int), ("max_suffix_tokens", C.c_int),
        ("min_context_tokens", C.c_int), ("acceptance", C.c_int), ("single_row_only", C.c_int),
        ("greedy_only", C.c_int),
    ]


class Sampling(C.Structure):
    _fields_ = [
        ("temperature", C.c_float), ("top_p", C.c_float), ("has_seed", C.c_int), ("seed", C.c_uint64),
        ("n_eos", C.c_int), ("eos", C.c_int32 * 8), ("reject_token", C.c_int32), ("top_k", C.c_int32),
        ("min_p", C.c_float), ("repetition_penalty", C.c_float), ("presence_penalty", C.c_float),
        ("frequency_penalty", C.c_float), ("min_tokens", C.c_int32), ("n_bias", C.c_int32),
        ("bias_token", C.c_int32 * 16), ("bias_value", C.c_float * 16),
    ]


class Stats(C.Structure):
    _fields_ = [("proposed", C.c_int64), ("accepted", C.c_int64), ("proposal_batches", C.c_int64),
                ("rejected_batches", C.c_int64)]


class Dist(C.Structure):
    _fields_ = [("total", C.c_uint64), ("max_logit", C.c_float), ("tau", C.c_float), ("filtered", C.c_int),
                ("min_p_log", C.c_float), ("topk_value", C.c_float), ("topk_index", C.c_int32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(LIB_PATH)
        P, I, U64, U32, F = C.c_void_p, C.c_int, C.c_uint64, C.c_uint32, C.c_float
        sig = {
            "or_mix64": (U64, [U64]),
            "or_uniform_u32": (U32, [U64, U64, U32, U32]),
            "or_f32_to_bf16": (C.c_uint16, [F]),
            "or_bf16_to_f32": (F, [C.c_uint16]),
            "or_gen_linear": (None, [U64, U64, I, I, I, P, P, P]),
            "or_gen_norm": (None, [U64, U64, I, P]),
            "or_tensor_id": (U64, [I, I]),
            "or_expert_tensor_id": (U64, [I, I, I]),
            "or_exp_neg": (F, [F]),
            "or_ngram_propose": (I, [P, I, I, I, I, P]),
            "or_argmax_bf16": (I, [P, I]),
            "or_dist_build": (None, [P, I, F, F, P]),
            "or_dist_mass": (U64, [P, P, F, I]),
            "or_dist_sample": (I, [P, P, I, F, U32, I]),
            "or_dist_build_f": (None, [P, I, F, F, I, F, P]),
            "or_dist_mass_f": (U64, [P, P, F, I]),
            "or_dist_sample_f": (I, [P, P, I, F, U32, I]),
            "or_min_p_log": (F, [F]),
            "or_process_logits": (I, [P, I, P, P, I, P]),
            "or_batch_trim": (I, [P, I, P, P, I]),
            "or_accept_row": (I, [P, I, P, I, P, P, I, U64, U64, P, I, I, I, P, P, P, P]),
            "or_qmatmul": (None, [P, P, P, I, I, P, I, P]),
            "or_model_create": (P, [P, U64, I, I]),
            "or_model_destroy": (None, [P]),
            "or_model_linear": (I, [P, I, I, I, P, P, P, P, P]),
            "or_model_rope_cos": (P, [P]),
            "or_model_rope_sin": (P, [P]),
            "or_kv_len": (I, [P, I]),
            "or_kv_set_len": (None, [P, I, I]),
            "or_kv_fill_synthetic": (None, [P, I, I, U64]),
            "or_kv_read": (None, [P, I, I, I, P]),
            "or_forward": (I, [P, I, P, P, P, P]),
            "or_forward_trace": (I, [P, I, P, P, P, P, P]),
            "or_forward_attn": (I, [P, I, P, P, P, P, P, P]),
            "or_set_threads": (None, [I]),
            "or_set_reduction_order": (None, [I]),
            "or_capture_router": (None, [P]),
            "or_generator_create": (P, [P, P, I, I, U64]),
            "or_generator_destroy": (None, [P]),
            "or_generator_insert": (I, [P, I, P, I, I, P, P]),
            "or_generator_insert_prefilled": (I, [P, I, P, I, I, P]),
            "or_generator_remove": (None, [P, I]),
            "or_generator_step": (I, [P, P, P, P, P]),
            "or_generator_stats": (None, [P, P]),
            "or_generator_call_widths": (I, [P, P, I]),
            "or_generator_active": (I, [P, I]),
            "or_generator_history": (I, [P, I, P, I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def i32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def ngram_propose(ctx, max_suffix: int, min_context: int, limit: int) -> list[int]:
    c = i32(ctx)
    out = np.zeros(max(limit, 1), dtype=np.int32)
    n = lib().or_ngram_propose(_p(c), len(c), max_suffix, min_context, limit, _p(out))
    return out[:n].tolist()


def gen_linear(seed: int, tid: int, N: int, K: int, scale_exp: int = -7):
    wq = np.zeros((N, K // 8), dtype=np.uint32)
    s = np.zeros((N, K // 64), dtype=np.uint16)
    b = np.zeros((N, K // 64), dtype=np.uint16)
    lib().or_gen_linear(seed, tid, N, K, scale_exp, _p(wq), _p(s), _p(b))
    return wq, s, b


def qmatmul(wq, s, b, x) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    N, K = wq.shape[0], wq.shape[1] * 8
    M = x.shape[0]
    y = np.zeros((M, N), dtype=np.float32)
    lib().or_qmatmul(_p(wq), _p(s), _p(b), N, K, _p(x), M, _p(y))
    return y


def accept_row(logits_bf16: np.ndarray, drafts, sampling: "Sampling", seed: int, counter: int, acceptance: int,
               forced_cap: int = -1, generated=(), uniforms=None, ext=None):
    """Acceptance of one row: logits_bf16 [P+1][V] uint16, drafts P tokens, `generated` the
    request's generated tokens so far, `uniforms` [P+1][2] caller draws (None = derived).
    `ext`: the history's token after the drafts (the forced schedule's continuation), or None.
    Returns (emitted tokens, kv_keep, n_accepted, rejected)."""
    lg = np.ascontiguousarray(logits_bf16, dtype=np.uint16)
    dr = i32(list(drafts) + ([ext] if ext is not None else [0]))
    P = len(drafts)
    assert lg.shape[0] == P + 1
    gen = i32(generated) if len(generated) else np.zeros(1, dtype=np.int32)
    u = None
    if uniforms is not None:
        u = np.ascontiguousarray(uniforms, dtype=np.uint32).reshape(-1)
        assert u.size >= 2 * (P + 1)
    out = np.zeros(P + 1, dtype=np.int32)
    keep, nacc, rej = C.c_int(), C.c_int(), C.c_int()
    n = lib().or_accept_row(_p(lg), lg.shape[1], _p(dr), P, C.byref(sampling), _p(gen), len(generated), seed,
                            counter, _p(u) if u is not None else None, acceptance, forced_cap,
                            1 if ext is not None else 0, _p(out), C.byref(keep), C.byref(nacc), C.byref(rej))
    return out[:n].tolist(), keep.value, nacc.value, rej.value


def process_logits(logits_bf16: np.ndarray, sampling: "Sampling", generated=()) -> np.ndarray:
    """The fp32 values one position samples from (bias, min_tokens mask, penalties)."""
    lg = np.ascontiguousarray(logits_bf16, dtype=np.uint16)
    gen = i32(generated) if len(generated) else np.zeros(1, dtype=np.int32)
    out = np.zeros(len(lg), dtype=np.float32)
    lib().or_process_logits(_p(lg), len(lg), C.byref(sampling), _p(gen), len(generated), _p(out))
    return out


def dist_build(logits_bf16: np.ndarray, temperature: float, top_p: float) -> Dist:
    lg = np.ascontiguousarray(logits_bf16, dtype=np.uint16)
    d = Dist()
    lib().or_dist_build(_p(lg), len(lg), temperature, top_p, C.byref(d))
    return d


def dist_build_f(values: np.ndarray, temperature: float, top_p: float = 0.0, top_k: int = 0,
                 min_p: float = 0.0) -> Dist:
    v = np.ascontiguousarray(values, dtype=np.float32)
    d = Dist()
    lib().or_dist_build_f(_p(v), len(v), temperature, top_p, top_k, lib().or_min_p_log(min_p), C.byref(d))
    return d


def kept_mask(d: Dist, values: np.ndarray) -> np.ndarray:
    """Tokens with positive mass at temperature 1 under the filters of d."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    return np.array([lib().or_dist_mass_f(C.byref(d), _p(v), 1.0, i) > 0 for i in range(len(v))])


class Model:
    def __init__(self, cfg: dict, seed: int, max_ctx: int, max_rows: int):
        self.cfg = Config(**cfg)
        self.h = lib().or_model_create(C.byref(self.cfg), seed, max_ctx, max_rows)
        self.max_ctx, self.max_rows = max_ctx, max_rows

    def close(self):
        if self.h:
            lib().or_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def linear(self, layer: int, which: int, expert: int = -1):
        wq, s, b = C.c_void_p(), C.c_void_p(), C.c_void_p()
        N, K = C.c_int(), C.c_int()
        rc = lib().or_model_linear(self.h, layer, which, expert, C.byref(wq), C.byref(s), C.byref(b),
                                   C.byref(N), C.byref(K))
        if rc:
            raise KeyError((layer, which, expert))
        n, k = N.value, K.value
        wq_a = np.ctypeslib.as_array(C.cast(wq, C.POINTER(C.c_uint32)), (n, k // 8)).copy()
        s_a = np.ctypeslib.as_array(C.cast(s, C.POINTER(C.c_uint16)), (n, k // 64)).copy()
        b_a = np.ctypeslib.as_array(C.cast(b, C.POINTER(C.c_uint16)), (n, k // 64)).copy()
        return wq_a, s_a, b_a

    def kv_len(self, row: int) -> int:
        return lib().or_kv_len(self.h, row)

    def set_kv_len(self, row: int, n: int) -> None:
        lib().or_kv_set_len(self.h, row, n)

    def fill_kv(self, row: int, n: int, seed: int) -> None:
        lib().or_kv_fill_synthetic(self.h, row, n, seed)

    def kv(self, layer: int, row: int, which_v: int) -> np.ndarray:
        c = self.cfg
        out = np.zeros((c.n_kv_heads, self.kv_len(row), c.head_dim), dtype=np.uint16)
        lib().or_kv_read(self.h, layer, row, which_v, _p(out))
        return out

    def forward(self, rows, counts, tokens, want_logits=True, trace=False, attention=False, router=False):
        """Logits [M][V]; with trace=True also the hidden states, with attention=True also each
        layer's attention output [layers][M][nq * d], with router=True also each layer's bf16
        router logits [layers][M][n_experts] (returned as a tuple in that order)."""
        rows, counts, tokens = i32(rows), i32(counts), i32(tokens)
        M = int(counts.sum())
        c = self.cfg
        lg = np.zeros((M, c.vocab), dtype=np.uint16) if want_logits else None
        hid = np.zeros((c.n_layers + 1, M, c.hidden), dtype=np.uint16) if trace else None
        att = np.zeros((c.n_layers, M, c.n_q_heads * c.head_dim), dtype=np.uint16) if attention else None
        rl = np.zeros((c.n_layers, M, max(1, c.n_experts)), dtype=np.uint16) if router else None
        if rl is not None:
            lib().or_capture_router(_p(rl))
        try:
            rc = lib().or_forward_attn(self.h, len(rows), _p(rows), _p(counts), _p(tokens),
                                       _p(lg) if lg is not None else None, _p(hid) if hid is not None else None,
                                       _p(att) if att is not None else None)
        finally:
            if rl is not None:
                lib().or_capture_router(None)
        if rc:
            raise RuntimeError(f"or_forward failed: {rc}")
        out = [lg] + ([hid] if trace else []) + ([att] if attention else []) + ([rl] if router else [])
        return tuple(out) if len(out) > 1 else lg


class reversed_reduction_order:
    """Context: every fp32 reduction of the oracle's forward runs in another order."""

    def __enter__(self):
        lib().or_set_reduction_order(1)
        return self

    def __exit__(self, *exc):
        lib().or_set_reduction_order(0)
        return False


def make_sampling(temperature=0.0, top_p=0.0, seed=None, eos=(), reject_token=-1, top_k=0, min_p=0.0,
                  repetition_penalty=1.0, presence_penalty=0.0, frequency_penalty=0.0, min_tokens=0,
                  logit_bias=None) -> Sampling:
    sp = Sampling()
    sp.temperature = temperature
    sp.top_p = top_p
    sp.has_seed = 0 if seed is None else 1
    sp.seed = 0 if seed is None else seed
    sp.n_eos = len(eos)
    for i, e in enumerate(eos):
        sp.eos[i] = e
    sp.reject_token = reject_token
    sp.top_k = top_k
    sp.min_p = min_p
    sp.repetition_penalty = repetition_penalty
    sp.presence_penalty = presence_penalty
    sp.frequency_penalty = frequency_penalty
    sp.min_tokens = max(0, min_tokens)
    bias = sorted((logit_bias or {}).items())
    assert len(bias) <= 16
    sp.n_bias = len(bias)
    for i, (t, b) in enumerate(bias):
        sp.bias_token[i] = t
        sp.bias_value[i] = b
    return sp


class Generator:
    """Restatement of ContinuousBatchGenerator + Scheduler.step over the oracle model."""

    def __init__(self, model: Model, spec: dict, max_rows: int, max_hist: int, global_seed: int = 7):
        self.model = model
        self.spec = SpecConfig(**spec)
        self.K = self.spec.max_proposal_tokens
        self.max_rows = max_rows
        self.h = lib().or_generator_create(model.h, C.byref(self.spec), max_rows, max_hist, global_seed)

    def close(self):
        if self.h:
            lib().or_generator_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def insert(self, row: int, prompt, max_tokens: int, sampling: Sampling):
        p = i32(prompt)
        fin = C.c_int(0)
        tok = lib().or_generator_insert(self.h, row, _p(p), len(p), max_tokens, C.byref(sampling), C.byref(fin))
        if tok < 0:
            raise RuntimeError(f"insert failed {tok}")
        return tok, fin.value

    def insert_prefilled(self, row: int, ctx, max_tokens: int, sampling: Sampling):
        c = i32(ctx)
        rc = lib().or_generator_insert_prefilled(self.h, row, _p(c), len(c), max_tokens, C.byref(sampling))
        if rc:
            raise RuntimeError(f"insert_prefilled failed {rc}")

    def step(self, forced_accept=None):
        K1 = max(self.K, 0) + 1
        toks = np.zeros((self.max_rows, K1), dtype=np.int32)
        counts = np.zeros(self.max_rows, dtype=np.int32)
        fin = np.zeros(self.max_rows, dtype=np.int32)
        fa = i32(forced_accept) if forced_accept is not None else None
        n = lib().or_generator_step(self.h, _p(toks), _p(counts), _p(fin), _p(fa) if fa is not None else None)
        if n < 0:
            raise RuntimeError("step failed")
        return toks, counts, fin

    def stats(self) -> dict:
        s = Stats()
        lib().or_generator_stats(self.h, C.byref(s))
        return {"proposed": s.proposed, "accepted": s.accepted, "proposal_batches": s.proposal_batches,
                "rejected_batches": s.rejected_batches}

    def call_widths(self) -> list[int]:
        out = np.zeros(4096, dtype=np.int32)
        n = lib().or_generator_call_widths(self.h, _p(out), 4096)
        return out[:n].tolist()

    def active(self, row: int) -> bool:
        return bool(lib().or_generator_active(self.h, row))

    def history(self, row: int) -> list[int]:
        out = np.zeros(1 << 16, dtype=np.int32)
        n = lib().or_generator_history(self.h, row, _p(out), len(out))
        return out[:n].tolist()
