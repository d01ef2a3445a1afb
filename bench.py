"""Benchmark of the n-gram speculative-decode step on one MI355X.

Workload (default): Qwen3-4B-shaped dense decoder (36 layers, hidden 2560, 32 q / 8 kv
heads, head_dim 128, intermediate 9728, vocab 151936, tied embeddings), random-init
weights in MLX 4-bit affine g64 format with bf16 scales/biases, batch 1, greedy,
n-gram drafts with K=5 and match length 3, a 2048-token seeded prompt with 40% of its
positions copied from earlier spans.  A step is one speculative step (n-gram proposal,
(K+1)-token verify forward, acceptance, KV rollback); the prompt is prefilled before
the timed region.  The same workload at batch 8 is reported beside it.

Prints one JSON line: accepted tokens/s at batch 1 (value), the batch-8 figure, the
verify-step latency, the live HBM roofline of the dominant kernel (the dequant GEMV, timed
with HIP events on its stream),
its measured HBM traffic per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, recorded in
profiles/), and the CPU oracle timed on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
QWEN3_4B = dict(arch=0, n_layers=36, hidden=2560, n_q_heads=32, n_kv_heads=8, head_dim=128, intermediate=9728,
                vocab=151936, tied_embeddings=1, rms_eps=1e-6, rope_theta=1e6, n_experts=0, n_experts_per_tok=0,
                moe_intermediate=0)
K_DRAFT, MATCH, PROMPT_LEN, DECODE, SEED = 5, 3, 2048, 256, 1234
# HBM bytes per launch of the verify GEMVs, measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
# (scaled by the same counters over a plain 256 MiB copy); the commands are in the
# summary beside this file
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qgemv_traffic_qwen3_4b_k5.json")


def measured_traffic(kernel: str):
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t.get("traffic_bytes_per_launch") if t.get("kernel") == kernel else None


def spec_cfg(rows: int) -> dict:
    return dict(enabled=1, max_proposal_tokens=K_DRAFT, max_suffix_tokens=MATCH, min_context_tokens=8,
                acceptance=1, single_row_only=0, greedy_only=0)


def step_bytes(cfg: dict, ctx_lens, M: int) -> float:
    """Algorithmic HBM bytes of one verify step: 4-bit g64 weights at 0.5625 B/weight,
    K/V read over each row's context, K/V written for the M verify tokens, bf16 logits."""
    H, d, nq, nkv, I, V, L = (cfg[k] for k in ("hidden", "head_dim", "n_q_heads", "n_kv_heads", "intermediate",
                                               "vocab", "n_layers"))
    per_layer = (nq + 2 * nkv) * d * H + H * nq * d + 2 * I * H + H * I
    weights = (L * per_layer + V * H) * 0.5625
    kv_tok = L * 2 * nkv * d * 2
    return weights + sum(ctx_lens) * kv_tok + M * kv_tok + M * V * 2


def run_gpu(rows: int, steps: int, warmup: int, profile: bool, forced: bool = False, decode: int = DECODE):
    """The 256-token decode of the workload: W warmup steps and an untimed prefix, then the
    timed steps, placed so that the timed window ends near token 256 (the rows' budget is
    256 plus the timed steps' worth, so no row finishes inside it).  forced: exactly L drafts
    accepted per row per step, L uniform in [0, K], then the history's next token (the
    survey's forced accept-length schedule: throughput at a known acceptance, whatever the
    random-init weights agree with)."""
    from mlxcat_amd import _lib as hip
    from mlxcat_amd.workloads import copy_span_prompt
    L = hip.load()
    if L.mc_set_device(0) < 0:
        raise RuntimeError(L.mc_last_error().decode())
    m = hip.Model(QWEN3_4B)
    m.init_synthetic(SEED)
    rng = np.random.default_rng(SEED + 17)
    max_new = decode + (steps + 1) * (K_DRAFT + 1)
    ctx = PROMPT_LEN + max_new + K_DRAFT + 16
    b = hip.Batch(m, rows, ctx, spec_cfg(rows))
    generated = np.ones(rows, dtype=np.int64)  # the first token, sampled at admission
    for r in range(rows):
        p = copy_span_prompt(SEED + r, PROMPT_LEN, QWEN3_4B["vocab"])
        b.insert(r, p, max_new, hip.make_sampling())
    fa = (lambda: rng.integers(0, K_DRAFT + 1, rows).astype(np.int32)) if forced else (lambda: None)
    for _ in range(warmup):
        generated += b.step(fa())[1]
    # untimed prefix: until the timed steps at the warm-up rate end at token DECODE
    rate = max(1.0, (generated.min() - 1) / max(1, warmup))
    prefix = 0
    while generated.min() < decode - steps * rate and prefix < 4 * decode:
        generated += b.step(fa())[1]
        prefix += 1
    st0 = b.stats()
    kv0 = [b.kv_len(r) for r in range(rows)]
    emitted = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        _, c, _ = b.step(fa())
        emitted += int(c.sum())
        generated += c
    dt = time.perf_counter() - t0
    st1 = b.stats()
    out = dict(tok_s=emitted / dt, ms_per_step=dt / steps * 1e3, tokens_per_step=emitted / steps / rows,
               proposed=st1["proposed"] - st0["proposed"], accepted=st1["accepted"] - st0["accepted"],
               batches=st1["proposal_batches"] - st0["proposal_batches"],
               bytes_per_step=step_bytes(QWEN3_4B, kv0, rows * (K_DRAFT + 1)),
               timed_tokens=[int(generated.min() - emitted // rows), int(generated.max())], prefix_steps=prefix)
    out["step_hbm_gbs"] = out["bytes_per_step"] / (out["ms_per_step"] * 1e-3) / 1e9
    if profile:
        # kind 0: the dequant GEMVs of the verify forward, each timed by the start and end events
        # of its own launch (hipExtLaunchKernel on the batch stream: the kernel's execution)
        b.set_profiling(True)
        acc = [0.0, 0.0, 0]
        for _ in range(3):
            b.step(fa())
            ms, by, n = b.profile(0)
            acc[0] += ms
            acc[1] += by
            acc[2] += n
        b.set_profiling(False)
        out["dominant"] = dict(ms=acc[0] / 3, bytes=acc[1] / 3, launches=acc[2] // 3, kernel="qgemv_kernel<1>")
    b.close()
    m.close()
    return out


def moe_step_bytes(cfg: dict, ctx_lens, M: int) -> float:
    """Algorithmic bytes of a Qwen3-MoE verify step: attention projections, router and the
    expected number of distinct experts M tokens touch under uniform routing,
    E (1 - (1 - k/E)^M), per layer; K/V and logits as for the dense decoder."""
    H, d, nq, nkv, V, L = (cfg[k] for k in ("hidden", "head_dim", "n_q_heads", "n_kv_heads", "vocab", "n_layers"))
    E, TK, MI = cfg["n_experts"], cfg["n_experts_per_tok"], cfg["moe_intermediate"]
    touched = E * (1.0 - (1.0 - TK / E) ** M)
    per_layer = (nq + 2 * nkv) * d * H + H * nq * d + E * H + touched * 3 * MI * H
    weights = (L * per_layer + V * H) * 0.5625
    kv_tok = L * 2 * nkv * d * 2
    return weights + sum(ctx_lens) * kv_tok + M * kv_tok + M * V * 2


# The survey's other workloads (parity-tested; measured here on demand, not the headline):
# (model, rows, K, context lengths (lo, hi), sampling per row, forced accept-length schedule)
CONFIGS = {
    "cfg3": ("llama3-8b", 8, 4, (512, 4096), "t0.7-topp0.95", False),
    "cfg4": ("qwen3-30b-a3b", 4, 4, (1024, 1024), "greedy", False),
    "cfg5": ("qwen3-8b", 32, 8, (16384, 16384), "even-greedy-odd-seeded", True),
}


def run_config(name: str, steps: int, warmup: int) -> dict:
    """One of CONFIGS: synthetic K/V for each row's context, seeded copy-span prompts, then
    speculative steps (a forced accept length uniform in [0, K] per row per step where the
    configuration asks for it)."""
    from mlxcat_amd import _lib as hip
    from mlxcat_amd.workloads import MODELS, copy_span_prompt
    model, rows, k, (lo, hi), samp, forced = CONFIGS[name]
    cfg = MODELS[model]
    L = hip.load()
    if L.mc_set_device(0) < 0:
        raise RuntimeError(L.mc_last_error().decode())
    m = hip.Model(cfg)
    m.init_synthetic(SEED)
    rng = np.random.default_rng(SEED)
    lens = [int(x) for x in rng.integers(lo, hi + 1, rows)]
    max_new = (warmup + steps + 4) * (k + 1) + 8
    spec = dict(enabled=1, max_proposal_tokens=k, max_suffix_tokens=MATCH, min_context_tokens=8, acceptance=1,
                single_row_only=0, greedy_only=0)
    b = hip.Batch(m, rows, max(lens) + max_new + k + 16, spec)
    for r in range(rows):
        if samp == "greedy" or (samp == "even-greedy-odd-seeded" and r % 2 == 0):
            sp = hip.make_sampling()
        elif samp == "even-greedy-odd-seeded":
            sp = hip.make_sampling(temperature=0.7, top_p=0.95, seed=SEED + r)
        else:
            sp = hip.make_sampling(temperature=0.7, top_p=0.95, seed=SEED + r)
        b.fill_synthetic_kv(r, lens[r] - 1, 99 + r)
        b.insert_prefilled(r, copy_span_prompt(SEED + r, lens[r], cfg["vocab"]), max_new, sp)
    fa = (lambda: rng.integers(0, k + 1, rows).astype(np.int32)) if forced else (lambda: None)
    for _ in range(warmup):
        b.step(fa())
    kv0 = [b.kv_len(r) for r in range(rows)]
    emitted = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        _, c, _ = b.step(fa())
        emitted += int(c.sum())
    dt = time.perf_counter() - t0
    M = rows * (k + 1)
    by = moe_step_bytes(cfg, kv0, M) if cfg["n_experts"] else step_bytes(cfg, kv0, M)
    ms = dt / steps * 1e3
    b.close()
    m.close()
    return {"config": {"workload": f"{model}-shape 4-bit g64 n-gram speculative step", "batch": rows, "k_draft": k,
                       "context": [lo, hi], "sampling": samp, "forced_accept_schedule": forced},
            "value": round(emitted / dt, 2), "unit": "tok/s", "ms_per_step": round(ms, 4), "steps": steps,
            "warmup": warmup, "tokens_per_step_per_row": round(emitted / steps / rows, 3), "verify_tokens": M,
            "verify_step_hbm": {"achieved": round(by / (ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_step": by},
            "dtype": "bf16", "data": "synthetic (random-init weights, synthetic K/V, seeded copy-span prompts)"}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run_cpu(rows: int = 1, budget_s: float = 15.0):
    """The oracle (CPU restatement, OpenMP) on a bounded sample of the same step: synthetic
    K/V for each row's 2047 prefilled positions, then speculative steps until the time
    budget is spent."""
    from mlxcat_amd.workloads import copy_span_prompt
    from oracle import pyoracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    O.lib().or_set_threads(threads)
    om = O.Model(QWEN3_4B, SEED, PROMPT_LEN + 128, rows)
    g = O.Generator(om, spec_cfg(rows), rows, PROMPT_LEN + 128)
    for r in range(rows):
        om.fill_kv(r, PROMPT_LEN - 1, 99 + r)
        g.insert_prefilled(r, copy_span_prompt(SEED + r, PROMPT_LEN, QWEN3_4B["vocab"]), 100, O.make_sampling())
    g.step()  # warm-up
    n_steps = emitted = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s and n_steps < 50:
        _, c, _ = g.step()
        emitted += int(c.sum())
        n_steps += 1
    dt = time.perf_counter() - t0
    om.close()
    return dict(value=emitted / dt, unit="tok/s", cores=threads, kind="port", cpu_model=cpu_model(),
                sample=f"{n_steps} speculative steps of the batch-{rows} Qwen3-4B-shape K=5 workload "
                       f"({emitted} tokens, {dt:.1f} s) after a synthetic 2047-position KV prefill per row")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-b8", action="store_true")
    ap.add_argument("--no-forced", action="store_true", help="skip the forced accept-length run")
    ap.add_argument("--decode", type=int, default=DECODE,
                    help="tokens decoded by the end of the timed window (shorter for counter runs, where every "
                         "launch is serialised)")
    ap.add_argument("--config", choices=sorted(CONFIGS), default=None,
                    help="measure one of the other workloads instead (its own JSON line)")
    ap.add_argument("--copy-ref", action="store_true",
                    help="only copy 256 MiB three times (a plain copy kernel of known size: the scale of the "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--read-probe", action="store_true",
                    help="only the HBM read ceiling: a streaming read of 9 MB .. 4 GiB per launch, each launch "
                         "from its own slice of a pool larger than the Infinity Cache")
    a = ap.parse_args()
    if a.read_probe:
        from mlxcat_amd import _lib as hip
        hip.load().mc_set_device(0)
        for nbytes, launches in ((9 << 20, 2000), (28 << 20, 1000), (64 << 20, 500), (219 << 20, 200),
                                 (1 << 30, 50), (4 << 30, 20)):
            us, gbs = hip.probe_hbm_read(nbytes, launches)
            print(json.dumps({"probe": "hbm_read", "bytes_per_launch": nbytes, "launches": launches,
                              "us_per_launch": round(us, 3), "GB_per_s": round(gbs, 1),
                              "frac_of_8TBs": round(gbs / HBM_PEAK_GBS, 4)}), flush=True)
        return
    if a.copy_ref:
        import torch
        src = torch.ones(256 << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("copied 3 x 256 MiB", flush=True)
        return
    if a.config:
        if a.gpus != 1:
            print("bench.py measures one GPU", file=sys.stderr)
            sys.exit(2)
        out = run_config(a.config, max(3, a.steps // 4), max(2, a.warmup // 2))
        out.update({"metric": f"accepted tok/s ({a.config})", "n_gpus": 1, "higher_is_better": True})
        print(json.dumps(out), flush=True)
        return
    if a.gpus != 1:
        print("bench.py measures one GPU: the speculative step is built and measured on a single MI355X "
              "(see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)
    b1 = run_gpu(1, a.steps, a.warmup, profile=True, decode=a.decode)
    b1f = None if a.no_forced else run_gpu(1, a.steps, a.warmup, profile=False, forced=True, decode=a.decode)
    b8 = None if a.no_b8 else run_gpu(8, max(8, a.steps // 2), a.warmup, profile=False, decode=a.decode)
    cpu = None if a.no_cpu else run_cpu(1)
    cpu8 = None if (a.no_cpu or a.no_b8) else run_cpu(8, budget_s=10.0)
    if cpu is not None and cpu8 is not None:
        cpu["batch8"] = {k: cpu8[k] for k in ("value", "unit", "sample")}
    g = b1["dominant"]
    achieved = g["bytes"] / (g["ms"] * 1e-3) / 1e9
    line = {
        "metric": "accepted tok/s (bs=1,8) Qwen3-4B-shape 4-bit K=5; verify HBM GB/s %peak",
        "value": round(b1["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(b1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init MLX 4-bit affine g64 weights, seeded copy-span prompts)",
        "config": {"workload": "Qwen3-4B-shape 4-bit g64 n-gram speculative step, batch 1, K=5, match 3, "
                               "2048-token prompt, greedy, 256-token decode", "batch": 1, "k_draft": K_DRAFT,
                   "prompt": PROMPT_LEN, "decode": a.decode, "timed_tokens": b1["timed_tokens"]},
        "tokens_per_step": round(b1["tokens_per_step"], 3),
        "draft_hit_rate": round(b1["batches"] / a.steps, 3),
        "accepted_drafts_per_step": round(b1["accepted"] / a.steps, 3),
        "verify_step_ms": round(b1["ms_per_step"], 4),
        "verify_step_hbm": {"achieved": round(b1["step_hbm_gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(b1["step_hbm_gbs"] / HBM_PEAK_GBS, 4),
                            "bytes_per_step": b1["bytes_per_step"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(g["kernel"]),
                     "kernel": g["kernel"], "launches_per_step": g["launches"],
                     "avg_launch_us": round(g["ms"] / max(1, g["launches"]) * 1e3, 3),
                     "alg_bytes_per_launch": round(g["bytes"] / max(1, g["launches"]))},
        "forced_accept": None if b1f is None else {"schedule": "exactly L ~ U[0, K] drafts accepted per step, then the history's next token "
                                      "(a stress of the speculative mechanics: the row keeps copying its history, "
                                      "so every step proposes; the tokens are not the model's)",
                          "tok_s": round(b1f["tok_s"], 2),
                          "ms_per_step": round(b1f["ms_per_step"], 4),
                          "tokens_per_step": round(b1f["tokens_per_step"], 3),
                          "accepted_drafts_per_step": round(b1f["accepted"] / a.steps, 3)},
        "batch8": None if b8 is None else {"tok_s": round(b8["tok_s"], 2), "ms_per_step": round(b8["ms_per_step"], 4),
                                           "tokens_per_step_per_row": round(b8["tokens_per_step"], 3),
                                           "step_hbm_frac": round(b8["step_hbm_gbs"] / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
