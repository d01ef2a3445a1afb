"""MLX-format checkpoint loader: config.json plus the safetensors shards of an mlx-community
4-bit model, into a device model through the C ABI (mc_model_set_linear / mc_model_set_norm).

The reference reads the model directory's config.json itself (model_type, the layer and head
counts, head_dim, hidden_size, with a text_config fallback:
Sources/MLXCatNative/NativeModelEngine.swift:1147-1231) and leaves the tensors to
mlx-swift-lm, whose Qwen3 / Llama / Qwen3-MoE modules hold every QuantizedLinear as a
.weight (uint32, 8 nibbles per word) / .scales / .biases (bf16, one per group of 64) triplet
and the MoE experts stacked along a leading expert axis (mlp.switch_mlp.*).  This module
restates that layout: names below are the mlx-lm module paths.
"""
from __future__ import annotations

import glob
import json
import os

import numpy as np

from ._lib import (ARCH_LLAMA, ARCH_QWEN3, ARCH_QWEN3_MOE, N_FINAL, N_INPUT, N_K, N_POST, N_Q, W_DOWN, W_EMBED,
                   W_GATE, W_K, W_LM_HEAD, W_O, W_Q, W_ROUTER, W_UP, W_V)

ARCHS = {"qwen3": ARCH_QWEN3, "llama": ARCH_LLAMA, "qwen3_moe": ARCH_QWEN3_MOE}

_ATTN = {"q_proj": W_Q, "k_proj": W_K, "v_proj": W_V, "o_proj": W_O}
_MLP = {"gate_proj": W_GATE, "up_proj": W_UP, "down_proj": W_DOWN}


class LoaderError(ValueError):
    pass


def read_config(path: str) -> dict:
    """The model configuration (mc_model_config fields) from <path>/config.json."""
    with open(os.path.join(path, "config.json")) as f:
        raw = json.load(f)
    text = raw.get("text_config") or {}

    def key(name, default=None):
        if name in raw:
            return raw[name]
        if name in text:
            return text[name]
        if default is not None:
            return default
        raise LoaderError(f"config.json: missing {name}")

    model_type = key("model_type")
    if model_type not in ARCHS:
        raise LoaderError(f"config.json: model_type {model_type!r} is not one of {sorted(ARCHS)}")
    q = raw.get("quantization") or raw.get("quantization_config") or {}
    if q.get("bits") != 4 or q.get("group_size") != 64 or q.get("mode", "affine") != "affine":
        raise LoaderError("only MLX 4-bit affine quantisation with group size 64 is supported "
                          f"(config.json quantization: {q})")
    # mlx-lm records modules quantised differently (an 8-bit MoE router, say) as per-path entries
    for name, v in q.items():
        if isinstance(v, dict) and (v.get("bits", 4) != 4 or v.get("group_size", 64) != 64):
            raise LoaderError(f"{name} is quantised as {v}: every linear must be 4-bit with group size 64")
        if v is False:
            raise LoaderError(f"{name} is not quantised: every linear must be 4-bit with group size 64")
    H, nq = int(key("hidden_size")), int(key("num_attention_heads"))
    cfg = dict(arch=ARCHS[model_type], n_layers=int(key("num_hidden_layers")), hidden=H, n_q_heads=nq,
               n_kv_heads=int(key("num_key_value_heads", nq)), head_dim=int(key("head_dim", H // nq)),
               intermediate=int(key("intermediate_size")), vocab=int(key("vocab_size")),
               tied_embeddings=int(bool(key("tie_word_embeddings", False))), rms_eps=float(key("rms_norm_eps")),
               rope_theta=float(_rope_theta(raw, text)), n_experts=0, n_experts_per_tok=0, moe_intermediate=0)
    if model_type == "qwen3_moe":
        cfg.update(n_experts=int(key("num_experts")), n_experts_per_tok=int(key("num_experts_per_tok")),
                   moe_intermediate=int(key("moe_intermediate_size")))
        if not key("norm_topk_prob", True):
            raise LoaderError("Qwen3-MoE without norm_topk_prob is not supported")
        if int(key("decoder_sparse_step", 1)) != 1 or key("mlp_only_layers", []) not in ([], None):
            raise LoaderError("Qwen3-MoE with dense layers between the sparse ones is not supported")
    return cfg


def _rope_theta(raw: dict, text: dict) -> float:
    for src in (raw, text):
        if "rope_theta" in src:
            return src["rope_theta"]
        rp = src.get("rope_parameters") or src.get("rope_scaling")
        if isinstance(rp, dict) and "rope_theta" in rp:
            if rp.get("rope_type", "default") not in ("default", None):
                raise LoaderError(f"rope scaling {rp.get('rope_type')!r} is not supported")
            return rp["rope_theta"]
    return 10000.0


def tensor_files(path: str) -> list[str]:
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            files = sorted(set(json.load(f)["weight_map"].values()))
        return [os.path.join(path, f) for f in files]
    files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    if not files:
        raise LoaderError(f"{path}: no safetensors files")
    return files


class Checkpoint:
    """The checkpoint's tensors, read one at a time (a 30B MoE is 17 GB of host memory when
    read whole): uint32 words as numpy uint32, bf16 as its uint16 bits."""

    def __init__(self, path: str):
        from safetensors import safe_open
        self._files = [safe_open(fn, framework="pt") for fn in tensor_files(path)]
        self._where = {k: f for f in self._files for k in f.keys()}

    def keys(self):
        return self._where.keys()

    def __getitem__(self, name: str) -> np.ndarray:
        import torch
        t = self._where[name].get_tensor(name)
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).numpy().view(np.uint16)
        if t.dtype == torch.uint32:
            return t.view(torch.int32).numpy().view(np.uint32)
        raise LoaderError(f"{name}: {t.dtype} tensor (4-bit words are uint32, scales, biases and norms bf16)")


def plan(cfg: dict, names) -> list:
    """(kind, layer, slot, expert, prefix) for every tensor the model needs, in load order;
    kind is "linear" (a .weight/.scales/.biases triplet at prefix) or "norm" (prefix.weight).
    Raises when the checkpoint lacks one."""
    names = set(names)
    steps = []

    def lin(layer, slot, prefix, expert=-1):
        for suf in ("weight", "scales", "biases"):
            if f"{prefix}.{suf}" not in names:
                raise LoaderError(f"checkpoint lacks {prefix}.{suf}")
        steps.append(("linear", layer, slot, expert, prefix))

    def norm(layer, slot, prefix):
        if f"{prefix}.weight" not in names:
            raise LoaderError(f"checkpoint lacks {prefix}.weight")
        steps.append(("norm", layer, slot, -1, prefix))

    lin(-1, W_EMBED, "model.embed_tokens")
    if not cfg["tied_embeddings"]:
        lin(-1, W_LM_HEAD, "lm_head")
    norm(-1, N_FINAL, "model.norm")
    for l in range(cfg["n_layers"]):
        p = f"model.layers.{l}"
        for nm, slot in _ATTN.items():
            lin(l, slot, f"{p}.self_attn.{nm}")
        norm(l, N_INPUT, f"{p}.input_layernorm")
        norm(l, N_POST, f"{p}.post_attention_layernorm")
        if cfg["arch"] in (ARCH_QWEN3, ARCH_QWEN3_MOE):
            norm(l, N_Q, f"{p}.self_attn.q_norm")
            norm(l, N_K, f"{p}.self_attn.k_norm")
        if cfg["arch"] == ARCH_QWEN3_MOE:
            lin(l, W_ROUTER, f"{p}.mlp.gate")
            for nm, slot in _MLP.items():
                lin(l, slot, f"{p}.mlp.switch_mlp.{nm}", expert=-2)  # every expert: stacked tensor
        else:
            for nm, slot in _MLP.items():
                lin(l, slot, f"{p}.mlp.{nm}")
    return steps


def load_model(path: str):
    """A device model (mlxcat_amd._lib.Model) holding the checkpoint at `path`."""
    from . import _lib as hip
    cfg = read_config(path)
    tensors = Checkpoint(path)
    steps = plan(cfg, tensors.keys())
    m = hip.Model(cfg)
    try:
        for kind, layer, slot, expert, prefix in steps:
            if kind == "norm":
                w = tensors[prefix + ".weight"]
                n = cfg["head_dim"] if slot in (N_Q, N_K) else cfg["hidden"]
                if w.shape != (n,) or w.dtype != np.uint16:
                    raise LoaderError(f"{prefix}.weight: expected bf16 ({n},), got {w.dtype.name} {w.shape}")
                m.set_norm(layer, slot, w)
                continue
            wq, s, b = (tensors[f"{prefix}.{x}"] for x in ("weight", "scales", "biases"))
            N, K = m._lshape(slot, 0 if expert == -2 else -1)
            lead = (cfg["n_experts"],) if expert == -2 else ()
            for t, suf, shape, dt in ((wq, "weight", (N, K // 8), np.uint32), (s, "scales", (N, K // 64), np.uint16),
                                      (b, "biases", (N, K // 64), np.uint16)):
                if t.shape != lead + shape or t.dtype != dt:
                    raise LoaderError(f"{prefix}.{suf}: expected {np.dtype(dt).name} {lead + shape}, "
                                      f"got {t.dtype.name} {t.shape}")
            if expert == -2:
                for e in range(cfg["n_experts"]):
                    m.set_linear(layer, slot, wq[e], s[e], b[e], expert=e)
            else:
                m.set_linear(layer, slot, wq, s, b)
    except Exception:
        m.close()
        raise
    return m
