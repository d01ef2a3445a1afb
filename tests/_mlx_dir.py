"""Writes an MLX-format model directory (config.json with mlx-lm's keys, 4-bit g64
.weight/.scales/.biases triplets, bf16 norms, MoE experts stacked under mlp.switch_mlp) from
the oracle's seeded synthetic weights, so the loader can be tested without a download."""
from __future__ import annotations

import json
import os

import numpy as np
import torch
from safetensors.torch import save_file

MODEL_TYPE = {0: "qwen3", 1: "llama", 2: "qwen3_moe"}
FINAL_NORM_TID = 0xE0000003


def _norm(O, seed, tid, n):
    w = np.zeros(n, dtype=np.uint16)
    O.lib().or_gen_norm(seed, tid, n, w.ctypes.data_as(__import__("ctypes").c_void_p))
    return w


def config_json(cfg: dict) -> dict:
    c = dict(model_type=MODEL_TYPE[cfg["arch"]], hidden_size=cfg["hidden"], num_hidden_layers=cfg["n_layers"],
             num_attention_heads=cfg["n_q_heads"], num_key_value_heads=cfg["n_kv_heads"], head_dim=cfg["head_dim"],
             intermediate_size=cfg["intermediate"], vocab_size=cfg["vocab"],
             tie_word_embeddings=bool(cfg["tied_embeddings"]), rms_norm_eps=cfg["rms_eps"],
             rope_theta=cfg["rope_theta"], max_position_embeddings=40960, torch_dtype="bfloat16",
             quantization={"group_size": 64, "bits": 4}, quantization_config={"group_size": 64, "bits": 4})
    if cfg["arch"] == 2:
        c.update(num_experts=cfg["n_experts"], num_experts_per_tok=cfg["n_experts_per_tok"],
                 moe_intermediate_size=cfg["moe_intermediate"], norm_topk_prob=True, decoder_sparse_step=1,
                 mlp_only_layers=[])
    return c


def mlx_tensors(O, m, cfg: dict, seed: int) -> dict:
    """name -> numpy array (uint32 words, bf16 bits as uint16) in mlx-lm's module paths."""
    out = {}

    def lin(prefix, layer, which, expert=-1):
        wq, s, b = m.linear(layer, which, expert)
        out[prefix + ".weight"], out[prefix + ".scales"], out[prefix + ".biases"] = wq, s, b

    lin("model.embed_tokens", -1, 0)
    if not cfg["tied_embeddings"]:
        lin("lm_head", -1, 1)
    out["model.norm.weight"] = _norm(O, seed, FINAL_NORM_TID, cfg["hidden"])
    tid = lambda l, w: O.lib().or_tensor_id(l, w)
    for l in range(cfg["n_layers"]):
        p = f"model.layers.{l}"
        for nm, w in (("q_proj", 0), ("k_proj", 1), ("v_proj", 2), ("o_proj", 3)):
            lin(f"{p}.self_attn.{nm}", l, w)
        out[f"{p}.input_layernorm.weight"] = _norm(O, seed, tid(l, 7), cfg["hidden"])
        out[f"{p}.post_attention_layernorm.weight"] = _norm(O, seed, tid(l, 8), cfg["hidden"])
        if cfg["arch"] in (0, 2):
            out[f"{p}.self_attn.q_norm.weight"] = _norm(O, seed, tid(l, 9), cfg["head_dim"])
            out[f"{p}.self_attn.k_norm.weight"] = _norm(O, seed, tid(l, 10), cfg["head_dim"])
        if cfg["arch"] == 2:
            lin(f"{p}.mlp.gate", l, 11)
            for nm, w in (("gate_proj", 4), ("up_proj", 5), ("down_proj", 6)):
                parts = [m.linear(l, w, e) for e in range(cfg["n_experts"])]
                for i, suf in enumerate(("weight", "scales", "biases")):
                    out[f"{p}.mlp.switch_mlp.{nm}.{suf}"] = np.stack([t[i] for t in parts])
        else:
            for nm, w in (("gate_proj", 4), ("up_proj", 5), ("down_proj", 6)):
                lin(f"{p}.mlp.{nm}", l, w)
    return out


def _torch(a: np.ndarray) -> torch.Tensor:
    if a.dtype == np.uint32:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).view(torch.uint32)
    assert a.dtype == np.uint16
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def write_mlx_dir(O, m, cfg: dict, seed: int, path: str, shards: int = 1, config_extra: dict | None = None) -> dict:
    """Write the directory; with shards > 1 the tensors are split over several files named by
    a model.safetensors.index.json, as mlx-lm saves large models."""
    os.makedirs(path, exist_ok=True)
    c = config_json(cfg)
    c.update(config_extra or {})
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(c, f)
    tensors = mlx_tensors(O, m, cfg, seed)
    names = sorted(tensors)
    if shards == 1:
        save_file({k: _torch(tensors[k]) for k in names}, os.path.join(path, "model.safetensors"))
        return tensors
    weight_map = {}
    for i in range(shards):
        fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        part = names[i::shards]
        save_file({k: _torch(tensors[k]) for k in part}, os.path.join(path, fn))
        weight_map.update({k: fn for k in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    return tensors
