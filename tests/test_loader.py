"""The MLX checkpoint loader's host side: config.json parsing (mlx-lm keys, text_config
fallback as NativeModelEngine.swift:1147-1231 reads them), the tensor plan covering every
tensor of a checkpoint exactly once, sharded checkpoints, and the errors for what the
device model cannot hold."""
import json
import os

import numpy as np
import pytest

from mlxcat_amd import mlx_loader as ml
from tests._common import TINY, TINY_LLAMA, TINY_MOE
from tests._mlx_dir import config_json, write_mlx_dir

SEED = 1234
CFGS = [TINY, TINY_LLAMA, TINY_MOE]
IDS = ["qwen3", "llama", "qwen3-moe"]


def _write_config(path, c):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(c, f)


@pytest.mark.parametrize("cfg", CFGS, ids=IDS)
def test_read_config_round_trip(tmp_path, cfg):
    _write_config(tmp_path, config_json(cfg))
    got = ml.read_config(str(tmp_path))
    for k, v in cfg.items():
        assert got[k] == pytest.approx(v), k


def test_text_config_fallback(tmp_path):
    """Keys missing at the top level are read from text_config (multimodal wrappers)."""
    c = config_json(TINY)
    inner = {k: c.pop(k) for k in ("hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
                                   "head_dim", "rope_theta")}
    c["text_config"] = inner
    _write_config(tmp_path, c)
    got = ml.read_config(str(tmp_path))
    assert (got["hidden"], got["n_layers"], got["n_q_heads"], got["n_kv_heads"], got["head_dim"]) == (256, 2, 4, 2, 64)
    assert got["rope_theta"] == 1e6


def test_head_dim_defaults_to_hidden_over_heads(tmp_path):
    c = config_json(TINY_LLAMA)
    del c["head_dim"]
    _write_config(tmp_path, c)
    assert ml.read_config(str(tmp_path))["head_dim"] == 64


@pytest.mark.parametrize("change,msg", [
    ({"model_type": "gemma3"}, "model_type"),
    ({"quantization": {"group_size": 32, "bits": 4}}, "group size 64"),
    ({"quantization": {"group_size": 64, "bits": 8}}, "group size 64"),
    ({"quantization": {"group_size": 64, "bits": 4, "mode": "mxfp4"}}, "affine"),
    ({"quantization": {"group_size": 64, "bits": 4, "model.layers.0.mlp.gate": {"group_size": 64, "bits": 8}}},
     "model.layers.0.mlp.gate"),
    ({"rope_theta": None, "rope_scaling": {"rope_type": "yarn", "rope_theta": 1e6}}, "rope scaling"),
])
def test_unsupported_configs_are_refused(tmp_path, change, msg):
    c = config_json(TINY)
    c.pop("quantization_config")
    c.update(change)
    if c.get("rope_theta", 0) is None:
        del c["rope_theta"]
    _write_config(tmp_path, c)
    with pytest.raises(ml.LoaderError, match=msg):
        ml.read_config(str(tmp_path))


def test_moe_without_topk_renormalisation_is_refused(tmp_path):
    c = config_json(TINY_MOE)
    c["norm_topk_prob"] = False
    _write_config(tmp_path, c)
    with pytest.raises(ml.LoaderError, match="norm_topk_prob"):
        ml.read_config(str(tmp_path))


@pytest.mark.parametrize("cfg", CFGS, ids=IDS)
@pytest.mark.parametrize("shards", [1, 3])
def test_plan_uses_every_tensor_once(tmp_path, oracle, cfg, shards):
    m = oracle.Model(cfg, SEED, 64, 1)
    tensors = write_mlx_dir(oracle, m, cfg, SEED, str(tmp_path), shards=shards)
    ck = ml.Checkpoint(str(tmp_path))
    assert set(ck.keys()) == set(tensors)
    steps = ml.plan(ml.read_config(str(tmp_path)), ck.keys())
    used = []
    for kind, _layer, _slot, _expert, prefix in steps:
        used += [prefix + ".weight"] if kind == "norm" else [f"{prefix}.{s}" for s in ("weight", "scales", "biases")]
    assert sorted(used) == sorted(tensors)
    # what is read back is what was written, bit for bit
    for k in ("model.embed_tokens.weight", "model.embed_tokens.scales", "model.norm.weight",
              "model.layers.1.self_attn.o_proj.biases"):
        assert np.array_equal(ck[k], tensors[k]) and ck[k].dtype == tensors[k].dtype


def test_missing_tensor_is_named(tmp_path, oracle):
    m = oracle.Model(TINY_LLAMA, SEED, 64, 1)
    tensors = write_mlx_dir(oracle, m, TINY_LLAMA, SEED, str(tmp_path))
    names = set(tensors) - {"model.layers.1.mlp.down_proj.scales"}
    with pytest.raises(ml.LoaderError, match=r"model\.layers\.1\.mlp\.down_proj\.scales"):
        ml.plan(TINY_LLAMA, names)
