"""The MLX checkpoint loader on the GPU: a directory written from the oracle's synthetic
weights (mlx-lm names, 4-bit g64 triplets, MoE experts stacked) loads into a device model
whose every linear exports back bit for bit, and whose verify logits are identical to
those of the model filled in place by the same seeded generator (which covers the norms)."""
import numpy as np
import pytest

from mlxcat_amd import mlx_loader as ml
from tests._common import TINY, TINY_LLAMA, TINY_MOE
from tests._mlx_dir import write_mlx_dir

pytestmark = pytest.mark.gpu
SEED = 1234
SPEC = dict(enabled=1, max_proposal_tokens=4, max_suffix_tokens=3, min_context_tokens=8, acceptance=1,
            single_row_only=0, greedy_only=0)


@pytest.mark.parametrize("cfg", [TINY, TINY_LLAMA, TINY_MOE], ids=["qwen3", "llama", "qwen3-moe"])
def test_loaded_model_equals_synthetic(hip, oracle, tmp_path, cfg):
    om = oracle.Model(cfg, SEED, 64, 1)
    tensors = write_mlx_dir(oracle, om, cfg, SEED, str(tmp_path), shards=2)
    loaded = ml.load_model(str(tmp_path))
    # every linear round-trips through the device tile layout unchanged
    for kind, layer, slot, expert, prefix in ml.plan(cfg, tensors.keys()):
        if kind != "linear":
            continue
        want = [tensors[f"{prefix}.{s}"] for s in ("weight", "scales", "biases")]
        for e in (range(cfg["n_experts"]) if expert == -2 else [-1]):
            got = loaded.get_linear(layer, slot, e)
            for g, w in zip(got, want):
                assert np.array_equal(g, w if e < 0 else w[e]), (prefix, e)
    synth = hip.Model(cfg)
    synth.init_synthetic(SEED)
    rng = np.random.default_rng(5)
    lens = [21, 9]
    toks = rng.integers(0, cfg["vocab"], sum(lens)).tolist()
    more = rng.integers(0, cfg["vocab"], 7).tolist()
    out = []
    for m in (loaded, synth):
        b = hip.Batch(m, 2, 128, SPEC)
        out.append((b.forward([0, 1], lens, toks), b.forward([0, 1], [4, 3], more)))
        b.close()
    for a, b in zip(*out):
        assert np.array_equal(a, b)
    loaded.close()
    synth.close()


def test_shape_mismatch_is_refused(hip, oracle, tmp_path):
    """A checkpoint whose tensors do not fit config.json fails before anything runs."""
    om = oracle.Model(TINY_LLAMA, SEED, 64, 1)
    write_mlx_dir(oracle, om, TINY_LLAMA, SEED, str(tmp_path), config_extra={"intermediate_size": 768})
    with pytest.raises(ml.LoaderError, match="gate_proj.weight"):
        ml.load_model(str(tmp_path))
