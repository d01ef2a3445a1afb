"""The oracle's decoder wiring against the published Hugging Face implementations of the
architectures the reference runs through mlx-swift-lm (Qwen3, Llama, Qwen3-MoE): the
transformers models are built from a config alone (no download) in float32 with eager
attention, loaded with the oracle's dequantised synthetic weights, and must give the
oracle's logits within the bf16 verify tolerance (2e-2 abs + 1e-2 rel).

This pins what the oracle's own restatement cannot: q/k-norm before RoPE, the rotate-half
RoPE convention, the tied head, the GQA head grouping and the Qwen3-MoE block (softmax
router, top-k, norm_topk_prob renormalisation, SwiGLU experts).  Each check is paired with
a deliberately miswired transformers model that must fail it, so the comparison can tell
a wiring mistake from rounding noise."""
import numpy as np
import pytest
import torch

from tests._common import ATOL, RTOL, TINY, TINY_LLAMA, TINY_MOE, bf16_to_f32
from tests.test_oracle_forward import SEED, dequant, norm_w

transformers = pytest.importorskip("transformers")


def hf_model(cfg, *, norm_topk_prob=True, arch=None):
    arch = cfg["arch"] if arch is None else arch
    common = dict(vocab_size=cfg["vocab"], hidden_size=cfg["hidden"], num_hidden_layers=cfg["n_layers"],
                  num_attention_heads=cfg["n_q_heads"], num_key_value_heads=cfg["n_kv_heads"],
                  head_dim=cfg["head_dim"], rms_norm_eps=cfg["rms_eps"], rope_theta=cfg["rope_theta"],
                  tie_word_embeddings=bool(cfg["tied_embeddings"]), max_position_embeddings=4096,
                  attention_bias=False, hidden_act="silu")
    if arch == 0:
        c = transformers.Qwen3Config(intermediate_size=cfg["intermediate"], **common)
        model_cls = transformers.Qwen3ForCausalLM
    elif arch == 1:
        c = transformers.LlamaConfig(intermediate_size=cfg["intermediate"], mlp_bias=False, **common)
        model_cls = transformers.LlamaForCausalLM
    else:
        c = transformers.Qwen3MoeConfig(intermediate_size=cfg["intermediate"], moe_intermediate_size=cfg["moe_intermediate"],
                                        num_experts=cfg["n_experts"], num_experts_per_tok=cfg["n_experts_per_tok"],
                                        norm_topk_prob=norm_topk_prob, decoder_sparse_step=1, mlp_only_layers=[],
                                        **common)
        model_cls = transformers.Qwen3MoeForCausalLM
    c._attn_implementation = "eager"
    torch.manual_seed(0)
    return model_cls(c).float().eval()


def interleave_rows(w, d):
    """Rows of a [heads * d, in] projection reordered from the rotate-half pairing (i, i + d/2)
    to the interleaved pairing (2i, 2i + 1): what a loader that confused the two RoPE
    conventions would produce."""
    heads = w.shape[0] // d
    perm = torch.cat([torch.stack([torch.arange(d // 2), torch.arange(d // 2) + d // 2], 1).reshape(-1) + h * d
                      for h in range(heads)])
    return w[perm]


def load_oracle_weights(O, m, hf, cfg, *, interleave=False):
    d, nq, nkv = cfg["head_dim"], cfg["n_q_heads"], cfg["n_kv_heads"]
    H = cfg["hidden"]
    tid = lambda l, w: O.lib().or_tensor_id(l, w)
    sd = {}
    sd["model.embed_tokens.weight"] = dequant(O, m, -1, 0)
    if not cfg["tied_embeddings"]:
        sd["lm_head.weight"] = dequant(O, m, -1, 1)
    sd["model.norm.weight"] = norm_w(O, SEED, 0xE0000003, H)
    for l in range(cfg["n_layers"]):
        p = f"model.layers.{l}."
        q, k = dequant(O, m, l, 0), dequant(O, m, l, 1)
        if interleave:
            q, k = interleave_rows(q, d), interleave_rows(k, d)
        sd[p + "self_attn.q_proj.weight"] = q
        sd[p + "self_attn.k_proj.weight"] = k
        sd[p + "self_attn.v_proj.weight"] = dequant(O, m, l, 2)
        sd[p + "self_attn.o_proj.weight"] = dequant(O, m, l, 3)
        sd[p + "input_layernorm.weight"] = norm_w(O, SEED, tid(l, 7), H)
        sd[p + "post_attention_layernorm.weight"] = norm_w(O, SEED, tid(l, 8), H)
        if cfg["arch"] in (0, 2) and hasattr(hf.model.layers[l].self_attn, "q_norm"):
            qn, kn = norm_w(O, SEED, tid(l, 9), d), norm_w(O, SEED, tid(l, 10), d)
            if interleave:
                qn, kn = interleave_rows(qn[:, None], d)[:, 0], interleave_rows(kn[:, None], d)[:, 0]
            sd[p + "self_attn.q_norm.weight"] = qn
            sd[p + "self_attn.k_norm.weight"] = kn
        if cfg["arch"] == 2:
            E = cfg["n_experts"]
            sd[p + "mlp.gate.weight"] = dequant(O, m, l, 11)
            sd[p + "mlp.experts.gate_up_proj"] = torch.stack(
                [torch.cat([dequant(O, m, l, 4, e), dequant(O, m, l, 5, e)], 0) for e in range(E)])
            sd[p + "mlp.experts.down_proj"] = torch.stack([dequant(O, m, l, 6, e) for e in range(E)])
        else:
            sd[p + "mlp.gate_proj.weight"] = dequant(O, m, l, 4)
            sd[p + "mlp.up_proj.weight"] = dequant(O, m, l, 5)
            sd[p + "mlp.down_proj.weight"] = dequant(O, m, l, 6)
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    # a tied head is the embedding; every other parameter came from the oracle
    assert set(missing) <= {"lm_head.weight"}, missing


def hf_logits(hf, tokens):
    with torch.no_grad():
        out = hf(input_ids=torch.tensor([tokens]), position_ids=torch.arange(len(tokens))[None], use_cache=False)
    return out.logits[0].double().numpy()


def inside(got_bf16, want_f64):
    g = bf16_to_f32(got_bf16).astype(np.float64)
    err = np.abs(g - want_f64)
    return float((err <= ATOL + RTOL * np.abs(want_f64)).mean()), float((err / (ATOL + RTOL * np.abs(want_f64))).max())


@pytest.mark.parametrize("cfg", [TINY, TINY_LLAMA, TINY_MOE], ids=["qwen3", "llama", "qwen3-moe"])
def test_oracle_matches_transformers(oracle, cfg):
    m = oracle.Model(cfg, SEED, 64, 1)
    rng = np.random.default_rng(11)
    toks = rng.integers(0, cfg["vocab"], 24).tolist()
    got = m.forward([0], [24], toks)
    hf = hf_model(cfg)
    load_oracle_weights(oracle, m, hf, cfg)
    want = hf_logits(hf, toks)
    frac, worst = inside(got, want)
    print(f"{cfg['arch']}: inside {frac:.5f}, worst {worst:.3f} x the bound")
    assert frac == 1.0 and worst < 0.75, (frac, worst)


def norm_after_rope(hf, monkeypatch):
    """The Qwen3 model with q/k-norm applied after the rotation instead of before it."""
    import transformers.models.qwen3.modeling_qwen3 as mq
    orig = mq.apply_rotary_pos_emb
    cur = {}

    def rotate_then_norm(q, k, cos, sin, *args, **kwargs):
        q, k = orig(q, k, cos, sin, *args, **kwargs)
        return cur["qn"](q), cur["kn"](k)

    for layer in hf.model.layers:
        attn = layer.self_attn
        qn, kn = attn.q_norm, attn.k_norm
        attn.q_norm, attn.k_norm = torch.nn.Identity(), torch.nn.Identity()
        attn.register_forward_pre_hook(lambda mod, args, qn=qn, kn=kn: cur.update(qn=qn, kn=kn))
    monkeypatch.setattr(mq, "apply_rotary_pos_emb", rotate_then_norm)


@pytest.mark.parametrize("variant", ["interleaved-rope", "no-qk-norm", "qk-norm-after-rope", "moe-without-norm-topk"])
def test_miswired_transformers_model_fails(oracle, variant, monkeypatch):
    """The comparison above detects each plausible wiring mistake."""
    cfg = TINY_MOE if variant == "moe-without-norm-topk" else TINY
    m = oracle.Model(cfg, SEED, 64, 1)
    rng = np.random.default_rng(11)
    toks = rng.integers(0, cfg["vocab"], 24).tolist()
    got = m.forward([0], [24], toks)
    if variant == "interleaved-rope":
        hf = hf_model(cfg)
        load_oracle_weights(oracle, m, hf, cfg, interleave=True)
    elif variant == "no-qk-norm":
        hf = hf_model(cfg, arch=1)  # Llama wiring: no q/k norm
        load_oracle_weights(oracle, m, hf, cfg)
    elif variant == "qk-norm-after-rope":
        hf = hf_model(cfg)
        load_oracle_weights(oracle, m, hf, cfg)
        norm_after_rope(hf, monkeypatch)
    else:
        hf = hf_model(cfg, norm_topk_prob=False)
        load_oracle_weights(oracle, m, hf, cfg)
    frac, worst = inside(got, hf_logits(hf, toks))
    print(f"{variant}: inside {frac:.5f}, worst {worst:.3f} x the bound")
    # the correct wiring puts every logit inside the bound (worst about half of it); each
    # mistake puts some outside, several times the bound away
    assert frac < 1.0 and worst > 2.0, (variant, frac, worst)
