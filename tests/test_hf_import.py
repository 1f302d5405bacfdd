"""The HuggingFace checkpoint importer (modelfile.read_hf: config.json + safetensors, as the reference's
HF path reads them, compiler/frontend/qhf.py:97-181). Tiny models with random weights are built and saved
by the transformers library itself (offline), imported, and the fp32 forward of the imported weights is
compared with transformers' own forward of the same model: equal logits within float32 rounding pin the
name mapping, the rotate-half -> interleaved-pair reordering of q / k (and the QK-norm gains), the MoE
layout, tied embeddings and the GELU-tanh gate."""
import os

import numpy as np
import pytest

import t2r_amd.config as C
from t2r_amd import modelfile as MF
from t2r_amd import weights as W

F = np.float32


def _build(kind, **over):
    import torch
    import transformers as T
    torch.manual_seed(7)
    common = dict(vocab_size=96, hidden_size=64, intermediate_size=96, num_hidden_layers=2, num_attention_heads=4,
                  num_key_value_heads=2, max_position_embeddings=64, rms_norm_eps=1e-5, rope_theta=10000.0,
                  tie_word_embeddings=False)
    common.update(over)
    if kind == "llama":
        cfg = T.LlamaConfig(**common)
        model = T.LlamaForCausalLM(cfg)
    elif kind == "qwen3":
        cfg = T.Qwen3Config(head_dim=32, **common)            # q_dim = 128 != hidden 64, QK-norm
        model = T.Qwen3ForCausalLM(cfg)
    else:
        cfg = T.MixtralConfig(num_local_experts=4, num_experts_per_tok=2, **common)
        model = T.MixtralForCausalLM(cfg)
    with torch.no_grad():                                     # norm gains away from 1: their mapping shows
        for n, p in model.named_parameters():
            if n.endswith("norm.weight") or "layernorm" in n:
                p.copy_(1 + 0.2 * torch.randn_like(p))
    return model.float().eval()


def _hf_logits(model, toks):
    import torch
    with torch.no_grad():
        return model(torch.tensor([toks])).logits[0].float().numpy()


def _ours(path):
    cfg = MF.hf_config(path, seq_len=64)
    w = MF.hf_weights(path, cfg)

    def weight(c, name, layer=-1):
        v = w[name]
        return np.asarray(v if layer < 0 or name in ("tok", "wcls", "rms_final") else v[layer], F)
    return cfg, w, weight


@pytest.mark.parametrize("kind,over", [("llama", {}), ("llama", {"tie_word_embeddings": True}),
                                       ("llama", {"hidden_act": "gelu_pytorch_tanh", "logits_scaling": 4.0}),
                                       ("qwen3", {}), ("mixtral", {})])
def test_import_matches_transformers(tmp_path, kind, over):
    model = _build(kind, **over)
    if "logits_scaling" in over:
        model.config.logits_scaling = over["logits_scaling"]
    model.save_pretrained(str(tmp_path))
    assert any(f.endswith(".safetensors") for f in os.listdir(tmp_path))
    cfg, w, weight = _ours(str(tmp_path))
    assert cfg.qk_norm == (kind == "qwen3") and cfg.moe == (kind == "mixtral")
    assert cfg.tied == bool(over.get("tie_word_embeddings", False))
    toks = [1, 17, 5, 88, 42, 3, 9, 60, 2, 31, 77, 4]
    want = _hf_logits(model, toks)
    if "logits_scaling" in over:
        want = want / over["logits_scaling"]                  # (transformers' Llama has no logits scaling)
        assert cfg.act == "gelu_tanh" and cfg.logits_scaling == over["logits_scaling"]
    got = W.fp32_logits(cfg, toks, weight)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 2e-5 * scale + 1e-6, np.abs(got - want).max() / scale
    # the reordering matters: q / k rows left in rotate-half order give different logits
    if kind != "mixtral":
        wrong = dict(w)
        wrong["wq"] = np.stack([MF._interleave_rows(x, cfg.heads, cfg.head_dim) for x in w["wq"]])

        def weight2(c, name, layer=-1):
            v = wrong[name]
            return np.asarray(v if layer < 0 or name in ("tok", "wcls", "rms_final") else v[layer], F)
        assert np.abs(W.fp32_logits(cfg, toks, weight2) - want).max() > 1e-3 * scale


def test_bf16_safetensors(tmp_path):
    """BF16 storage is read as its float32 widening (the top 16 bits)."""
    import torch
    model = _build("llama").to(torch.bfloat16)
    model.save_pretrained(str(tmp_path))
    t = {}
    for f in os.listdir(tmp_path):
        if f.endswith(".safetensors"):
            t.update(MF.read_safetensors(str(tmp_path / f)))
    sd = model.state_dict()
    for n in ("model.embed_tokens.weight", "model.layers.1.mlp.down_proj.weight", "model.norm.weight"):
        assert np.array_equal(t[n], sd[n].float().numpy())


def test_read_hf_quantises(tmp_path):
    """read_hf: the W8A8 model of the imported weights (rows, scales, calibrated KV scales) and the
    refusals of what the datapath cannot express."""
    import json
    model = _build("qwen3")
    model.save_pretrained(str(tmp_path))
    qm = MF.read_hf(str(tmp_path), seq_len=64, calib_tokens=[1, 5, 9, 13])
    cfg, w, _ = _ours(str(tmp_path))
    q, s = W.quantize_rows(np.concatenate([w["wq"][1], w["wk"][1], w["wv"][1]]))
    assert np.array_equal(qm.wqkv[1], q) and np.array_equal(qm.s_wqkv[1], s)
    assert np.array_equal(qm.q_norm, w["q_norm"]) and qm.kv_scales.shape == (2, 2)
    qm2 = MF.read_hf(str(tmp_path), seq_len=64, calib_tokens=[1, 5, 9, 13], kv_channel="k")
    assert qm2.kv_scales.shape == (2, 2, cfg.kv_dim) and (qm2.kv_flags == 1).all()
    c = json.load(open(tmp_path / "config.json"))
    for bad in ({"attention_bias": True}, {"hidden_act": "relu"}, {"rope_scaling": {"rope_type": "linear", "factor": 2.0}},
                {"architectures": ["GPT2LMHeadModel"]}):
        d = tmp_path / ("bad" + str(len(os.listdir(tmp_path))))
        d.mkdir()
        json.dump({**c, **bad}, open(d / "config.json", "w"))
        with pytest.raises(ValueError):
            MF.hf_config(str(d))
