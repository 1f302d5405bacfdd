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


def _compressed(model, path, bf16_scales=False):
    """Save `model` as a compressed-tensors W8A8 checkpoint (llm-compressor's int-quantized format): every
    decoder Linear as int8 rows [N, K] (symmetric, s = max|w| / 127.5, so the most negative values round to
    -128) with weight_scale [N, 1]; lm_head ignored. Returns {module name: (q, s)}."""
    import json
    import torch
    from safetensors.numpy import save_file
    model.save_pretrained(str(path))
    sd = {}                                                   # the checkpoint's own tensor names
    for f in os.listdir(path):
        if f.endswith(".safetensors"):
            sd.update({k: np.array(v) for k, v in MF.read_safetensors(os.path.join(path, f)).items()})
    out, stored = {}, {}
    for k, v in sd.items():
        mod = k[:-len(".weight")]
        if k.endswith(".weight") and v.ndim == 2 and "layers." in k and "norm" not in k and ".gate." not in k:
            s = (np.abs(v).max(axis=1) / F(127.5)).astype(F)
            q = np.clip(np.rint(v / s[:, None]), -128, 127).astype(np.int8)
            out[k] = q
            sc = s[:, None]
            if bf16_scales:                                   # stored as bf16: the scale is its bf16 value
                sc = (sc.view(np.uint32) & np.uint32(0xFFFF0000)).view(F)
                out[mod + ".weight_scale"] = torch.from_numpy(sc).to(torch.bfloat16).view(torch.int16).numpy()
            else:
                out[mod + ".weight_scale"] = sc
            stored[mod] = (q, sc[:, 0])
        else:
            out[k] = v
    for f in os.listdir(path):
        if f.endswith(".safetensors"):
            os.remove(os.path.join(path, f))
    if bf16_scales:                                           # (save_file has no bf16: write the header by hand)
        _save_with_bf16(out, os.path.join(path, "model.safetensors"), [k for k in out if k.endswith("weight_scale")])
    else:
        save_file(out, os.path.join(path, "model.safetensors"))
    c = json.load(open(os.path.join(path, "config.json")))
    scheme = {"type": "int", "num_bits": 8, "symmetric": True, "group_size": None, "block_structure": None}
    c["quantization_config"] = {
        "quant_method": "compressed-tensors", "format": "int-quantized", "quantization_status": "compressed",
        "config_groups": {"group_0": {"targets": ["Linear"],
                                      "weights": {**scheme, "dynamic": False, "strategy": "channel", "actorder": None},
                                      "input_activations": {**scheme, "dynamic": True, "strategy": "token"}}},
        "ignore": ["lm_head", "re:.*block_sparse_moe.gate$"]}
    json.dump(c, open(os.path.join(path, "config.json"), "w"))
    return stored


def _save_with_bf16(tensors, path, bf16):
    import json
    header, blobs, off = {}, [], 0
    for k, v in tensors.items():
        v = np.ascontiguousarray(v)
        dt = "BF16" if k in bf16 else {np.dtype(np.float32): "F32", np.dtype(np.int8): "I8"}[v.dtype]
        header[k] = {"dtype": dt, "shape": list(v.shape), "data_offsets": [off, off + v.nbytes]}
        blobs.append(v.tobytes())
        off += v.nbytes
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


@pytest.mark.parametrize("kind,bf16", [("llama", False), ("qwen3", True), ("mixtral", False)])
def test_compressed_tensors_checkpoint(tmp_path, kind, bf16):
    """A compressed-tensors W8A8 checkpoint (ct_import.py:1-27) keeps its own int8 rows (-128 included) and
    scales: the imported model's q | k | v, o, FFN / expert rows are the stored ones (q / k reordered into
    RoPE pairs with their scales), the ignored classifier is quantized here, and the dequantized model's
    fp32 forward equals transformers' forward with the same dequantized weights."""
    import torch
    model = _build(kind)
    stored = _compressed(model, tmp_path, bf16_scales=bf16)
    assert any((q == -128).any() for q, _ in stored.values())
    cfg = MF.hf_config(str(tmp_path), seq_len=64)
    qm = MF.read_hf(str(tmp_path), seq_len=64, calib_tokens=[1, 5, 9])
    hd, L = cfg.head_dim, cfg.layers
    perm = lambda x, h: MF._interleave_rows(np.asarray(x, F)[:, None] if x.ndim == 1 else x.astype(F), h, hd)
    for l in range(L):
        a = f"model.layers.{l}.self_attn."
        q = np.concatenate([perm(stored[a + "q_proj"][0], cfg.heads), perm(stored[a + "k_proj"][0], cfg.kv_heads),
                            stored[a + "v_proj"][0]]).astype(np.int8)
        s = np.concatenate([perm(stored[a + "q_proj"][1], cfg.heads)[:, 0], perm(stored[a + "k_proj"][1], cfg.kv_heads)[:, 0],
                            stored[a + "v_proj"][1]])
        assert np.array_equal(qm.wqkv[l], q) and np.array_equal(qm.s_wqkv[l], s)
        assert np.array_equal(qm.wo[l], stored[a + "o_proj"][0]) and np.array_equal(qm.s_wo[l], stored[a + "o_proj"][1])
        if kind == "mixtral":
            e = f"model.layers.{l}.block_sparse_moe.experts.1."
            assert np.array_equal(qm.wg[l, 1], stored[e + "w1"][0]) and np.array_equal(qm.s_wd[l, 1], stored[e + "w2"][1])
        else:
            m = f"model.layers.{l}.mlp."
            assert np.array_equal(qm.w1[l], stored[m + "gate_proj"][0]) and np.array_equal(qm.s_w2[l], stored[m + "down_proj"][1])
    head_q, head_s = W.quantize_rows(model.lm_head.weight.detach().float().numpy())
    assert np.array_equal(qm.cls_q, head_q) and np.array_equal(qm.cls_s, head_s)
    # the dequantized checkpoint, loaded by transformers, gives the fp32 forward of the imported weights
    import json
    import transformers as T
    from safetensors.numpy import save_file
    deq = tmp_path / "dequantized"
    deq.mkdir()
    t = MF.read_safetensors(str(tmp_path / "model.safetensors"))
    plain = {k: np.array(v, F) for k, v in t.items() if not k.endswith("weight_scale") and t[k].dtype != np.int8}
    for mod, (q, s) in stored.items():
        plain[mod + ".weight"] = (q.astype(F) * s[:, None]).astype(F)
    save_file(plain, str(deq / "model.safetensors"))
    c = json.load(open(tmp_path / "config.json"))
    del c["quantization_config"]
    json.dump(c, open(deq / "config.json", "w"))
    ref = T.AutoModelForCausalLM.from_pretrained(str(deq), dtype=torch.float32).eval()
    cfg2, w, weight = _ours(str(tmp_path))
    toks = [1, 17, 5, 88, 42, 3, 9, 60]
    want = _hf_logits(ref, toks)
    got = W.fp32_logits(cfg2, toks, weight)
    assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max() + 1e-6


def test_compressed_tensors_refusals(tmp_path):
    """What the datapath cannot take as stored is refused (ct_import.py:63-105): static activations, groups,
    asymmetric weights, a KV cache scheme, a non-zero zero point."""
    import json
    model = _build("llama")
    _compressed(model, tmp_path)
    c = json.load(open(tmp_path / "config.json"))
    g = c["quantization_config"]["config_groups"]["group_0"]
    for change in ({"input_activations": {**g["input_activations"], "dynamic": False}},
                   {"weights": {**g["weights"], "group_size": 128}},
                   {"weights": {**g["weights"], "symmetric": False}}):
        bad = json.loads(json.dumps(c))
        bad["quantization_config"]["config_groups"]["group_0"].update(change)
        json.dump(bad, open(tmp_path / "config.json", "w"))
        with pytest.raises(ValueError):
            MF.hf_config(str(tmp_path))
    bad = json.loads(json.dumps(c))
    bad["quantization_config"]["kv_cache_scheme"] = {"num_bits": 8}
    json.dump(bad, open(tmp_path / "config.json", "w"))
    with pytest.raises(ValueError):
        MF.hf_config(str(tmp_path))
