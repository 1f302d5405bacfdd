#!/usr/bin/env python3
"""Writes the fixtures of tests/golden/ that pin the generalised datapath (q_dim != dim, GQA, QK-norm,
theta / eps per model, the float64 RoPE tables, MoE routing and the ordered expert combine) and the
runtime pieces beside it, from the reference itself.

Run in a checkout next to the reference (it imports /root/reference/compiler/frontend/qhf.py and
hf_generic.py, torch + transformers, and /root/reference/llm, NumPy only). The fixtures are data: the
inputs and the reference's outputs, committed so the tests never need the reference.

  qhf_golden.json      - qhf.rope_tables (compiler/frontend/qhf.py:183-189) of every f64-method config:
                         sha256 of the cos / sin bits;
                       - qhf.QModel (qhf.py:254-409) on synthetic models of t2r_amd.config, decode steps
                         (forward) and prompt chunks (prefill), run in the device's numerics: EXP / RECIP /
                         RSQRT by qhf.device_sfu() (the reference's own switch to llm/ref_model.SfuExact,
                         qhf.py:52-64) and the two fp32 sums QModel takes (RMSNorm's sum of squares and the
                         softmax denominator, qhf.py:300-317) in the device's lane order, the reference's
                         own DeviceModel.red_sum (llm/ref_model.py:179-186). QModel says it "matches the sa
                         device up to reduction order" (qhf.py:34-36): with both substitutions it is the
                         device form of the generalised decoder, in the reference's structure;
                       - per position: the token fed, sha256 of the logits bits, the argmax, the first
                         logits' bits; per run the int8 KV cache's sha256, the int8 tables' sha256.
  moe_golden.npz       hf_generic.QMixtralMoe (compiler/frontend/hf_generic.py:602-663) built from a
                       transformers MixtralSparseMoeBlock holding the synthetic expert weights of a config,
                       route() and _row() on seeded input rows, in the device's numerics: torch.exp /
                       torch.reciprocal as SfuExact's EXP / RECIP, the route's sum over the k weights in the
                       lane order (DeviceModel.red_sum), and the expert activation SiLU as
                       g * RECIP(1 + EXP(-g)) (llm/ref_model.py:246-250). Inputs, ids, weights, outputs.
  w8a8_tiny.w8a8       llm/export_w8a8.export (llm/export_w8a8.py:102-130) of the tiny model at D = 8.
  tokenizer_golden.*   a synthetic tokenizer.bin (written here: pieces, scores including <= -1e10 and NaN,
                       byte pieces, multi-byte UTF-8) and llm/tokenizer.Tokenizer's ids and text for it.
  sampler_golden.json  llm/runtime.Sampler (llm/runtime.py:37-72) draws on seeded logits at several
                       temperatures, top-p values and seeds.
  hfopt_golden.npz     the HF path's numerics options as hf_generic computes them, in the device's numerics
                       (torch.exp / torch.reciprocal as SfuExact's EXP / RECIP, as write_moe does; the only
                       sum, qsum's total of the int8 probabilities, is exact in any order):
                       - SaCache (compiler/frontend/hf_generic.py:136-229) built from per-layer or per-channel
                         KV scales: its constants (1/s_k, s_k, a_k, 1/s_v, a_v) and the int8 cache rows its
                         update() writes from seeded fp32 K / V rows (V_PACKED off: the row layout);
                       - sa_attention (:231-293) of seeded query rows at several positions over that cache
                         (qsum normalisation; K per channel folded into q; V per channel);
                       - SaGELUTanh (:840-852) on a sweep through EXP overflow and the specials;
                       - the logits_scaling fold (:909-917) of seeded classifier scales.
  hf_tokenizer_golden.json  hf_tokenizer.BpeTokenizer (compiler/frontend/hf_tokenizer.py:11-205) on a
                       synthetic byte-level tokenizer.json: ids and decoded text of sample texts.

    python3 tests/golden/make_golden_hf.py [--reference /root/reference]
        [--only rope qmodel moe w8a8 tok sampler hfopt hftok]
"""
import argparse
import contextlib
import hashlib
import json
import os
import struct
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
F = np.float32


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# ------------------------------------------------------------------ the device's fp32 sum, from the reference
def device_sum(D):
    """A torch.sum over the last axis in the lane order of DeviceModel.red_sum (called on a bare DeviceModel
    whose only state is its lane width)."""
    import torch
    from ref_model import DeviceModel
    dm = object.__new__(DeviceModel)
    dm.d = D

    def dsum(x, dim=None, keepdim=False, **kw):
        assert dim in (-1, x.dim() - 1) and not kw and x.dtype == torch.float32, (dim, kw, x.dtype)
        rows = x.detach().reshape(-1, x.shape[-1]).numpy()
        out = np.array([dm.red_sum(r) for r in rows], F).reshape(x.shape[:-1] + ((1,) if keepdim else ()))
        return torch.from_numpy(out)
    return dsum


@contextlib.contextmanager
def patched(obj, name, fn):
    old = getattr(obj, name)
    setattr(obj, name, fn)
    try:
        yield
    finally:
        setattr(obj, name, old)


# ------------------------------------------------------------------ RoPE tables
def write_rope(qhf, out):
    import t2r_amd.config as C
    from t2r_amd import weights as W
    recs = []
    for cfg in list(C.CONFIGS.values()) + list(C.TINY_CONFIGS.values()):
        if cfg.rope_method != "f64":
            continue
        hc = type("HC", (), {})()
        hc.head_size, hc.theta, hc.seq_len = cfg.head_dim, float(cfg.theta), cfg.seq_len
        cos, sin = qhf.rope_tables(hc)
        mc, ms = W.rope_tables(cfg)
        recs.append({"config": cfg.name, "theta": cfg.theta, "head_dim": cfg.head_dim, "seq_len": cfg.seq_len,
                     "sha": sha(cos, sin), "equal_here": bool(np.array_equal(cos.view(np.uint32), mc.view(np.uint32))
                                                          and np.array_equal(sin.view(np.uint32), ms.view(np.uint32)))})
        print(f"rope {cfg.name}: reference == t2r_amd.weights: {recs[-1]['equal_here']}", flush=True)
    out["rope"] = recs


# ------------------------------------------------------------------ QModel in the device's numerics
QMODEL_PLAN = [
    # (config, overrides, D, decode positions before the chunks, prefill chunks (start, rows), decode after)
    ("tiny-qwen", {}, 16, 32, [], 0),
    ("tiny-qwen", {}, 8, 6, [(6, 10), (16, 4)], 6),
    ("tiny-qwen", {"name": "tiny-gqa-t5e5", "heads": 4, "kv_heads": 2, "head_dim": 16, "qk_norm": False,
                   "theta": 5e5, "eps": 1e-5, "seed_w": 91}, 16, 8, [(8, 16)], 8),
    ("tiny-qwen", {"name": "tiny-g3-t1e5", "dim": 48, "heads": 6, "kv_heads": 2, "head_dim": 16, "qk_norm": False,
                   "theta": 1e5, "eps": 1e-5, "seed_w": 92}, 16, 8, [(8, 12)], 6),
    ("c2-smollm2-135m", {}, 16, 6, [(6, 16)], 3),
    ("c3-qwen3-0.6b", {}, 16, 6, [(6, 16)], 3),
    ("c4-llama3.2-1b", {}, 16, 4, [(4, 16)], 3),
]


def hf_config(qhf, cfg):
    c = {"architectures": ["Qwen3ForCausalLM" if cfg.qk_norm else "LlamaForCausalLM"], "hidden_size": cfg.dim,
         "intermediate_size": cfg.hidden, "num_hidden_layers": cfg.layers, "num_attention_heads": cfg.heads,
         "num_key_value_heads": cfg.kv_heads, "head_dim": cfg.head_dim, "vocab_size": cfg.vocab,
         "rope_theta": cfg.theta, "rms_norm_eps": cfg.eps, "tie_word_embeddings": True,
         "max_position_embeddings": cfg.seq_len}
    with tempfile.TemporaryDirectory() as tmp:
        json.dump(c, open(os.path.join(tmp, "config.json"), "w"))
        hc = qhf.HFConfig(tmp, seq_len=cfg.seq_len)
    assert (hc.q_dim, hc.kv_dim, hc.qk_norm, hc.theta, hc.eps) == (cfg.q_dim, cfg.kv_dim, cfg.qk_norm, cfg.theta,
                                                                      cfg.eps)
    return hc


def qmodel_weights(cfg):
    """The synthetic fp32 weights of t2r_amd.weights in qhf's dict (already in interleaved-pair order)."""
    from t2r_amd import weights as W
    L = cfg.layers
    w = {"tok": W.fp32_tensor(cfg, "tok"), "rms_final": W.fp32_tensor(cfg, "rms_final")}
    names = ["rms_att", "rms_ffn", "wq", "wk", "wv", "wo", "w1", "w2", "w3"] + (["q_norm", "k_norm"] if cfg.qk_norm
                                                                              else [])
    for n in names:
        w[n] = np.stack([W.fp32_tensor(cfg, n, l) for l in range(L)])
    w["wcls"] = w["tok"]
    return w


def run_qmodel(qhf, base, over, D, n_dec0, chunks, n_dec1):
    import torch
    import t2r_amd.config as C
    from t2r_amd import weights as W
    cfg = C.get(base).with_(**over) if over else C.get(base)
    cfg = cfg.with_(D=D, rope_method="f64")
    t0 = time.time()
    w = qmodel_weights(cfg)
    kv = W.stored_kv_scales(cfg) if cfg.name in C.CONFIGS else W.calibrate_kv(cfg)
    kv = np.asarray(kv, F).reshape(cfg.layers, 2)
    qm = qhf.QModel(hf_config(qhf, cfg), w, kv)
    del w
    mine = W.QuantModel(cfg, kv_scales=kv)
    tables_equal = bool(np.array_equal(qm.emb_q.numpy(), mine.emb_q) and np.array_equal(qm.emb_s.numpy(), mine.emb_s)
                        and all(np.array_equal(qm.wqkv[l].numpy(), mine.wqkv[l]) and
                                np.array_equal(qm.s_wqkv[l].numpy(), mine.s_wqkv[l]) for l in range(cfg.layers)))
    consts_equal = bool(np.array_equal(np.asarray([qm.inv_sk, qm.inv_sv, qm.a_k, qm.a_v], F).T, mine.kvc))
    del mine
    prompt = cfg.prompt() if cfg.prompt_len else []
    rng = np.random.default_rng(4242 + D)
    need = n_dec0 + sum(m for _, m in chunks) + n_dec1
    toks = (prompt + rng.integers(0, cfg.vocab, max(0, need - len(prompt))).tolist())[:need]
    calls, fed = [], []
    pos = 0
    T_of = lambda p: torch.zeros(p + 1, dtype=torch.int64)

    def record(kind, p0, rows, lg):
        lg = lg.detach().numpy().astype(F).reshape(-1)
        calls.append({"kind": kind, "pos": p0, "rows": rows, "logits_sha": sha(lg), "argmax": int(np.argmax(lg)),
                      "head": [int(b) for b in lg.view(np.uint32)[:8]]})
        return int(np.argmax(lg))

    with qhf.device_sfu(), patched(torch, "sum", device_sum(D)), torch.no_grad():
        nxt = None
        for _ in range(n_dec0):
            t = toks[pos]
            fed.append(t)
            nxt = record("decode", pos, 1, qm.forward(torch.tensor([t]), torch.tensor([pos]), T_of(pos)))
            pos += 1
        for start, M in chunks:
            assert start == pos
            tk = toks[start:start + M]
            fed.extend(tk)
            lg = qm.prefill(torch.tensor(tk), torch.arange(start, start + M), T_of(start + M - 1))
            nxt = record("prefill", start, M, lg)
            pos += M
        for _ in range(n_dec1):               # greedy from here (the reference's argmax)
            fed.append(nxt)
            nxt = record("decode", pos, 1, qm.forward(torch.tensor([nxt]), torch.tensor([pos]), T_of(pos)))
            pos += 1
    L, S = cfg.layers, cfg.seq_len
    kc = qm.kc.numpy().reshape(L, S, cfg.kv_dim)[:, :pos]
    vc = qm.vc.numpy().reshape(L, S, cfg.kv_dim)[:, :pos]
    rec = {"config": base, "overrides": over, "D": D, "kv_bits": [int(b) for b in kv.view(np.uint32).ravel()],
           "tokens": [int(t) for t in fed], "calls": calls, "kv_sha": sha(kc, vc),
           "tables_equal_here": tables_equal, "kv_consts_equal_here": consts_equal,
           "seconds": round(time.time() - t0, 1)}
    print(f"QModel {cfg.name} D={D}: {len(calls)} calls, {pos} positions in {rec['seconds']} s; tables equal here: "
          f"{tables_equal}, kv constants: {consts_equal}", flush=True)
    return rec


# ------------------------------------------------------------------ QMixtralMoe in the device's numerics
MOE_PLAN = [("tiny-moe", 0, 6), ("tiny-moe", 1, 4), ("c5-granite-1b-a400m", 0, 4)]


def device_silu(ref_sfu):
    import torch

    class Silu(torch.nn.Module):
        def forward(self, g):
            gn = g.detach().numpy().astype(F)
            sig = ref_sfu.recip((F(1) + ref_sfu.exp((gn * F(-1)).astype(F))).astype(F))
            return torch.from_numpy((gn * sig).astype(F))
    return Silu()


def write_moe(hfg, out_path, D=16):
    import torch
    from transformers import MixtralConfig
    from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock
    from ref_model import SfuExact
    import t2r_amd.config as C
    from t2r_amd import weights as W
    arrays, meta = {}, []
    dsum = device_sum(D)
    tensor_sum = torch.Tensor.sum

    def tsum(self, dim=None, keepdim=False, **kw):
        return dsum(self, dim=dim, keepdim=keepdim, **kw)
    for i, (name, layer, rows) in enumerate(MOE_PLAN):
        cfg = C.get(name)
        E, k, d, Fe = cfg.n_experts, cfg.top_k, cfg.dim, cfg.hidden
        mc = MixtralConfig(hidden_size=d, intermediate_size=Fe, num_local_experts=E, num_experts_per_tok=k,
                           hidden_act="silu", num_hidden_layers=1, num_attention_heads=cfg.heads,
                           num_key_value_heads=cfg.kv_heads, vocab_size=cfg.vocab)
        blk = MixtralSparseMoeBlock(mc)
        wg, wu, wd = (W.fp32_tensor(cfg, n, layer) for n in ("wg", "wu", "wd"))
        with torch.no_grad():
            blk.gate.weight.copy_(torch.from_numpy(W.fp32_tensor(cfg, "router", layer)))
            blk.experts.gate_up_proj.copy_(torch.from_numpy(np.concatenate([wg, wu], axis=1)))
            blk.experts.down_proj.copy_(torch.from_numpy(wd))
        moe = hfg.QMixtralMoe(blk)
        moe.act_fn = device_silu(SfuExact)
        rng = np.random.default_rng(777 + i)
        x = (rng.standard_normal((rows, d)) * (1.0 + 0.5 * rng.random((rows, 1)))).astype(F)
        ids, wts, ys = [], [], []
        sfu_exp = lambda t: torch.from_numpy(SfuExact.exp(t.detach().numpy().astype(F)))
        sfu_rec = lambda t: torch.from_numpy(SfuExact.recip(t.detach().numpy().astype(F)))
        with torch.no_grad(), patched(torch, "exp", sfu_exp), patched(torch, "reciprocal", sfu_rec), \
                patched(torch.Tensor, "sum", tsum):
            for r in range(rows):
                xr = torch.from_numpy(x[r:r + 1])
                _, idr, wr = moe.route(xr)
                y = moe._row(xr)
                ids.append(idr.numpy().reshape(-1))
                wts.append(wr.numpy().astype(F).reshape(-1))
                ys.append(y.numpy().astype(F).reshape(-1))
        assert torch.Tensor.sum is tensor_sum
        key = f"m{i}"
        arrays[key + "_x"] = x
        arrays[key + "_ids"] = np.asarray(ids, np.int32)
        arrays[key + "_w"] = np.asarray(wts, F)
        arrays[key + "_y"] = np.asarray(ys, F)
        tabs = [moe.rq, moe.rs, moe.gq, moe.gs, moe.uq, moe.us, moe.dq, moe.ds]
        mine = [W.quantize_rows(W.fp32_tensor(cfg, "router", layer))] + [W.quantize_rows(t) for t in (wg, wu, wd)]
        # the router's rows past E are QMixtralMoe's padding (scores -inf, never selected)
        eq = all(np.array_equal(a.detach().numpy()[:len(q)], b) for (q, s), (a, b2) in
                 zip(mine, [(moe.rq, moe.rs), (moe.gq, moe.gs), (moe.uq, moe.us), (moe.dq, moe.ds)])
                 for a, b in ((a, q), (b2, s)))
        meta.append({"key": key, "config": name, "layer": layer, "rows": rows, "D": D,
                     "tables_sha": sha(*[t.detach().numpy() for t in tabs]), "tables_equal_here": eq})
        print(f"QMixtralMoe {name} layer {layer}: {rows} rows; ids {arrays[key + '_ids'][0].tolist()}; "
              f"tables equal here: {eq}", flush=True)
    np.savez_compressed(out_path, meta=np.frombuffer(json.dumps(meta).encode(), np.uint8), **arrays)


# ------------------------------------------------------------------ the HF path's numerics options
# (name, heads, kv heads, head dim, cache rows T, query positions, per-channel parts, KV spread, seed)
HFOPT_PLAN = [
    ("g2-hd16-layer", 4, 2, 16, 40, [0, 1, 15, 16, 17, 39], "", 1.0, 1),
    ("g2-hd16-k", 4, 2, 16, 40, [0, 1, 15, 16, 17, 39], "k", 1.0, 2),
    ("g1-hd32-v", 2, 2, 32, 33, [0, 7, 31, 32], "v", 1.0, 3),
    ("g4-hd64-kv", 8, 2, 64, 70, [0, 5, 63, 64, 69], "kv", 1.0, 4),
    ("g2-hd128-kv", 4, 2, 128, 300, [0, 100, 255, 256, 299], "kv", 1.0, 5),
    ("g3-hd64-k-wide", 6, 2, 64, 90, [3, 50, 89], "k", 40.0, 6),        # scores spread past EXP's underflow
]


def write_hfopt(hfg, out_path):
    """SaCache constants and cache rows, sa_attention outputs, SaGELUTanh and the logits fold (see the module
    docstring), with torch.exp / torch.reciprocal as the device SFU."""
    import torch
    from types import SimpleNamespace
    from transformers import LlamaConfig
    from ref_model import SfuExact
    assert not hfg.V_PACKED, "run with SA_V_PACKED=0: the row layout of the V cache"
    sfu_exp = lambda t: torch.from_numpy(SfuExact.exp(t.detach().numpy().astype(F)))
    sfu_rec = lambda t: torch.from_numpy(SfuExact.recip(t.detach().numpy().astype(F)))
    arrays, meta = {}, []
    for name, H, Hk, hd, T, positions, parts, spread, seed in HFOPT_PLAN:
        rng = np.random.default_rng(3100 + seed)
        kv_dim = Hk * hd
        kf = (rng.standard_normal((T, kv_dim)) * rng.uniform(0.2, 3.0, kv_dim) * spread).astype(F)
        vf = (rng.standard_normal((T, kv_dim)) * rng.uniform(0.2, 3.0, kv_dim)).astype(F)
        q = (rng.standard_normal((len(positions), H * hd)) * 2.0).astype(F)
        amax = np.stack([np.abs(kf).max(0), np.abs(vf).max(0)])                    # (2, kv_dim)
        kv = (np.maximum(amax, 1e-8) / 127.0).astype(F)
        for j, part in enumerate("kv"):
            if part not in parts:
                kv[j] = kv[j].max()                                                # one value: per layer
        kv = kv[None]                                                              # (L = 1, 2, kv_dim)
        cfg = LlamaConfig(hidden_size=H * hd, intermediate_size=16, num_hidden_layers=1, num_attention_heads=H,
                          num_key_value_heads=Hk, head_dim=hd, vocab_size=32, max_position_embeddings=T)
        owner = SimpleNamespace(kc=torch.zeros((T, kv_dim), dtype=torch.int8),
                                vc=torch.zeros((T, kv_dim), dtype=torch.int8))
        cache = hfg.SaCache(cfg, T, owner, kv)
        assert (cache.k_ch[0], cache.v_ch[0]) == ("k" in parts, "v" in parts)
        with torch.no_grad(), patched(torch, "exp", sfu_exp), patched(torch, "reciprocal", sfu_rec):
            # the cache rows through the reference's update (key_states [1, Hk, M, hd])
            cache.positions = torch.arange(T)
            ks = torch.from_numpy(kf).reshape(T, Hk, hd).transpose(0, 1)[None]
            vs = torch.from_numpy(vf).reshape(T, Hk, hd).transpose(0, 1)[None]
            cache.layers[0].update(ks, vs)
            key, value = owner.kc[0:T], owner.vc[0:T]
            module = SimpleNamespace(sa_cache=cache, layer_idx=0)
            outs = []
            for m, p in enumerate(positions):
                cache.positions = torch.tensor([p])
                query = torch.from_numpy(q[m]).reshape(H, hd)[None, :, None, :]
                o, _ = hfg.sa_attention(module, query, key, value, None)
                outs.append(o.reshape(-1).numpy().astype(F))
        f32 = lambda v: np.asarray(v.numpy() if torch.is_tensor(v) else v, F).reshape(-1)
        key_ = f"a{len(meta)}"
        arrays.update({key_ + "_kf": kf, key_ + "_vf": vf, key_ + "_q": q, key_ + "_kv": kv,
                       key_ + "_kc": owner.kc.numpy().copy(), key_ + "_vc": owner.vc.numpy().copy(),
                       key_ + "_out": np.asarray(outs, F),
                       key_ + "_inv_sk": f32(cache.inv_sk[0]), key_ + "_inv_sv": f32(cache.inv_sv[0]),
                       key_ + "_a_k": f32(cache.a_k[0]),
                       key_ + "_a_v": f32(cache.a_v[0]),           # per channel: [Hk, G, hd], per query head
                       key_ + "_sk": f32(cache.sk[0]) if cache.sk[0] is not None else np.zeros(0, F)})
        meta.append({"key": key_, "name": name, "H": H, "Hk": Hk, "hd": hd, "T": T, "positions": positions,
                     "parts": parts})
        print(f"sa_attention {name}: {len(positions)} rows over {T} cache rows (K per channel {cache.k_ch[0]}, "
              f"V per channel {cache.v_ch[0]})", flush=True)
    # SaGELUTanh: a dense sweep through EXP's overflow (x < about -10.1) plus specials and extremes
    rng = np.random.default_rng(3200)
    xs = [np.linspace(-14.0, 14.0, 56001, dtype=np.float64).astype(F), (rng.standard_normal(20000) * 6).astype(F),
          np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 1e-30, -1e-30, 1e19, -1e19, 1e20, -1e20,
                    3e38, -3e38, -10.5, -10.0, -10.1, -10.2, 10.5, 89.0, -89.0], F)]
    x = np.concatenate(xs).astype(F)
    with torch.no_grad(), patched(torch, "exp", sfu_exp), patched(torch, "reciprocal", sfu_rec), \
            np.errstate(over="ignore", invalid="ignore"):
        g = hfg.SaGELUTanh()(torch.from_numpy(x)).numpy().astype(F)
    arrays["gelu_x"], arrays["gelu_y"] = x, g
    arrays["gelu_AB"] = np.array([hfg.SaGELUTanh.A, hfg.SaGELUTanh.B], F)
    # the logits_scaling fold: head.s_w / float(ls) on a float32 tensor
    s_w = (np.abs(rng.standard_normal(4096)) * 0.01 + 1e-4).astype(F)
    folds = {}
    for ls in (8.0, 3.0, 0.7, 1.0 / 3.0, 16.0, 10.0):
        folds[repr(ls)] = (torch.from_numpy(s_w) / float(ls)).numpy().astype(F)
    arrays["fold_s_w"] = s_w
    arrays["fold_ls"] = np.array(list(map(float, folds)), np.float64)
    arrays["fold_out"] = np.stack(list(folds.values()))
    print(f"SaGELUTanh: {len(x)} inputs; logits fold: {len(folds)} scalings", flush=True)
    np.savez_compressed(out_path, meta=np.frombuffer(json.dumps(meta).encode(), np.uint8), **arrays)


# ------------------------------------------------------------------ .w8a8, tokenizer, sampler
def write_w8a8(path):
    import checkpoint
    from export_w8a8 import export
    import t2r_amd.config as C
    from t2r_amd import weights as W
    cfg = C.TINY
    rc = checkpoint.Config(cfg.dim, cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads, cfg.vocab, cfg.seq_len)
    w = {"tok": W.fp32_tensor(cfg, "tok"), "rms_final": W.fp32_tensor(cfg, "rms_final")}
    for n in ("rms_att", "rms_ffn", "wq", "wk", "wv", "wo", "w1", "w2", "w3"):
        w[n] = np.stack([W.fp32_tensor(cfg, n, l) for l in range(cfg.layers)])
    w["wcls"] = w["tok"]
    kv = W.calibrate_kv(cfg)
    n = export(rc, w, np.asarray(kv, F).reshape(cfg.layers, 2), 8, path)
    print(f"w8a8: {path} {n} bytes, sha {sha(np.fromfile(path, np.uint8))[:16]}", flush=True)


def synthetic_tokenizer(path):
    """A tokenizer.bin in llama2.c's layout (max_token_length, then per id: f32 score, i32 length, bytes)."""
    pieces = [(b"<unk>", 0.0), (b"\n<s>\n", 0.0), (b"\n</s>\n", 0.0)]
    pieces += [(("<0x%02X>" % b).encode(), 0.0) for b in range(256)]
    singles = [b" ", b"a", b"b", b"c", b"d", b"e", b"h", b"l", b"o", b"t", b"w", b"r", b"!", b",",
               "é".encode(), "世".encode(), b"\n"]
    pieces += [(s, -1000.0 - i) for i, s in enumerate(singles)]
    merges = [(b"he", -1.0), (b"ll", -2.0), (b"hell", -3.0), (b"hello", -0.5), (b" h", -5.0), (b" hello", -0.25),
              (b"wo", -7.0), (b"or", -6.0), (b"wor", -4.0), (b"ld", -8.0), (b"world", -2.5), (b" world", -1.5),
              (b"ab", -1e10), (b"abc", -2e10), (b"cd", float("nan")), (b"de", -1e10 + 1e4), (b"ee", -20.0),
              (b"tt", -20.0), (b"  ", -30.0), ("éé".encode(), -9.0), (b"to", -12.0), (b"ot", -12.0),
              (b"oto", -11.0), (b"tot", -11.0)]
    pieces += merges
    pieces += [(b"hello", -99.0)]          # a duplicate piece: the first id wins
    mx = max(len(p) for p, _ in pieces)
    with open(path, "wb") as f:
        f.write(struct.pack("i", mx))
        for p, s in pieces:
            f.write(struct.pack("fi", s, len(p)))
            f.write(p)
    return len(pieces)


def write_tokenizer(bin_path, json_path):
    from tokenizer import Tokenizer
    n = synthetic_tokenizer(bin_path)
    tk = Tokenizer(bin_path, vocab_size=n)
    texts = ["", "hello", "hello world", " hello world!", "abcd", "abcde", "cdde", "eeee", "tttt", "toto tot",
             "ééé", "世界", "hello\nworld", "a  b", "xÿĀz", "de de", "\U0001F600!",
             "\xe9t\xe9 à l'hôtel"]
    cases = []
    for t in texts:
        ids = tk.encode(t, bos=True, eos=False)
        cases.append({"text": t, "ids": ids, "ids_eos": tk.encode(t, bos=False, eos=True),
                      "decoded": tk.decode(ids)})
    json.dump({"vocab_size": n, "cases": cases}, open(json_path, "w"), indent=0, ensure_ascii=True)
    print(f"tokenizer: {n} pieces, {len(cases)} texts", flush=True)


def write_sampler(json_path):
    from runtime import Sampler
    rng = np.random.default_rng(99)
    runs = []
    for i, (V, t, p, seed) in enumerate([(40, 0.0, 0.9, 1), (40, 1.0, 0.9, 1), (40, 0.7, 0.9, 12345),
                                         (40, 1.3, 0.5, 7), (40, 1.0, 0.0, 3), (40, 1.0, 1.0, 3),
                                         (500, 0.8, 0.95, 2026), (500, 1.0, 0.2, 99), (7, 2.0, 0.999, 5),
                                         (64, 0.01, 0.9, 11)]):
        logits = (rng.standard_normal((12, V)) * rng.uniform(0.5, 6.0)).astype(F)
        s = Sampler(temperature=t, topp=p, seed=seed)
        draws = [s(lg) for lg in logits]
        runs.append({"V": V, "temperature": t, "topp": p, "seed": seed,
                     "logits_bits": [int(b) for b in logits.view(np.uint32).ravel()], "draws": draws,
                     "state": str(s.state)})
    json.dump({"runs": runs}, open(json_path, "w"), indent=0)
    print(f"sampler: {len(runs)} runs", flush=True)


HFTOK_CORPUS = ["hello world, hello there! The quick brown fox jumps over the lazy dog 12345 times.",
                "Tokenizers split text into pieces; byte-level BPE keeps every byte: caf\u00e9, na\u00efve, \u4e16\u754c.",
                "   leading spaces, trailing spaces   \n\nnew lines\ttabs and 2024-12-02 dates 3.14159",
                "It's we're they've I'm you'll he'd -- punctuation!!! ??? ... $100 #tag @user"] * 4
HFTOK_TEXTS = ["", "hello world", " hello  world ", "The quick brown fox.", "It's 2024: caf\u00e9 \u4e16\u754c!",
               "\n\n  tabs\tand\nnewlines  ", "12345678901234567890", "unseen words zyxwv qqq",
               "<|begin|>hello<|end|> world<|begin|>", "e\u0301 composed (NFC)", "\U0001F600 emoji!!",
               "they've we'll I'd ... $$$"]


def hftok_files():
    """Two synthetic byte-level tokenizer.json files, trained here with the `tokenizers` library on a small
    corpus: GPT-2 style (ByteLevel's own split) and Llama-3 style (NFC, a Split regex then ByteLevel
    without its regex, ignore_merges), each with two added special tokens."""
    from tokenizers import Regex, Tokenizer, decoders, models, normalizers, pre_tokenizers, trainers
    out = []
    for style in ("gpt2", "llama3"):
        tk = Tokenizer(models.BPE(ignore_merges=style == "llama3"))
        if style == "gpt2":
            tk.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
        else:
            tk.normalizer = normalizers.NFC()
            split = r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+"
            tk.pre_tokenizer = pre_tokenizers.Sequence([
                pre_tokenizers.Split(Regex(split), behavior="isolated"),
                pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
        tk.decoder = decoders.ByteLevel()
        trainer = trainers.BpeTrainer(vocab_size=420, special_tokens=["<|begin|>", "<|end|>"],
                                      initial_alphabet=pre_tokenizers.ByteLevel.alphabet(), show_progress=False)
        tk.train_from_iterator(HFTOK_CORPUS, trainer)
        out.append((style, tk.to_str()))
    return out


def write_hftok(json_path):
    import hf_tokenizer
    recs = []
    for style, text in hftok_files():
        with tempfile.TemporaryDirectory() as tmp:
            with open(os.path.join(tmp, "tokenizer.json"), "w") as f:
                f.write(text)
            ref = hf_tokenizer.BpeTokenizer(tmp)
            assert ref.exact, "the regex module is needed for the exact Unicode classes"
            cases = []
            for t in HFTOK_TEXTS:
                ids = ref.encode(t)
                cases.append({"text": t, "ids": ids, "decoded": ref.decode(ids)})
        recs.append({"style": style, "tokenizer_json": text, "cases": cases})
        print(f"hf_tokenizer {style}: {len(cases)} texts", flush=True)
    json.dump({"generator": "tests/golden/make_golden_hf.py", "tokenizers": recs}, open(json_path, "w"), indent=0)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--only", nargs="*")
    args = ap.parse_args()
    ref = args.reference
    for p in (os.path.join(ref, "llm"), os.path.join(ref, "driver"), os.path.join(ref, "compiler", "frontend")):
        sys.path.insert(0, p)
    only = set(args.only or ["rope", "qmodel", "moe", "w8a8", "tok", "sampler", "hfopt", "hftok"])
    os.environ["SA_V_PACKED"] = "0"      # hf_generic's V cache in the row layout (its flag is read at import)
    path = os.path.join(HERE, "qhf_golden.json")
    out = json.load(open(path)) if os.path.exists(path) else {}
    out["generator"] = "tests/golden/make_golden_hf.py"
    if "rope" in only or "qmodel" in only:
        import qhf
        if "rope" in only:
            write_rope(qhf, out)
        if "qmodel" in only:
            out["qmodel"] = [run_qmodel(qhf, *p) for p in QMODEL_PLAN]
        json.dump(out, open(path, "w"), indent=0)
    if "moe" in only:
        import hf_generic
        write_moe(hf_generic, os.path.join(HERE, "moe_golden.npz"))
    if "hfopt" in only:
        import hf_generic
        write_hfopt(hf_generic, os.path.join(HERE, "hfopt_golden.npz"))
    if "w8a8" in only:
        write_w8a8(os.path.join(HERE, "w8a8_tiny.w8a8"))
    if "hftok" in only:
        write_hftok(os.path.join(HERE, "hf_tokenizer_golden.json"))
    if "tok" in only:
        write_tokenizer(os.path.join(HERE, "tokenizer_golden.bin"), os.path.join(HERE, "tokenizer_golden.json"))
    if "sampler" in only:
        write_sampler(os.path.join(HERE, "sampler_golden.json"))


if __name__ == "__main__":
    main()
