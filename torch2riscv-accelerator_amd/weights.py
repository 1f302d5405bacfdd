"""Host-side model data: seeded synthetic fp32 weights, their W8A8 quantisation,
the RoPE tables and the per-layer KV constants.

Everything here runs once per model on the host, as the reference's exporter
does (llm/export_w8a8.py:75-95): the device only ever sees int8 weight rows
with one fp32 scale per row, fp32 norm gains, the RoPE tables and four fp32
constants per layer.

- Weights: N(0, std) in float32 from one NumPy generator per tensor, seeded by
  (seed_w, tensor id, layer), so any tensor can be regenerated alone.
- Quantisation: symmetric per output row, s = max|w| / 127 in float32 and
  q = to_i8(w / s) (llm/ref_model.py:136-148).
- RoPE tables: (seq_len, head_dim / 2) cos and sin; pair i of every head at
  position p rotates by p * theta^(-2i / head_dim). Method "f32" evaluates it
  in float32 as llama2.c's run.c does (llm/ref_model.py:34-41), "f64" in float64
  then rounds (compiler/frontend/qhf.py:183-189).
- KV constants per layer from the static scales (s_k, s_v):
  1/s_k, 1/s_v, a_k = s_k / sqrt(head_dim), a_v = s_v / 127, each computed in
  float64 and rounded once (llm/export_w8a8.py:68-72).
- Per-channel KV scales (cfg.kv_channel; compiler/frontend/hf_generic.py:153-187,
  466-491): scales [L, 2, kv_dim]; a layer whose K (or V) row holds one value is
  per layer. A K-per-channel layer multiplies q by s_k per channel before its
  quantisation and scales the scores by a_k = f32(1 / sqrt(head_dim)) only; the
  cache takes to_i8(F(k * F(1 / s_k))) per channel (a float32 division). A
  V-per-channel layer quantises with F(1 / s_v) per channel and scales the output
  channel by a_v = F(s_v * f32(1 / 127)) (a float32 product).
- logits_scaling: the classifier's row scales divided by it, F(s / f32(ls)) (the
  float32 division of hf_generic.py:909-917); a tied classifier keeps the
  embedding's int8 rows and gets scales of its own.
"""
import hashlib
import json
import os

import numpy as np

F = np.float32
HERE = os.path.dirname(os.path.abspath(__file__))

_TENSOR_ID = {"tok": 1, "wq": 2, "wk": 3, "wv": 4, "wo": 5, "w1": 6, "w3": 7, "w2": 8, "router": 9,
              "rms_att": 10, "rms_ffn": 11, "rms_final": 12, "q_norm": 13, "k_norm": 14, "wcls": 15,
              "wg": 16, "wu": 17, "wd": 18}


def to_i8(x):
    """fp32 -> int8: round half to even, saturate to [-127, 127], NaN -> 0 (llm/ref_model.py:136-139)."""
    y = np.rint(np.asarray(x, F))
    return np.clip(np.nan_to_num(y, nan=0.0, posinf=127, neginf=-127), -127, 127).astype(np.int8)


def quantize_rows(w):
    """Symmetric int8 per row: (q int8, s float32) with s = max|row| / 127 and q = to_i8(w / s)
    (llm/ref_model.py:142-148). w / s is finite except 0 / 0 on an all-zero row (NaN -> 0), so the
    in-place rint + clip below is to_i8 exactly."""
    w = np.asarray(w, F)
    s = (np.abs(w).max(axis=-1) / F(127)).astype(F)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.divide(w, s[..., None])
    np.rint(q, out=q)
    np.clip(q, -127, 127, out=q)
    q = q.astype(np.int8)
    zero = s == 0
    if zero.any():
        q[zero] = 0
    return q, s


def _gen(cfg, name, layer, shape, fan_in):
    rng = np.random.default_rng([cfg.seed_w, _TENSOR_ID[name], layer + 1])
    std = cfg.weight_std if cfg.weight_std is not None else 1.0 / np.sqrt(fan_in)
    return (rng.standard_normal(shape, dtype=F) * F(std)).astype(F)


def _gain(cfg, name, layer, n):
    if cfg.gain_std == 0:
        return np.ones(n, F)
    rng = np.random.default_rng([cfg.seed_w, _TENSOR_ID[name], layer + 1])
    return (F(1) + F(cfg.gain_std) * rng.standard_normal(n, dtype=F)).astype(F)


def fp32_tensor(cfg, name, layer=-1):
    """One fp32 tensor of the synthetic model (PyTorch orientation: linear weights are (out, in))."""
    d, q, kv, f = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden
    E = cfg.n_experts
    shapes = {"tok": ((cfg.vocab, d), d), "wcls": ((cfg.vocab, d), d), "wq": ((q, d), d), "wk": ((kv, d), d), "wv": ((kv, d), d),
              "wo": ((d, q), q), "w1": ((f, d), d), "w3": ((f, d), d), "w2": ((d, f), f),
              "router": ((E, d), d), "wg": ((E, f, d), d), "wu": ((E, f, d), d), "wd": ((E, d, f), f)}
    if name in ("rms_att", "rms_ffn", "rms_final"):
        return _gain(cfg, name, layer, d)
    if name in ("q_norm", "k_norm"):
        return _gain(cfg, name, layer, cfg.head_dim)
    shape, fan_in = shapes[name]
    w = _gen(cfg, name, layer, shape, fan_in)
    if name == "tok" and cfg.emb_scale != 1.0:
        w = (w * F(cfg.emb_scale)).astype(F)
    return w


def rope_tables(cfg):
    """(cos, sin), each float32 (seq_len, head_dim // 2)."""
    hs = cfg.head_dim
    if cfg.rope_method == "f32":
        hd = np.arange(0, hs, 2).astype(F)
        freq = F(1.0) / np.power(F(cfg.theta), hd / F(hs))
        val = np.arange(cfg.seq_len, dtype=F)[:, None] * freq[None, :]
        return np.cos(val).astype(F), np.sin(val).astype(F)
    freq = 1.0 / np.power(float(cfg.theta), np.arange(0, hs, 2, dtype=np.float64) / hs)
    val = np.arange(cfg.seq_len, dtype=np.float64)[:, None] * freq[None, :]
    return np.cos(val).astype(F), np.sin(val).astype(F)


def kv_channel_flags(cfg, kv_scales):
    """(L,) int32: bit 0 K per channel, bit 1 V per channel, for scales (L, 2) (none) or (L, 2, kv_dim):
    a layer's row is per channel unless it holds one value (compiler/frontend/hf_generic.py:155-160)."""
    kv = np.asarray(kv_scales, F)
    flags = np.zeros(cfg.layers, np.int32)
    if kv.ndim == 3:
        for l in range(cfg.layers):
            for j in (0, 1):
                if not np.all(kv[l, j] == kv[l, j, 0]):
                    flags[l] |= 1 << j
    return flags


def kv_constants(cfg, kv_scales):
    """(L, 4) float32 per layer: 1/s_k, 1/s_v, a_k, a_v. a_k = s_k / sqrt(head_dim), or 1 / sqrt(head_dim) on a
    K-per-channel layer; a_v = s_v / 127 (hf_generic.py:172-186). With scales (L, 2, kv_dim) a layer's value is
    its channel 0 (the per-layer case, every channel equal)."""
    kv = np.asarray(kv_scales, F)
    flags = kv_channel_flags(cfg, kv)
    kv1 = kv[:, :, 0] if kv.ndim == 3 else kv.reshape(cfg.layers, 2)
    out = np.empty((cfg.layers, 4), F)
    for l, (sk, sv) in enumerate(kv1):
        a_k = F(1.0 / np.sqrt(cfg.head_dim)) if flags[l] & 1 else F(float(sk) / np.sqrt(cfg.head_dim))
        out[l] = [F(1.0 / float(sk)), F(1.0 / float(sv)), a_k, F(float(sv) / 127.0)]
    return out


def kv_channel_constants(cfg, kv_scales):
    """(L, 4, kv_dim) float32 per cache channel: s_k (the q multiplier), F(1 / s_k), F(1 / s_v),
    F(s_v * f32(1 / 127)) (float32 operations, hf_generic.py:169-186), or None for per-layer scales."""
    kv = np.asarray(kv_scales, F)
    if kv.ndim != 3:
        return None
    one = F(1.0)
    with np.errstate(divide="ignore"):
        out = np.stack([kv[:, 0], (one / kv[:, 0]).astype(F), (one / kv[:, 1]).astype(F),
                        (kv[:, 1] * F(1.0 / 127.0)).astype(F)], axis=1)
    return np.ascontiguousarray(out, F)


def fold_logits_scaling(cls_s, ls):
    """Classifier row scales with the logits' division folded in: F(s / f32(ls)) (hf_generic.py:909-917)."""
    if ls == 1.0:
        return cls_s
    return (np.asarray(cls_s, F) / F(ls)).astype(F)


class QuantModel:
    """The quantised model as the device consumes it (host NumPy arrays).

    Linear layers are int8 row-major (out, in) with a float32 scale per row:
    wqkv (L, q + 2 kv, d) = the q | k | v rows; wo (L, d, q); w1, w3 (L, F, d);
    w2 (L, d, F); MoE: router (L, E, d), wg / wu (L, E, F, d), wd (L, E, d, F).
    The classifier is the embedding (tied) unless cfg.tied is False.
    """

    def __init__(self, cfg, kv_scales=None, layers=None):
        cfg.validate()
        self.cfg = c = cfg
        L = c.layers
        # tensors are independent (one generator each): generate them in parallel threads (NumPy
        # releases the GIL in its random fills and ufuncs)
        from concurrent.futures import ThreadPoolExecutor
        pool = ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4))
        emb = pool.submit(lambda: quantize_rows(fp32_tensor(c, "tok")))
        cls = None if c.tied else pool.submit(lambda: quantize_rows(fp32_tensor(c, "wcls")))
        self.rms_final = fp32_tensor(c, "rms_final")
        self.rms_att = np.stack([fp32_tensor(c, "rms_att", l) for l in range(L)])
        self.rms_ffn = np.stack([fp32_tensor(c, "rms_ffn", l) for l in range(L)])
        hd = c.head_dim
        self.q_norm = np.stack([fp32_tensor(c, "q_norm", l) for l in range(L)]) if c.qk_norm else np.ones((L, hd), F)
        self.k_norm = np.stack([fp32_tensor(c, "k_norm", l) for l in range(L)]) if c.qk_norm else np.ones((L, hd), F)

        def stack(fn):
            qs = list(pool.map(fn, range(L)))
            return np.stack([a for a, _ in qs]), np.stack([b for _, b in qs])
        self.wqkv, self.s_wqkv = stack(lambda l: quantize_rows(np.concatenate(
            [fp32_tensor(c, "wq", l), fp32_tensor(c, "wk", l), fp32_tensor(c, "wv", l)])))
        self.wo, self.s_wo = stack(lambda l: quantize_rows(fp32_tensor(c, "wo", l)))
        if c.moe:
            self.router, self.s_router = stack(lambda l: quantize_rows(fp32_tensor(c, "router", l)))
            self.wg, self.s_wg = stack(lambda l: quantize_rows(fp32_tensor(c, "wg", l)))
            self.wu, self.s_wu = stack(lambda l: quantize_rows(fp32_tensor(c, "wu", l)))
            self.wd, self.s_wd = stack(lambda l: quantize_rows(fp32_tensor(c, "wd", l)))
        else:
            self.w1, self.s_w1 = stack(lambda l: quantize_rows(fp32_tensor(c, "w1", l)))
            self.w3, self.s_w3 = stack(lambda l: quantize_rows(fp32_tensor(c, "w3", l)))
            self.w2, self.s_w2 = stack(lambda l: quantize_rows(fp32_tensor(c, "w2", l)))
        self.emb_q, self.emb_s = emb.result()
        if c.tied:
            self.cls_q, self.cls_s = self.emb_q, self.emb_s
        else:
            self.cls_q, self.cls_s = cls.result()
        self.cls_s = fold_logits_scaling(self.cls_s, c.logits_scaling)
        pool.shutdown()
        self.cos, self.sin = rope_tables(c)
        if kv_scales is None:
            kv_scales = stored_kv_scales(c)
        self._set_kv(kv_scales)

    def _set_kv(self, kv_scales):
        c = self.cfg
        kv = np.asarray(kv_scales, F)
        self.kv_scales = kv if kv.ndim == 3 else kv.reshape(c.layers, 2)
        if self.kv_scales.ndim == 3 and self.kv_scales.shape != (c.layers, 2, c.kv_dim):
            raise ValueError(f"{c.name}: kv_scales shape {self.kv_scales.shape}")
        self.kvc = kv_constants(c, self.kv_scales)
        self.kvch = kv_channel_constants(c, self.kv_scales)
        self.kv_flags = kv_channel_flags(c, self.kv_scales)

    # the arrays a model consists of (dense; MoE replaces w1 / w3 / w2 with router / wg / wu / wd)
    DENSE = ("w1", "s_w1", "w3", "s_w3", "w2", "s_w2")
    MOE = ("router", "s_router", "wg", "s_wg", "wu", "s_wu", "wd", "s_wd")
    COMMON = ("emb_q", "emb_s", "rms_final", "rms_att", "rms_ffn", "q_norm", "k_norm", "wqkv", "s_wqkv", "wo",
              "s_wo", "cls_q", "cls_s", "cos", "sin", "kv_scales", "kvc")

    @classmethod
    def from_arrays(cls, cfg, arrays):
        """A model from given arrays (a model file's), no synthetic generation: every name of COMMON
        and of DENSE or MOE, with the shapes the class docstring states; q_norm / k_norm may be None
        (gains of 1), kvc may be None (computed from kv_scales), cos / sin may be None (computed)."""
        cfg.validate()
        self = cls.__new__(cls)
        self.cfg = c = cfg
        L, hd = c.layers, c.head_dim
        for k in cls.COMMON + (cls.MOE if c.moe else cls.DENSE):
            v = arrays.get(k)
            if v is None and k in ("q_norm", "k_norm"):
                v = np.ones((L, hd), F)
            if v is None and k in ("cos", "sin", "kvc"):
                continue
            if v is None:
                raise ValueError(f"{cfg.name}: array {k} missing")
            setattr(self, k, np.ascontiguousarray(v))
        # a tied classifier stays the embedding's arrays (one copy on the device)
        if arrays.get("cls_q") is arrays.get("emb_q"):
            self.cls_q = self.emb_q
        if arrays.get("cls_s") is arrays.get("emb_s"):
            self.cls_s = self.emb_s
        if getattr(self, "cos", None) is None or getattr(self, "sin", None) is None:
            self.cos, self.sin = rope_tables(c)
        kvc = getattr(self, "kvc", None)
        self._set_kv(self.kv_scales)
        if kvc is not None:
            self.kvc = np.asarray(kvc, F)
        expect = {"emb_q": (c.vocab, c.dim), "wqkv": (L, c.q_dim + 2 * c.kv_dim, c.dim), "wo": (L, c.dim, c.q_dim),
                  "cls_q": (c.vocab, c.dim), "cos": (c.seq_len, hd // 2), "sin": (c.seq_len, hd // 2),
                  "kvc": (L, 4), "rms_att": (L, c.dim), "rms_ffn": (L, c.dim), "rms_final": (c.dim,)}
        if not c.moe:
            expect.update({"w1": (L, c.hidden, c.dim), "w3": (L, c.hidden, c.dim), "w2": (L, c.dim, c.hidden)})
        for k, shp in expect.items():
            if getattr(self, k).shape != shp:
                raise ValueError(f"{cfg.name}: {k} has shape {getattr(self, k).shape}, expected {shp}")
        return self

    def digest(self):
        """sha256 over every array (a fingerprint of the model data)."""
        h = hashlib.sha256()
        for k in sorted(vars(self)):
            v = getattr(self, k)
            if isinstance(v, np.ndarray):
                h.update(k.encode())
                h.update(np.ascontiguousarray(v).tobytes())
        return h.hexdigest()


# ------------------------------------------------------------------ KV calibration
def _fp32_forward_rows(cfg, tokens, amax_out, weight=None):
    """Causal fp32 forward of `tokens` at positions 0.. (all rows at once, torch on the CPU),
    recording max|k| and max|v| per layer and cache channel into amax_out [L, 2, kv_dim] (after RoPE for
    k); returns the logits [M, vocab]. llama2.c run.c semantics (llm/ref_model.py:45-91) generalised as
    compiler/frontend/qhf.py:206-243; cfg.act "gelu_tanh" gates with GELU's tanh form."""
    import torch
    c = cfg
    fp32_tensor = weight if weight is not None else globals()["fp32_tensor"]
    M = len(tokens)
    t = lambda a: torch.from_numpy(np.require(a, F, requirements=["C", "W"]))   # (a read-only map: copied)
    H, Hk, hd = c.heads, c.kv_heads, c.head_dim
    G = H // Hk
    cos, sin = rope_tables(c)
    cos = t(np.repeat(cos[:M], 2, axis=1))
    sin = t(np.repeat(sin[:M], 2, axis=1))

    def rms(x, g):
        return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + c.eps) * g

    def swapneg(v):
        p = v.reshape(v.shape[:-1] + (-1, 2))
        return torch.stack((-p[..., 1], p[..., 0]), dim=-1).reshape(v.shape)

    if c.act == "gelu_tanh":
        act = lambda h: torch.nn.functional.gelu(h, approximate="tanh")
    else:
        act = torch.nn.functional.silu

    with torch.no_grad():
        x = t(fp32_tensor(c, "tok", -1))[torch.tensor(tokens)]
        mask = torch.tril(torch.ones(M, M, dtype=torch.bool))
        for l in range(c.layers):
            xb = rms(x, t(fp32_tensor(c, "rms_att", l)))
            q = (xb @ t(fp32_tensor(c, "wq", l)).T).reshape(M, H, hd)
            k = (xb @ t(fp32_tensor(c, "wk", l)).T).reshape(M, Hk, hd)
            v = xb @ t(fp32_tensor(c, "wv", l)).T
            if c.qk_norm:
                q = rms(q, t(fp32_tensor(c, "q_norm", l)))
                k = rms(k, t(fp32_tensor(c, "k_norm", l)))
            q = q * cos[:, None] + swapneg(q) * sin[:, None]
            k = k * cos[:, None] + swapneg(k) * sin[:, None]
            amax_out[l, 0] = np.maximum(amax_out[l, 0], k.reshape(M, -1).abs().amax(0).double().numpy())
            amax_out[l, 1] = np.maximum(amax_out[l, 1], v.abs().amax(0).double().numpy())
            kk = k.repeat_interleave(G, dim=1)                        # (M, H, hd)
            vv = v.reshape(M, Hk, hd).repeat_interleave(G, dim=1)
            s = torch.einsum("mhd,thd->hmt", q, kk) / np.sqrt(hd)
            s = s.masked_fill(~mask[None], float("-inf"))
            att = torch.einsum("hmt,thd->mhd", torch.softmax(s, dim=-1), vv).reshape(M, -1)
            x = x + att @ t(fp32_tensor(c, "wo", l)).T
            xb = rms(x, t(fp32_tensor(c, "rms_ffn", l)))
            if c.moe:
                sc = xb @ t(fp32_tensor(c, "router", l)).T               # (M, E)
                vals, ids = torch.topk(sc, c.top_k, dim=-1)
                wts = torch.softmax(vals, dim=-1)
                wg, wu, wd = (t(fp32_tensor(c, n, l)) for n in ("wg", "wu", "wd"))
                y = torch.zeros_like(x)
                for m in range(M):
                    for j in range(c.top_k):
                        e = int(ids[m, j])
                        h = act(wg[e] @ xb[m]) * (wu[e] @ xb[m])
                        y[m] += wts[m, j] * (wd[e] @ h)
                x = x + y
            else:
                h = act(xb @ t(fp32_tensor(c, "w1", l)).T) * (xb @ t(fp32_tensor(c, "w3", l)).T)
                x = x + h @ t(fp32_tensor(c, "w2", l)).T
        cls = fp32_tensor(c, "wcls") if not c.tied else fp32_tensor(c, "tok")
        logits = rms(x, t(fp32_tensor(c, "rms_final"))) @ t(cls).T
        if c.logits_scaling != 1.0:
            logits = logits / c.logits_scaling
        return logits.numpy()


def fp32_logits(cfg, tokens, weight=None):
    """Logits [M, vocab] of the causal fp32 forward of `tokens` at positions 0.. (the calibration run's
    model; weight(cfg, name, layer) as in calibrate_kv)."""
    amax = np.zeros((cfg.layers, 2, cfg.kv_dim), np.float64)
    return _fp32_forward_rows(cfg, list(tokens), amax, weight)


def calibrate_kv(cfg, tokens=None, chunk=None, weight=None, channel=None):
    """Static KV scales: max(absmax, 1e-8) / 127 over an fp32 run of the prompt, per layer [L, 2]
    (llm/test_l4.py:51-55, compiler/frontend/qhf.py:246-251), or with channel "k" / "v" / "kv"
    (default cfg.kv_channel) those parts per cache channel [L, 2, kv_dim], the others' rows the layer's
    single value (compiler/frontend/hf_generic.py:466-491). A text longer than seq_len is calibrated
    window by window. weight(cfg, name, layer): the fp32 tensors (default: the synthetic ones of
    fp32_tensor)."""
    channel = cfg.kv_channel if channel is None else channel
    tokens = cfg.prompt() if tokens is None else list(tokens)
    amax = np.zeros((cfg.layers, 2, cfg.kv_dim), np.float64)
    # tokens beyond seq_len: windows of seq_len, each from position 0 (a fresh cache), the max over them
    # (compiler/frontend/hf_generic.py:472-484)
    for w in range(0, max(len(tokens), 1), cfg.seq_len):
        _fp32_forward_rows(cfg, tokens[w:w + cfg.seq_len], amax, weight)
    if not channel:
        return (np.maximum(amax.max(-1), 1e-8) / 127.0).astype(F)
    out = np.repeat(amax.max(-1, keepdims=True), cfg.kv_dim, -1)
    for j, part in enumerate("kv"):
        if part in channel:
            out[:, j] = amax[:, j]
    return (np.maximum(out, 1e-8) / 127.0).astype(F)


_KV_FILE = os.path.join(HERE, "kv_scales.json")


def stored_kv_scales(cfg):
    """The recorded calibration of a named config (kv_scales.json, float32 bit patterns); the tiny
    test models are calibrated on the fly."""
    if os.path.exists(_KV_FILE):
        with open(_KV_FILE) as f:
            table = json.load(f)
        if cfg.name in table and table[cfg.name]["seed_w"] == cfg.seed_w and not cfg.kv_channel:
            return np.array(table[cfg.name]["bits"], np.uint32).view(F).reshape(cfg.layers, 2)
    if cfg.layers * cfg.dim <= 1 << 16:
        return calibrate_kv(cfg)
    raise FileNotFoundError(f"no recorded KV scales for {cfg.name}; run `python -m t2r_amd.weights --calibrate "
                            f"{cfg.name}` in a checkout that has the reference data")


def _main():
    import argparse
    import sys
    sys.path.insert(0, os.path.dirname(HERE))
    ap = argparse.ArgumentParser(description="record the static KV scales of the named configs")
    ap.add_argument("--calibrate", nargs="+", required=True)
    args = ap.parse_args()
    from t2r_amd import config as C
    table = json.load(open(_KV_FILE)) if os.path.exists(_KV_FILE) else {}
    for name in args.calibrate:
        cfg = C.get(name)
        kv = calibrate_kv(cfg)
        table[cfg.name] = {"seed_w": cfg.seed_w, "prompt_len": cfg.prompt_len,
                           "bits": [int(b) for b in kv.view(np.uint32).ravel()],
                           "values": [float(v) for v in kv.ravel()]}
        print(cfg.name, kv.ravel()[:6], "...", flush=True)
        with open(_KV_FILE, "w") as f:
            json.dump(table, f, indent=1)


if __name__ == "__main__":
    _main()
