"""Model configurations of the W8A8 decoder datapath.

One dataclass covers the five shapes the datapath is measured on plus the tiny
test models. The reference describes a model with llama2.c's `Config`
(llm/checkpoint.py:14-30: head_size = dim // heads) and, for HF models, with
`HFConfig` (compiler/frontend/qhf.py:97-121: head_dim, q_dim != dim, theta,
eps, tied embeddings, QK-norm). This one carries every field either needs, and
the numerics choices the reference leaves to the caller:

- `D`: the reduction lane width of the vector engine (sums run lane-wise over
  groups of D, then a pairwise tree; llm/ref_model.py:179-186). It changes
  RMSNorm / softmax results, so it is part of the model.
- `rope_method`: how the host builds the RoPE tables. "f32" is llama2.c run.c's
  float32 formula (llm/ref_model.py:34-41), "f64" the float64 one of
  compiler/frontend/qhf.py:183-189.
- MoE: `n_experts` experts with top-`top_k` routing; `hidden` is then the
  per-expert FFN width (compiler/frontend/hf_generic.py:602-663).
- The HF path's numerics options (compiler/frontend/hf_generic.py), all off by
  default (DeviceModel's form):
  - `attn_norm` "qsum": int8 probabilities eq = to_i8(F(e * 127)) and the
    output F(F(f32(sum eq V) * F(RECIP(f32(sum eq)) * 127)) * a_v) instead of
    p = F(e * RECIP(red_sum(e))) (:265-292);
  - `kv_channel` "k" / "v" / "kv": static K and / or V scales per cache channel
    (calibrated per channel, :466-491); K's folded into q before its
    quantisation, V's applied per output channel (:153-187);
  - `act` "gelu_tanh": the FFN gate's activation is GELU's tanh approximation
    from EXP and RECIP (GeGLU, :840-852) instead of SiLU;
  - `logits_scaling`: the logits divided by it, folded into the classifier's
    row scales as F(s / F(ls)) (:909-917).
"""
from dataclasses import dataclass, replace

import numpy as np


@dataclass(frozen=True)
class ModelConfig:
    name: str
    dim: int
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    seq_len: int
    theta: float = 10000.0
    eps: float = 1e-5
    qk_norm: bool = False
    tied: bool = True
    n_experts: int = 0
    top_k: int = 0
    rope_method: str = "f64"
    D: int = 16
    # synthetic weights: N(0, weight_std) (None: 1 / sqrt(fan_in)); norm gains 1 + gain_std * N(0, 1)
    weight_std: float = 0.02
    gain_std: float = 0.0
    emb_scale: float = 1.0
    seed_w: int = 0
    seed_p: int = 0
    prompt_len: int = 0
    decode_steps: int = 0
    attn_norm: str = "device"
    kv_channel: str = ""
    act: str = "silu"
    logits_scaling: float = 1.0

    @property
    def q_dim(self):
        return self.heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim

    @property
    def group(self):
        return self.heads // self.kv_heads

    @property
    def moe(self):
        return self.n_experts > 0

    def validate(self):
        if self.heads % self.kv_heads:
            raise ValueError(f"{self.name}: {self.heads} heads not a multiple of {self.kv_heads} KV heads")
        if self.head_dim % 2:
            raise ValueError(f"{self.name}: head_dim {self.head_dim} is odd (RoPE rotates pairs)")
        if self.D not in (8, 16):
            raise ValueError(f"{self.name}: D = {self.D} (8 or 16)")
        if self.rope_method not in ("f32", "f64"):
            raise ValueError(f"{self.name}: rope_method {self.rope_method!r}")
        if self.attn_norm not in ("device", "qsum"):
            raise ValueError(f"{self.name}: attn_norm {self.attn_norm!r} (device or qsum)")
        if self.kv_channel not in ("", "k", "v", "kv"):
            raise ValueError(f"{self.name}: kv_channel {self.kv_channel!r} ('', k, v or kv)")
        if self.act not in ("silu", "gelu_tanh"):
            raise ValueError(f"{self.name}: act {self.act!r} (silu or gelu_tanh)")
        if not (np.isfinite(self.logits_scaling) and self.logits_scaling != 0):
            raise ValueError(f"{self.name}: logits_scaling {self.logits_scaling}")
        if self.moe and not 1 <= self.top_k <= min(self.n_experts, 8):
            raise ValueError(f"{self.name}: top-{self.top_k} of {self.n_experts} experts")
        for n in ("dim", "hidden", "q_dim", "kv_dim"):
            if getattr(self, n) % 16:
                raise ValueError(f"{self.name}: {n} = {getattr(self, n)} not a multiple of 16")
        return self

    def with_(self, **kw):
        return replace(self, **kw).validate()

    def weight_bytes_per_token(self):
        """int8 weight bytes one decode step reads (the classifier included)."""
        d, q, kv, f = self.dim, self.q_dim, self.kv_dim, self.hidden
        per = (q + 2 * kv) * d + d * q
        if self.moe:
            per += self.n_experts * d + self.top_k * (2 * f * d + d * f)
        else:
            per += 2 * f * d + d * f
        return self.layers * per + self.vocab * d

    def prompt(self):
        """The seeded prompt: prompt_len uniform token ids."""
        return [int(t) for t in np.random.default_rng(self.seed_p).integers(0, self.vocab, self.prompt_len)]


# The five measured shapes (random weights; BASELINE.json "configs").
C1 = ModelConfig("c1-stories15m", dim=288, hidden=768, layers=6, heads=6, kv_heads=6, head_dim=48, vocab=32000,
                 seq_len=256, theta=10000.0, eps=1e-5, rope_method="f32", seed_w=1001, seed_p=2001,
                 prompt_len=32, decode_steps=128)
C2 = ModelConfig("c2-smollm2-135m", dim=576, hidden=1536, layers=30, heads=9, kv_heads=3, head_dim=64, vocab=49152,
                 seq_len=2048, theta=1e5, eps=1e-5, seed_w=1002, seed_p=2002, prompt_len=40, decode_steps=256)
C3 = ModelConfig("c3-qwen3-0.6b", dim=1024, hidden=3072, layers=28, heads=16, kv_heads=8, head_dim=128,
                 vocab=151936, seq_len=2048, theta=1e6, eps=1e-6, qk_norm=True, seed_w=1003, seed_p=2003,
                 prompt_len=2032, decode_steps=16)
C4 = ModelConfig("c4-llama3.2-1b", dim=2048, hidden=8192, layers=16, heads=32, kv_heads=8, head_dim=64,
                 vocab=128256, seq_len=2048, theta=5e5, eps=1e-5, seed_w=1004, seed_p=2004, prompt_len=512,
                 decode_steps=256)
C5 = ModelConfig("c5-granite-1b-a400m", dim=1024, hidden=512, layers=24, heads=16, kv_heads=8, head_dim=64,
                 vocab=49155, seq_len=2048, theta=1e4, eps=1e-6, n_experts=32, top_k=8, seed_w=1005, seed_p=2005,
                 prompt_len=64, decode_steps=256)

# Tiny models for the tests: the reference's co-simulation shapes (llm/test_l4.py:41-55, 159-162) and tiny
# versions of every generalisation (q_dim != dim, QK-norm, MoE).
TINY = ModelConfig("tiny", dim=32, hidden=64, layers=2, heads=2, kv_heads=2, head_dim=16, vocab=64, seq_len=16,
                   rope_method="f32", weight_std=None, gain_std=0.1, emb_scale=4.0, seed_w=3, seed_p=7,
                   prompt_len=4, decode_steps=12)
TINY_GQA = TINY.with_(name="tiny-gqa", heads=4, kv_heads=2, head_dim=8, seed_w=11)
TINY_QWEN = ModelConfig("tiny-qwen", dim=32, hidden=96, layers=2, heads=4, kv_heads=2, head_dim=16, vocab=80,
                        seq_len=40, theta=1e6, eps=1e-6, qk_norm=True, weight_std=None, gain_std=0.1,
                        emb_scale=4.0, seed_w=21, seed_p=22, prompt_len=20, decode_steps=12)
TINY_MOE = ModelConfig("tiny-moe", dim=32, hidden=32, layers=2, heads=4, kv_heads=2, head_dim=8, vocab=70,
                       seq_len=24, theta=1e4, eps=1e-6, n_experts=8, top_k=4, weight_std=None, gain_std=0.1,
                       emb_scale=4.0, seed_w=31, seed_p=32, prompt_len=6, decode_steps=10)

# the HF path's numerics options on tiny models: every option, and each kind of per-channel scale
TINY_HF = TINY_QWEN.with_(name="tiny-hf", attn_norm="qsum", kv_channel="k", act="gelu_tanh", logits_scaling=8.0,
                          seed_w=41)
TINY_HF_KV = TINY_GQA.with_(name="tiny-hf-kv", attn_norm="qsum", kv_channel="kv", logits_scaling=3.0, seed_w=51)
TINY_HF_V = TINY.with_(name="tiny-hf-v", kv_channel="v", act="gelu_tanh", seed_w=61)
TINY_HF_MOE = TINY_MOE.with_(name="tiny-hf-moe", attn_norm="qsum", kv_channel="k", act="gelu_tanh", seed_w=71)

CONFIGS = {c.name: c.validate() for c in (C1, C2, C3, C4, C5)}
TINY_CONFIGS = {c.name: c.validate() for c in (TINY, TINY_GQA, TINY_QWEN, TINY_MOE, TINY_HF, TINY_HF_KV, TINY_HF_V,
                                                TINY_HF_MOE)}


def hf_options(cfg, name=None):
    """cfg with every HF-path option on (qsum, K per channel, GELU-tanh gate, logits scaling 8), as the
    reference's HF builds compute (compiler/frontend/hf_generic.py); named name or cfg.name + "-hf"."""
    return cfg.with_(name=name or cfg.name + "-hf", attn_norm="qsum", kv_channel="k", act="gelu_tanh",
                     logits_scaling=8.0)


def get(name):
    for table in (CONFIGS, TINY_CONFIGS):
        if name in table:
            return table[name]
    short = {"c1": C1, "c2": C2, "c3": C3, "c4": C4, "c5": C5}
    if name in short:
        return short[name]
    if name.endswith("-hf") and name[:-3] in CONFIGS:
        return hf_options(CONFIGS[name[:-3]])
    raise KeyError(f"unknown config {name!r}")
