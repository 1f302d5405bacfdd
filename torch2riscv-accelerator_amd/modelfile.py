"""Model files and tokenizers of the reference's runtime, read (and written) on the host.

- `.w8a8` device files (llm/export_w8a8.py:15-30 layout, :97-128 writer, :131-167 reader): a
  64-byte header, a table of 32-byte entries, then every tensor 64-byte aligned; per-layer
  tensors at layer_base + l * layer_stride. Linear weights are stored as D-wide B tiles
  (out / D, in, D): tile t holds output rows [t D, (t + 1) D) transposed. Version 1 is the
  reference's llama2.c-shaped model. Version 2 (this package's extension, which a version-1 reader
  refuses) adds what version 1 cannot express: q_dim != dim, QK-norm, MoE, theta / eps, the RoPE
  method, an untied classifier and the HF path's numerics options (qsum, the GELU-tanh gate, the
  logits scaling folded into s_wcls, per-channel KV scales as a per-layer `kvch` tensor), in a `cfg`
  entry and extra named tensors; its linear weights are row-major (out, in) int8 (the B tiles serve
  the reference's matrix engine, not this device).
- llama2.c legacy fp32 checkpoints (llm/checkpoint.py:30-59): 7 int32 (dim, hidden, layers, heads,
  kv_heads, vocab, seq_len; vocab < 0: separate classifier), then the fp32 tensors in run.c's order.
- `tokenizer.bin`, llama2.c's SentencePiece-style BPE (llm/tokenizer.py:10-67).
- HuggingFace `tokenizer.json` through the `tokenizers` library, which the reference's own port
  (compiler/frontend/hf_tokenizer.py:1-20) states it is identical to.
"""
import dataclasses
import heapq
import os
import re
import struct

import numpy as np

from . import config as C
from . import weights as W

F = np.float32
MAGIC = b"W8A8LLM\0"
HEADER = struct.Struct("<8s12I")      # magic, version, D, dim, hidden, layers, heads, kv_heads, vocab,
#                                       seq_len, n_entries, layer_base, layer_stride (padded to 64 bytes)
ENTRY = struct.Struct("<16s4I")       # name, offset, bytes, per_layer, reserved
ALIGN = 64
V1_LAYER = ("rms_att", "rms_ffn", "wqkv", "s_wqkv", "wo", "s_wo", "w13", "s_w13", "w2", "s_w2", "kvp")
INT8 = {"emb_q", "wcls", "wqkv", "wo", "w13", "w2", "router", "wg", "wu", "wd"}
BOS, EOS = 1, 2


def _up(n):
    return (n + ALIGN - 1) // ALIGN * ALIGN


# ------------------------------------------------------------------ B tiles
def to_tiles(q, d):
    """int8 rows (out, in) -> D-wide B tiles (out / d, in, d): tiles[t, k, j] = q[t d + j, k]."""
    out, k = q.shape
    if out % d or k % d:
        raise ValueError(f"linear {out} x {k} is not a multiple of D = {d}")
    return np.ascontiguousarray(np.swapaxes(q.reshape(out // d, d, k), 1, 2))


def from_tiles(tiles):
    """B tiles (n, in, d) -> rows (n d, in)."""
    n, k, d = tiles.shape
    return np.ascontiguousarray(np.swapaxes(tiles, 1, 2).reshape(n * d, k))


# ------------------------------------------------------------------ .w8a8
def _rope_wide(t, width):
    """Per-head table (seq, hd / 2) -> (seq, width): column c holds pair c // 2 of its head (each value
    twice, for both elements of its rotation pair)."""
    hp = t.shape[1]
    return np.ascontiguousarray(t[:, (np.arange(width) // 2) % hp]).astype(F)


def _rope_head(wide, hd):
    """(seq, width) -> the per-head table (seq, hd / 2); every head's columns must agree."""
    hp = hd // 2
    first = wide[:, 0:hd:2]
    for h in range(1, wide.shape[1] // hd):
        if not np.array_equal(wide[:, h * hd:(h + 1) * hd:2].view(np.uint32), first.view(np.uint32)):
            raise ValueError("RoPE table differs between heads")
    if not np.array_equal(wide[:, 1:hd:2].view(np.uint32), first.view(np.uint32)):
        raise ValueError("RoPE table pair elements differ")
    return np.ascontiguousarray(first[:, :hp]).astype(F)


def _kvp(qm):
    """(L, 8) float32: s_k, s_v, 1/s_k, 1/s_v, a_k, a_v, 0, 0 per layer (per-channel scales: channel 0's
    values here, the rows in `kvch`)."""
    out = np.zeros((qm.cfg.layers, 8), F)
    out[:, 0:2] = qm.kv_scales[:, :, 0] if qm.kv_scales.ndim == 3 else qm.kv_scales
    out[:, 2:6] = qm.kvc
    return out


_CFG_WORDS = 16


def _cfg_block(c):
    """Words 0-5 head_dim, qk_norm, tied, n_experts, top_k, RoPE method; 6-9 eps, theta (float64);
    10 qsum, 11 the gate (1 GELU-tanh), 12 per-channel KV (bit 0 K, bit 1 V), 13-14 logits_scaling
    (float64; already folded into s_wcls)."""
    w = np.zeros(_CFG_WORDS, np.uint32)
    w[0:6] = [c.head_dim, int(c.qk_norm), int(c.tied), c.n_experts, c.top_k, 1 if c.rope_method == "f64" else 0]
    w[6:8] = np.array([c.eps], np.float64).view(np.uint32)       # float64: the config's values exactly
    w[8:10] = np.array([c.theta], np.float64).view(np.uint32)
    w[10:13] = [int(c.attn_norm == "qsum"), int(c.act == "gelu_tanh"),
                ("k" in c.kv_channel) | (("v" in c.kv_channel) << 1)]
    w[13:15] = np.array([c.logits_scaling], np.float64).view(np.uint32)
    return w


def is_v1(cfg):
    """Whether the reference's version-1 layout can hold the model (llama2.c shape: q_dim == dim,
    head_dim = dim / heads, no QK-norm, no MoE)."""
    c = cfg
    return (c.q_dim == c.dim and c.head_dim * c.heads == c.dim and not c.qk_norm and not c.moe
            and c.eps == 1e-5 and c.rope_method == "f32" and c.theta == 10000.0 and c.attn_norm == "device"
            and not c.kv_channel and c.act == "silu" and c.logits_scaling == 1.0)


def write_w8a8(qm, path, d=None):
    """Write a QuantModel as a .w8a8 file (version 1 when the model fits it, else 2); returns bytes."""
    c = qm.cfg
    d = d or c.D
    v1 = is_v1(c)
    width = c.dim if v1 else c.head_dim
    lin = (lambda q: to_tiles(q, d)) if v1 else (lambda q: q)
    glob = [("emb_q", qm.emb_q), ("emb_s", qm.emb_s), ("rms_final", qm.rms_final),
            ("wcls", lin(qm.cls_q)), ("s_wcls", qm.cls_s),
            ("rope_cos", _rope_wide(qm.cos, width)), ("rope_sin", _rope_wide(qm.sin, width))]
    if not v1:
        glob.append(("cfg", _cfg_block(c)))
    kvp = _kvp(qm)

    def layer(l):
        t = [("rms_att", qm.rms_att[l]), ("rms_ffn", qm.rms_ffn[l]), ("wqkv", lin(qm.wqkv[l])),
             ("s_wqkv", qm.s_wqkv[l]), ("wo", lin(qm.wo[l])), ("s_wo", qm.s_wo[l])]
        if c.moe:
            t += [("router", qm.router[l]), ("s_router", qm.s_router[l]), ("wg", qm.wg[l]), ("s_wg", qm.s_wg[l]),
                  ("wu", qm.wu[l]), ("s_wu", qm.s_wu[l]), ("wd", qm.wd[l]), ("s_wd", qm.s_wd[l])]
        else:
            t += [("w13", lin(np.concatenate([qm.w1[l], qm.w3[l]]))),
                  ("s_w13", np.concatenate([qm.s_w1[l], qm.s_w3[l]])),
                  ("w2", lin(qm.w2[l])), ("s_w2", qm.s_w2[l])]
        t.append(("kvp", kvp[l]))
        if qm.kv_scales.ndim == 3:
            t.append(("kvch", qm.kv_scales[l]))
        if c.qk_norm:
            t += [("q_norm", qm.q_norm[l]), ("k_norm", qm.k_norm[l])]
        return [(n, np.ascontiguousarray(a)) for n, a in t]

    first = layer(0)
    n_entries = len(glob) + len(first)
    offs, pos = [], _up(64 + ENTRY.size * n_entries)
    for n, a in glob:
        offs.append((n, pos, a.nbytes, 0))
        pos = _up(pos + a.nbytes)
    layer_base, rel = pos, 0
    for n, a in first:
        offs.append((n, rel, a.nbytes, 1))
        rel = _up(rel + a.nbytes)
    stride = rel
    total = layer_base + stride * c.layers
    with open(path, "wb") as f:
        f.truncate(total)
        f.seek(0)
        f.write(HEADER.pack(MAGIC, 1 if v1 else 2, d, c.dim, c.hidden, c.layers, c.heads, c.kv_heads, c.vocab,
                            c.seq_len, n_entries, layer_base, stride))
        f.seek(64)
        for n, o, nb, per in offs:
            f.write(ENTRY.pack(n.encode().ljust(16, b"\0"), o, nb, per, 0))
        for (n, a), (_, o, _, _) in zip(glob, offs):
            f.seek(o)
            f.write(a.tobytes())
        for l in range(c.layers):
            for (n, a), (_, o, nb, _) in zip(layer(l) if l else first, offs[len(glob):]):
                if a.nbytes != nb:
                    raise ValueError(f"layer {l}: {n} has {a.nbytes} bytes, layer 0 {nb}")
                f.seek(layer_base + l * stride + o)
                f.write(a.tobytes())
    return total


class W8A8File:
    """A .w8a8 file, memory-mapped: header fields, the entry table and each tensor as a view."""

    def __init__(self, path):
        self.path = path
        self.raw = np.memmap(path, dtype=np.uint8, mode="r")
        if self.raw.size < 64:
            raise ValueError(f"{path}: not a w8a8 file")
        h = HEADER.unpack(self.raw[:HEADER.size].tobytes())
        if h[0] != MAGIC or h[1] not in (1, 2):
            raise ValueError(f"{path}: not a w8a8 v1 / v2 file")
        (self.version, self.d, self.dim, self.hidden, self.layers, self.heads, self.kv_heads, self.vocab,
         self.seq_len, n, self.layer_base, self.layer_stride) = h[1:]
        self.entries = {}
        for i in range(n):
            name, off, nb, per, _ = ENTRY.unpack(self.raw[64 + i * ENTRY.size:64 + (i + 1) * ENTRY.size].tobytes())
            self.entries[name.rstrip(b"\0").decode()] = (off, nb, bool(per))
        end = self.layer_base + self.layer_stride * self.layers
        if end > self.raw.size:
            raise ValueError(f"{path}: {self.raw.size} bytes, the layers need {end}")

    def offset(self, name, layer=None):
        off, _, per = self.entries[name]
        if per:
            if layer is None:
                raise ValueError(f"{name} is per layer")
            return self.layer_base + layer * self.layer_stride + off
        return off

    def get(self, name, layer=None):
        """The tensor's bytes as a flat view of its element type (int8 weights, uint32 cfg, float32)."""
        off, nb = self.offset(name, layer), self.entries[name][1]
        dt = np.int8 if name in INT8 else (np.uint32 if name == "cfg" else F)
        return self.raw[off:off + nb].view(dt)

    def config(self, name=None):
        """The ModelConfig the file describes."""
        name = name or os.path.splitext(os.path.basename(self.path))[0]
        base = dict(name=name, dim=self.dim, hidden=self.hidden, layers=self.layers, heads=self.heads,
                    kv_heads=self.kv_heads, vocab=self.vocab, seq_len=self.seq_len, D=self.d)
        if self.version == 1:
            return C.ModelConfig(head_dim=self.dim // self.heads, theta=10000.0, eps=1e-5, rope_method="f32",
                                 tied=False, **base)
        w = self.get("cfg")
        ls = float(np.array(w[13:15]).view(np.float64)[0])
        return C.ModelConfig(head_dim=int(w[0]), qk_norm=bool(w[1]), tied=bool(w[2]), n_experts=int(w[3]),
                             top_k=int(w[4]), rope_method="f64" if w[5] else "f32",
                             eps=float(np.array(w[6:8]).view(np.float64)[0]),
                             theta=float(np.array(w[8:10]).view(np.float64)[0]),
                             attn_norm="qsum" if w[10] else "device", act="gelu_tanh" if w[11] else "silu",
                             kv_channel=("k" if w[12] & 1 else "") + ("v" if w[12] & 2 else ""),
                             logits_scaling=ls if ls else 1.0, **base)

    def quant_model(self, name=None):
        """The QuantModel (row-major int8 weights) of the file. A version-1 classifier equal to the
        embedding rows becomes a tied one (one copy on the device)."""
        c = self.config(name)
        L, d, hd = c.layers, self.d, c.head_dim

        def rows(x, n_out, k):                     # a linear's int8 rows from its stored form
            return from_tiles(x.reshape(n_out // d, k, d)) if self.version == 1 else np.asarray(x).reshape(n_out, k)
        a = {"emb_q": self.get("emb_q").reshape(c.vocab, c.dim), "emb_s": self.get("emb_s"),
             "rms_final": self.get("rms_final")}
        cls_q = rows(self.get("wcls"), c.vocab, c.dim)
        cls_s = np.array(self.get("s_wcls"))
        if self.version == 1 and np.array_equal(cls_q, a["emb_q"]) and np.array_equal(
                cls_s.view(np.uint32), a["emb_s"].view(np.uint32)):
            c = dataclasses.replace(c, tied=True)
        a["cls_q"], a["cls_s"] = (a["emb_q"], a["emb_s"]) if c.tied else (cls_q, cls_s)
        if c.tied and not np.array_equal(cls_s.view(np.uint32), a["emb_s"].view(np.uint32)):
            a["cls_s"] = cls_s                     # the embedding's rows with the logits scaling folded in
        a["cos"] = _rope_head(self.get("rope_cos").reshape(c.seq_len, -1), hd)
        a["sin"] = _rope_head(self.get("rope_sin").reshape(c.seq_len, -1), hd)

        def per(n, f=lambda x: x):
            return np.stack([f(self.get(n, l)) for l in range(L)])
        a["rms_att"], a["rms_ffn"] = per("rms_att"), per("rms_ffn")
        a["wqkv"] = per("wqkv", lambda x: rows(x, c.q_dim + 2 * c.kv_dim, c.dim))
        a["s_wqkv"] = per("s_wqkv")
        a["wo"] = per("wo", lambda x: rows(x, c.dim, c.q_dim))
        a["s_wo"] = per("s_wo")
        if c.moe:
            E, Fh = c.n_experts, c.hidden
            a["router"], a["s_router"] = per("router", lambda x: x.reshape(E, c.dim)), per("s_router")
            a["wg"], a["s_wg"] = per("wg", lambda x: x.reshape(E, Fh, c.dim)), per("s_wg", lambda x: x.reshape(E, Fh))
            a["wu"], a["s_wu"] = per("wu", lambda x: x.reshape(E, Fh, c.dim)), per("s_wu", lambda x: x.reshape(E, Fh))
            a["wd"], a["s_wd"] = per("wd", lambda x: x.reshape(E, c.dim, Fh)), per("s_wd", lambda x: x.reshape(E, c.dim))
        else:
            w13 = per("w13", lambda x: rows(x, 2 * c.hidden, c.dim))
            s13 = per("s_w13")
            a["w1"], a["w3"] = w13[:, :c.hidden], w13[:, c.hidden:]
            a["s_w1"], a["s_w3"] = s13[:, :c.hidden], s13[:, c.hidden:]
            a["w2"] = per("w2", lambda x: rows(x, c.dim, c.hidden))
            a["s_w2"] = per("s_w2")
        kvp = per("kvp")
        a["kv_scales"], a["kvc"] = kvp[:, 0:2], kvp[:, 2:6]
        if "kvch" in self.entries:
            a["kv_scales"] = per("kvch", lambda x: x.reshape(2, c.kv_dim))
        if c.qk_norm:
            a["q_norm"], a["k_norm"] = per("q_norm"), per("k_norm")
        return W.QuantModel.from_arrays(c, a)


def read_w8a8(path, name=None):
    """QuantModel of a .w8a8 file."""
    return W8A8File(path).quant_model(name)


# ------------------------------------------------------------------ llama2.c checkpoints
def read_llama2c(path):
    """(ModelConfig, {name: float32 array}) of a llama2.c legacy checkpoint, memory-mapped.
    Names: tok, rms_att, wq, wk, wv, wo, rms_ffn, w1, w2, w3, rms_final, wcls (the embedding
    when shared); linear weights (out, in) per layer."""
    raw = np.memmap(path, dtype=F, mode="r")
    if raw.size < 7:
        raise ValueError(f"{path}: not a llama2.c checkpoint")
    dim, hidden, layers, heads, kv_heads, vocab, seq = struct.unpack("<7i", raw[:7].tobytes())
    shared = vocab > 0
    vocab = abs(vocab)
    if min(dim, hidden, layers, heads, kv_heads, vocab, seq) <= 0 or dim % heads:
        raise ValueError(f"{path}: header {dim, hidden, layers, heads, kv_heads, vocab, seq} is not a llama2.c one")
    hs = dim // heads
    kv = kv_heads * hs
    order = [("tok", (vocab, dim)), ("rms_att", (layers, dim)), ("wq", (layers, dim, dim)), ("wk", (layers, kv, dim)),
             ("wv", (layers, kv, dim)), ("wo", (layers, dim, dim)), ("rms_ffn", (layers, dim)),
             ("w1", (layers, hidden, dim)), ("w2", (layers, dim, hidden)), ("w3", (layers, hidden, dim)),
             ("rms_final", (dim,)), ("rope", (seq * hs,))]       # run.c's (unused) precomputed RoPE floats
    if not shared:
        order.append(("wcls", (vocab, dim)))
    w, pos = {}, 7
    for name, shape in order:
        n = int(np.prod(shape))
        w[name] = raw[pos:pos + n].reshape(shape)
        pos += n
    if pos != raw.size:
        raise ValueError(f"{path}: {raw.size} floats, a llama2.c checkpoint of this header has {pos}")
    del w["rope"]
    if shared:
        w["wcls"] = w["tok"]
    cfg = C.ModelConfig(name=os.path.splitext(os.path.basename(path))[0], dim=dim, hidden=hidden, layers=layers,
                        heads=heads, kv_heads=kv_heads, head_dim=hs, vocab=vocab, seq_len=seq, theta=10000.0,
                        eps=1e-5, rope_method="f32", tied=shared)
    return cfg, w


def quant_model_from_fp32(cfg, w, kv_scales=None, calib_tokens=None, stored=None):
    """Quantise fp32 llama2.c-named weights (read_llama2c, hf_weights) as the reference's exporters do
    (llm/export_w8a8.py:75-95, compiler/frontend/hf_generic.py:872-917: per-row int8 of every linear,
    q | k | v rows stacked; MoE experts row by row; the logits scaling folded into the classifier's
    scales). Extra names: q_norm / k_norm [L, hd] (QK-norm), router [L, E, d], wg / wu [L, E, F, d],
    wd [L, E, d, F] (MoE). kv_scales (layers, 2) or (layers, 2, kv_dim) as the reference's --kv file;
    None: calibrated by an fp32 run of calib_tokens (per channel as cfg.kv_channel says). stored: int8 rows
    and scales to take as they are instead of quantizing ({name: (q, s)}, a compressed-tensors checkpoint's)."""
    L = cfg.layers
    stored = stored or {}

    def quant(name, l=None):
        if name in stored:
            q, sc = stored[name]
            return (q, sc) if l is None else (q[l], sc[l])
        return W.quantize_rows(w[name] if l is None else w[name][l])

    def stack(fn):
        qs = [fn(l) for l in range(L)]
        return np.stack([q for q, _ in qs]), np.stack([s for _, s in qs])
    a = {}
    a["emb_q"], a["emb_s"] = W.quantize_rows(w["tok"])
    if cfg.tied:
        a["cls_q"], a["cls_s"] = a["emb_q"], a["emb_s"]
    else:
        a["cls_q"], a["cls_s"] = quant("wcls")
    a["cls_s"] = W.fold_logits_scaling(a["cls_s"], cfg.logits_scaling)
    a["rms_final"] = np.array(w["rms_final"], F)
    a["rms_att"], a["rms_ffn"] = np.array(w["rms_att"], F), np.array(w["rms_ffn"], F)
    if cfg.qk_norm:
        a["q_norm"], a["k_norm"] = np.array(w["q_norm"], F), np.array(w["k_norm"], F)
    def qkv(l):
        parts = [quant(n, l) for n in ("wq", "wk", "wv")]
        return np.concatenate([q for q, _ in parts]), np.concatenate([s_ for _, s_ in parts])
    a["wqkv"], a["s_wqkv"] = stack(qkv)
    for n in ("wo",) + (("router", "wg", "wu", "wd") if cfg.moe else ("w1", "w3", "w2")):
        a[n], a["s_" + n] = stack(lambda l, n=n: quant(n, l))
    if kv_scales is None:
        def weight(c, name, layer=-1):
            v = w[name]
            return np.asarray(v if layer < 0 or name in ("tok", "wcls", "rms_final") else v[layer], F)
        toks = list(calib_tokens) if calib_tokens is not None else [BOS] + list(range(3, 3 + min(31, cfg.vocab - 3)))
        kv_scales = W.calibrate_kv(cfg, toks, weight=weight)
    kv = np.asarray(kv_scales, F)
    a["kv_scales"] = kv if kv.ndim == 3 else kv.reshape(L, 2)
    return W.QuantModel.from_arrays(cfg, a)


def write_llama2c(path, cfg, w):
    """Write fp32 weights as a llama2.c legacy checkpoint (the layout read_llama2c reads)."""
    hs = cfg.dim // cfg.heads
    with open(path, "wb") as f:
        f.write(struct.pack("<7i", cfg.dim, cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads,
                            cfg.vocab if cfg.tied else -cfg.vocab, cfg.seq_len))
        for n in ("tok", "rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3", "rms_final"):
            f.write(np.ascontiguousarray(w[n], F).tobytes())
        f.write(np.zeros(cfg.seq_len * hs, F).tobytes())
        if not cfg.tied:
            f.write(np.ascontiguousarray(w["wcls"], F).tobytes())


# ------------------------------------------------------------------ tokenizers
class Llama2cTokenizer:
    """tokenizer.bin of llama2.c: int32 max_token_length, then per id a float32 score, an int32
    length and the piece's bytes; a piece listed twice maps to its first id.

    encode() gives run.c's ids (llm/tokenizer.py:24-52): BOS, a " " dummy prefix for non-empty
    text, one piece per UTF-8 code point (at most 4 bytes; an unknown one as its bytes, id = byte
    + 3), then merges: each step joins the adjacent pair (BOS included) whose joined piece is in
    the vocabulary with the highest score above -1e10 (a NaN score never qualifies), the leftmost
    such pair on equal scores, until none is left. Here the pairs wait in a heap keyed by (score,
    position of the left token) over a linked list of the tokens; a merge keeps the left token's
    position, so the positions still order the live tokens, and a popped pair is used only if both
    tokens are still live, adjacent and unchanged. That picks the same pair as a rescan of the list
    at every step, in O(n log n) rather than O(n^2).

    decode() prints as run.c (llm/tokenizer.py:54-67): after BOS a piece loses one leading space;
    a piece "<0xHH>" is the byte HH; a single byte that is neither printable ASCII nor C whitespace
    prints nothing."""
    _HEX = frozenset(b"0123456789abcdefABCDEF")
    _SPACE = frozenset(b" \t\n\r\x0b\x0c")

    def __init__(self, path, vocab_size):
        with open(path, "rb") as f:
            blob = memoryview(f.read())
        (self.max_token_length,) = struct.unpack_from("<i", blob, 0)
        self.pieces, self.scores = [], []
        at = 4
        for _ in range(vocab_size):
            score, n = struct.unpack_from("<fi", blob, at)
            self.scores.append(score)
            self.pieces.append(bytes(blob[at + 8:at + 8 + n]))
            at += 8 + n
        self.ids = {}
        for i in range(vocab_size - 1, -1, -1):    # lowest id last, so it is the one kept
            self.ids[self.pieces[i]] = i
        self._shown = {}

    def _code_points(self, data):
        out, i = [], 0
        while i < len(data):
            j = i + 1
            while j < min(len(data), i + 4) and data[j] >> 6 == 2:   # continuation bytes 10xxxxxx
                j += 1
            tid = self.ids.get(data[i:j])
            if tid is None:
                out.extend(c + 3 for c in data[i:j])
            else:
                out.append(tid)
            i = j
        return out

    def _merge(self, tok):
        n = len(tok)
        nxt, prv, live = list(range(1, n + 1)), list(range(-1, n - 1)), [True] * n
        heap = []

        def offer(a):                              # the pair (a, its right neighbour), if it merges
            b = nxt[a]
            if b < n:
                m = self.ids.get(self.pieces[tok[a]] + self.pieces[tok[b]])
                if m is not None and self.scores[m] > -1e10:
                    heapq.heappush(heap, (-self.scores[m], a, b, tok[a], tok[b], m))

        for a in range(n - 1):
            offer(a)
        while heap:
            _, a, b, ta, tb, m = heapq.heappop(heap)
            if not live[a] or nxt[a] != b or tok[a] != ta or tok[b] != tb:
                continue                           # stale: a neighbour merged since it was offered
            tok[a], live[b] = m, False
            nxt[a] = nxt[b]
            if nxt[a] < n:
                prv[nxt[a]] = a
            if prv[a] >= 0:
                offer(prv[a])
            offer(a)
        out, a = [], 0
        while a < n:
            out.append(tok[a])
            a = nxt[a]
        return out

    def encode(self, text, bos=True, eos=False):
        data = text.encode("utf-8")
        tok = ([BOS] if bos else []) + ([self.ids[b" "]] if data else []) + self._code_points(data)
        tok = self._merge(tok)
        return tok + [EOS] if eos else tok

    def _printed(self, p):
        if len(p) == 6 and p[:3] == b"<0x" and p[5:] == b">" and p[3] in self._HEX and p[4] in self._HEX:
            p = bytes([int(p[3:5].decode(), 16)])
        if len(p) == 1 and not (32 <= p[0] <= 126 or p[0] in self._SPACE):
            return b""
        return p

    def piece(self, prev, token):
        """The bytes run.c prints for `token` when `prev` came before it."""
        p = self.pieces[token]
        if prev == BOS and p[:1] == b" ":
            return self._printed(p[1:])
        if token not in self._shown:
            self._shown[token] = self._printed(p)
        return self._shown[token]

    def decode(self, tokens):
        """Text of a token sequence that starts with BOS (what run.c prints for tokens[1:])."""
        return b"".join(self.piece(a, b) for a, b in zip(tokens, tokens[1:])).decode("utf-8", "replace")


class HFTokenizer:
    """A HuggingFace tokenizer.json (a file, or a directory holding one) through the `tokenizers`
    library: encode() without the file's post-processor (BOS only when asked), decode() keeping
    special tokens, as the reference's port does (compiler/frontend/hf_tokenizer.py:149-205)."""

    def __init__(self, path, bos_id=None):
        from tokenizers import Tokenizer
        if os.path.isdir(path):
            path = os.path.join(path, "tokenizer.json")
        self.tk = Tokenizer.from_file(path)
        self.bos_id = bos_id

    def encode(self, text, bos=True, eos=False):
        ids = self.tk.encode(text, add_special_tokens=False).ids
        return ([self.bos_id] if bos and self.bos_id is not None else []) + ids

    def decode(self, tokens):
        return self.tk.decode(list(tokens), skip_special_tokens=False)


def open_tokenizer(path, vocab_size, bos_id=None):
    """tokenizer.bin (llama2.c, BOS = 1) or tokenizer.json / a directory with one (HuggingFace; BOS
    prepended only when bos_id is given, as the reference's callers do)."""
    if os.path.isdir(path) or path.endswith(".json"):
        return HFTokenizer(path, bos_id=bos_id)
    return Llama2cTokenizer(path, vocab_size)


# ------------------------------------------------------------------ HuggingFace checkpoints
# A model directory with config.json and *.safetensors, as the reference's HF path reads it
# (compiler/frontend/qhf.py:97-181): the fp32 weights (F32 / F16 / BF16 stored), q / k rows (and
# QK-norm gains) reordered from HF's rotate-half halves to the interleaved RoPE pairs this datapath
# rotates, then W8A8-quantised like every other source. Mixtral-style MoE blocks as
# compiler/frontend/hf_generic.py:602-663 reads them.
HF_ARCHS = ("LlamaForCausalLM", "MistralForCausalLM", "Qwen3ForCausalLM", "MixtralForCausalLM")
_HF_ACT = {"silu": "silu", "swish": "silu", "gelu_pytorch_tanh": "gelu_tanh", "gelu_tanh": "gelu_tanh"}


def read_safetensors(path):
    """{name: float32 array} of a .safetensors file (8-byte little-endian header length, a JSON header,
    the raw tensors; F32 kept memory-mapped, F16 / BF16 widened; I8 (a compressed-tensors checkpoint's
    weights) kept int8). Executes nothing from the file."""
    import json
    raw = np.memmap(path, dtype=np.uint8, mode="r")
    n = int(raw[:8].view("<u8")[0])
    header = json.loads(bytes(raw[8:8 + n]).decode("utf-8"))
    base = 8 + n
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        a, b = info["data_offsets"]
        buf = raw[base + a:base + b]
        dt = info["dtype"]
        if dt == "F32":
            v = buf.view("<f4")
        elif dt == "F16":
            v = buf.view("<f2").astype(F)
        elif dt == "BF16":
            v = (buf.view("<u2").astype(np.uint32) << 16).view(F)
        elif dt == "I8":
            v = buf.view(np.int8)
        else:
            raise ValueError(f"{path}: {name} has dtype {dt} (F32, F16, BF16 or I8)")
        out[name] = v.reshape(info["shape"])
    return out


def hf_config(path, seq_len=2048, name=None, D=16, **options):
    """The ModelConfig of an HF model directory (config.json; qhf.py:97-121). options: the HF path's
    numerics options (attn_norm, kv_channel); act and logits_scaling come from the config."""
    import json
    c = json.load(open(os.path.join(path, "config.json")))
    arch = (c.get("architectures") or ["LlamaForCausalLM"])[0]
    if arch not in HF_ARCHS:
        raise ValueError(f"{path}: architecture {arch} (supported: {', '.join(HF_ARCHS)})")
    rp = c.get("rope_parameters") or {}
    scaling = c.get("rope_scaling") or ({k: v for k, v in rp.items() if k != "rope_theta"}
                                        if rp.get("rope_type", "default") != "default" else None)
    if scaling:
        raise ValueError(f"{path}: rope scaling {scaling} is not supported")
    if c.get("attention_bias") or c.get("mlp_bias"):
        raise ValueError(f"{path}: linear biases are not supported (W8A8 rows with one scale each)")
    act = c.get("hidden_act", c.get("hidden_activation", "silu"))
    if act not in _HF_ACT:
        raise ValueError(f"{path}: activation {act} (supported: {', '.join(_HF_ACT)})")
    if c.get("quantization_config") is not None:
        CompressedScheme(c["quantization_config"])          # refuses what the datapath cannot take as it is
    heads = c["num_attention_heads"]
    moe = arch == "MixtralForCausalLM"
    cfg = C.ModelConfig(
        name=name or os.path.basename(os.path.normpath(path)), dim=c["hidden_size"], hidden=c["intermediate_size"],
        layers=c["num_hidden_layers"], heads=heads, kv_heads=c.get("num_key_value_heads") or heads,
        head_dim=c.get("head_dim") or c["hidden_size"] // heads, vocab=c["vocab_size"],
        seq_len=min(seq_len, c.get("max_position_embeddings", seq_len)),
        theta=float(c.get("rope_theta", rp.get("rope_theta", 10000.0))), eps=float(c.get("rms_norm_eps", 1e-5)),
        qk_norm=arch.startswith("Qwen3"), tied=bool(c.get("tie_word_embeddings", False)),
        n_experts=c["num_local_experts"] if moe else 0, top_k=c["num_experts_per_tok"] if moe else 0,
        rope_method="f64", D=D, act=_HF_ACT[act], logits_scaling=float(c.get("logits_scaling", 1.0) or 1.0),
        **options)
    return cfg.validate()


def _interleave_rows(w, heads, hd):
    """HF's rotate-half order (per head: the first halves of the pairs, then the second halves) -> the
    interleaved pairs (x0, x1), (x2, x3), ... this datapath rotates (qhf.py:123-130)."""
    w = np.asarray(w, F)
    return np.ascontiguousarray(np.swapaxes(w.reshape(heads, 2, hd // 2, *w.shape[1:]), 1, 2).reshape(w.shape))


class CompressedScheme:
    """A compressed-tensors quantization_config (llm-compressor W8A8, as the reference's
    compiler/frontend/ct_import.py:1-27, 63-105 accepts it): int-quantized, compressed; weights int8
    static per output channel, symmetric; input activations int8 dynamic per token, symmetric (the
    datapath's own quant_act). Anything else raises. `quantized(module name)`: whether a Linear's weight
    is stored as int8 rows with scales."""
    WEIGHTS = {"type": "int", "num_bits": 8, "dynamic": False, "strategy": "channel", "symmetric": True}
    INPUTS = {"type": "int", "num_bits": 8, "dynamic": True, "strategy": "token", "symmetric": True}
    UNSET = ("group_size", "block_structure")

    def __init__(self, qc):
        bad = lambda what: ValueError(f"compressed-tensors: {what}")
        if qc.get("quant_method") != "compressed-tensors":
            raise bad(f"quant_method {qc.get('quant_method')!r} (supported: compressed-tensors)")
        if qc.get("format") != "int-quantized":
            raise bad(f"format {qc.get('format')!r} (supported: int-quantized)")
        if qc.get("quantization_status", "compressed") != "compressed":
            raise bad(f"quantization_status {qc.get('quantization_status')!r} (supported: compressed)")
        if qc.get("kv_cache_scheme"):
            raise bad("kv_cache_scheme set (the KV scales are calibrated here)")
        self.targets = []
        for name, g in (qc.get("config_groups") or {}).items():
            for kind, want in (("weights", self.WEIGHTS), ("input_activations", self.INPUTS)):
                a = g.get(kind)
                if a is None:
                    raise bad(f"group {name}: no {kind} scheme")
                for k, v in want.items():
                    if a.get(k) != v:
                        raise bad(f"group {name}: {kind}.{k} = {a.get(k)!r} (supported: {v!r})")
                for k in self.UNSET:
                    if a.get(k) not in (None, False, {}):
                        raise bad(f"group {name}: {kind}.{k} = {a.get(k)!r} (supported: unset)")
                if kind == "weights" and a.get("actorder") not in (None, False, "static"):
                    raise bad(f"group {name}: weights.actorder = {a.get('actorder')!r} (supported: none, static)")
            if g.get("output_activations"):
                raise bad(f"group {name}: output_activations set")
            self.targets += g.get("targets") or []
        if not self.targets:
            raise bad("no config_groups with targets")
        self.ignore = qc.get("ignore") or []

    @staticmethod
    def _match(name, pats):
        return any(re.fullmatch(p[3:], name) if p.startswith("re:") else p in (name, "Linear") for p in pats)

    def quantized(self, name):
        return self._match(name, self.targets) and not self._match(name, self.ignore)


def _stored_qs(t, name, shape):
    """(int8 rows [N, K], fp32 scales [N]) of a compressed-tensors linear layer, checked
    (ct_import.py:150-167): the int8 values as stored (-128 included)."""
    q, sc = t.get(name + ".weight"), t.get(name + ".weight_scale")
    if q is None or sc is None:
        raise ValueError(f"compressed-tensors: {name}: weight / weight_scale missing")
    if q.dtype != np.int8 or tuple(q.shape) != tuple(shape):
        raise ValueError(f"compressed-tensors: {name}.weight: {q.dtype} {tuple(q.shape)}, expected int8 {tuple(shape)}")
    if sc.size != shape[0] or (sc.ndim == 2 and sc.shape[1] != 1) or sc.ndim > 2:
        raise ValueError(f"compressed-tensors: {name}.weight_scale: shape {tuple(sc.shape)}, expected ({shape[0]}, 1)")
    zp = t.get(name + ".weight_zero_point")
    if zp is not None and np.any(np.asarray(zp) != 0):
        raise ValueError(f"compressed-tensors: {name}.weight_zero_point non-zero (supported: symmetric)")
    for k in ("weight_g_idx", "input_scale", "input_zero_point"):
        if name + "." + k in t:
            raise ValueError(f"compressed-tensors: {name}.{k} present (supported: no act-order, dynamic inputs)")
    return np.ascontiguousarray(q), np.ascontiguousarray(np.asarray(sc, F).reshape(shape[0]))


def hf_weights(path, cfg, stored=None):
    """{llama2.c name: float32 array} of an HF model directory (qhf.py:159-181): tok, wcls, rms_final,
    per layer (stacked) wq, wk, wv, wo, rms_att, rms_ffn, w1 / w3 / w2 (gate / up / down) or the MoE
    router, wg, wu, wd, and q_norm / k_norm (QK-norm), q / k in interleaved pair order. A compressed-tensors
    checkpoint's quantized linears come as q * s (the fp32 model of the KV calibration); their int8 rows
    and scales, reordered with them, go into `stored` (a dict): {name: (q [L, ...], s [L, ...])}."""
    import json
    t = {}
    for f in sorted(os.listdir(path)):
        if f.endswith(".safetensors"):
            t.update(read_safetensors(os.path.join(path, f)))
    if not t:
        raise ValueError(f"{path}: no .safetensors files")
    qc = json.load(open(os.path.join(path, "config.json"))).get("quantization_config")
    scheme = CompressedScheme(qc) if qc is not None else None
    L, hd, d = cfg.layers, cfg.head_dim, cfg.dim
    shapes = {"self_attn.q_proj": (cfg.q_dim, d), "self_attn.k_proj": (cfg.kv_dim, d),
              "self_attn.v_proj": (cfg.kv_dim, d), "self_attn.o_proj": (d, cfg.q_dim),
              "mlp.gate_proj": (cfg.hidden, d), "mlp.up_proj": (cfg.hidden, d), "mlp.down_proj": (d, cfg.hidden),
              "block_sparse_moe.gate": (cfg.n_experts, d), "w1": (cfg.hidden, d), "w3": (cfg.hidden, d),
              "w2": (d, cfg.hidden)}
    qs = {}

    def lin(full, kind):
        """fp32 weight of a Linear (dequantized when the checkpoint stores it as int8 rows)."""
        if scheme is not None and scheme.quantized(full):
            q, sc = _stored_qs(t, full, shapes[kind])
            qs[full] = (q, sc)
            return (q.astype(F) * sc[:, None]).astype(F)
        if full + ".weight" not in t:
            raise ValueError(f"{path}: tensor {full}.weight missing")
        v = np.asarray(t[full + ".weight"])
        if v.dtype == np.int8:
            raise ValueError(f"{full}.weight is int8 but the scheme does not quantize it")
        return np.asarray(v, F)
    g = lambda n: np.asarray(t[n], F)
    w = {"tok": g("model.embed_tokens.weight"), "rms_final": g("model.norm.weight")}
    shapes["lm_head"] = (cfg.vocab, d)
    w["wcls"] = w["tok"] if cfg.tied or "lm_head.weight" not in t else lin("lm_head", "lm_head")
    gains = {"rms_att": "input_layernorm", "rms_ffn": "post_attention_layernorm"}
    if cfg.qk_norm:
        gains.update({"q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm"})
    for k, n in gains.items():
        w[k] = np.stack([g(f"model.layers.{l}.{n}.weight") for l in range(L)])
    linears = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj", "wo": "self_attn.o_proj"}
    if not cfg.moe:
        linears.update({"w1": "mlp.gate_proj", "w3": "mlp.up_proj", "w2": "mlp.down_proj"})
    for k, n in linears.items():
        w[k] = np.stack([lin(f"model.layers.{l}.{n}", n) for l in range(L)])
    if cfg.moe:
        E = cfg.n_experts
        moe = lambda l, n: f"model.layers.{l}.block_sparse_moe.{n}"
        w["router"] = np.stack([lin(moe(l, "gate"), "block_sparse_moe.gate") for l in range(L)])
        for k, n in (("wg", "w1"), ("wu", "w3"), ("wd", "w2")):
            w[k] = np.stack([np.stack([lin(moe(l, f"experts.{e}.{n}"), n) for e in range(E)]) for l in range(L)])
    perm = lambda x, heads: _interleave_rows(x, heads, hd)
    w["wq"] = np.stack([perm(x, cfg.heads) for x in w["wq"]])
    w["wk"] = np.stack([perm(x, cfg.kv_heads) for x in w["wk"]])
    if cfg.qk_norm:
        w["q_norm"] = np.stack([_interleave_rows(x, 1, hd) for x in w["q_norm"]])
        w["k_norm"] = np.stack([_interleave_rows(x, 1, hd) for x in w["k_norm"]])
    if stored is not None and qs:
        # the stored int8 rows under this datapath's names (q / k rows and scales reordered like the weights)
        def rows(names, heads=None):
            q = np.stack([qs[n][0] for n in names])
            sc = np.stack([qs[n][1] for n in names])
            if heads is not None:
                q = np.stack([_interleave_rows(x, heads, hd).astype(np.int8) for x in q.astype(F)]).astype(np.int8)
                sc = np.stack([_interleave_rows(x[:, None], heads, hd)[:, 0] for x in sc])
            return q, sc
        for k, n in linears.items():
            names = [f"model.layers.{l}.{n}" for l in range(L)]
            if all(x in qs for x in names):
                heads = cfg.heads if k == "wq" else cfg.kv_heads if k == "wk" else None
                stored[k] = rows(names, heads)
        if cfg.moe:
            for k, n in (("wg", "w1"), ("wu", "w3"), ("wd", "w2")):
                names = [[f"model.layers.{l}.block_sparse_moe.experts.{e}.{n}" for e in range(cfg.n_experts)]
                         for l in range(L)]
                if all(x in qs for r in names for x in r):
                    stored[k] = (np.stack([np.stack([qs[x][0] for x in r]) for r in names]),
                                 np.stack([np.stack([qs[x][1] for x in r]) for r in names]))
            names = [f"model.layers.{l}.block_sparse_moe.gate" for l in range(L)]
            if all(x in qs for x in names):
                stored["router"] = rows(names)
        if "lm_head" in qs:
            stored["wcls"] = qs["lm_head"]
    return w


def read_hf(path, seq_len=2048, kv_scales=None, calib_tokens=None, name=None, **options):
    """QuantModel of an HF model directory: hf_config + hf_weights + quant_model_from_fp32 (KV scales
    calibrated on calib_tokens unless given). A compressed-tensors W8A8 checkpoint keeps its own int8
    rows and scales; the layers its scheme ignores are quantized here."""
    cfg = hf_config(path, seq_len=seq_len, name=name, **options)
    stored = {}
    w = hf_weights(path, cfg, stored)
    return quant_model_from_fp32(cfg, w, kv_scales=kv_scales, calib_tokens=calib_tokens, stored=stored)
