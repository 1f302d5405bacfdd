"""Model files and tokenizers (t2r_amd.modelfile): the reference's .w8a8 layout
(llm/export_w8a8.py:15-30, 97-167), llama2.c checkpoints (llm/checkpoint.py:30-59), tokenizer.bin
BPE (llm/tokenizer.py:10-67) and HuggingFace tokenizer.json.

The layout checks read bytes at offsets derived from the documented format by hand (header field
order, entry order, 64-byte alignment, the B-tile transpose, the paired RoPE columns, the KV
parameter block); the tokenizer cases are known answers worked out from run.c's rules on a small
vocabulary. No reference file of either kind ships with the reference, so these are the pins."""
import os
import struct

import numpy as np
import pytest

import t2r_amd.config as C
from t2r_amd import modelfile as MF
from t2r_amd import weights as W

F = np.float32


def arrays(qm):
    names = W.QuantModel.COMMON + (W.QuantModel.MOE if qm.cfg.moe else W.QuantModel.DENSE)
    return {k: np.asarray(getattr(qm, k)) for k in names}


def same_model(a, b):
    A, B = arrays(a), arrays(b)
    assert A.keys() == B.keys()
    for k in A:
        assert A[k].shape == B[k].shape, k
        assert np.array_equal(A[k].view(np.uint8), B[k].view(np.uint8)), k


@pytest.mark.parametrize("name,version", [("tiny", 1), ("tiny-gqa", 1), ("tiny-qwen", 2), ("tiny-moe", 2),
                                          ("tiny-hf", 2), ("tiny-hf-kv", 2), ("tiny-hf-v", 2), ("tiny-hf-moe", 2),
                                          ("c1-stories15m", 1)])
def test_w8a8_round_trip(tmp_path, name, version):
    cfg = C.get(name)
    qm = W.QuantModel(cfg)
    path = str(tmp_path / "m.w8a8")
    n = MF.write_w8a8(qm, path)
    assert os.path.getsize(path) == n
    f = MF.W8A8File(path)
    assert f.version == version
    back = f.quant_model()
    assert back.cfg.tied == cfg.tied and back.cfg.D == cfg.D and back.cfg.head_dim == cfg.head_dim
    assert back.cfg.qk_norm == cfg.qk_norm and back.cfg.n_experts == cfg.n_experts and back.cfg.eps == cfg.eps
    same_model(qm, back)


def test_w8a8_v1_layout(tmp_path):
    """tiny (dim 32, hidden 64, 2 layers, 2 heads, vocab 64, seq 16, D 16) at hand-computed offsets."""
    cfg = C.get("tiny")
    qm = W.QuantModel(cfg)
    path = str(tmp_path / "tiny.w8a8")
    MF.write_w8a8(qm, path)
    raw = open(path, "rb").read()
    assert raw[:8] == b"W8A8LLM\0"
    version, D, dim, hidden, layers, heads, kv_heads, vocab, seq, n, base, stride = struct.unpack_from("<12I", raw, 8)
    assert (version, D, dim, hidden, layers, heads, kv_heads, vocab, seq) == (1, 16, 32, 64, 2, 2, 2, 64, 16)
    names = ["emb_q", "emb_s", "rms_final", "wcls", "s_wcls", "rope_cos", "rope_sin", "rms_att", "rms_ffn", "wqkv",
             "s_wqkv", "wo", "s_wo", "w13", "s_w13", "w2", "s_w2", "kvp"]
    assert n == len(names)
    ent = {}
    for i in range(n):
        nm, off, nb, per, res = struct.unpack_from("<16s4I", raw, 64 + 32 * i)
        assert nm.rstrip(b"\0").decode() == names[i] and res == 0
        assert off % 64 == 0
        ent[names[i]] = (off, nb, per)
    sizes = {"emb_q": 64 * 32, "emb_s": 64 * 4, "rms_final": 32 * 4, "wcls": 64 * 32, "s_wcls": 64 * 4,
             "rope_cos": 16 * 32 * 4, "rope_sin": 16 * 32 * 4, "rms_att": 32 * 4, "rms_ffn": 32 * 4,
             "wqkv": 96 * 32, "s_wqkv": 96 * 4, "wo": 32 * 32, "s_wo": 32 * 4, "w13": 128 * 32, "s_w13": 128 * 4,
             "w2": 32 * 64, "s_w2": 32 * 4, "kvp": 32}
    for k, v in sizes.items():
        assert ent[k][1] == v, k
        assert ent[k][2] == (1 if k in ("rms_att", "rms_ffn", "wqkv", "s_wqkv", "wo", "s_wo", "w13", "s_w13", "w2",
                                        "s_w2", "kvp") else 0)
    # global tensors packed in order from the first 64-byte boundary after the 18 entries
    pos = (64 + 32 * 18 + 63) // 64 * 64
    for k in names[:7]:
        assert ent[k][0] == pos
        pos = (pos + sizes[k] + 63) // 64 * 64
    assert base == pos
    rel = 0
    for k in names[7:]:
        assert ent[k][0] == rel
        rel = (rel + sizes[k] + 63) // 64 * 64
    assert stride == rel and len(raw) == base + 2 * stride

    def byte(off):
        return struct.unpack_from("<b", raw, off)[0]
    # B tiles: byte (t, k, j) of a linear = W[t D + j, k]
    for l in range(2):
        for (t, k, j) in ((0, 0, 0), (0, 5, 3), (1, 31, 15), (5, 17, 9)):
            assert byte(base + l * stride + ent["wqkv"][0] + (t * 32 + k) * 16 + j) == qm.wqkv[l][t * 16 + j, k]
        # w13: the W1 rows, then the W3 rows (output rows 64 .. 127 of the stacked matrix)
        assert byte(base + l * stride + ent["w13"][0] + (4 * 32 + 7) * 16 + 2) == qm.w3[l][2, 7]
        assert byte(base + l * stride + ent["w2"][0] + (1 * 64 + 50) * 16 + 4) == qm.w2[l][20, 50]
        kvp = np.frombuffer(raw, F, 8, base + l * stride + ent["kvp"][0])
        sk, sv = qm.kv_scales[l]
        want = [sk, sv, F(1.0 / float(sk)), F(1.0 / float(sv)), F(float(sk) / np.sqrt(16)), F(float(sv) / 127.0), 0, 0]
        assert np.array_equal(kvp.view(np.uint32), np.array(want, F).view(np.uint32))
    assert byte(ent["wcls"][0] + (3 * 32 + 11) * 16 + 6) == qm.emb_q[3 * 16 + 6, 11]
    # RoPE: column c of position p is cos / sin of p * 10000^(-2 ((c // 2) % 8) / 16), both pair elements
    cos = np.frombuffer(raw, F, 16 * 32, ent["rope_cos"][0]).reshape(16, 32)
    sin = np.frombuffer(raw, F, 16 * 32, ent["rope_sin"][0]).reshape(16, 32)
    for p in (0, 1, 7, 15):
        for c in (0, 1, 6, 7, 17, 30, 31):
            ang = p * 10000.0 ** (-2.0 * ((c // 2) % 8) / 16)
            assert abs(cos[p, c] - np.cos(ang)) < 4e-6 and abs(sin[p, c] - np.sin(ang)) < 4e-6


def test_w8a8_rejects(tmp_path):
    p = tmp_path / "bad.w8a8"
    p.write_bytes(b"W8A8LLM\0" + struct.pack("<12I", 3, *([0] * 11)) + bytes(8))
    with pytest.raises(ValueError):
        MF.W8A8File(str(p))
    p.write_bytes(b"NOTAFILE" + bytes(120))
    with pytest.raises(ValueError):
        MF.W8A8File(str(p))


def fp32_weights(cfg):
    L = cfg.layers
    w = {"tok": W.fp32_tensor(cfg, "tok"), "rms_final": W.fp32_tensor(cfg, "rms_final")}
    for n in ("rms_att", "rms_ffn", "wq", "wk", "wv", "wo", "w1", "w2", "w3"):
        w[n] = np.stack([W.fp32_tensor(cfg, n, l) for l in range(L)])
    w["wcls"] = w["tok"] if cfg.tied else W.fp32_tensor(cfg, "wcls")
    return w


@pytest.mark.parametrize("tied", [True, False])
def test_llama2c_checkpoint(tmp_path, tied):
    cfg = C.get("tiny").with_(tied=tied)
    w = fp32_weights(cfg)
    path = str(tmp_path / "tiny.bin")
    MF.write_llama2c(path, cfg, w)
    raw = open(path, "rb").read()
    hs = cfg.dim // cfg.heads
    # the header: 7 int32, vocab negative for a separate classifier
    assert struct.unpack_from("<7i", raw) == (32, 64, 2, 2, 2, 64 if tied else -64, 16)
    floats = 64 * 32 + 2 * 32 + 2 * (32 * 32 * 4) + 2 * 32 + 3 * 2 * 64 * 32 + 32 + 16 * hs + (0 if tied else 64 * 32)
    assert len(raw) == 4 * (7 + floats)
    # tensor order: tok, rms_att, wq, wk, wv, wo, rms_ffn, w1, w2, w3, rms_final, RoPE floats, [wcls]
    wq_off = 4 * (7 + 64 * 32 + 2 * 32)
    assert np.frombuffer(raw, F, 1, wq_off + 4 * (32 * 32 + 5 * 32 + 7))[0] == w["wq"][1][5, 7]
    c2, w2 = MF.read_llama2c(path)
    assert (c2.dim, c2.hidden, c2.layers, c2.heads, c2.kv_heads, c2.vocab, c2.seq_len, c2.tied) == \
        (32, 64, 2, 2, 2, 64, 16, tied)
    for k in w:
        assert np.array_equal(np.asarray(w2[k]), w[k]), k
    # quantised as the synthetic model is (same quantize_rows), with the same KV scales
    qm = W.QuantModel(cfg)
    back = MF.quant_model_from_fp32(c2.with_(D=cfg.D), w2, kv_scales=qm.kv_scales)
    same_model(qm, back)
    with open(path, "ab") as f:
        f.write(bytes(4))
    with pytest.raises(ValueError):
        MF.read_llama2c(path)


def test_llama2c_calibration_matches_synthetic():
    """KV scales calibrated over a checkpoint's arrays equal those over the same synthetic tensors."""
    cfg = C.get("tiny")
    w = fp32_weights(cfg)
    toks = cfg.prompt()

    def weight(c, name, layer=-1):
        return w[name] if layer < 0 or name == "tok" else w[name][layer]
    a = W.calibrate_kv(cfg, toks, weight=weight)
    b = W.calibrate_kv(cfg, toks)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------------------ tokenizer.bin
PIECES = [b"<unk>", b"\n<s>\n", b"\n</s>\n"] + [b"<0x%02X>" % i for i in range(256)] + \
    [b" ", b"a", b"b", b"c", b"ab", b" a", b" ab", b"bc", b"abc", b"\xc3\xa9", b"ca", b"aa"]
SCORES = [0.0] * 259 + [-1.0, -2.0, -2.0, -2.0, -3.0, -1.5, -0.5, -3.0, -5.0, -2.0, -3.0, -4.0]


def tok_file(tmp_path):
    path = tmp_path / "tokenizer.bin"
    with open(path, "wb") as f:
        f.write(struct.pack("<i", max(len(p) for p in PIECES)))
        for p, s in zip(PIECES, SCORES):
            f.write(struct.pack("<fi", s, len(p)))
            f.write(p)
    return str(path)


def tid(p):
    return PIECES.index(p)


def test_llama2c_tokenizer_known_answers(tmp_path):
    t = MF.Llama2cTokenizer(tok_file(tmp_path), len(PIECES))
    assert t.max_token_length == 6
    # [BOS, " ", a, b]: " a" (-1.5) beats "ab" (-3), then " a" + b = " ab" (-0.5)
    assert t.encode("ab") == [1, tid(b" ab")]
    # [BOS, " ", b, c]: "bc" (-3) is the only merge; " b" is not a piece
    assert t.encode("bc") == [1, tid(b" "), tid(b"bc")]
    # [BOS, " ", c, a, a]: "ca" (-3) and "aa" (-4): "ca" first, then nothing (" ca", "caa" absent)
    assert t.encode("caa") == [1, tid(b" "), tid(b"ca"), tid(b"a")]
    # equal scores, the leftmost pair first: [" ", a, a, a, a] -> [" a", a, a, a] -> [" a", "aa", a]
    assert t.encode("aaaa", bos=False) == [tid(b" a"), tid(b"aa"), tid(b"a")]
    # code points: e-acute is one piece; z (absent) falls back to its byte + 3; a 4-byte code point too
    assert t.encode("éz", bos=False) == [tid(b" "), tid(b"\xc3\xa9"), ord("z") + 3]
    assert t.encode("\U0001F600", bos=False, eos=True) == [tid(b" "), 0xF0 + 3, 0x9F + 3, 0x98 + 3, 0x80 + 3, 2]
    assert t.encode("") == [1]
    # decode: the space after BOS dropped, byte pieces as bytes, unprintable single bytes dropped
    assert t.decode([1, tid(b" ab"), tid(b"c")]) == "abc"
    assert t.decode([5, tid(b" ab")]) == " ab"
    assert t.decode([1, 0x41 + 3, 0x07 + 3, 0x0A + 3]) == "A\n"
    assert t.decode([1, tid(b" "), tid(b"\xc3\xa9")]) == "é"


def _merge_by_rescan(t, tok):
    """run.c's merge loop as written there: rescan every adjacent pair at each step, keep the first
    one with the highest score above -1e10, join it."""
    while True:
        best, at, mid = -1e10, -1, -1
        for k in range(len(tok) - 1):
            m = t.ids.get(t.pieces[tok[k]] + t.pieces[tok[k + 1]])
            if m is not None and t.scores[m] > best:
                best, at, mid = t.scores[m], k, m
        if at < 0:
            return tok
        tok = tok[:at] + [mid] + tok[at + 2:]


def test_llama2c_tokenizer_heap_merge_equals_rescan(tmp_path):
    """The heap-ordered merge picks the same pair as a full rescan at every step: random vocabularies
    with many equal scores, NaN and sub-floor scores and chains of merges, random texts."""
    rng = np.random.default_rng(11)
    alpha = ["a", "b", "c", " ", "é"]
    for trial in range(40):
        extra = sorted({"".join(rng.choice(alpha, int(rng.integers(2, 5)))).encode() for _ in range(50)})
        pieces = PIECES[:259] + [b" ", b"a", b"b", b"c", b"\xc3\xa9"] + extra
        scores = [float(np.float32(s)) for s in rng.integers(-3, 3, len(pieces))]
        for q in rng.integers(264, len(pieces), 4):
            scores[q] = float("nan") if q % 2 else -3e10
        path = tmp_path / f"t{trial}.bin"
        with open(path, "wb") as f:
            f.write(struct.pack("<i", 8))
            for p, s in zip(pieces, scores):
                f.write(struct.pack("<fi", s, len(p)) + p)
        t = MF.Llama2cTokenizer(str(path), len(pieces))
        for _ in range(10):
            text = "".join(rng.choice(alpha, int(rng.integers(0, 40))))
            start = [1] + ([t.ids[b" "]] + t._code_points(text.encode()) if text else [])
            assert t.encode(text) == _merge_by_rescan(t, start), (trial, text)


def test_hf_tokenizer(tmp_path):
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, processors
    vocab = {"<s>": 0}
    for i, ch in enumerate(pre_tokenizers.ByteLevel.alphabet()):
        vocab[ch] = i + 1
    merges = [("h", "e"), ("l", "l"), ("he", "ll"), ("hell", "o")]
    for a, b in merges:
        vocab[a + b] = len(vocab)
    tk = Tokenizer(models.BPE(vocab, merges))
    tk.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tk.decoder = decoders.ByteLevel()
    tk.add_special_tokens(["<s>"])
    tk.post_processor = processors.TemplateProcessing(single="<s> $A", special_tokens=[("<s>", 0)])
    path = str(tmp_path / "tokenizer.json")
    tk.save(path)
    t = MF.open_tokenizer(path, len(vocab))
    ids = t.encode("hello hello")
    assert ids[0] == vocab["hello"] and 0 not in ids              # no post-processor BOS
    assert t.decode(ids) == "hello hello"
    t2 = MF.open_tokenizer(str(tmp_path), len(vocab), bos_id=0)  # a directory; BOS on request
    assert t2.encode("hello") == [0, vocab["hello"]]
    assert t2.decode([0, vocab["hello"]]) == "<s>hello"


@pytest.mark.parametrize("name", ["tiny-hf", "tiny-hf-kv", "tiny-hf-moe"])
def test_w8a8_hf_options_round_trip(tmp_path, name):
    """The HF options survive a version-2 file: the config fields, the per-channel KV scales (`kvch`) and
    their constants, and a tied classifier's own folded scales beside the shared int8 rows."""
    cfg = C.get(name)
    qm = W.QuantModel(cfg)
    p = str(tmp_path / "m.w8a8")
    MF.write_w8a8(qm, p)
    back = MF.read_w8a8(p)
    for f in ("attn_norm", "act", "kv_channel", "logits_scaling"):
        assert getattr(back.cfg, f) == getattr(cfg, f), f
    assert back.kv_scales.shape == (cfg.layers, 2, cfg.kv_dim)
    assert np.array_equal(back.kvch, qm.kvch) and np.array_equal(back.kv_flags, qm.kv_flags)
    assert np.array_equal(back.kvc.view(np.uint32), qm.kvc.view(np.uint32))
    assert np.array_equal(back.cls_s.view(np.uint32), qm.cls_s.view(np.uint32))
    if cfg.tied:
        assert back.cls_q is back.emb_q
        assert (cfg.logits_scaling == 1.0) == (back.cls_s is back.emb_s)


def test_reference_w8a8_file_through_oracle_equals_device_model_run():
    """The reference exporter's file (tests/golden/w8a8_tiny.w8a8) read by W8A8File / read_w8a8 and run by the
    oracle reproduces the reference's DeviceModel(SfuExact) run of the same model (model_golden.json, tiny at
    D = 8): every position's logits bytes and the KV cache. The GPU test runs the same file through LlamaDevice."""
    import hashlib
    import json
    from oracle import OracleModel
    gold_dir = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    gold = json.load(open(os.path.join(gold_dir, "model_golden.json")))
    run = next(r for r in gold["device_model"] if r["config"] == "tiny" and r["D"] == 8)
    qm = MF.read_w8a8(os.path.join(gold_dir, "w8a8_tiny.w8a8"))
    assert qm.cfg.D == 8
    sha = lambda *a: hashlib.sha256(b"".join(np.ascontiguousarray(x).tobytes() for x in a)).hexdigest()
    om = OracleModel(qm)
    for rec in run["positions"]:
        assert sha(om.forward(rec["token"], rec["pos"])) == rec["logits_sha"], rec["pos"]
    n = run["steps"]
    assert sha(om.kc[:, :n], om.vc[:, :n]) == run["kv_sha"]
