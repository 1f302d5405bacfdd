"""LlamaDevice on model files: a .w8a8 (version 1 and 2) with a tokenizer.bin next to it runs the
same numbers as the in-memory model, and generate() takes text and yields text pieces
(llm/runtime.py:75-146)."""
import os
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

LETTERS = [chr(c).encode() for c in range(ord("a"), ord("z") + 1)]


def tokenizer_bin(path, vocab):
    """A tokenizer.bin of exactly `vocab` pieces: <unk>, <s>, </s>, " ", a..z, " a".." z", then
    two-letter pieces (scores favour the " x" merges)."""
    pieces = [b"<unk>", b"\n<s>\n", b"\n</s>\n", b" "] + LETTERS + [b" " + c for c in LETTERS]
    scores = [0.0] * 4 + [-5.0] * 26 + [-1.0] * 26
    extra = [a + b for a in LETTERS for b in LETTERS]
    pieces += extra[:vocab - len(pieces)]
    scores += [-3.0] * (vocab - len(scores))
    assert len(pieces) == vocab
    with open(path, "wb") as f:
        f.write(struct.pack("<i", 8))
        for p, s in zip(pieces, scores):
            f.write(struct.pack("<fi", s, len(p)))
            f.write(p)


@pytest.mark.parametrize("name", ["tiny", "tiny-qwen"])
def test_llamadevice_from_w8a8(tmp_path, name):
    import t2r_amd.config as C
    from t2r_amd import modelfile as MF
    from t2r_amd import weights as W
    from t2r_amd.runtime import LlamaDevice
    cfg = C.get(name)
    qm = W.QuantModel(cfg)
    path = str(tmp_path / f"{name}.w8a8")
    MF.write_w8a8(qm, path)
    tokenizer_bin(str(tmp_path / "tokenizer.bin"), cfg.vocab)
    print(f"{name}: files written", flush=True)
    a = LlamaDevice(qm)
    b = LlamaDevice(path)                                  # tokenizer.bin found next to the model
    assert b.tok is not None and b.cfg.vocab == cfg.vocab
    toks = b.tok.encode("ab c")
    assert toks[0] == 1 and len(toks) >= 3
    for t in toks[:6]:
        la, lb = a.forward(t), b.forward(t)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    got = list(b.generate("ab c", steps=min(12, cfg.seq_len)))
    want = list(a.generate(toks, steps=min(12, cfg.seq_len)))
    assert [t for t, _ in got] == [t for t, _ in want]
    assert all(isinstance(s, str) for _, s in got)
    with pytest.raises(ValueError):
        next(a.generate("text without a tokenizer"))
    a.close()
    b.close()


def test_llamadevice_from_llama2c_checkpoint(tmp_path):
    """A llama2.c fp32 checkpoint is quantised on load (the KV scales calibrated over an fp32 run):
    its greedy tokens equal those of the same arrays through QuantModel.from_arrays."""
    import t2r_amd.config as C
    from t2r_amd import modelfile as MF
    from t2r_amd import weights as W
    from t2r_amd.runtime import LlamaDevice
    cfg = C.get("tiny")
    w = {"tok": W.fp32_tensor(cfg, "tok"), "rms_final": W.fp32_tensor(cfg, "rms_final")}
    for n in ("rms_att", "rms_ffn", "wq", "wk", "wv", "wo", "w1", "w2", "w3"):
        w[n] = np.stack([W.fp32_tensor(cfg, n, l) for l in range(cfg.layers)])
    path = str(tmp_path / "tiny.bin")
    MF.write_llama2c(path, cfg, w)
    dev = LlamaDevice(path)
    c2, w2 = MF.read_llama2c(path)
    qm = MF.quant_model_from_fp32(c2, w2)
    ref = LlamaDevice(qm)
    assert dev.tok is None
    prompt = [1, 5, 9, 17]
    assert [t for t, _ in dev.generate(prompt, steps=10)] == [t for t, _ in ref.generate(prompt, steps=10)]
    dev.close()
    ref.close()


@pytest.mark.parametrize("kind", ["qwen3", "mixtral"])
def test_hf_checkpoint_on_device(tmp_path, kind):
    """An HF checkpoint directory (transformers' own tiny random model, saved as safetensors) through
    LlamaDevice(path): the imported W8A8 model decodes on the device bit-identically to the oracle."""
    from oracle import OracleModel
    from t2r_amd.runtime import LlamaDevice
    from test_hf_import import _build
    model = _build(kind)
    model.save_pretrained(str(tmp_path))
    dev = LlamaDevice(str(tmp_path))
    assert dev.cfg.qk_norm == (kind == "qwen3") and dev.cfg.moe == (kind == "mixtral")
    om = OracleModel(dev.qm)
    for pos, t in enumerate([1, 17, 5, 88, 42, 3, 9, 60]):
        want = om.forward(t, pos)
        got = dev.forward(t)
        assert np.array_equal(np.asarray(got, np.float32).view(np.uint32), want.view(np.uint32)), f"pos {pos}"
    dev.close()


@pytest.mark.parametrize("kind", ["llama", "mixtral"])
def test_compressed_tensors_on_device(tmp_path, kind):
    """A compressed-tensors W8A8 checkpoint (int8 rows with -128 values, kept as stored) decodes and
    prefills on the device bit-identically to the oracle."""
    from oracle import OracleModel
    from t2r_amd.runtime import LlamaDevice
    from test_hf_import import _build, _compressed
    stored = _compressed(_build(kind), tmp_path)
    assert any((q == -128).any() for q, _ in stored.values())
    dev = LlamaDevice(str(tmp_path))
    assert (dev.qm.wqkv == -128).any() or (dev.qm.wo == -128).any()
    om = OracleModel(dev.qm)
    toks = [1, 17, 5, 88, 42, 3, 9, 60, 11, 4]
    for pos, t in enumerate(toks):
        want = om.forward(t, pos)
        got = dev.forward(t)
        assert np.array_equal(np.asarray(got, np.float32).view(np.uint32), want.view(np.uint32)), f"pos {pos}"
    dev.m.reset()
    pre = dev.m.prefill(toks).cpu().numpy()
    assert np.array_equal(pre.view(np.uint32), want.view(np.uint32))
    dev.close()


def test_reference_w8a8_file_equals_device_model_run():
    """The reference exporter's own file (tests/golden/w8a8_tiny.w8a8: llm/export_w8a8.export of the tiny
    model at D = 8) through LlamaDevice, the reference's consumer path (llm/runtime.py:76-99, the file read
    as llm/export_w8a8.py:133-167 lays it out), against the reference's DeviceModel(SfuExact) run of the
    same model in model_golden.json: every position's logits (sha256 of the bytes), the argmax, and the
    int8 KV cache."""
    import hashlib
    import json
    from t2r_amd.runtime import LlamaDevice
    gold = json.load(open(os.path.join(GOLD, "model_golden.json")))
    run = next(r for r in gold["device_model"] if r["config"] == "tiny" and r["D"] == 8)
    dev = LlamaDevice(os.path.join(GOLD, "w8a8_tiny.w8a8"), tokenizer_path=None)
    assert dev.cfg.D == 8 and dev.cfg.layers == 2
    assert np.array_equal(np.asarray(dev.qm.kv_scales, np.float32).reshape(-1).view(np.uint32),
                          np.array(run["kv_bits"], np.uint32))
    sha = lambda *a: hashlib.sha256(b"".join(np.ascontiguousarray(x).tobytes() for x in a)).hexdigest()
    print(f"reference w8a8 file: {run['steps']} positions", flush=True)
    for rec in run["positions"]:
        assert dev.pos == rec["pos"]
        lg = dev.forward(rec["token"])
        assert sha(lg) == rec["logits_sha"], f"pos {rec['pos']}: logits differ from the reference's run"
        assert int(np.argmax(lg)) == rec["argmax"]
    n = run["steps"]
    assert sha(dev.m.kc[:, :n].cpu().numpy(), dev.m.vc[:, :n].cpu().numpy()) == run["kv_sha"]
    dev.close()
