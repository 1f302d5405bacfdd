"""The oracle's generalised datapath and the host runtime pieces against fixtures written by the reference
itself (tests/golden/make_golden_hf.py):

- the float64 RoPE tables of qhf.rope_tables (compiler/frontend/qhf.py:183-189), bit for bit;
- qhf.QModel (compiler/frontend/qhf.py:254-409: q_dim != dim, GQA, QK-norm before RoPE, theta and eps per
  model, prefill chunks) run in the device's numerics: every logit's bits, the greedy tokens and the int8 KV
  cache of OracleModel equal the reference's, on tiny models and on the C2 / C3 / C4 shapes;
- hf_generic.QMixtralMoe.route / _row (compiler/frontend/hf_generic.py:641-657) in the device's numerics:
  the selected ids, the route weights and the ordered combine's output, bit for bit;
- the .w8a8 bytes of llm/export_w8a8.export, llm/tokenizer.Tokenizer's ids and text, and
  llm/runtime.Sampler's draws.

Each QModel run also checks planted mistakes in the oracle (eps, theta, QK-norm after RoPE, the KV head of a
query head) against the same fixture: each must fail it."""
import hashlib
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
F = np.float32


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


@pytest.fixture(scope="module")
def qhf_gold():
    return json.load(open(os.path.join(GOLD, "qhf_golden.json")))


def test_rope_tables_f64_equal_reference(qhf_gold):
    import t2r_amd.config as C
    from t2r_amd import weights as W
    assert len(qhf_gold["rope"]) >= 4
    for r in qhf_gold["rope"]:
        cfg = C.get(r["config"])
        assert (cfg.theta, cfg.head_dim, cfg.seq_len) == (r["theta"], r["head_dim"], r["seq_len"])
        assert sha(*W.rope_tables(cfg)) == r["sha"], r["config"]


def run_cfg(rec):
    import t2r_amd.config as C
    base = C.get(rec["config"])
    cfg = base.with_(**rec["overrides"]) if rec["overrides"] else base
    return cfg.with_(D=rec["D"], rope_method="f64")


def replay(om, rec):
    """The fixture's calls through the oracle; returns the first mismatch (or None) and the KV sha."""
    om.reset()
    toks = rec["tokens"]
    i = 0
    for c in rec["calls"]:
        if c["kind"] == "decode":
            lg = om.forward(toks[i], c["pos"])
            i += 1
        else:
            lg = om.prefill(toks[i:i + c["rows"]], start=c["pos"])
            i += c["rows"]
        lg = np.asarray(lg, F)
        if sha(lg) != c["logits_sha"] or int(np.argmax(lg)) != c["argmax"]:
            return f"{c['kind']} at {c['pos']}: head {lg.view(np.uint32)[:4].tolist()} vs {c['head'][:4]}"
    n = len(toks)
    return None if sha(om.kc[:, :n], om.vc[:, :n]) == rec["kv_sha"] else "KV cache"


def model_of(rec, cfg=None):
    from t2r_amd import weights as W
    cfg = cfg or run_cfg(rec)
    kv = np.array(rec["kv_bits"], np.uint32).view(F).reshape(cfg.layers, 2)
    return W.QuantModel(cfg, kv_scales=kv)


QRUNS = list(range(7))


@pytest.mark.parametrize("idx", QRUNS)
def test_oracle_equals_qmodel_device_form(qhf_gold, idx):
    from oracle import OracleModel
    rec = qhf_gold["qmodel"][idx]
    assert rec["tables_equal_here"] and rec["kv_consts_equal_here"]
    om = OracleModel(model_of(rec))
    assert replay(om, rec) is None, f"{rec['config']} {rec['overrides'].get('name', '')} D={rec['D']}"


class _NormAfterRope:
    """OracleModel with QK-norm applied after RoPE (a planted mistake)."""

    @staticmethod
    def make(om):
        import types
        from oracle import numerics as N

        def qkv_rows(self, l, qkv, positions):
            c, qm = self.cfg, self.qm
            hd, M = c.head_dim, qkv.shape[0]
            q = qkv[:, :c.q_dim].reshape(M, c.heads, hd)
            k = qkv[:, c.q_dim:c.q_dim + c.kv_dim].reshape(M, c.kv_heads, hd)
            v = qkv[:, c.q_dim + c.kv_dim:]
            pos = np.asarray(positions)
            cs, sn = qm.cos[pos][:, None, :], qm.sin[pos][:, None, :]
            q, k = N.rope(q, cs, sn), N.rope(k, cs, sn)
            q = N.rmsnorm(q, qm.q_norm[l], c.eps, self.D).reshape(M, c.q_dim)
            k = N.rmsnorm(k, qm.k_norm[l], c.eps, self.D).reshape(M, c.kv_dim)
            self.kc[l, pos] = N.to_i8((k * qm.kvc[l, 0]).astype(F))
            self.vc[l, pos] = N.to_i8((v * qm.kvc[l, 1]).astype(F))
            return q
        om.qkv_rows = types.MethodType(qkv_rows, om)
        return om


class _WrongKvHead:
    """OracleModel whose query head h reads KV head h % Hk instead of h // G (a planted mistake): the heads
    are permuted into the slots of the wrong KV head around the real attention."""

    @staticmethod
    def make(om):
        import types
        c = om.cfg
        H, Hk, hd, G = c.heads, c.kv_heads, c.head_dim, c.group
        perm = np.array([(h % Hk) * G + h // Hk for h in range(H)])
        base = type(om).attention

        def attention(self, l, q, pos):
            qp = np.empty((H, hd), F)
            qp[perm] = q.reshape(H, hd)
            return base(self, l, qp.reshape(-1), pos).reshape(H, hd)[perm].reshape(-1)
        om.attention = types.MethodType(attention, om)
        return om


@pytest.mark.parametrize("mistake", ["eps", "theta", "norm_after_rope", "kv_head"])
def test_planted_mistakes_fail_qmodel_fixture(qhf_gold, mistake):
    """A plausible mistake in the generalised structure, planted in the oracle, fails the reference fixture
    (the fixtures are sensitive to what they pin)."""
    from oracle import OracleModel
    rec = qhf_gold["qmodel"][0]                      # tiny-qwen: QK-norm, q_dim != dim, theta 1e6, eps 1e-6
    cfg = run_cfg(rec)
    assert cfg.qk_norm and cfg.q_dim != cfg.dim and cfg.group == 2
    if mistake == "eps":
        qm = model_of(rec, cfg.with_(eps=1e-5))
    elif mistake == "theta":
        qm = model_of(rec, cfg.with_(theta=1e4))
    else:
        qm = model_of(rec)
    om = OracleModel(qm)
    if mistake == "norm_after_rope":
        om = _NormAfterRope.make(om)
    elif mistake == "kv_head":
        om = _WrongKvHead.make(om)
    assert replay(om, rec) is not None


def moe_gold():
    z = np.load(os.path.join(GOLD, "moe_golden.npz"))
    return json.loads(bytes(z["meta"]).decode()), z


@pytest.mark.parametrize("idx", range(3))
def test_moe_equals_qmixtralmoe_device_form(idx):
    """The route (ids in order, weights) and the ordered combine of k expert outputs equal the reference's
    QMixtralMoe in the device's numerics, bit for bit (top-8 of 32 at the C5 shape)."""
    import t2r_amd.config as C
    from oracle import numerics as N
    from oracle.model import _Lin, moe_row
    from t2r_amd import weights as W
    meta, z = moe_gold()
    m = meta[idx]
    cfg = C.get(m["config"])
    l = m["layer"]
    q = lambda n: W.quantize_rows(W.fp32_tensor(cfg, n, l))
    router = _Lin(*q("router"))
    tabs = [q(n) for n in ("wg", "wu", "wd")]
    experts = [tuple(_Lin(t[0][e], t[1][e]) for t in tabs) for e in range(cfg.n_experts)]
    x = z[m["key"] + "_x"]
    for r in range(m["rows"]):
        xq, s_x = N.quant_act(x[r])
        y, ids, w = moe_row(router, experts, xq, s_x, cfg.top_k, m["D"], cfg.act, cfg.dim)
        assert list(ids) == z[m["key"] + "_ids"][r].tolist(), f"row {r}"
        assert np.array_equal(np.asarray(w, F).view(np.uint32), z[m["key"] + "_w"][r].view(np.uint32)), f"row {r}"
        assert np.array_equal(np.asarray(y, F).view(np.uint32), z[m["key"] + "_y"][r].view(np.uint32)), f"row {r}"


def test_moe_fixture_detects_combine_order():
    """Adding the expert outputs in id order instead of the route's order misses the fixture: the test above
    pins the combine order, not only the set of experts."""
    import t2r_amd.config as C
    from oracle import numerics as N
    from oracle.model import _Lin
    from t2r_amd import weights as W
    meta, z = moe_gold()
    m = meta[2]
    cfg = C.get(m["config"])
    q = lambda n: W.quantize_rows(W.fp32_tensor(cfg, n, m["layer"]))
    tabs = [q(n) for n in ("wg", "wu", "wd")]
    x = z[m["key"] + "_x"]
    missed = 0
    for r in range(m["rows"]):
        ids = z[m["key"] + "_ids"][r]
        w = z[m["key"] + "_w"][r]
        xq, s_x = N.quant_act(x[r])
        y = np.zeros(cfg.dim, F)
        for j in np.argsort(ids):
            e = ids[j]
            g, u, d = (_Lin(t[0][e], t[1][e]) for t in tabs)
            hq, s_h = N.quant_act(N.gate_mul(g(xq, s_x), u(xq, s_x), cfg.act))
            y = (y + (w[j] * d(hq, s_h)).astype(F)).astype(F)
        missed += not np.array_equal(y.view(np.uint32), z[m["key"] + "_y"][r].view(np.uint32))
    assert missed > 0


def test_w8a8_bytes_equal_reference_export(tmp_path):
    """write_w8a8 of the tiny model at D = 8 reproduces llm/export_w8a8.export's file byte for byte, and
    read_w8a8 of the reference's file gives the model's int8 tables, scales and KV constants."""
    import t2r_amd.config as C
    from t2r_amd import modelfile as MF
    from t2r_amd import weights as W
    ref = os.path.join(GOLD, "w8a8_tiny.w8a8")
    cfg = C.TINY
    qm = W.QuantModel(cfg)
    out = tmp_path / "mine.w8a8"
    MF.write_w8a8(qm, str(out), d=8)
    a, b = np.fromfile(ref, np.uint8), np.fromfile(str(out), np.uint8)
    assert a.size == b.size and np.array_equal(a, b)
    back = MF.read_w8a8(ref)
    for n in ("emb_q", "emb_s", "wqkv", "s_wqkv", "wo", "s_wo", "w1", "s_w1", "w3", "s_w3", "w2", "s_w2", "kvc",
              "rms_att", "rms_ffn", "rms_final"):
        assert np.array_equal(np.asarray(getattr(back, n)), np.asarray(getattr(qm, n))), n


def test_tokenizer_equals_reference():
    """Llama2cTokenizer on a synthetic tokenizer.bin: ids (BOS / EOS, dummy prefix, byte fallback, merges by
    score with run.c's -1e10 floor and NaN scores never merging, a duplicated piece) and printed text equal
    llm/tokenizer.Tokenizer's."""
    from t2r_amd.modelfile import Llama2cTokenizer
    gold = json.load(open(os.path.join(GOLD, "tokenizer_golden.json")))
    tk = Llama2cTokenizer(os.path.join(GOLD, "tokenizer_golden.bin"), gold["vocab_size"])
    for c in gold["cases"]:
        assert tk.encode(c["text"], bos=True, eos=False) == c["ids"], c["text"]
        assert tk.encode(c["text"], bos=False, eos=True) == c["ids_eos"], c["text"]
        assert tk.decode(c["ids"]) == c["decoded"], c["text"]


def test_sampler_equals_reference():
    """Sampler (run.c's xorshift*, temperature, top-p) draws the reference's ids from the same logits, seeds,
    temperatures and top-p values, and ends in the same generator state."""
    from t2r_amd.runtime import Sampler
    gold = json.load(open(os.path.join(GOLD, "sampler_golden.json")))
    for r in gold["runs"]:
        lg = np.array(r["logits_bits"], np.uint32).view(F).reshape(-1, r["V"])
        s = Sampler(temperature=r["temperature"], topp=r["topp"], seed=r["seed"])
        assert [s(x) for x in lg] == r["draws"], (r["temperature"], r["topp"], r["seed"])
        assert str(s.state) == r["state"]
