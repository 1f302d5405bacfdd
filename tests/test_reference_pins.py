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

- the HF path's numerics options as hf_generic computes them in the device's numerics: SaCache's per-layer
  and per-channel KV constants and the int8 rows its update() writes, sa_attention's outputs (qsum
  normalisation, K per channel folded into q, V per channel), SaGELUTanh through EXP overflow and the logits
  scaling fold, bit for bit; hf_tokenizer.BpeTokenizer's ids and text on two synthetic byte-level
  tokenizer.json files against modelfile.HFTokenizer.

Each QModel run also checks planted mistakes in the oracle (eps, theta, QK-norm after RoPE, the KV head of a
query head) against the same fixture: each must fail it; so do the attention mistakes of
numerics.PLANTS and an expanded GELU-tanh exponent against the HF-option fixtures."""
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


# ------------------------------------------------------------------ the HF path's numerics options
@pytest.fixture(scope="module")
def hfopt():
    z = np.load(os.path.join(GOLD, "hfopt_golden.npz"))
    return json.loads(bytes(z["meta"]).decode()), z


def _hf_case(z, rec):
    """The oracle's constants and cache rows for one sa_attention case, from the case's KV scales."""
    from types import SimpleNamespace
    from t2r_amd import weights as W
    k = rec["key"]
    kv = z[k + "_kv"]
    cfg = SimpleNamespace(layers=1, head_dim=rec["hd"], kv_dim=rec["Hk"] * rec["hd"])
    flags = W.kv_channel_flags(cfg, kv)
    kvc = W.kv_constants(cfg, kv)[0]                       # 1/s_k, 1/s_v, a_k, a_v per layer
    ch = W.kv_channel_constants(cfg, kv)[0]                # s_k, 1/s_k, 1/s_v, a_v per channel
    return int(flags[0]), kvc, ch


def test_hf_kv_constants_and_cache_equal_sacache(hfopt):
    """SaCache's constants (hf_generic.py:153-187) and the int8 rows its update() writes (:203-218) equal
    weights.kv_constants / kv_channel_constants and the oracle's append to_i8(F(k * inv_s))."""
    from oracle import numerics as N
    meta, z = hfopt
    u = lambda a: np.asarray(a, F).view(np.uint32)
    for rec in meta:
        k, fl, (kvc, ch) = rec["key"], *(lambda t: (t[0], t[1:]))(_hf_case(z, rec))
        G = rec["H"] // rec["Hk"]
        want_isk = ch[1] if fl & 1 else kvc[0:1]
        want_isv = ch[2] if fl & 2 else kvc[1:2]
        assert np.array_equal(u(z[k + "_inv_sk"]), u(want_isk)), rec["name"]
        assert np.array_equal(u(z[k + "_inv_sv"]), u(want_isv)), rec["name"]
        assert np.array_equal(u(z[k + "_a_k"]), u(kvc[2:3])), rec["name"]
        if fl & 1:
            want_sk = np.repeat(ch[0].reshape(rec["Hk"], 1, rec["hd"]), G, 1).reshape(-1)    # per query head
            assert np.array_equal(u(z[k + "_sk"]), u(want_sk)), rec["name"]
        want_av = np.repeat(ch[3].reshape(rec["Hk"], 1, rec["hd"]), G, 1).reshape(-1) if fl & 2 else kvc[3:4]
        assert np.array_equal(u(z[k + "_a_v"]), u(want_av)), rec["name"]
        kc = N.to_i8((z[k + "_kf"] * want_isk).astype(F))
        vc = N.to_i8((z[k + "_vf"] * want_isv).astype(F))
        assert np.array_equal(kc, z[k + "_kc"]) and np.array_equal(vc, z[k + "_vc"]), rec["name"]


def _hf_attention(z, rec, plant=None):
    """numerics.attention (qsum, the case's per-channel options) of every query row of a case: [rows, H hd]."""
    from oracle import numerics as N
    k = rec["key"]
    fl, kvc, ch = _hf_case(z, rec)
    out = []
    for m, p in enumerate(rec["positions"]):
        out.append(N.attention(z[k + "_q"][m], z[k + "_kc"][:p + 1], z[k + "_vc"][:p + 1], rec["H"], rec["Hk"],
                               kvc[2], kvc[3], 16, qsum=True, ch_sk=ch[0] if fl & 1 else None,
                               ch_av=ch[3] if fl & 2 else None, plant=plant))
    return np.asarray(out, F)


def test_hf_attention_equals_sa_attention(hfopt):
    """sa_attention (hf_generic.py:231-293) with the device SFU: every output bit, on GQA groups of 1-4, head
    dims 16-128, per-layer, K, V and K+V per-channel scales, positions at and past D-lane boundaries, and a
    case whose scores spread past EXP's underflow."""
    meta, z = hfopt
    for rec in meta:
        got = _hf_attention(z, rec)
        want = z[rec["key"] + "_out"]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rec["name"]


@pytest.mark.parametrize("plant", ["rq_av_first", "qsum_e", "fold_head0", "fold_after_quant"])
def test_hf_attention_planted_mistakes_fail(hfopt, plant):
    from oracle import numerics as N
    assert plant in N.PLANTS
    meta, z = hfopt
    caught = [rec["name"] for rec in meta
              if not np.array_equal(_hf_attention(z, rec, plant).view(np.uint32), z[rec["key"] + "_out"].view(np.uint32))]
    assert caught, f"{plant}: no sa_attention case tells it from the reference"


def test_gelu_tanh_equals_sagelutanh(hfopt):
    """SaGELUTanh (hf_generic.py:840-852) with the device SFU on 76k inputs (a dense sweep over [-14, 14]
    through EXP's overflow, random values, specials): every bit (NaN as NaN); its constants A and B; and an
    expanded exponent F(F(x A) + F(F(F(x x) x) B)) misses the fixture."""
    from oracle import numerics as N
    _, z = hfopt
    x, want = z["gelu_x"], z["gelu_y"]
    assert np.array_equal(z["gelu_AB"].view(np.uint32), np.array([N.GELU_A, N.GELU_B], F).view(np.uint32))
    got = N.gelu_tanh(x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    with np.errstate(over="ignore", invalid="ignore"):
        zexp = ((x * N.GELU_A).astype(F) + ((((x * x).astype(F) * x).astype(F)) * N.GELU_B).astype(F)).astype(F)
        bad = (x * N.sfu_recip((N.sfu_exp(zexp) + F(1)).astype(F))).astype(F)
    assert not np.array_equal(bad[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_logits_fold_equals_reference(hfopt):
    """head.s_w / float(ls) (hf_generic.py:909-917) equals weights.fold_logits_scaling bit for bit."""
    from t2r_amd import weights as W
    _, z = hfopt
    for ls, want in zip(z["fold_ls"], z["fold_out"]):
        got = W.fold_logits_scaling(z["fold_s_w"], float(ls))
        assert np.array_equal(np.asarray(got, F).view(np.uint32), want.view(np.uint32)), ls


def test_hf_tokenizer_equals_reference_port(tmp_path):
    """modelfile.HFTokenizer (the tokenizers library) equals the reference's own byte-level BPE port
    (compiler/frontend/hf_tokenizer.py:11-205) on a GPT-2-style and a Llama-3-style tokenizer.json: ids and
    decoded text of every sample (added tokens, NFC, digits, whitespace runs, multi-byte characters)."""
    from t2r_amd.modelfile import HFTokenizer
    gold = json.load(open(os.path.join(GOLD, "hf_tokenizer_golden.json")))
    for rec in gold["tokenizers"]:
        d = tmp_path / rec["style"]
        d.mkdir()
        (d / "tokenizer.json").write_text(rec["tokenizer_json"])
        tk = HFTokenizer(str(d))
        for case in rec["cases"]:
            assert tk.encode(case["text"], bos=False) == case["ids"], (rec["style"], case["text"])
            assert tk.decode(case["ids"]) == case["decoded"], (rec["style"], case["text"])
