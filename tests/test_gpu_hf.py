"""The HF path's numerics options on the HIP datapath (compiler/frontend/hf_generic.py): qsum
attention normalisation, per-channel K / V scales, the GELU-tanh gate and the logits scaling, against
the CPU restatement (bit-exact logits, greedy tokens and int8 KV cache), and each of the datapath's
kernels with the options against the others (decode, prefill, batched decode)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = np.float32


@pytest.fixture(scope="module")
def env():
    import torch

    from oracle import numerics as N
    from t2r_amd import abi, ops
    abi.load()
    dev = torch.device("cuda:0")
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    H = lambda t: t.cpu().numpy()
    return torch, N, ops, T, H


def quant_model(cfg, calib=64):
    """The model with KV scales calibrated on the first `calib` prompt tokens (per channel as cfg says);
    calib 0: the whole prompt (the tiny models' default calibration)."""
    from t2r_amd import weights as W
    kv = W.calibrate_kv(cfg, tokens=cfg.prompt()[:calib]) if calib else None
    return W.QuantModel(cfg, kv_scales=kv)


# ------------------------------------------------------------------ op level
def test_attention_options_equal_sa_attention(env):
    """t2r_attn_decode_opt and t2r_attn_prefill (qsum; K / V per channel as each case has them) on the cache
    rows the reference's SaCache wrote, against sa_attention's outputs in the device numerics
    (tests/golden/hfopt_golden.npz, compiler/frontend/hf_generic.py:231-293): every bit."""
    import json
    import os
    from types import SimpleNamespace
    from t2r_amd import weights as W
    torch, N, ops, T, H = env
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hfopt_golden.npz"))
    for rec in json.loads(bytes(z["meta"]).decode()):
        k, Hh, Hk, hd = rec["key"], rec["H"], rec["Hk"], rec["hd"]
        kv = z[k + "_kv"]
        cfg = SimpleNamespace(layers=1, head_dim=hd, kv_dim=Hk * hd)
        fl, kvc, ch = int(W.kv_channel_flags(cfg, kv)[0]), W.kv_constants(cfg, kv)[0], W.kv_channel_constants(cfg, kv)[0]
        args = dict(qsum=True, ch_sk=T(ch[0]) if fl & 1 else None, ch_av=T(ch[3]) if fl & 2 else None)
        kc, vc, q = T(z[k + "_kc"]), T(z[k + "_vc"]), T(z[k + "_q"])
        pos = T(np.asarray(rec["positions"], np.int32))
        want = z[k + "_out"].view(np.uint32)
        print(f"sa_attention case {rec['name']}", flush=True)
        got = H(ops.attention_opt(q, kc, vc, pos, Hh, Hk, kvc[2], kvc[3], 16, **args))
        assert np.array_equal(got.view(np.uint32), want), rec["name"]
        got = H(ops.attention_prefill(q, kc, vc, pos, Hh, Hk, kvc[2], kvc[3], 16, **args))
        assert np.array_equal(got.view(np.uint32), want), rec["name"] + " (prefill kernel)"


def test_gated_ffn_gelu(env):
    """t2r_gated_ffn_w8a8 with the GELU-tanh gate over h1 out to about +-100 (EXP overflow to +inf, RECIP
    of +inf, signed zeros past +-10.5) against numerics.gelu_mul, and act 0 against the SiLU gate."""
    torch, N, ops, T, H = env
    rng = np.random.default_rng(12)
    F_, K = 1024, 256
    w1 = rng.integers(-127, 128, (F_, K)).astype(np.int8)
    w3 = rng.integers(-127, 128, (F_, K)).astype(np.int8)
    s1 = np.exp(rng.uniform(np.log(1e-5), np.log(5e-2), F_)).astype(F)
    s3 = rng.uniform(1e-4, 1e-3, F_).astype(F)
    xq = rng.integers(-127, 128, K).astype(np.int8)
    s_x = np.array([0.01], F)
    h1 = N.linear(xq, s_x[0], w1, s1)
    h3 = N.linear(xq, s_x[0], w3, s3)
    assert (h1 < -11).sum() > 10 and (h1 > 11).sum() > 10         # both saturated ends are exercised
    for act in ("gelu_tanh", "silu"):
        u, hq, s_h = ops.gated_ffn(act, T(w1), T(s1), T(w3), T(s3), T(xq), T(s_x))
        uw = N.gate_mul(h1, h3, act)
        hw, sw = N.quant_act(uw)
        assert np.array_equal(H(u).view(np.uint32), uw.view(np.uint32)), act
        assert np.array_equal(H(hq), hw) and H(s_h)[0] == sw


def test_kv_append_per_channel(env):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(4)
    S, kv = 32, 96
    k = (rng.standard_normal((3, kv)) * 4).astype(F)
    v = rng.standard_normal((3, kv)).astype(F)
    isk = (F(1) / np.exp(rng.uniform(-6, -1, kv)).astype(F)).astype(F)
    isv = (F(1) / np.exp(rng.uniform(-6, -1, kv)).astype(F)).astype(F)
    pos = np.array([0, 7, 31], np.int32)
    for vk, vv in ((isk, isv), (isk, F(50.0)), (F(20.0), isv)):
        kc = torch.zeros((S, kv), dtype=torch.int8, device="cuda:0")
        vc = torch.zeros_like(kc)
        arg = lambda x: T(x) if isinstance(x, np.ndarray) else x
        ops.kv_append_ch(T(k), T(v), arg(vk), arg(vv), kc, vc, T(pos))
        assert np.array_equal(H(kc)[pos], N.to_i8((k * vk).astype(F)))
        assert np.array_equal(H(vc)[pos], N.to_i8((v * vv).astype(F)))
        assert not np.delete(H(kc), pos, axis=0).any()


@pytest.mark.parametrize("H_,Hk,hd,S,D", [(6, 6, 48, 256, 16), (4, 2, 8, 16, 8), (9, 3, 64, 2048, 16),
                                         (16, 8, 128, 2048, 16)])
@pytest.mark.parametrize("qsum,kch,vch", [(True, False, False), (False, True, False), (False, False, True),
                                          (True, True, True)])
def test_attention_options(env, H_, Hk, hd, S, D, qsum, kch, vch):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(H_ * hd + 7 * kch + 3 * vch)
    kc = rng.integers(-127, 128, (S, Hk * hd)).astype(np.int8)
    vc = rng.integers(-127, 128, (S, Hk * hd)).astype(np.int8)
    positions = sorted({0, D - 1, D, 255 % S, S - 1, S // 3})
    q = (rng.standard_normal((len(positions), H_ * hd)) * 2).astype(F)
    sk = np.exp(rng.uniform(-5, 0, Hk * hd)).astype(F) if kch else None      # a 150x spread of channel scales
    av = (np.exp(rng.uniform(-6, -2, Hk * hd)) / 127).astype(F) if vch else None
    a_k = F(1 / np.sqrt(hd)) if kch else F(0.02 / np.sqrt(hd))
    a_v = F(0.03 / 127)
    got = H(ops.attention_opt(T(q), T(kc), T(vc), T(np.array(positions, np.int32)), H_, Hk, a_k, a_v, D,
                              qsum=qsum, ch_sk=None if sk is None else T(sk), ch_av=None if av is None else T(av)))
    for i, p in enumerate(positions):
        want = N.attention(q[i], kc[:p + 1], vc[:p + 1], H_, Hk, a_k, a_v, D, qsum=qsum, ch_sk=sk, ch_av=av)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"pos {p}"


# ------------------------------------------------------------------ model level
@pytest.mark.parametrize("name", ["tiny-hf", "tiny-hf-kv", "tiny-hf-v", "tiny-hf-moe"])
def test_hf_decode_vs_oracle(name):
    import t2r_amd.config as C
    from oracle import OracleModel
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = quant_model(cfg, calib=0)
    rm = ResidentModel(qm)
    om = OracleModel(qm)
    seq = list(cfg.prompt())
    print(f"{name}: {cfg.prompt_len + cfg.decode_steps} positions", flush=True)
    for pos in range(cfg.prompt_len + cfg.decode_steps):
        want = om.forward(seq[pos], pos)
        got = rm.decode(seq[pos], pos).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{name} pos {pos}"
        assert int(rm.next.item()) == int(np.argmax(want))
        if pos + 1 >= len(seq):
            seq.append(int(np.argmax(want)))
    n = len(seq) - 1
    assert np.array_equal(rm.kc[:, :n].cpu().numpy(), om.kc[:, :n])
    assert np.array_equal(rm.vc[:, :n].cpu().numpy(), om.vc[:, :n])
    rm.close()


@pytest.mark.parametrize("name,steps", [("c2-smollm2-135m-hf", 6), ("c3-qwen3-0.6b-hf", 4), ("c5-granite-1b-a400m-hf", 3)])
def test_hf_full_shape_decode_vs_oracle(name, steps):
    """The full-size decode kernels with the options (head dims 64 and 128, groups of 3 and 2 query
    heads, QK-norm, and C5's 32-expert MoE with the GELU-tanh expert gate) against the CPU restatement
    on the first positions."""
    import t2r_amd.config as C
    from oracle import OracleModel
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = quant_model(cfg, calib=16 if cfg.moe else 64)    # (the fp32 MoE calibration runs row by row)
    rm = ResidentModel(qm, max_rows=16)
    om = OracleModel(qm)
    toks = cfg.prompt()[:steps]
    print(f"{name}: {steps} positions", flush=True)
    for pos, t in enumerate(toks):
        want = om.forward(t, pos)
        got = rm.decode(t, pos).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{name} pos {pos}"
    assert np.array_equal(rm.kc[:, :steps].cpu().numpy(), om.kc[:, :steps])
    assert np.array_equal(rm.vc[:, :steps].cpu().numpy(), om.vc[:, :steps])
    rm.close()


@pytest.mark.parametrize("name,P", [("tiny-hf", 20), ("tiny-hf-kv", 16), ("tiny-hf-v", 16), ("tiny-hf-moe", 20),
                                    ("c2-smollm2-135m-hf", 40), ("c3-qwen3-0.6b-hf", 300)])
def test_hf_prefill_equals_decode(name, P):
    """The prompt through t2r_prefill (all rows, and 8-row chunks) gives the decode-only logits and KV
    cache bit for bit (the prefill attention kernel with the options against the decode one)."""
    import t2r_amd.config as C
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = quant_model(cfg, calib=0 if cfg.name.startswith("tiny") else 64)
    rm = ResidentModel(qm, max_rows=max(P, 64))
    toks = (cfg.prompt() * 8)[:P]
    print(f"{name}: {P} rows", flush=True)
    for p, t in enumerate(toks):
        dec = rm.decode(t, p).cpu().numpy()
    kd = rm.kc[:, :P].cpu().numpy(), rm.vc[:, :P].cpu().numpy()
    rm.reset()
    pre = rm.prefill(toks).cpu().numpy()
    assert np.array_equal(pre.view(np.uint32), dec.view(np.uint32))
    assert np.array_equal(rm.kc[:, :P].cpu().numpy(), kd[0]) and np.array_equal(rm.vc[:, :P].cpu().numpy(), kd[1])
    rm.reset()
    ch = rm.prefill_chunks(toks, M=8).cpu().numpy()
    assert np.array_equal(ch.view(np.uint32), dec.view(np.uint32))
    rm.close()


@pytest.mark.parametrize("name,B", [("tiny-hf", 4), ("tiny-hf-kv", 3), ("tiny-hf-moe", 3), ("c2-smollm2-135m-hf", 4),
                                    ("c3-qwen3-0.6b-hf", 3)])
def test_hf_decode_batch_equals_single(name, B):
    import torch
    import t2r_amd.config as C
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = quant_model(cfg, calib=0 if cfg.name.startswith("tiny") else 64)
    rm = ResidentModel(qm, max_rows=B)
    rng = np.random.default_rng(6)
    steps = min(cfg.seq_len, 10)
    seqs = [rng.integers(0, cfg.vocab, steps + B).tolist() for _ in range(B)]
    kc, vc = rm.batch_caches(B)
    nxt = torch.zeros(B, dtype=torch.int32, device=rm.device)
    got = [[] for _ in range(B)]
    print(f"{name}: B = {B}", flush=True)
    for s in range(steps + B - 1):
        poses = [s - b if 0 <= s - b < steps else 0 for b in range(B)]
        live = [0 <= s - b < steps for b in range(B)]
        toks = [seqs[b][poses[b]] if live[b] else 1 for b in range(B)]
        lg = rm.decode_batch(toks, poses, kc, vc, next_tokens=nxt).cpu().numpy()
        nx = nxt.cpu().numpy()
        for b in range(B):
            if live[b]:
                got[b].append(lg[b].copy())
                assert nx[b] == int(np.argmax(lg[b]))
    for b in range(B):
        rm.reset()
        for p in range(steps):
            want = rm.decode(seqs[b][p], p).cpu().numpy()
            assert np.array_equal(got[b][p].view(np.uint32), want.view(np.uint32)), f"sequence {b} pos {p}"
    rm.close()


@pytest.mark.parametrize("name,lens", [("c3-qwen3-0.6b-hf", [35, 1100]), ("c2-smollm2-135m-hf", [1500, 64])])
def test_hf_long_context(name, lens):
    """Past one 1024-key pass of the decode kernels: each slot's cache holds a prefilled prompt; one
    batched step (grouped attention) equals the single decode (per-head attention) at that position,
    and the prefill's last logits equal the single decode's at its last row."""
    import torch
    import t2r_amd.config as C
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = quant_model(cfg)
    B = len(lens)
    rm = ResidentModel(qm, max_rows=max(lens))
    rng = np.random.default_rng(10)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in lens]
    nxt = [int(rng.integers(0, cfg.vocab)) for _ in lens]
    kc, vc = rm.batch_caches(B)
    print(f"{name}: positions {lens}", flush=True)
    for b, p in enumerate(prompts):
        rm.reset()
        rm.prefill(p, logits=False)
        kc[b].copy_(rm.kc)
        vc[b].copy_(rm.vc)
    got = rm.decode_batch(nxt, lens, kc, vc).cpu().numpy()
    for b, p in enumerate(prompts):
        rm.reset()
        last = rm.prefill(p).cpu().numpy()
        want = rm.decode(nxt[b], lens[b]).cpu().numpy()
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), f"sequence {b} at {lens[b]}"
        assert torch.equal(kc[b, :, lens[b]], rm.kc[:, lens[b]])
        rm.reset()                                 # the last prompt row decoded on the prefilled cache
        rm.prefill(p[:-1], logits=False)
        dec_last = rm.decode(p[-1], len(p) - 1).cpu().numpy()
        assert np.array_equal(last.view(np.uint32), dec_last.view(np.uint32)), f"prefill {b} last row"
    rm.close()


def test_logits_scaling_folded(env):
    """logits_scaling divides the logits through the classifier's row scales F(s / f32(ls)) (a tied
    classifier gets scales of its own): the device logits equal the oracle's, and the tied embedding's
    scales are untouched."""
    import t2r_amd.config as C
    from oracle import OracleModel
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    base = C.get("tiny-qwen")
    cfg = base.with_(name="tiny-qwen-ls", logits_scaling=3.0)
    qm0, qm = W.QuantModel(base), W.QuantModel(cfg)
    assert np.array_equal(qm.emb_s, qm0.emb_s) and qm.cls_q is qm.emb_q
    assert np.array_equal(qm.cls_s, (qm0.cls_s / F(3.0)).astype(F))
    rm = ResidentModel(qm)
    om = OracleModel(qm)
    for pos, t in enumerate(cfg.prompt()[:6]):
        want = om.forward(t, pos)
        got = rm.decode(t, pos).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"pos {pos}"
    rm.close()
