"""Attention at op level: t2r_attn_prefill (the prompt chunk's attention, SahlExpandKernels.cpp:1702,
qhf.py:356-409) row by row against the CPU restatement (numerics.attention) and against the decode op
on the same rows, bit for bit: consecutive prompt rows and scattered positions, head dims that take the
multi-row MFMA kernel and ones that do not, GQA groups, D = 8 and 16, the HF options; and scores whose
spread underflows EXP (x <= -104 gives +0) in the default instantiations of the prefill, decode and
grouped decode kernels."""
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


def caches(rng, S, kvd):
    return rng.integers(-127, 128, (S, kvd)).astype(np.int8), rng.integers(-127, 128, (S, kvd)).astype(np.int8)


@pytest.mark.parametrize("H_,Hk,hd,S,D", [(6, 6, 48, 256, 16), (9, 3, 64, 2048, 16), (16, 8, 128, 2048, 16),
                                         (32, 8, 64, 2048, 16), (4, 2, 32, 512, 8), (4, 2, 8, 16, 8),
                                         (6, 2, 24, 96, 16), (8, 2, 128, 2048, 8), (4, 4, 128, 1000, 16),
                                         (32, 8, 64, 512, 16), (8, 2, 64, 500, 8), (9, 3, 64, 96, 16)])
@pytest.mark.parametrize("layout", ["chunk", "scattered"])
def test_attn_prefill_vs_oracle(env, H_, Hk, hd, S, D, layout):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(H_ * hd + S)
    kc, vc = caches(rng, S, Hk * hd)
    if layout == "chunk":                         # a prompt chunk: consecutive rows ending at the cache's end
        M = min(37, S)
        pos = np.arange(S - M, S, dtype=np.int32)
    else:
        M = min(21, S)
        pos = np.sort(rng.choice(S, M, replace=False)).astype(np.int32)[::-1].copy()
    q = (rng.standard_normal((M, H_ * hd)) * 2).astype(F)
    a_k, a_v = F(0.02 / np.sqrt(hd)), F(0.03 / 127)
    print(f"H {H_} Hk {Hk} hd {hd} S {S} D {D} {layout}: {M} rows", flush=True)
    got = H(ops.attention_prefill(T(q), T(kc), T(vc), T(pos), H_, Hk, a_k, a_v, D))
    dec = H(ops.attention(T(q), T(kc), T(vc), T(pos), H_, Hk, a_k, a_v, D))
    for i, p in enumerate(pos):
        want = N.attention(q[i], kc[:p + 1], vc[:p + 1], H_, Hk, a_k, a_v, D)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"row {i} pos {p}"
    assert np.array_equal(got.view(np.uint32), dec.view(np.uint32))


@pytest.mark.parametrize("H_,Hk,hd,S", [(9, 3, 64, 512), (16, 8, 128, 512)])
@pytest.mark.parametrize("qsum,kch,vch", [(True, False, False), (False, True, True), (True, True, True)])
def test_attn_prefill_options_vs_oracle(env, H_, Hk, hd, S, qsum, kch, vch):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(7 * H_ + hd)
    kc, vc = caches(rng, S, Hk * hd)
    M = 40
    pos = np.arange(S - M - 3, S - 3, dtype=np.int32)
    q = (rng.standard_normal((M, H_ * hd)) * 2).astype(F)
    a_k, a_v = F(1.0 / np.sqrt(hd)), F(0.03 / 127)
    ch_sk = np.exp(rng.uniform(-4, 1, Hk * hd)).astype(F) * F(0.01) if kch else None
    ch_av = np.exp(rng.uniform(-3, 2, Hk * hd)).astype(F) * F(1e-3) if vch else None
    if not kch:
        a_k = F(0.02 / np.sqrt(hd))
    t = lambda a: None if a is None else T(a)
    got = H(ops.attention_prefill(T(q), T(kc), T(vc), T(pos), H_, Hk, a_k, a_v, 16, qsum, t(ch_sk), t(ch_av)))
    for i, p in enumerate(pos):
        want = N.attention(q[i], kc[:p + 1], vc[:p + 1], H_, Hk, a_k, a_v, 16, qsum=qsum, ch_sk=ch_sk, ch_av=ch_av)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"row {i} pos {p}"


@pytest.mark.parametrize("H_,Hk,hd,S", [(6, 6, 48, 256), (32, 8, 64, 1024), (16, 8, 128, 1024)])
def test_attention_exp_underflow(env, H_, Hk, hd, S):
    """Scores spread far beyond EXP's -104 cut: most keys' e is +0 (default numerics, not the OPT
    kernels); prefill op, decode op and a batched decode step (the grouped kernel) against the oracle."""
    torch, N, ops, T, H = env
    rng = np.random.default_rng(hd + S)
    kc, vc = caches(rng, S, Hk * hd)
    pos = np.array([S - 1, S // 2, 40, 3], np.int32)
    q = (rng.standard_normal((len(pos), H_ * hd)) * 2).astype(F)
    a_k, a_v = F(0.5 / np.sqrt(hd)), F(0.03 / 127)
    # the spread: quant_act(q) . K scaled, per head; at least one head of every row reaches x <= -104
    G = H_ // Hk
    for i, p in enumerate(pos):
        qq, s_q = N.quant_act(q[i].reshape(H_, hd))
        Kh = kc[:p + 1].reshape(p + 1, Hk, hd).astype(np.int64)
        sc = np.stack([((Kh[:, h // G] @ qq[h].astype(np.int64)).astype(F) * s_q[h]).astype(F) * a_k
                       for h in range(H_)])
        if p > 3:
            assert (sc - sc.max(axis=1, keepdims=True)).min() <= -104.0
    want = [N.attention(q[i], kc[:p + 1], vc[:p + 1], H_, Hk, a_k, a_v, 16) for i, p in enumerate(pos)]
    pre = H(ops.attention_prefill(T(q), T(kc), T(vc), T(pos), H_, Hk, a_k, a_v, 16))
    dec = H(ops.attention(T(q), T(kc), T(vc), T(pos), H_, Hk, a_k, a_v, 16))
    for i in range(len(pos)):
        assert np.array_equal(pre[i].view(np.uint32), want[i].view(np.uint32)), f"prefill row {i}"
        assert np.array_equal(dec[i].view(np.uint32), want[i].view(np.uint32)), f"decode row {i}"


@pytest.mark.parametrize("H_,Hk,hd,S", [(32, 8, 64, 512), (16, 8, 128, 512)])
def test_attention_special_scores(env, H_, Hk, hd, S):
    """Rows whose q holds NaN or +-inf (NaN scores: every EXP NaN, every probability 0) beside finite
    rows, through the prefill kernel (eight and sixteen waves: the row maximum folded into the score
    pass, the softmax form of EXP) and the decode op, against the oracle (np.max: NaN propagates)."""
    torch, N, ops, T, H = env
    rng = np.random.default_rng(11 * hd + H_)
    kc, vc = caches(rng, S, Hk * hd)
    M = 20
    pos = np.arange(S - M, S, dtype=np.int32)
    q = (rng.standard_normal((M, H_ * hd)) * 2).astype(F)
    q[2, 5] = np.nan                                  # head 0 of row 2
    q[7, hd + 1] = np.inf                             # head 1 of row 7
    q[11, :] = -np.inf                                # every head of row 11
    q[15, 3 * hd:4 * hd] = np.nan                     # a whole head of row 15
    a_k, a_v = F(0.5 / np.sqrt(hd)), F(0.03 / 127)
    with np.errstate(invalid="ignore", over="ignore"):
        want = [N.attention(q[i], kc[:p + 1], vc[:p + 1], H_, Hk, a_k, a_v, 16) for i, p in enumerate(pos)]
    pre = H(ops.attention_prefill(T(q), T(kc), T(vc), T(pos), H_, Hk, a_k, a_v, 16))
    dec = H(ops.attention(T(q), T(kc), T(vc), T(pos), H_, Hk, a_k, a_v, 16))
    for i in range(M):
        assert np.array_equal(pre[i].view(np.uint32), want[i].view(np.uint32)), f"prefill row {i}"
        assert np.array_equal(dec[i].view(np.uint32), want[i].view(np.uint32)), f"decode row {i}"


@pytest.mark.parametrize("name", ["c4-llama3.2-1b", "c2-smollm2-135m", "c3-qwen3-0.6b"])
def test_model_exp_underflow(name):
    """The fused decode attention (k_attn_dec), the grouped batched kernel (k_attn_gqa) and the prefill
    kernels inside the model, with KV scales 40x the calibrated ones (scores spread past EXP's cut):
    decode steps, a prefill and a batched step against the oracle."""
    import torch
    import t2r_amd.config as C
    from oracle import OracleModel
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = C.get(name).with_(layers=2)
    kv = np.asarray(W.calibrate_kv(cfg, tokens=cfg.prompt()[:16]), F).reshape(cfg.layers, 2)
    kv[:, 0] *= F(40.0)                                   # a_k 40x: q.K scores 40x wider
    qm = W.QuantModel(cfg, kv_scales=kv)
    om = OracleModel(qm)
    rm = ResidentModel(qm, max_rows=48)
    toks = np.random.default_rng(3).integers(0, cfg.vocab, 48).tolist()
    want = om.prefill(toks)
    got = rm.prefill(toks).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(rm.kc[:, :48].cpu().numpy(), om.kc[:, :48])
    for p in (48, 49):
        want = om.forward(toks[p - 40], p)
        got = rm.decode(toks[p - 40], p).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"decode at {p}"
    # a batched step: slot 0 the sequence above at 50, slot 1 a copy of its cache at 30
    kc, vc = rm.batch_caches(2)
    for b in range(2):
        kc[b].copy_(rm.kc)
        vc[b].copy_(rm.vc)
    snap = (om.kc.copy(), om.vc.copy())
    w0 = om.forward(7, 50)
    om.kc[:], om.vc[:] = snap
    w1 = om.forward(9, 30)
    got = rm.decode_batch([7, 9], [50, 30], kc, vc).cpu().numpy()
    assert np.array_equal(got[0].view(np.uint32), w0.view(np.uint32))
    assert np.array_equal(got[1].view(np.uint32), w1.view(np.uint32))
    assert torch.equal(kc[1, :, 30].cpu(), torch.from_numpy(om.kc[:, 30]))


@pytest.mark.parametrize("D", [16, 8])
def test_attn_prefill_c4_prompt(env, D):
    """C4's attention shape over its whole 512-row prompt at once (32 query heads, 8 KV heads, head dim
    64, a 512-position cache: the 32-row kernel's head-dim-64 form, 16 blocks of 32 rows): every row
    against the decode op, and rows at both ends of several blocks against the oracle."""
    torch, N, ops, T, H = env
    H_, Hk, hd, S, M = 32, 8, 64, 512, 512
    rng = np.random.default_rng(512 + D)
    kc, vc = caches(rng, S, Hk * hd)
    pos = np.arange(M, dtype=np.int32)
    q = (rng.standard_normal((M, H_ * hd)) * 2).astype(F)
    a_k, a_v = F(0.05 / np.sqrt(hd)), F(0.03 / 127)
    print(f"C4 prompt shape, D {D}: {M} rows", flush=True)
    Tq, Tk, Tv, Tp = T(q), T(kc), T(vc), T(pos)
    got = H(ops.attention_prefill(Tq, Tk, Tv, Tp, H_, Hk, a_k, a_v, D))
    dec = H(ops.attention(Tq, Tk, Tv, Tp, H_, Hk, a_k, a_v, D))
    bad = np.flatnonzero((got.view(np.uint32) != dec.view(np.uint32)).any(axis=1))
    assert bad.size == 0, f"rows {bad[:8]} differ from the decode op"
    for i in (0, 1, 31, 32, 255, 256, 479, 480, 511):
        want = N.attention(q[i], kc[:i + 1], vc[:i + 1], H_, Hk, a_k, a_v, D)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"row {i}"


@pytest.mark.parametrize("D", [16, 8])
def test_attn_prefill_c3_prompt(env, D):
    """C3's attention shape over its whole 2032-row prompt at once (16 query heads, 8 KV heads, head dim
    128, every row attending to all earlier positions: 64 blocks of 32 rows, the longest 2032 keys):
    every row against the decode op, and rows spread over the blocks (both ends of each of several
    blocks) against the oracle."""
    torch, N, ops, T, H = env
    H_, Hk, hd, S, M = 16, 8, 128, 2048, 2032
    rng = np.random.default_rng(2032 + D)
    kc, vc = caches(rng, S, Hk * hd)
    pos = np.arange(M, dtype=np.int32)
    q = (rng.standard_normal((M, H_ * hd)) * 2).astype(F)
    a_k, a_v = F(0.05 / np.sqrt(hd)), F(0.03 / 127)
    print(f"C3 prompt shape, D {D}: {M} rows", flush=True)
    Tq, Tk, Tv, Tp = T(q), T(kc), T(vc), T(pos)
    got = H(ops.attention_prefill(Tq, Tk, Tv, Tp, H_, Hk, a_k, a_v, D))
    dec = H(ops.attention(Tq, Tk, Tv, Tp, H_, Hk, a_k, a_v, D))
    bad = np.flatnonzero((got.view(np.uint32) != dec.view(np.uint32)).any(axis=1))
    assert bad.size == 0, f"rows {bad[:8]} differ from the decode op"
    for i in (0, 1, 31, 32, 63, 500, 1023, 1024, 1535, 2000, 2015, 2016, 2031):
        want = N.attention(q[i], kc[:i + 1], vc[:i + 1], H_, Hk, a_k, a_v, D)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"row {i}"
