"""Op-level parity of the HIP kernels (through the C-ABI) with the CPU restatement and the
reference's golden vectors: bit-exact for every integer, int8 and fp32 output."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = np.float32
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


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


def bits_t(T, a):
    return T(np.asarray(a, np.uint32).view(np.int32))


def test_sfu_tables_on_device(env):
    from t2r_amd import abi
    rom = json.load(open(os.path.join(GOLD, "sfu_tables.json")))
    out = np.zeros(512, np.uint32)
    abi.check("t2r_sfu_tables", abi.load().t2r_sfu_tables(out.ctypes.data))
    want = np.concatenate([rom["exp"]["T"], rom["exp"]["S"], rom["recip"]["T"], rom["recip"]["S"],
                           rom["rsqrt"]["T"], rom["rsqrt"]["S"]]).astype(np.uint32)
    assert np.array_equal(out, want)


@pytest.mark.parametrize("name", ["exp", "recip", "rsqrt"])
def test_sfu_golden(env, name):
    torch, N, ops, T, H = env
    g = np.load(os.path.join(GOLD, "sfu_golden.npz"))
    x, y = g[name + "_x"], g[name + "_y"]
    got = H(ops.sfu(name, bits_t(T, x))).view(np.uint32)
    bad = np.flatnonzero(got != y)
    assert bad.size == 0, [(hex(x[i]), hex(got[i]), hex(y[i])) for i in bad[:6]]


@pytest.mark.parametrize("name", ["exp", "recip", "rsqrt"])
def test_sfu_sweep_vs_oracle(env, name):
    """2^21 inputs: random bit patterns over every exponent, the working ranges, and the flush-to-zero
    boundary (subnormal and near-2^-126 results)."""
    torch, N, ops, T, H = env
    rng = np.random.default_rng(11)
    n = 1 << 19
    parts = [rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32),
             N.bits(rng.uniform(-110, 95, n).astype(F)),
             N.bits(np.exp(rng.uniform(-90, 90, n)).astype(F)),
             (rng.integers(0, 2, n).astype(np.uint32) << 31) | rng.integers(0, 0x02000000, n).astype(np.uint32)]
    x = np.concatenate(parts)
    fn = {"exp": N.sfu_exp_bits, "recip": N.sfu_recip_bits, "rsqrt": N.sfu_rsqrt_bits}[name]
    want = fn(x)
    got = H(ops.sfu(name, bits_t(T, x))).view(np.uint32)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(x[i]), hex(got[i]), hex(want[i])) for i in bad[:6]]


@pytest.mark.parametrize("name", ["exp", "recip", "rsqrt", "exp_np", "recip_ge1", "exp_sm", "exp_g", "recip_g1"])
def test_sfu_exhaustive_vs_literal_sequence(env, name):
    """All 2^32 inputs: the datapath SFU (plain IEEE steps where the FTZ rule cannot change a result)
    equals the per-operation FTZ sequence of llm/sfu.py, which the sweep above pins to the oracle.
    'exp_np', the attention softmax's EXP, over its whole domain (x <= 0 and NaN: 2^31 + 2^23 inputs);
    'recip_ge1', the SwiGLU / GeGLU gates' RECIP, over its (x >= 1 and NaN); 'exp_sm', the prefill
    softmax's EXP under a finite row maximum, over its (x <= 0: 2^31 + 1 inputs); 'exp_g' and
    'recip_g1', the prefill gate epilogues' pair-table forms, over every non-NaN input and x >= 1."""
    torch, N, ops, T, H = env
    bad, first = ops.sfu_check(name)
    assert bad == 0, (name, bad, None if first is None else hex(first))


def test_fp32_primitives(env):
    torch, N, ops, T, H = env
    g = np.load(os.path.join(GOLD, "sfu_golden.npz"))
    rng = np.random.default_rng(5)
    n = 1 << 18
    a = np.concatenate([g["bin_a"], rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32),
                        (rng.integers(0, 2, n).astype(np.uint32) << 31) | rng.integers(0x00400000, 0x0A000000, n).astype(np.uint32)])
    b = np.concatenate([g["bin_b"], rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32),
                        (rng.integers(0, 2, n).astype(np.uint32) << 31) | rng.integers(0x1F000000, 0x3F800000, n).astype(np.uint32)])
    A, B = bits_t(T, a), bits_t(T, b)
    for op in ("add", "sub", "mul"):
        got = H(ops.fp32_op(op, A, B)).view(np.uint32)
        want = getattr(N, op)(a, b)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, (op, [(hex(a[i]), hex(b[i]), hex(got[i]), hex(want[i])) for i in bad[:5]])
    nn = rng.integers(-300, 301, a.size).astype(np.int32)
    got = H(ops.fp32_op("ldexp", A, T(nn))).view(np.uint32)
    assert np.array_equal(got, N.ldexp(a, nn))
    got = H(ops.fp32_op("floor", A, B)).astype(np.int64)
    assert np.array_equal(got, N.to_int(a, -2 ** 31, 2 ** 31 - 1, "floor"))
    got = H(ops.fp32_op("to_i8", A, B)).astype(np.int64)
    with np.errstate(invalid="ignore"):
        assert np.array_equal(got, N.to_i8(N.val(a)).astype(np.int64))
    ints = g["from_int_x"].astype(np.int32)
    got = H(ops.fp32_op("from_int", T(ints), T(ints))).view(np.uint32)
    assert np.array_equal(got, g["from_int"])


def test_ieee_vector_steps_keep_subnormals(env):
    """The vector steps are NumPy float32 arithmetic: IEEE with gradual underflow, no fusion."""
    torch, N, ops, T, H = env
    rng = np.random.default_rng(6)
    n = 1 << 18
    a = (rng.integers(0, 2, n).astype(np.uint32) << 31) | rng.integers(0, 0x20000000, n).astype(np.uint32)
    b = (rng.integers(0, 2, n).astype(np.uint32) << 31) | rng.integers(0x00000000, 0x40000000, n).astype(np.uint32)
    with np.errstate(all="ignore"):
        fa, fb = N.val(a), N.val(b)
        wm, wa = (fa * fb).view(np.uint32), (fa + fb).view(np.uint32)
    gm = H(ops.fp32_op("ieee_mul", bits_t(T, a), bits_t(T, b))).view(np.uint32)
    ga = H(ops.fp32_op("ieee_add", bits_t(T, a), bits_t(T, b))).view(np.uint32)
    nan = np.isnan(N.val(wm))
    assert np.array_equal(gm[~nan], wm[~nan]) and np.array_equal(ga, wa)
    assert ((wm & 0x7F800000) == 0).sum() > 1000                             # subnormal products were exercised


@pytest.mark.parametrize("N_,K,M", [(1, 16, 1), (37, 288, 1), (300, 2048, 1), (129, 8192, 1), (64, 1040, 3),
                                     (257, 3072, 5), (3072, 2048, 512), (40, 48, 77), (130, 288, 33),
                                     (2048, 8192, 130), (16, 16, 1000), (200, 576, 70), (1536, 1600, 260),
                                     (960, 576, 40), (576, 1536, 64), (96, 8192, 63), (3072, 2048, 48),
                                     (200, 1024, 100), (3500, 512, 300)])
def test_linear_exact(env, N_, K, M):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(N_ * 7 + K)
    w = rng.integers(-127, 128, (N_, K)).astype(np.int8)
    s_w = rng.uniform(1e-4, 1e-2, N_).astype(F)
    xq = rng.integers(-127, 128, (M, K)).astype(np.int8)
    xq[0, :16] = 127
    w[0, :16] = -127
    s_x = rng.uniform(1e-3, 1e-1, M).astype(F)
    res = rng.standard_normal((M, N_)).astype(F)
    acc_want = xq.astype(np.int64) @ w.astype(np.int64).T
    xin = T(xq) if M > 1 else T(xq[0])
    y, acc = ops.linear(T(w), T(s_w), xin, T(s_x), acc=True)
    assert np.array_equal(H(acc).reshape(M, N_).astype(np.int64), acc_want)
    assert np.array_equal(H(y).reshape(M, N_).view(np.uint32), N.dequant(acc_want, s_w, s_x).view(np.uint32))
    y2 = ops.linear(T(w), T(s_w), xin, T(s_x), residual=T(res if M > 1 else res[0]))
    want = (res + N.dequant(acc_want, s_w, s_x)).astype(F)
    assert np.array_equal(H(y2).reshape(M, N_).view(np.uint32), want.view(np.uint32))
    y3 = ops.linear(T(w), T(s_w), xin, T(s_x))           # no int32 copy: the GEMM's staged epilogue
    assert np.array_equal(H(y3).reshape(M, N_).view(np.uint32), N.dequant(acc_want, s_w, s_x).view(np.uint32))


@pytest.mark.parametrize("N_,K,M", [(64, 256, 1), (64, 256, 40), (512, 2048, 300)])
def test_linear_residual_signed_zeros(env, N_, K, M):
    """Residual rows of -0 with products of +0 and of -0 (zero weight rows, negative scales): IEEE gives
    -0 + +0 = +0 and -0 + -0 = -0, as NumPy's float32 does."""
    torch, N, ops, T, H = env
    rng = np.random.default_rng(N_ + M)
    w = rng.integers(-127, 128, (N_, K)).astype(np.int8)
    w[::3] = 0                                            # acc = 0: the product is +-0 by the scale's sign
    s_w = rng.uniform(1e-4, 1e-2, N_).astype(F)
    s_w[::2] *= -1
    xq = rng.integers(-127, 128, (M, K)).astype(np.int8)
    s_x = rng.uniform(1e-3, 1e-1, M).astype(F)
    res = rng.standard_normal((M, N_)).astype(F)
    res[:, ::3] = -0.0
    acc_want = xq.astype(np.int64) @ w.astype(np.int64).T
    want = (res + N.dequant(acc_want, s_w, s_x)).astype(F)
    assert (want.view(np.uint32) == 0x80000000).any() and ((want == 0) & (want.view(np.uint32) == 0)).any()
    xin = T(xq) if M > 1 else T(xq[0])
    got = ops.linear(T(w), T(s_w), xin, T(s_x), residual=T(res if M > 1 else res[0]))
    assert np.array_equal(H(got).reshape(M, N_).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n", [16, 288, 2048, 8192])
def test_quant_act(env, n):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((4, n)) * np.array([[1e-3], [1.0], [30.0], [0.0]])).astype(F)
    x[1, 3] = 2.5 * (np.abs(x[1]).max() / 127)                              # a tie in units of s_x
    xq, s = ops.quant_act(T(x))
    wq, ws = N.quant_act(x)
    assert np.array_equal(H(xq), wq) and np.array_equal(H(s).view(np.uint32), ws.view(np.uint32))
    assert not H(xq)[3].any() and H(s)[3] == 0


@pytest.mark.parametrize("n,D", [(1, 16), (7, 8), (15, 16), (16, 16), (17, 16), (48, 8), (128, 16), (288, 16),
                                 (2048, 16), (2048, 8), (1000, 16)])
def test_rmsnorm(env, n, D):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(n + D)
    x = (rng.standard_normal((3, n)) * np.array([[1e-3], [1.0], [40.0]])).astype(F)
    g = (1 + 0.1 * rng.standard_normal(n)).astype(F)
    for eps in (1e-5, 1e-6):
        got = H(ops.rmsnorm(T(x), T(g), eps, D))
        assert np.array_equal(got.view(np.uint32), N.rmsnorm(x, g, eps, D).view(np.uint32))


def test_rope_and_kv_append(env):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(3)
    S, hd, heads = 64, 48, 6
    ang = rng.uniform(-3, 3, (S, hd // 2))
    cos, sin = np.cos(ang).astype(F), np.sin(ang).astype(F)
    v = rng.standard_normal((5, heads * hd)).astype(F)
    pos = np.array([0, 3, 17, 63, 40], np.int32)
    got = H(ops.rope(T(v), T(cos), T(sin), T(pos)))
    want = N.rope(v.reshape(5, heads, hd), cos[pos][:, None], sin[pos][:, None]).reshape(5, -1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    kc = torch.zeros((S, heads * hd), dtype=torch.int8, device="cuda:0")
    vc = torch.zeros_like(kc)
    k, vv = rng.standard_normal((5, heads * hd)).astype(F) * 3, rng.standard_normal((5, heads * hd)).astype(F)
    ops.kv_append(T(k), T(vv), F(1 / 0.02), F(1 / 0.03), kc, vc, T(pos))
    kh, vh = H(kc), H(vc)
    assert np.array_equal(kh[pos], N.to_i8((k * F(1 / 0.02)).astype(F)))
    assert np.array_equal(vh[pos], N.to_i8((vv * F(1 / 0.03)).astype(F)))
    assert not np.delete(kh, pos, axis=0).any()


def _attn_ref(N, q, kc, vc, pos, H_, Hk, a_k, a_v, D):
    hd = q.shape[-1] // H_
    G = H_ // Hk
    T_ = pos + 1
    K = kc[:T_].reshape(T_, Hk, hd).astype(np.int64)
    V = vc[:T_].reshape(T_, Hk, hd).astype(np.int64)
    out = np.empty(H_ * hd, F)
    for h in range(H_):
        qq, s_q = N.quant_act(q[h * hd:(h + 1) * hd])
        sc = ((K[:, h // G] @ qq.astype(np.int64)).astype(F) * s_q).astype(F)
        sc = (sc * F(a_k)).astype(F)
        e = N.sfu_exp((sc - sc.max()).astype(F))
        r = N.sfu_recip(N.red_sum(e, D))
        pq = N.to_i8(((e * r).astype(F) * F(127)).astype(F)).astype(np.int64)
        out[h * hd:(h + 1) * hd] = ((pq @ V[:, h // G]).astype(F) * F(a_v)).astype(F)
    return out


@pytest.mark.parametrize("H_,Hk,hd,S,D", [(6, 6, 48, 256, 16), (4, 2, 8, 16, 8), (9, 3, 64, 2048, 16),
                                         (16, 8, 128, 2048, 16), (32, 8, 64, 2048, 16)])
def test_attention(env, H_, Hk, hd, S, D):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(H_ * hd)
    kc = rng.integers(-127, 128, (S, Hk * hd)).astype(np.int8)
    vc = rng.integers(-127, 128, (S, Hk * hd)).astype(np.int8)
    positions = sorted({0, D - 2, D - 1, D, 255 % S, S - 1, S // 3})
    q = (rng.standard_normal((len(positions), H_ * hd)) * 2).astype(F)
    a_k, a_v = F(0.02 / np.sqrt(hd)), F(0.03 / 127)
    got = H(ops.attention(T(q), T(kc), T(vc), T(np.array(positions, np.int32)), H_, Hk, a_k, a_v, D))
    for i, p in enumerate(positions):
        want = _attn_ref(N, q[i], kc, vc, p, H_, Hk, a_k, a_v, D)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"pos {p}"


def test_swiglu(env):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(8)
    F_, K = 768, 288
    w1 = rng.integers(-127, 128, (F_, K)).astype(np.int8)
    w3 = rng.integers(-127, 128, (F_, K)).astype(np.int8)
    s1, s3 = rng.uniform(1e-4, 1e-3, F_).astype(F), rng.uniform(1e-4, 1e-3, F_).astype(F)
    xq = rng.integers(-127, 128, K).astype(np.int8)
    s_x = np.array([0.01], F)
    u, hq, s_h = ops.swiglu(T(w1), T(s1), T(w3), T(s3), T(xq), T(s_x))
    h1 = N.linear(xq, s_x[0], w1, s1)
    h3 = N.linear(xq, s_x[0], w3, s3)
    uw = N.silu_mul(h1, h3)
    hw, sw = N.quant_act(uw)
    assert np.array_equal(H(u).view(np.uint32), uw.view(np.uint32))
    assert np.array_equal(H(hq), hw) and H(s_h)[0] == sw


def test_moe_route(env):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(4)
    sc = rng.standard_normal((6, 32)).astype(F)
    sc[1, [3, 9, 20]] = 2.5                                                  # ties: lower id first
    sc[2, :] = 1.0
    sc[3, 5] = np.nan                                                        # NaN after every number
    sc[4, 30] = -0.0
    sc[4, 2] = 0.0
    wide = rng.standard_normal((4, 64)).astype(F)                            # E = 64: every lane an expert
    wide[0, [1, 40, 63]] = np.nan
    wide[1, :] = np.nan                                                      # all NaN: ids in order
    wide[2, ::3] = 7.0
    wide[3, 60:] = np.inf
    for scores, k, D in ((sc, 8, 16), (sc, 2, 8), (sc, 1, 16), (wide, 8, 16), (wide, 5, 8), (sc[:, :8], 8, 16)):
        scores = np.ascontiguousarray(scores)
        ids, w = ops.moe_route(T(scores), k, D)
        ids, w = H(ids), H(w)
        for r in range(scores.shape[0]):
            want = N.topk_desc(scores[r], k)
            assert list(ids[r]) == list(want)
            v = scores[r][want]
            e = N.sfu_exp((v - v[0]).astype(F))
            ww = (e * N.sfu_recip(N.red_sum(e, D))).astype(F)
            assert np.array_equal(w[r].view(np.uint32), ww.view(np.uint32))


def test_argmax_first_index(env):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 151936)).astype(F)
    x[1, [10, 70000, 151935]] = 9.0
    x[2, :] = 0.0
    x[2, 5] = -0.0
    x[3, [100, 200]] = np.nan
    x[4, 0] = np.inf
    got = H(ops.argmax(T(x)))
    assert list(got) == [int(np.argmax(r)) for r in x]


def test_requant(env):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(1)
    r = rng.integers(-2 ** 31, 2 ** 31, 4096).astype(np.int32)
    r[:4] = [0, -1, 2 ** 31 - 1, -2 ** 31]
    for scale, shift, zp, lo, hi in ((1, 0, 0, -2 ** 31, 2 ** 31 - 1), (-32768, 31, 3, -100, 100),
                                     (123, 12, -5, -128, 127), (7, 1, 0, 0, 50)):
        got = H(ops.requant(T(r), scale, shift, zp, lo, hi))
        assert np.array_equal(got, N.requant_int(r, scale, shift, zp, lo, hi))


def test_embed(env):
    torch, N, ops, T, H = env
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, (100, 48)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-1, 100).astype(F)
    toks = np.array([0, 99, 42, 42], np.int32)
    got = H(ops.embed(T(q), T(s), T(toks)))
    assert np.array_equal(got.view(np.uint32), (q[toks].astype(F) * s[toks][:, None]).astype(F).view(np.uint32))


def test_shape_errors_raise(env):
    torch, N, ops, T, H = env
    with pytest.raises(ValueError):
        ops.linear(T(np.zeros((4, 24), np.int8)), T(np.ones(4, F)), T(np.zeros(24, np.int8)), T(np.ones(1, F)))
    with pytest.raises(ValueError):
        ops.moe_route(T(np.zeros((1, 70), F)), 4, 16)
