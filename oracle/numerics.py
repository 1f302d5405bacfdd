"""CPU restatement of the W8A8 decoder's numerics: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import
this package, and only as the checker (or as the timed CPU baseline). The
product path (the HIP extension) never calls it.

What it restates (reference file:line for each function below):

- binary32 arithmetic of the device's fp32 units with flush-to-zero
  (llm/fp32.py:1-19, 78-209): RNE; a subnormal input counts as a signed zero; a
  result whose exponent, after rounding to 24 bits with an unbounded exponent
  range, is below the normal range becomes a signed zero; overflow gives +-inf;
  every NaN is 0x7FC00000. The method here is float64: a sum or product of two
  binary32 values is computed exactly (product) or with one innocuous rounding
  (sum: 53 >= 2*24 + 2 bits) in float64, then rounded to 24 significant bits
  with np.rint on the float64 significand. The reference uses integer
  significands; the two are independent ways to the same function.
- the SFU (llm/sfu.py:42-118): EXP / RECIP / RSQRT as table lookup, linear
  interpolation and one Newton step, built from those operations.
- the vector-engine primitives of DeviceModel (llm/ref_model.py:136-214): to_i8,
  the D-lane ordered sum, quant_act, the W8A8 linear layer, RMSNorm, RoPE.
  DeviceModel runs these in NumPy float32 (IEEE, gradual underflow); so does
  this restatement, with the bit-exact SFU for exp / recip / rsqrt
  (DeviceModel(sfu=SfuExact), llm/ref_model.py:115-133).

Parity pins (tests/test_oracle.py): IEEE float32 where IEEE and FTZ agree, the
literal KATs of llm/test_fp32.py:79-105, the SFU tables of
rtl/sysarray/sa_sfu_tables.vh, golden SFU outputs and golden DeviceModel runs
written by tests/golden/make_golden.py from the reference itself.
"""
import numpy as np

F = np.float32
U32 = np.uint32
QNAN = 0x7FC00000
PINF = 0x7F800000
NINF = 0xFF800000
_TWO24 = float(2 ** 24)
_MIN_NORMAL = 2.0 ** -126
_OVERFLOW = 2.0 ** 128


def bits(x):
    """float32 values -> uint32 bit patterns."""
    return np.asarray(x, F).view(U32)


def val(b):
    """uint32 bit patterns -> float32 values."""
    return np.asarray(b, U32).view(F)


def ftz(b):
    """Subnormal -> zero of the same sign (llm/fp32.py:206-209)."""
    b = np.asarray(b, U32)
    return np.where((b & U32(0x7F800000)) == 0, b & U32(0x80000000), b).astype(U32)


def _f64(b):
    return val(ftz(b)).astype(np.float64)


def _to_bits(r64):
    """A float64 result -> binary32 bits: round to 24 bits (unbounded exponent), FTZ, overflow, QNAN."""
    r64 = np.asarray(r64, np.float64)
    nan = np.isnan(r64)
    fin = np.isfinite(r64)
    m, e = np.frexp(np.where(fin, r64, 0.0))
    r = np.ldexp(np.rint(m * _TWO24) / _TWO24, e)               # 24 significant bits, RNE
    neg = np.signbit(r64).astype(np.uint64).astype(U32) << U32(31)
    with np.errstate(over="ignore"):
        out = bits(np.where(np.abs(r) < _OVERFLOW, r, 0.0).astype(F))
    out = np.where(np.abs(r) < _MIN_NORMAL, neg, out)            # below normal after rounding: signed zero
    out = np.where(~fin | (np.abs(r) >= _OVERFLOW), neg | U32(PINF), out)
    return np.where(nan, U32(QNAN), out).astype(U32)


def add(a, b):
    """a + b, binary32 bits (llm/fp32.py:78-118)."""
    with np.errstate(invalid="ignore"):
        return _to_bits(_f64(a) + _f64(b))


def sub(a, b):
    """a - b (llm/fp32.py:125)."""
    return add(a, np.asarray(b, U32) ^ U32(0x80000000))


def mul(a, b):
    """a * b (llm/fp32.py:129-144); the float64 product of two 24-bit significands is exact."""
    with np.errstate(invalid="ignore"):
        return _to_bits(_f64(a) * _f64(b))


def ldexp(a, n):
    """a * 2^n as an exponent-field add (llm/fp32.py:147-151): FTZ below, +-inf above the normal
    range; zero and inf pass through, NaN -> QNAN."""
    a = ftz(a).astype(np.int64)
    n = np.asarray(n, np.int64)
    s, e, m = a >> 31, (a >> 23) & 0xFF, a & 0x7FFFFF
    e2 = e + n
    out = np.where(e2 < 1, s << 31, np.where(e2 > 254, (s << 31) | PINF, (s << 31) | (np.clip(e2, 0, 255) << 23) | m))
    out = np.where((e == 0) | ((e == 255) & (m == 0)), a, out)
    out = np.where((e == 255) & (m != 0), QNAN, out)
    return out.astype(U32)


def from_int(i):
    """int32 -> binary32, RNE (llm/fp32.py:154-166): exact in float64, one rounding to float32."""
    return bits(np.asarray(i, np.int64).astype(np.float64).astype(F))


def to_int(a, lo, hi, mode="rne"):
    """binary32 -> integer, RNE or floor, saturated to [lo, hi]; NaN -> 0 (llm/fp32.py:169-189)."""
    v = _f64(a)
    with np.errstate(invalid="ignore"):
        r = np.rint(v) if mode == "rne" else np.floor(v)
        r = np.clip(np.nan_to_num(r, nan=0.0, posinf=hi, neginf=lo), lo, hi)
    return r.astype(np.int64)


# ------------------------------------------------------------------ SFU
def sfu_tables():
    """{"exp" | "recip" | "rsqrt": (T, S)} uint32: segment start values and slopes, computed in
    float64 and rounded to float32 (llm/sfu.py:42-56)."""
    k = np.arange(64, dtype=np.float64)
    te = np.exp2(k / 64)
    se = np.exp2((k + 1) / 64) - te
    tr = 1.0 / (1.0 + k / 64)
    sr = 1.0 / (1.0 + (k + 1) / 64) - tr
    m2 = np.concatenate([1.0 + k / 64, 2.0 * (1.0 + k / 64)])
    step = np.concatenate([np.full(64, 1 / 64), np.full(64, 2 / 64)])
    tq = 1.0 / np.sqrt(m2)
    sq = 1.0 / np.sqrt(m2 + step) - tq
    return {n: (bits(t.astype(F)), bits(s.astype(F))) for n, t, s in
            (("exp", te, se), ("recip", tr, sr), ("rsqrt", tq, sq))}


_TAB = sfu_tables()
_LOG2E = bits(F(1.4426950408889634))
_C64, _C2, _C1_5, _C0_5 = bits(F(64.0)), bits(F(2.0)), bits(F(1.5)), bits(F(0.5))


def _fields(x):
    x = np.asarray(x, U32).astype(np.int64)
    return x >> 31, (x >> 23) & 0xFF, x & 0x7FFFFF


def _frac17(frac):
    """(frac & 0x1FFFF) / 2^17 as binary32 (exact)."""
    return ldexp(from_int(frac & 0x1FFFF), -17)


def sfu_exp_bits(x):
    """EXP (llm/sfu.py:7-11, 69-82): t = x log2e, n = floor(t), f = t - n, u = 64 f, i = floor(u),
    r = u - i, y = T[i] + r S[i], y 2^n; x >= 89 -> +inf, x <= -104 -> +0, NaN -> QNAN."""
    x = ftz(x)
    T, S = _TAB["exp"]
    t = mul(x, _LOG2E)
    n = to_int(t, -2 ** 31, 2 ** 31 - 1, "floor")
    f = sub(t, from_int(n))
    u = mul(f, _C64)
    i = np.clip(to_int(u, 0, 63, "floor"), 0, 63)
    r = sub(u, from_int(i))
    y = add(T[i], mul(r, S[i]))
    res = ldexp(y, np.clip(n, -300, 300))
    xf = val(x).astype(np.float64)
    res = np.where(xf >= 89, U32(PINF), np.where(xf <= -104, U32(0), res))
    return np.where(np.isnan(xf), U32(QNAN), res).astype(U32)


def sfu_recip_bits(x):
    """RECIP (llm/sfu.py:12-15, 85-96): 6-bit table index, 17-bit interpolation, one Newton step
    y1 = y0 (2 - m y0), exponent 127 - e; +-0 -> +-inf, +-inf -> +-0, NaN -> QNAN."""
    x = ftz(x)
    T, S = _TAB["recip"]
    s, e, frac = _fields(x)
    i = frac >> 17
    m = (frac | 0x3F800000).astype(U32)
    y0 = add(T[i], mul(_frac17(frac), S[i]))
    y1 = mul(y0, sub(_C2, mul(m, y0)))
    res = ldexp(y1, 127 - e) | (s << 31).astype(U32)
    res = np.where(e == 0, ((s << 31) | PINF).astype(U32), res)
    res = np.where((e == 255) & (frac == 0), (s << 31).astype(U32), res)
    return np.where((e == 255) & (frac != 0), U32(QNAN), res).astype(U32)


def sfu_rsqrt_bits(x):
    """RSQRT (llm/sfu.py:16-20, 99-114): mantissa m or 2m by exponent parity, 128-entry table,
    y1 = y0 (1.5 - (m' y0^2) 0.5), exponent -(E - odd) / 2; +-0 -> +inf, x < 0 -> QNAN,
    +inf -> +0, NaN -> QNAN."""
    x = ftz(x)
    T, S = _TAB["rsqrt"]
    s, e, frac = _fields(x)
    E = e - 127
    odd = E & 1
    j = odd * 64 + (frac >> 17)
    m2 = (frac | ((127 + odd) << 23)).astype(U32)
    y0 = add(T[j], mul(_frac17(frac), S[j]))
    y1 = mul(y0, sub(_C1_5, mul(mul(m2, mul(y0, y0)), _C0_5)))
    res = ldexp(y1, -((E - odd) // 2))
    res = np.where(e == 0, U32(PINF), res)
    res = np.where((s == 1) & (e != 0), U32(QNAN), res)
    res = np.where((s == 0) & (e == 255) & (frac == 0), U32(0), res)
    return np.where((e == 255) & (frac != 0), U32(QNAN), res).astype(U32)


def sfu_exp(x):
    return val(sfu_exp_bits(bits(x)))


def sfu_recip(x):
    return val(sfu_recip_bits(bits(x)))


def sfu_rsqrt(x):
    return val(sfu_rsqrt_bits(bits(x)))


# ------------------------------------------------------------------ vector-engine primitives
def to_i8(x):
    """fp32 -> int8: RNE, saturate to +-127, NaN -> 0, +-inf -> +-127 (llm/ref_model.py:136-139)."""
    y = np.rint(np.asarray(x, F))
    return np.clip(np.nan_to_num(y, nan=0.0, posinf=127, neginf=-127), -127, 127).astype(np.int8)


def red_sum(v, D):
    """The device's ordered fp32 sum over the last axis (llm/ref_model.py:179-186,
    compiler/tests/oracle.py:588-600): +0 padding to a multiple of D, lane l accumulates
    v[l], v[D + l], v[2D + l], ... in order, then pairs of lanes (0+1, 2+3, ...) until one remains."""
    v = np.asarray(v, F)
    n = v.shape[-1]
    pad = (-n) % D
    if pad or n == 0:
        v = np.concatenate([v, np.zeros(v.shape[:-1] + (pad if n else D,), F)], axis=-1)
    g = v.reshape(v.shape[:-1] + (-1, D))
    acc = g[..., 0, :].copy()
    for i in range(1, g.shape[-2]):
        acc = (acc + g[..., i, :]).astype(F)
    while acc.shape[-1] > 1:
        acc = (acc[..., 0::2] + acc[..., 1::2]).astype(F)
    return acc[..., 0]


def quant_act(x):
    """Per-row dynamic int8 (llm/ref_model.py:191-196): amax = max|x|, s = amax * F(1/127),
    xq = to_i8(x * recip(s)). Rows are the last axis; returns (xq, s) with s of shape x.shape[:-1]."""
    x = np.asarray(x, F)
    amax = np.max(np.abs(x), axis=-1)
    s = (amax * F(1 / 127)).astype(F)
    inv = sfu_recip(s)
    with np.errstate(invalid="ignore", over="ignore"):
        return to_i8((x * inv[..., None]).astype(F)), s


def int_dot(xq, wq):
    """Exact int32 products: xq [..., K] int8 . wq [N, K] int8 -> int64 [..., N]."""
    return np.asarray(xq, np.int64) @ np.asarray(wq, np.int64).T


def dequant(acc, s_w, s_x):
    """y = F(F(f32(acc) * s_w) * s_x) (llm/ref_model.py:198-202); s_x per row of acc."""
    y = (np.asarray(acc).astype(np.float64).astype(F) * np.asarray(s_w, F)).astype(F)
    return (y * np.asarray(s_x, F)[..., None]).astype(F)


def linear(xq, s_x, wq, s_w, wq_f64=None):
    """The W8A8 linear layer on rows xq [..., K] with scales s_x [...]. wq_f64: the same int8 weights
    as float64 (the exact float64 matmul of llm/ref_model.py:162, 200), for speed."""
    if wq_f64 is not None:
        acc = (np.asarray(xq).astype(np.float64) @ wq_f64.T).astype(np.int64)
    else:
        acc = int_dot(xq, wq)
    return dequant(acc, s_w, s_x)


def rmsnorm(x, g, eps, D):
    """Per row (last axis) (llm/ref_model.py:204-207): ss = red_sum(x*x); r = rsqrt(ss * F(1/n) + F(eps));
    out = (x * r) * g."""
    x = np.asarray(x, F)
    n = x.shape[-1]
    ss = red_sum((x * x).astype(F), D)
    r = sfu_rsqrt(((ss * F(1.0 / n)).astype(F) + F(eps)).astype(F))
    return ((x * r[..., None]).astype(F) * np.asarray(g, F)).astype(F)


def rope(v, c, s):
    """Rotate interleaved pairs (2i, 2i+1) of the last axis (llm/ref_model.py:209-214):
    out = F(F(v * c) + F(sw * s)), sw = (-v1, v0); c, s per pair (broadcast over the pairs' heads)."""
    v = np.asarray(v, F)
    c2 = np.repeat(np.asarray(c, F), 2, axis=-1)
    s2 = np.repeat(np.asarray(s, F), 2, axis=-1)
    sw = np.empty_like(v)
    sw[..., 0::2], sw[..., 1::2] = -v[..., 1::2], v[..., 0::2]
    return ((v * c2).astype(F) + (sw * s2).astype(F)).astype(F)


def silu_mul(h1, h3):
    """u = F(F(h1 * recip(F(1 + exp(F(h1 * -1))))) * h3) (llm/ref_model.py:249-250)."""
    h1 = np.asarray(h1, F)
    sig = sfu_recip((F(1) + sfu_exp((h1 * F(-1)).astype(F))).astype(F))
    return ((h1 * sig).astype(F) * np.asarray(h3, F)).astype(F)


# GELU's tanh approximation as the device computes it (compiler/frontend/hf_generic.py:840-852):
# x * 0.5 * (1 + tanh(u)) = x * RECIP(F(EXP(z) + 1)), z = F(x * F(A + F(F(x * x) * B))),
# u = sqrt(2 / pi) * (x + 0.044715 x^3), A = f32(-2 sqrt(2 / pi)), B = f32(A * 0.044715) (float64
# constants rounded once).
GELU_A = F(-2.0 * np.sqrt(2.0 / np.pi))
GELU_B = F(-2.0 * np.sqrt(2.0 / np.pi) * 0.044715)


def gelu_tanh(x):
    """F(x * RECIP(F(EXP(z) + 1))) with z as above (hf_generic.py:848-852)."""
    x = np.asarray(x, F)
    with np.errstate(over="ignore", invalid="ignore"):     # |x| > 1.8e19: x * x -> inf, as on the device
        z = (x * (GELU_A + ((x * x).astype(F) * GELU_B).astype(F)).astype(F)).astype(F)
        return (x * sfu_recip((sfu_exp(z) + F(1)).astype(F))).astype(F)


def gelu_mul(h1, h3):
    """The GELU-tanh gate of a GeGLU FFN: u = F(gelu_tanh(h1) * h3) (the gate's activation in place of
    SiLU, llm/ref_model.py:249-250's product order)."""
    return (gelu_tanh(h1) * np.asarray(h3, F)).astype(F)


def gate_mul(h1, h3, act):
    """act "silu" (SwiGLU) or "gelu_tanh" (GeGLU)."""
    return gelu_mul(h1, h3) if act == "gelu_tanh" else silu_mul(h1, h3)


# Mistakes the tests plant in attention() to show that the reference fixtures catch them (test use only):
# "rq_av_first" F(att * F(rq * a_v)); "qsum_e" qsum's total over the exps instead of the int8
# probabilities; "fold_head0" the K fold with KV head 0's scales for every head; "fold_after_quant" q
# quantised, dequantised, folded and quantised again.
PLANTS = ("rq_av_first", "qsum_e", "fold_head0", "fold_after_quant")


def attention(q, K, V, H, Hk, a_k, a_v, D, qsum=False, ch_sk=None, ch_av=None, plant=None):
    """One query row q [H * hd] against the int8 cache rows K, V [T, Hk * hd] (llm/ref_model.py:230-243,
    GQA as compiler/frontend/qhf.py:304-319): per head quant_act(q), exact int32 scores
    F(F(f32(dot) * s_q) * a_k), e = EXP(F(s - max)), then
    - DeviceModel's form: pq = to_i8(F(F(e * RECIP(red_sum(e))) * 127)), out = F(f32(pq . V) * a_v);
    - qsum (compiler/frontend/hf_generic.py:265-292): pq = to_i8(F(e * 127)),
      out = F(F(f32(pq . V) * F(RECIP(f32(sum pq)) * 127)) * a_v).
    ch_sk [Hk * hd]: K's per-channel scales, q = F(q * s_k) before its quant_act (hf_generic.py:252-254);
    ch_av [Hk * hd]: a_v per output channel (hf_generic.py:183-186, 292). plant: one of PLANTS (tests)."""
    assert plant in (None,) + PLANTS
    T = K.shape[0]
    hd = q.shape[-1] // H
    G = H // Hk
    per_head = lambda v: np.repeat(np.asarray(v, F).reshape(Hk, hd), G, axis=0)   # (H, hd)
    # int8 products summed in float64 are exact: |dot| <= 127^2 hd and |P.V| <= 127^2 T, far below 2^53
    Kg = np.asarray(K).reshape(T, Hk, hd).transpose(1, 0, 2).astype(np.float64)      # (Hk, T, hd)
    Vg = np.asarray(V).reshape(T, Hk, hd).transpose(1, 0, 2).astype(np.float64)
    qh = np.asarray(q, F).reshape(H, hd)
    if ch_sk is not None and plant == "fold_after_quant":
        qq, s_q = quant_act(qh)
        qh = ((qq.astype(F) * s_q[:, None]).astype(F) * per_head(ch_sk)).astype(F)
    elif ch_sk is not None:
        sk = np.tile(np.asarray(ch_sk, F).reshape(Hk, hd)[:1], (H, 1)) if plant == "fold_head0" else per_head(ch_sk)
        qh = (qh * sk).astype(F)
    qq, s_q = quant_act(qh)                                                          # (H, hd), (H,)
    qg = qq.astype(np.float64).reshape(Hk, G, hd)
    dots = np.matmul(qg, Kg.transpose(0, 2, 1)).reshape(H, T)                        # (H, T) exact
    sc = (dots.astype(F) * s_q[:, None]).astype(F)
    sc = (sc * F(a_k)).astype(F)
    e = sfu_exp((sc - np.max(sc, axis=-1, keepdims=True)).astype(F))
    if qsum:
        pq = to_i8((e * F(127)).astype(F)).astype(np.int64)
        tot = red_sum(e, D) if plant == "qsum_e" else pq.sum(-1).astype(F)
        rq = (sfu_recip(tot) * F(127)).astype(F)                                    # (H,), the sum exact
    else:
        r = sfu_recip(red_sum(e, D))
        pq = to_i8(((e * r[:, None]).astype(F) * F(127)).astype(F)).astype(np.int64)
    att = np.matmul(pq.astype(np.float64).reshape(Hk, G, T), Vg).reshape(H, hd).astype(F)   # exact sums
    av = per_head(ch_av) if ch_av is not None else F(a_v)
    if qsum and plant == "rq_av_first":
        return (att * (rq[:, None] * av).astype(F)).astype(F).reshape(H * hd)
    if qsum:
        att = (att * rq[:, None]).astype(F)
    return (att * av).astype(F).reshape(H * hd)


def topk_desc(scores, k):
    """Top-k ids of a score vector: descending values, an equal value placed before a larger id, NaN
    never selected (compiler/tests/oracle.py:558-585). A stable sort on -value does exactly this."""
    s = np.asarray(scores, F).astype(np.float64)
    key = np.where(np.isnan(s), np.inf, -s)
    return np.argsort(key, kind="stable")[:k]


def requant_int(r, scale, shift, zp, lo, hi):
    """The integer VE REQUANT (llm/sa_funcsim.py:265-274): q = ((r * scale + 2^(shift-1)) >> shift) + zp,
    clamp to [lo, hi], then to int8 range. scale is a signed 16-bit value; arithmetic shift."""
    r = np.asarray(r, np.int64)
    q = (r * int(scale) + ((1 << (shift - 1)) if shift else 0)) >> shift
    q = q + int(zp)
    q = np.clip(q, lo, hi)
    return np.clip(q, -128, 127).astype(np.int8)
