"""Op-level calls on torch device tensors: one C-ABI call (one or two HIP launches) per piece of
the reference's token list (llm/compile_model.py:147-349), each step for step the DeviceModel
method it names (llm/ref_model.py:191-255). Inputs must be contiguous tensors on a HIP device
with the dtypes below; outputs are allocated here (the C-ABI itself never allocates)."""
import torch

from . import abi

I8, I32, F32 = torch.int8, torch.int32, torch.float32


def _dev(*ts):
    for t in ts:
        if t is not None and (not t.is_cuda or not t.is_contiguous()):
            raise ValueError("op arguments must be contiguous tensors on a HIP device")


def _s():
    return abi.stream_ptr()


def _u32(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t


def sfu(fn, x_bits):
    """fn 'exp' | 'recip' | 'rsqrt' | 'abs' on fp32 bit patterns (int32 tensor) -> bit patterns."""
    _dev(x_bits)
    code = {"exp": 0, "recip": 1, "rsqrt": 2, "abs": 3}[fn]
    y = torch.empty_like(x_bits)
    abi.call("t2r_sfu", code, abi.ptr(x_bits), abi.ptr(y), x_bits.numel(), _s())
    return y


def sfu_check(fn, first=0, count=1 << 32):
    """Inputs [first, first + count) through the datapath SFU and the literal FTZ sequence; returns
    (number of differing results, smallest differing input or None). 'exp_np': the softmax's EXP,
    checked against EXP on its domain (x <= 0 and NaN); 'recip_ge1': the gates' RECIP, against RECIP
    on its domain (x >= 1 and NaN); 'exp_sm': the softmax's EXP under a finite maximum, against EXP
    on its domain (x <= 0); 'exp_g' / 'recip_g1': the gates' pair-table EXP (x not NaN) and RECIP
    (x >= 1, not NaN), against EXP and RECIP; other inputs skipped."""
    code = {"exp": 0, "recip": 1, "rsqrt": 2, "exp_np": 3, "recip_ge1": 4, "exp_sm": 5, "exp_g": 6, "recip_g1": 7}[fn]
    out = torch.empty(2, dtype=torch.int32, device="cuda")
    abi.call("t2r_sfu_check", code, first, count, abi.ptr(out), _s())
    n, lo = (int(v) & 0xFFFFFFFF for v in out.cpu().tolist())
    return n, (None if n == 0 else lo)


def fp32_op(op, a_bits, b_bits):
    """The fp32 primitives on bit patterns: 'add', 'sub', 'mul', 'ldexp', 'floor', 'to_i8', 'from_int',
    'ieee_mul', 'ieee_add' (see include/t2r.h t2r_fp32_op)."""
    _dev(a_bits, b_bits)
    code = ["add", "sub", "mul", "ldexp", "floor", "to_i8", "from_int", "ieee_mul", "ieee_add"].index(op)
    y = torch.empty_like(a_bits)
    abi.call("t2r_fp32_op", code, abi.ptr(a_bits), abi.ptr(b_bits), abi.ptr(y), a_bits.numel(), _s())
    return y


def requant(r, scale, shift, zp, lo, hi):
    _dev(r)
    out = torch.empty(r.shape, dtype=I8, device=r.device)
    abi.call("t2r_requant", abi.ptr(r), r.numel(), int(scale), int(shift), int(zp), int(lo), int(hi), abi.ptr(out), _s())
    return out


def embed(emb_q, emb_s, tokens):
    _dev(emb_q, emb_s, tokens)
    V, d = emb_q.shape
    x = torch.empty((tokens.numel(), d), dtype=F32, device=emb_q.device)
    abi.call("t2r_embed", abi.ptr(emb_q), abi.ptr(emb_s), abi.ptr(tokens), tokens.numel(), d, V, abi.ptr(x), None, _s())
    return x


def rmsnorm(x, g, eps, D):
    _dev(x, g)
    out = torch.empty_like(x)
    n = x.shape[-1]
    abi.call("t2r_rmsnorm", abi.ptr(x), abi.ptr(g), x.numel() // n, n, float(eps), int(D), abi.ptr(out), _s())
    return out


def quant_act(x):
    _dev(x)
    n = x.shape[-1]
    rows = x.numel() // n
    xq = torch.empty(x.shape, dtype=I8, device=x.device)
    s = torch.empty(x.shape[:-1] if x.dim() > 1 else (1,), dtype=F32, device=x.device)
    abi.call("t2r_quant_act", abi.ptr(x), rows, n, abi.ptr(xq), abi.ptr(s), _s())
    return xq, s


def linear(w, s_w, xq, s_x, residual=None, acc=False):
    """W8A8 linear of rows xq [M, K] (or [K]); returns y (and the int32 accumulators with acc=True)."""
    _dev(w, s_w, xq, s_x, residual)
    N, K = w.shape
    M = xq.numel() // K
    y = torch.empty((M, N) if xq.dim() > 1 else (N,), dtype=F32, device=w.device)
    a = torch.empty(y.shape, dtype=I32, device=w.device) if acc else None
    name = "t2r_gemv_w8a8" if xq.dim() == 1 else "t2r_gemm_w8a8"
    args = [abi.ptr(w), abi.ptr(s_w), abi.ptr(xq), abi.ptr(s_x)] + ([] if xq.dim() == 1 else [M]) + \
        [N, K, abi.ptr(y), abi.ptr(a), abi.ptr(residual), _s()]
    abi.call(name, *args)
    return (y, a) if acc else y


def rope(v, cos_t, sin_t, pos):
    """RoPE of rows v [rows, n] in place (heads of head_dim = 2 * cos_t.shape[1])."""
    _dev(v, cos_t, sin_t, pos)
    n = v.shape[-1]
    abi.call("t2r_rope", abi.ptr(v), abi.ptr(cos_t), abi.ptr(sin_t), abi.ptr(pos), v.numel() // n, n,
             cos_t.shape[1], cos_t.shape[0], _s())
    return v


def kv_append(k, v, inv_sk, inv_sv, kc, vc, pos):
    _dev(k, v, kc, vc, pos)
    kv = kc.shape[-1]
    abi.call("t2r_kv_append", abi.ptr(k), abi.ptr(v), float(inv_sk), float(inv_sv), abi.ptr(kc), abi.ptr(vc),
             abi.ptr(pos), k.numel() // kv, kv, kc.shape[0], _s())


def kv_append_ch(k, v, inv_sk, inv_sv, kc, vc, pos):
    """KV append with per-channel inverse scales: inv_sk / inv_sv are [kv_dim] device tensors or scalars."""
    _dev(k, v, kc, vc, pos)
    kv = kc.shape[-1]
    vec = lambda x: abi.ptr(x) if isinstance(x, torch.Tensor) else None
    sca = lambda x: 0.0 if isinstance(x, torch.Tensor) else float(x)
    abi.call("t2r_kv_append_ch", abi.ptr(k), abi.ptr(v), sca(inv_sk), sca(inv_sv), vec(inv_sk), vec(inv_sv),
             abi.ptr(kc), abi.ptr(vc), abi.ptr(pos), k.numel() // kv, kv, kc.shape[0], _s())


def attention(q, kc, vc, pos, H, Hk, a_k, a_v, D):
    """Attention of rows q [rows, H * hd] at positions pos over the int8 caches [S, Hk * hd]."""
    _dev(q, kc, vc, pos)
    hd = q.shape[-1] // H
    rows = q.numel() // q.shape[-1]
    att = torch.empty_like(q)
    abi.call("t2r_attn_decode", abi.ptr(q), abi.ptr(kc), abi.ptr(vc), abi.ptr(pos), rows, H, Hk, hd, kc.shape[0],
             float(a_k), float(a_v), int(D), abi.ptr(att), _s())
    return att


def attention_opt(q, kc, vc, pos, H, Hk, a_k, a_v, D, qsum=False, ch_sk=None, ch_av=None):
    """attention() with the HF path's options: qsum normalisation, K per channel (ch_sk [Hk * hd]: q
    multiplied before its quantisation), V per channel (ch_av [Hk * hd] in place of a_v)."""
    _dev(q, kc, vc, pos)
    hd = q.shape[-1] // H
    rows = q.numel() // q.shape[-1]
    att = torch.empty_like(q)
    abi.call("t2r_attn_decode_opt", abi.ptr(q), abi.ptr(kc), abi.ptr(vc), abi.ptr(pos), rows, H, Hk, hd,
             kc.shape[0], float(a_k), float(a_v), int(D), abi.T2R_ATTN_QSUM if qsum else 0, abi.ptr(ch_sk),
             abi.ptr(ch_av), abi.ptr(att), _s())
    return att


def attention_prefill(q, kc, vc, pos, H, Hk, a_k, a_v, D, qsum=False, ch_sk=None, ch_av=None):
    """Prefill attention of prompt rows q [M, H * hd] at positions pos [M] (t2r_attn_prefill): each row
    as attention_opt computes it, the rows on the multi-row kernel where the shape allows."""
    _dev(q, kc, vc, pos)
    hd = q.shape[-1] // H
    rows = q.numel() // q.shape[-1]
    att = torch.empty_like(q)
    abi.call("t2r_attn_prefill", abi.ptr(q), abi.ptr(kc), abi.ptr(vc), abi.ptr(pos), rows, H, Hk, hd,
             kc.shape[0], float(a_k), float(a_v), int(D), abi.T2R_ATTN_QSUM if qsum else 0, abi.ptr(ch_sk),
             abi.ptr(ch_av), abi.ptr(att), _s())
    return att


def swiglu(w1, s_w1, w3, s_w3, xq, s_x):
    _dev(w1, s_w1, w3, s_w3, xq, s_x)
    F_, K = w1.shape
    u = torch.empty(F_, dtype=F32, device=w1.device)
    hq = torch.empty(F_, dtype=I8, device=w1.device)
    s_h = torch.empty(1, dtype=F32, device=w1.device)
    abi.call("t2r_swiglu_w8a8", abi.ptr(w1), abi.ptr(s_w1), abi.ptr(w3), abi.ptr(s_w3), abi.ptr(xq), abi.ptr(s_x),
             F_, K, abi.ptr(u), abi.ptr(hq), abi.ptr(s_h), _s())
    return u, hq, s_h


def gated_ffn(act, w1, s_w1, w3, s_w3, xq, s_x):
    """The gated up-projection with gate activation act ("silu" or "gelu_tanh"), then quant_act."""
    _dev(w1, s_w1, w3, s_w3, xq, s_x)
    F_, K = w1.shape
    u = torch.empty(F_, dtype=F32, device=w1.device)
    hq = torch.empty(F_, dtype=I8, device=w1.device)
    s_h = torch.empty(1, dtype=F32, device=w1.device)
    code = {"silu": 0, "gelu_tanh": 1}[act]
    abi.call("t2r_gated_ffn_w8a8", code, abi.ptr(w1), abi.ptr(s_w1), abi.ptr(w3), abi.ptr(s_w3), abi.ptr(xq),
             abi.ptr(s_x), F_, K, abi.ptr(u), abi.ptr(hq), abi.ptr(s_h), _s())
    return u, hq, s_h


def moe_route(scores, k, D):
    _dev(scores)
    E = scores.shape[-1]
    rows = scores.numel() // E
    ids = torch.empty((rows, k), dtype=I32, device=scores.device)
    w = torch.empty((rows, k), dtype=F32, device=scores.device)
    abi.call("t2r_moe_route", abi.ptr(scores), rows, E, int(k), int(D), abi.ptr(ids), abi.ptr(w), _s())
    return ids, w


def argmax(x):
    _dev(x)
    n = x.shape[-1]
    rows = x.numel() // n
    idx = torch.empty(rows, dtype=I32, device=x.device)
    abi.call("t2r_argmax", abi.ptr(x), rows, n, abi.ptr(idx), _s())
    return idx
