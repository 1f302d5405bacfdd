"""CPU restatement of the whole W8A8 decoder: TEST INFRASTRUCTURE ONLY (the checker
for the HIP path, and bench.py's timed CPU baseline). Never imported by the product.

`OracleModel` is the reference's DeviceModel (llm/ref_model.py:151-255) with its
numerics unchanged (NumPy float32 vector steps, bit-exact SFU, D-lane ordered sums,
int8 KV cache with static per-layer scales, int8 softmax probabilities), generalised
to the structure the reference's HF path adds (compiler/frontend/qhf.py:321-409):

- head_dim and q_dim = heads * head_dim independent of dim, grouped KV heads;
- per-head RMSNorm of q and k before RoPE (QK-norm), eps and theta per model;
- a tied classifier (the embedding's int8 rows and scales);
- a top-k mixture-of-experts FFN (compiler/frontend/hf_generic.py:641-657) with the
  device's top-k order (compiler/tests/oracle.py:558-585) and the route weights
  e = EXP(v - v0), w = e * RECIP(red_sum(e)).

The HF path's numerics options (compiler/frontend/hf_generic.py; cfg.attn_norm,
cfg.kv_channel, cfg.act, cfg.logits_scaling, the last folded into the classifier's
scales by the model data) change these steps, with the device's primitives:
- qsum (hf_generic.py:265-292): eq = to_i8(F(e * 127)), att = sum eq V (int32),
  rq = F(RECIP(f32(sum eq)) * 127) (the sum exact in float32), out = F(F(f32(att) * rq) * a_v);
- K per channel (hf_generic.py:153-187, 252-254): q = F(q * s_k) per channel before its
  quant_act, a_k = f32(1 / sqrt(hd)); the cache row to_i8(F(k * inv_sk[c]));
- V per channel: to_i8(F(v * inv_sv[c])), and a_v[c] per output channel;
- GELU-tanh gate (hf_generic.py:840-852): numerics.gelu_mul in place of silu_mul.

With q_dim = dim, no QK-norm, theta 1e4 (float32 tables), eps 1e-5, a dense FFN and no
options it computes exactly DeviceModel(sfu=SfuExact); tests/golden holds runs of the
reference that pin that. The generalised parts (QK-norm, q_dim != dim, MoE routing, the
HF options) have no runnable reference implementation with these numerics: they are
pinned by properties and by float64 attention / GELU within stated tolerances (see the
tests that cover them), not by reference vectors.

Prefill (qhf.QModel.prefill, compiler/frontend/qhf.py:356-409): every row is a decode
step at its own position; rows only share the linear layers, whose numerics are
per row, so a prefill gives the decode-only logits and KV cache bit for bit.
"""
import numpy as np

from . import numerics as N

F = np.float32
_KCHUNK = 1024          # int8 products summed in float32 stay exact while K-chunk * 127^2 < 2^24


class _Lin:
    """int8 weights (N, K) with scales; the product as exact chunked float32 GEMMs."""

    def __init__(self, q, s):
        self.q, self.s = np.asarray(q, np.int8), np.asarray(s, F)
        self._f = None

    def acc(self, xq):
        if self._f is None:
            self._f = self.q.astype(F)
        xq = np.asarray(xq)
        xf = xq.astype(F)
        K = self.q.shape[1]
        out = np.zeros(xq.shape[:-1] + (self.q.shape[0],), np.int64)
        for k0 in range(0, K, _KCHUNK):
            out += (xf[..., k0:k0 + _KCHUNK] @ self._f[:, k0:k0 + _KCHUNK].T).astype(np.int64)
        return out

    def __call__(self, xq, s_x):
        return N.dequant(self.acc(xq), self.s, s_x)


def moe_row(router, experts, xq, s_x, k, D, act="silu", dim=None):
    """One row's top-k mixture of experts (QMixtralMoe.route / _row, compiler/frontend/hf_generic.py:641-657,
    in the device's numerics): scores = linear(router); the k largest in descending order (equal scores:
    lower id first, NaN never chosen); e = EXP(F(v - v0)); w = F(e * RECIP(red_sum(e))); then per k in
    order y = F(y + F(w_k * linear(quant_act(gate(g_k, u_k)), down_k))). router: a _Lin; experts[e] =
    (gate, up, down) _Lins. Returns (y, ids, w)."""
    sc = router(xq, s_x)
    ids = N.topk_desc(sc, k)
    v = sc[ids]
    e = N.sfu_exp((v - v[0]).astype(F))
    w = (e * N.sfu_recip(N.red_sum(e, D))).astype(F)
    y = np.zeros(dim if dim is not None else experts[0][2].q.shape[0], F)
    for j, i in enumerate(ids):
        g_l, u_l, d_l = experts[i]
        h = N.gate_mul(g_l(xq, s_x), u_l(xq, s_x), act)
        hq, s_h = N.quant_act(h)
        y = (y + (w[j] * d_l(hq, s_h)).astype(F)).astype(F)
    return y, ids, w


class OracleModel:
    def __init__(self, qm, D=None):
        """qm: the model data (int8 weights, scales, gains, RoPE tables, KV constants); attribute names as
        t2r_amd.weights.QuantModel."""
        self.qm, self.cfg = qm, qm.cfg
        c = self.cfg
        self.D = D or c.D
        L = c.layers
        self.emb_q, self.emb_s = qm.emb_q, qm.emb_s
        self.cls = _Lin(qm.cls_q, qm.cls_s)
        self.wqkv = [_Lin(qm.wqkv[l], qm.s_wqkv[l]) for l in range(L)]
        self.wo = [_Lin(qm.wo[l], qm.s_wo[l]) for l in range(L)]
        if c.moe:
            self.router = [_Lin(qm.router[l], qm.s_router[l]) for l in range(L)]
            self.experts = [[(_Lin(qm.wg[l, e], qm.s_wg[l, e]), _Lin(qm.wu[l, e], qm.s_wu[l, e]),
                              _Lin(qm.wd[l, e], qm.s_wd[l, e])) for e in range(c.n_experts)] for l in range(L)]
        else:
            self.w1 = [_Lin(qm.w1[l], qm.s_w1[l]) for l in range(L)]
            self.w3 = [_Lin(qm.w3[l], qm.s_w3[l]) for l in range(L)]
            self.w2 = [_Lin(qm.w2[l], qm.s_w2[l]) for l in range(L)]
        self.last_route = None
        self.reset()

    def reset(self):
        c = self.cfg
        self.kc = np.zeros((c.layers, c.seq_len, c.kv_dim), np.int8)
        self.vc = np.zeros((c.layers, c.seq_len, c.kv_dim), np.int8)

    # ------------------------------------------------------------ pieces
    def embed(self, tokens):
        t = np.asarray(tokens)
        return (self.emb_q[t].astype(F) * self.emb_s[t][..., None]).astype(F)

    def norm_quant(self, x, g):
        return N.quant_act(N.rmsnorm(x, g, self.cfg.eps, self.D))

    def qkv_rows(self, l, qkv, positions):
        """QK-norm, RoPE and the KV append of rows qkv [M, q + 2 kv] at their positions; returns q [M, q_dim]."""
        c, qm = self.cfg, self.qm
        hd, M = c.head_dim, qkv.shape[0]
        q = qkv[:, :c.q_dim].reshape(M, c.heads, hd)
        k = qkv[:, c.q_dim:c.q_dim + c.kv_dim].reshape(M, c.kv_heads, hd)
        v = qkv[:, c.q_dim + c.kv_dim:]
        if c.qk_norm:
            q = N.rmsnorm(q, qm.q_norm[l], c.eps, self.D)
            k = N.rmsnorm(k, qm.k_norm[l], c.eps, self.D)
        pos = np.asarray(positions)
        cs, sn = qm.cos[pos][:, None, :], qm.sin[pos][:, None, :]
        q = N.rope(q, cs, sn).reshape(M, c.q_dim)
        k = N.rope(k, cs, sn).reshape(M, c.kv_dim)
        inv_sk, inv_sv = qm.kvc[l, 0], qm.kvc[l, 1]
        fl = int(qm.kv_flags[l]) if getattr(qm, "kv_flags", None) is not None else 0
        if fl & 1:
            inv_sk = qm.kvch[l, 1]
        if fl & 2:
            inv_sv = qm.kvch[l, 2]
        self.kc[l, pos] = N.to_i8((k * inv_sk).astype(F))
        self.vc[l, pos] = N.to_i8((v * inv_sv).astype(F))
        return q

    def attention(self, l, q, pos):
        """One query row q [q_dim] at position pos against the cache rows 0..pos (llm/ref_model.py:230-243;
        the HF options as numerics.attention states them)."""
        c, qm = self.cfg, self.qm
        T = pos + 1
        fl = int(qm.kv_flags[l]) if getattr(qm, "kv_flags", None) is not None else 0
        return N.attention(q, self.kc[l, :T], self.vc[l, :T], c.heads, c.kv_heads, qm.kvc[l, 2], qm.kvc[l, 3],
                           self.D, qsum=c.attn_norm == "qsum", ch_sk=qm.kvch[l, 0] if fl & 1 else None,
                           ch_av=qm.kvch[l, 3] if fl & 2 else None)

    def moe(self, l, xq, s_x):
        """Top-k MoE FFN of one row (compiler/frontend/hf_generic.py:641-657 with device numerics)."""
        c = self.cfg
        y, ids, w = moe_row(self.router[l], self.experts[l], xq, s_x, c.top_k, self.D, c.act, c.dim)
        self.last_route = (ids, w)
        return y

    def layer(self, l, x, positions):
        """One decoder layer on rows x [M, d] at positions [M] (each row a decode step)."""
        c, qm = self.cfg, self.qm
        xq, s_x = self.norm_quant(x, qm.rms_att[l])
        qkv = self.wqkv[l](xq, s_x)
        q = self.qkv_rows(l, qkv, positions)
        att = np.stack([self.attention(l, q[m], int(p)) for m, p in enumerate(positions)])
        aq, s_a = N.quant_act(att)
        x = (x + self.wo[l](aq, s_a)).astype(F)
        xq, s_x = self.norm_quant(x, qm.rms_ffn[l])
        if c.moe:
            y = np.stack([self.moe(l, xq[m], s_x[m]) for m in range(x.shape[0])])
        else:
            u = N.gate_mul(self.w1[l](xq, s_x), self.w3[l](xq, s_x), c.act)
            hq, s_h = N.quant_act(u)
            y = self.w2[l](hq, s_h)
        return (x + y).astype(F)

    def final(self, x):
        xq, s_x = self.norm_quant(x, self.qm.rms_final)
        return self.cls(xq, s_x)

    # ------------------------------------------------------------ model
    def forward(self, token, pos, n_layers=None):
        """Logits of `token` at `pos` (a decode step); with n_layers, x after that many layers."""
        x = self.embed([token])
        for l in range(self.cfg.layers if n_layers is None else n_layers):
            x = self.layer(l, x, [pos])
        if n_layers is not None:
            return x[0]
        return self.final(x)[0]

    def prefill(self, tokens, start=0):
        """Rows tokens at positions start..start+M-1 through the layers together; logits of the last row."""
        M = len(tokens)
        positions = list(range(start, start + M))
        x = self.embed(tokens)
        for l in range(self.cfg.layers):
            x = self.layer(l, x, positions)
        return self.final(x[M - 1:M])[0]


def greedy(model, prompt, steps):
    """Prompt tokens fed one by one, then the argmax (first maximal index) of each step's logits; no stop
    token (BOS may occur among random ids). Returns (tokens fed, logits of every step)."""
    model.reset()
    toks, out = [prompt[0]], []
    for pos in range(min(steps, model.cfg.seq_len)):
        lg = model.forward(toks[-1], pos)
        out.append(lg)
        if pos + 1 < len(prompt):
            toks.append(prompt[pos + 1])
        else:
            toks.append(int(np.argmax(lg)))
    return toks, out
