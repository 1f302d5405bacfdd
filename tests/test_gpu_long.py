"""Long context: caches of 8192 positions (the datapath's kMaxS), past the 2048 of the measured
configs. The decode kernels then take several passes over the keys, the prefill attention falls back
to the per-(head, row) kernel when a chunk's score rows do not fit in LDS, and the batched step to
per-head attention. Each is checked against the CPU restatement or the others, bit for bit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = np.float32


@pytest.mark.parametrize("qsum,kch", [(False, False), (True, True)])
def test_attention_op_8k(qsum, kch):
    import torch
    from oracle import numerics as N
    from t2r_amd import ops
    rng = np.random.default_rng(21)
    H_, Hk, hd, S, D = 8, 2, 64, 8192, 16
    kc = rng.integers(-127, 128, (S, Hk * hd)).astype(np.int8)
    vc = rng.integers(-127, 128, (S, Hk * hd)).astype(np.int8)
    positions = [2047, 2048, 4100, 6001, 8191]
    q = (rng.standard_normal((len(positions), H_ * hd)) * 2).astype(F)
    sk = np.exp(rng.uniform(-5, 0, Hk * hd)).astype(F) if kch else None
    a_k, a_v = (F(1 / np.sqrt(hd)) if kch else F(0.02 / np.sqrt(hd))), F(0.03 / 127)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    got = ops.attention_opt(T(q), T(kc), T(vc), T(np.array(positions, np.int32)), H_, Hk, a_k, a_v, D, qsum=qsum,
                            ch_sk=None if sk is None else T(sk)).cpu().numpy()
    for i, p in enumerate(positions):
        want = N.attention(q[i], kc[:p + 1], vc[:p + 1], H_, Hk, a_k, a_v, D, qsum=qsum, ch_sk=sk)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"pos {p}"


def _long_tiny(qsum):
    import t2r_amd.config as C
    # head_dim 64 and two query heads per KV head: the full-size decode kernels' shapes on a tiny model
    return C.ModelConfig("tiny-long" + ("-hf" if qsum else ""), dim=128, hidden=256, layers=2, heads=4, kv_heads=2,
                         head_dim=64, vocab=96, seq_len=8192, theta=5e5, eps=1e-5, weight_std=None, gain_std=0.1,
                         emb_scale=4.0, seed_w=81, seed_p=82, prompt_len=64,
                         attn_norm="qsum" if qsum else "device", kv_channel="k" if qsum else "").validate()


@pytest.mark.parametrize("qsum", [False, True])
def test_long_tiny_vs_oracle(qsum):
    """A 2600-token prompt (three 1024-key passes of the decode kernels) through the oracle and through
    t2r_prefill (1024-row chunks), then decode steps at 2600..2603 and one batched step at positions
    (2604, 2100, 17): logits and every KV byte equal."""
    import torch
    from oracle import OracleModel
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = _long_tiny(qsum)
    qm = W.QuantModel(cfg)
    rng = np.random.default_rng(23)
    P = 2600
    toks = rng.integers(0, cfg.vocab, P + 4).tolist()
    om = OracleModel(qm)
    want = om.prefill(toks[:P])
    rm = ResidentModel(qm, max_rows=1024)
    print(f"{cfg.name}: prefill {P} rows", flush=True)
    got = rm.prefill(toks[:P]).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(rm.kc[:, :P].cpu().numpy(), om.kc[:, :P])
    assert np.array_equal(rm.vc[:, :P].cpu().numpy(), om.vc[:, :P])
    for pos in range(P, P + 4):
        w = om.forward(toks[pos], pos)
        g = rm.decode(toks[pos], pos).cpu().numpy()
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"decode at {pos}"
    # batched: slot 0 continues the sequence, slots 1 and 2 hold its first 2100 / 17 positions
    B, lens = 3, [P + 4, 2100, 17]
    kc, vc = rm.batch_caches(B)
    for b in range(B):
        kc[b, :, :lens[b]].copy_(rm.kc[:, :lens[b]])
        vc[b, :, :lens[b]].copy_(rm.vc[:, :lens[b]])
    nxt = [int(t) for t in rng.integers(0, cfg.vocab, B)]
    out = rm.decode_batch(nxt, lens, kc, vc).cpu().numpy()
    for b in range(B):
        om.kc[:, :lens[b]], om.vc[:, :lens[b]] = rm.kc[:, :lens[b]].cpu().numpy(), rm.vc[:, :lens[b]].cpu().numpy()
        w = om.forward(nxt[b], lens[b])
        assert np.array_equal(out[b].view(np.uint32), w.view(np.uint32)), f"batched row {b} at {lens[b]}"
        assert np.array_equal(kc[b, :, lens[b]].cpu().numpy(), om.kc[:, lens[b]])
    rm.close()


def test_c4_8k_paths_agree():
    """C4's shape with an 8192-position cache (its recorded KV scales): a 6000-token prompt prefilled in
    1024-row chunks equals the prefill of its first 5999 rows plus a decode step of the last, and one
    batched step at positions (6000, 200) equals the single decode of each."""
    import torch
    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    base = C.get("c4-llama3.2-1b")
    cfg = base.with_(name="c4-8k", seq_len=8192)
    qm = W.QuantModel(cfg, kv_scales=W.stored_kv_scales(base))
    rm = ResidentModel(qm, max_rows=1024)
    rng = np.random.default_rng(25)
    P = 6000
    toks = rng.integers(0, cfg.vocab, P).tolist()
    print("c4-8k: prefill 6000 rows", flush=True)
    full = rm.prefill(toks).cpu().numpy()
    kv_full = rm.kc[:, :P].clone(), rm.vc[:, :P].clone()
    rm.reset()
    rm.prefill(toks[:-1], logits=False)
    last = rm.decode(toks[-1], P - 1).cpu().numpy()
    assert np.array_equal(full.view(np.uint32), last.view(np.uint32))
    assert torch.equal(rm.kc[:, :P], kv_full[0]) and torch.equal(rm.vc[:, :P], kv_full[1])
    B, lens = 2, [P, 200]
    kc, vc = rm.batch_caches(B)
    for b in range(B):
        kc[b, :, :lens[b]].copy_(kv_full[0][:, :lens[b]])
        vc[b, :, :lens[b]].copy_(kv_full[1][:, :lens[b]])
    nxt = [int(t) for t in rng.integers(0, cfg.vocab, B)]
    out = rm.decode_batch(nxt, lens, kc, vc).cpu().numpy()
    for b in range(B):
        rm.reset()
        rm.kc[:, :lens[b]].copy_(kv_full[0][:, :lens[b]])
        rm.vc[:, :lens[b]].copy_(kv_full[1][:, :lens[b]])
        want = rm.decode(nxt[b], lens[b]).cpu().numpy()
        assert np.array_equal(out[b].view(np.uint32), want.view(np.uint32)), f"batched row {b} at {lens[b]}"
        assert torch.equal(kc[b, :, lens[b]], rm.kc[:, lens[b]])
    rm.close()
