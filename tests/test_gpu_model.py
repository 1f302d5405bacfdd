"""Model-level parity of the HIP datapath: decode steps and prefills through t2r_decode_step /
t2r_prefill against the reference's own runs (DeviceModel and SaFuncSim fixtures) and against
the CPU restatement for the generalised shapes (q_dim != dim, QK-norm, MoE). Bit-exact logits,
greedy tokens and int8 KV cache."""
import hashlib
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = np.float32
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


@pytest.fixture(scope="module")
def gold():
    return json.load(open(os.path.join(GOLD, "model_golden.json")))


def resident(cfg, kv=None, D=None, max_rows=None):
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    qm = W.QuantModel(cfg, kv_scales=kv)
    return qm, ResidentModel(qm, D=D, max_rows=max_rows)


def kv_host(rm, n):
    return rm.kc[:, :n].cpu().numpy(), rm.vc[:, :n].cpu().numpy()


@pytest.mark.parametrize("idx", range(6))
def test_decode_equals_reference_runs(gold, idx):
    """Every step's logits (sha256 of the bytes), the greedy token and the KV cache of the reference's
    DeviceModel(SfuExact) runs; for c1-stories15m D=16 that is the whole config-1 run (32-token prompt,
    128 greedy steps), which SaFuncSim reproduces on its first positions (the fixture checks that)."""
    import t2r_amd.config as C
    run = gold["device_model"][idx]
    cfg = C.get(run["config"])
    kv = np.array(run["kv_bits"], np.uint32).view(F).reshape(cfg.layers, 2)
    qm, rm = resident(cfg, kv, D=run["D"])
    print(f"{cfg.name} D={run['D']}: {run['steps']} steps", flush=True)
    for rec in run["positions"]:
        lg = rm.decode(rec["token"], rec["pos"]).cpu().numpy()
        assert sha(lg) == rec["logits_sha"], f"{cfg.name} D={run['D']} pos {rec['pos']}: logits differ"
        assert int(np.argmax(lg)) == rec["argmax"]
        assert int(rm.next.item()) == rec["argmax"]                         # the device-side argmax
    assert sha(*kv_host(rm, run["steps"])) == run["kv_sha"]
    rm.close()


@pytest.mark.parametrize("name", ["tiny-qwen", "tiny-moe", "tiny-gqa"])
def test_generalised_decode_vs_oracle(name):
    import t2r_amd.config as C
    from oracle import OracleModel
    cfg = C.get(name)
    qm, rm = resident(cfg)
    om = OracleModel(qm)
    toks = cfg.prompt()
    seq = list(toks)
    for pos in range(cfg.prompt_len + cfg.decode_steps):
        t = seq[pos]
        want = om.forward(t, pos)
        got = rm.decode(t, pos).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{name} pos {pos}"
        if pos + 1 >= len(seq):
            seq.append(int(np.argmax(want)))
    n = len(seq) - 1
    kc, vc = kv_host(rm, n)
    assert np.array_equal(kc, om.kc[:, :n]) and np.array_equal(vc, om.vc[:, :n])


@pytest.mark.parametrize("dim,hidden,D", [(2048, 8176, 16), (1024, 8192, 8)])
def test_wide_ffn_decode_vs_oracle(dim, hidden, D):
    """FFNs of about 8192 rows (the largest a model takes: W2's K) fill a grid of one block per CU or
    more, so their SwiGLU GEMV is the form with a prologue wave. 8176 rows need 2044 waves of
    four-row tiles: the last of the 256 blocks has rows for four of its eight streaming waves. dim
    1024 takes the one-chunk register slice, D = 8 the eight-lane ordered sum; the norm gains are not
    all ones. Logits and KV bit-exact with the oracle."""
    import t2r_amd.config as C
    from oracle import OracleModel
    cfg = C.ModelConfig(f"wide-{dim}-{hidden}", dim=dim, hidden=hidden, layers=1, heads=8, kv_heads=4, head_dim=64,
                        vocab=1024, seq_len=64, gain_std=0.1, D=D, seed_w=77, seed_p=78, prompt_len=2,
                        decode_steps=2).validate()
    qm, rm = resident(cfg, D=D)
    om = OracleModel(qm)
    seq = list(cfg.prompt())
    print(f"{cfg.name} D={D}", flush=True)
    for pos in range(cfg.prompt_len + cfg.decode_steps):
        want = om.forward(seq[pos], pos)
        got = rm.decode(seq[pos], pos).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{cfg.name} pos {pos}"
        if pos + 1 >= len(seq):
            seq.append(int(np.argmax(want)))
    n = len(seq) - 1
    kc, vc = kv_host(rm, n)
    assert np.array_equal(kc, om.kc[:, :n]) and np.array_equal(vc, om.vc[:, :n])
    rm.close()


@pytest.mark.parametrize("name", ["tiny", "tiny-qwen", "tiny-moe", "c1-stories15m"])
def test_prefill_equals_decode(name):
    """A prompt through t2r_prefill (all rows at once, and the reference's 16-row chunk schedule with
    its overlapping last chunk) gives the decode-only logits and KV cache bit for bit."""
    import t2r_amd.config as C
    cfg = C.get(name)
    qm, rm = resident(cfg, max_rows=64)
    toks = cfg.prompt() if cfg.prompt_len >= 8 else (cfg.prompt() * 8)[:min(cfg.seq_len, 20)]
    P = len(toks)
    for p, t in enumerate(toks):
        dec = rm.decode(t, p).cpu().numpy()
    kd = kv_host(rm, P)
    rm.reset()
    pre = rm.prefill(toks).cpu().numpy()
    assert sha(pre) == sha(dec)
    kp = kv_host(rm, P)
    assert np.array_equal(kp[0], kd[0]) and np.array_equal(kp[1], kd[1])
    if P > 8:
        rm.reset()
        ch = rm.prefill_chunks(toks, M=8).cpu().numpy()
        assert sha(ch) == sha(dec)
        kc = kv_host(rm, P)
        assert np.array_equal(kc[0], kd[0]) and np.array_equal(kc[1], kd[1])


def test_moe_grouped_prefill_many_routes():
    """The grouped MoE prefill (routes listed per expert, each expert's linears over its routes in
    groups of 32) with more routes than 32 per expert: 160 rows x 8 routes over 32 experts puts at
    least 33 on some expert in every layer, so second groups run. Prefill (one call, and 64-row
    chunks) gives the decode-only logits and KV cache bit for bit."""
    import t2r_amd.config as C
    cfg = C.C5.with_(name="c5-2l-160", layers=2, prompt_len=160)
    assert cfg.prompt_len * cfg.top_k > 32 * cfg.n_experts
    qm, rm = resident(cfg, max_rows=160)
    toks = cfg.prompt()
    P = len(toks)
    print(f"{cfg.name}: {P} rows", flush=True)
    for p, t in enumerate(toks):
        dec = rm.decode(t, p).cpu().numpy()
    kd = kv_host(rm, P)
    rm.reset()
    pre = rm.prefill(toks).cpu().numpy()
    assert sha(pre) == sha(dec)
    kp = kv_host(rm, P)
    assert np.array_equal(kp[0], kd[0]) and np.array_equal(kp[1], kd[1])
    rm.reset()
    ch = rm.prefill_chunks(toks, M=64).cpu().numpy()
    assert sha(ch) == sha(dec)
    rm.close()


def test_greedy_on_device_c1(gold):
    """The config-1 run as LlamaDevice.greedy_on_device does it (prefill, then argmax and pos += 1 on the
    device, no host round trip): the same 160 tokens as the reference's run."""
    import t2r_amd.config as C
    from t2r_amd.runtime import LlamaDevice
    run = next(r for r in gold["device_model"] if r["config"] == "c1-stories15m" and r["D"] == 16)
    cfg = C.get(run["config"])
    kv = np.array(run["kv_bits"], np.uint32).view(F).reshape(cfg.layers, 2)
    from t2r_amd import weights as W
    dev = LlamaDevice(W.QuantModel(cfg, kv_scales=kv), max_rows=64)
    toks = dev.greedy_on_device(run["prompt"], run["steps"])
    assert toks == run["tokens"]
    assert sha(*kv_host(dev.m, run["steps"])) == run["kv_sha"]
    dev.close()


def test_llamadevice_api():
    """forward() / generate() / reset() and the errors of llm/runtime.py:107-148."""
    import t2r_amd.config as C
    from t2r_amd.runtime import LlamaDevice
    dev = LlamaDevice(C.TINY)
    out = list(dev.generate([5, 6, 7], steps=10, stop_at_bos=False))
    assert len(out) == 10 and all(isinstance(t, int) for t, _ in out)
    again = list(dev.generate([5, 6, 7], steps=10, stop_at_bos=False))
    assert again == out                                                      # reset() restores the state
    dev.reset()
    for _ in range(C.TINY.seq_len):
        dev.forward(3)
    with pytest.raises(ValueError):
        dev.forward(3)
    forced = list(dev.generate(None, steps=6, forced=[1, 2, 3, 4]))
    assert len(forced) == 4 and forced[0][1].shape == (C.TINY.vocab,)
    dev.close()


@pytest.mark.parametrize("name", ["tiny-qwen", "c1-stories15m"])
def test_prefill_at_equals_prefill_with_positions(name):
    """t2r_prefill_at (positions start.., score rows sized by start + M) and t2r_prefill (positions
    passed in, score rows sized by the cache length) write the same KV rows and logits."""
    import torch
    import t2r_amd.config as C
    from t2r_amd import abi
    cfg = C.get(name)
    qm, rm = resident(cfg, max_rows=32)
    toks = (cfg.prompt() * 4)[:min(24, cfg.seq_len - 4)]
    M, start = len(toks) - 4, 4
    rm.reset()
    rm.prefill(toks[:start])
    rm.prefill(toks[start:], start=start)
    a_lg, a_k, a_v = rm.logits.cpu().numpy().copy(), rm.kc.cpu().numpy().copy(), rm.vc.cpu().numpy().copy()
    rm.reset()
    rm.prefill(toks[:start])
    rm.rows_tok[:M].copy_(torch.tensor(toks[start:], dtype=torch.int32))
    rm.rows_pos[:M].copy_(torch.arange(start, start + M, dtype=torch.int32))
    abi.check("t2r_prefill", rm.lib.t2r_prefill(rm.handle, abi.ptr(rm.rows_tok), abi.ptr(rm.rows_pos), M,
                                                abi.ptr(rm.logits), None, abi.stream_ptr()))
    assert np.array_equal(rm.logits.cpu().numpy().view(np.uint32), a_lg.view(np.uint32))
    assert np.array_equal(rm.kc.cpu().numpy(), a_k) and np.array_equal(rm.vc.cpu().numpy(), a_v)
    with pytest.raises(ValueError):
        rm.prefill([1] * 4, start=cfg.seq_len - 2)
    rm.close()


def test_status_word_and_token_range():
    """Token ids outside the vocabulary: the host calls refuse them (ValueError, as the reference's
    runtime raises for bad arguments); one that reaches the device anyway (through the step's device
    token) reads row 0 and sets bit 0 of the model's status word, which t2r_model_status reports and
    clears."""
    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = C.get("tiny-qwen")
    rm = ResidentModel(W.QuantModel(cfg), max_rows=8)
    with pytest.raises(ValueError):
        rm.decode(cfg.vocab, 0)
    with pytest.raises(ValueError):
        rm.prefill([1, -1, 3])
    with pytest.raises(ValueError):
        rm.decode_batch([2, cfg.vocab + 7], [0, 0], *rm.batch_caches(2))
    rm.decode(3, 0)
    assert rm.status() == 0
    rm.tok.fill_(cfg.vocab + 5)
    rm.pos.fill_(1)
    rm.step()
    assert rm.status() == 1
    assert rm.status() == 0
    rm.close()


@pytest.mark.parametrize("name", ["tiny-qwen", "c2-smollm2-135m"])
def test_prefill_graph_replays_equal_eager(name):
    """ResidentModel.capture_prefill: a HIP graph of one t2r_prefill_at call, replayed three times with eager
    work between the replays (the cache cleared, an eager decode step), each replay's last logits, greedy
    token and KV rows equal to the eager prefill's."""
    import torch
    import t2r_amd.config as C
    cfg = C.get(name)
    toks = cfg.prompt()[:40]
    qm, rm = resident(cfg, max_rows=len(toks))
    rm.reset()
    want = rm.prefill(toks).cpu().numpy().copy()
    nxt = int(rm.next.item())
    kv = kv_host(rm, len(toks))
    g = rm.capture_prefill(toks)
    for i in range(3):
        rm.reset()
        rm.logits.zero_()
        print(f"{name}: prefill graph replay {i}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        got = rm.logits.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {i}"
        assert int(rm.next.item()) == nxt
        a, b = kv_host(rm, len(toks))
        assert np.array_equal(a, kv[0]) and np.array_equal(b, kv[1])
        rm.decode(nxt, len(toks))                          # eager work between the replays
    assert rm.status() == 0
    rm.close()
