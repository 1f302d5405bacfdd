"""The measured shapes at full size (config 1 is covered by the reference
runs in test_gpu_model.py): the HIP datapath against the CPU restatement on the first positions,
bit for bit, and the long-context properties that need no CPU run (prefill == chunked prefill ==
decode-only, deterministic greedy streams up to T = 2048)."""
import hashlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = np.float32
FULL = ["c2-smollm2-135m", "c3-qwen3-0.6b", "c4-llama3.2-1b", "c5-granite-1b-a400m"]


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def build(name, max_rows=64):
    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = W.QuantModel(cfg)
    return cfg, qm, ResidentModel(qm, max_rows=max_rows)


@pytest.mark.parametrize("name", FULL)
def test_full_config_vs_oracle(name):
    """A 6-token prefill, then 3 greedy decode steps: logits of every step and the KV rows equal the
    CPU restatement's."""
    from oracle import OracleModel
    cfg, qm, rm = build(name)
    print(f"{name}: weights ready", flush=True)
    om = OracleModel(qm)
    toks = cfg.prompt()[:6]
    got = rm.prefill(toks).cpu().numpy()
    want = om.prefill(toks)
    assert sha(got) == sha(want), f"{name}: prefill logits differ"
    tok, pos = int(np.argmax(want)), len(toks)
    for _ in range(3):
        got = rm.decode(tok, pos).cpu().numpy()
        want = om.forward(tok, pos)
        assert sha(got) == sha(want), f"{name}: decode at {pos} differs"
        assert int(rm.next.item()) == int(np.argmax(want))
        tok, pos = int(np.argmax(want)), pos + 1
    assert np.array_equal(rm.kc[:, :pos].cpu().numpy(), om.kc[:, :pos])
    assert np.array_equal(rm.vc[:, :pos].cpu().numpy(), om.vc[:, :pos])
    rm.close()


def test_c3_long_context():
    """Config 3's 2032-token prompt: all rows in one prefill and the reference's 16-row chunk schedule
    (chunks at 0, 16, ..., 2016) give the same last-row logits and the same 2032 KV rows; the 16 greedy
    steps to T = 2048 then repeat exactly."""
    cfg, qm, rm = build("c3-qwen3-0.6b", max_rows=2048)
    prompt = cfg.prompt()
    P = len(prompt)
    full = rm.prefill(prompt).cpu().numpy()
    kv_full = (rm.kc[:, :P].cpu().numpy(), rm.vc[:, :P].cpu().numpy())
    rm.reset()
    chunked = rm.prefill_chunks(prompt, M=16).cpu().numpy()
    assert sha(chunked) == sha(full)
    assert np.array_equal(rm.kc[:, :P].cpu().numpy(), kv_full[0])
    assert np.array_equal(rm.vc[:, :P].cpu().numpy(), kv_full[1])
    streams = []
    for _ in range(2):
        rm.tok.copy_(rm.next)
        rm.pos.fill_(P)
        first = int(rm.next.item())
        out = [first]
        for _ in range(cfg.seq_len - P):
            rm.step(logits=False, advance=True)
            out.append(int(rm.tok.item()))
        streams.append(out)
        rm.reset()
        rm.prefill(prompt)
    assert streams[0] == streams[1] and len(streams[0]) == 17
    rm.close()


def test_c5_prefill_equals_decode():
    """MoE rows in one prefill equal the same rows fed one decode step at a time (routing, ordered expert
    combine and KV rows included)."""
    cfg, qm, rm = build("c5-granite-1b-a400m")
    toks = cfg.prompt()[:24]
    for p, t in enumerate(toks):
        dec = rm.decode(t, p).cpu().numpy()
    kd = rm.kc[:, :24].cpu().numpy()
    rm.reset()
    pre = rm.prefill(toks).cpu().numpy()
    assert sha(pre) == sha(dec)
    assert np.array_equal(rm.kc[:, :24].cpu().numpy(), kd)
    rm.close()
