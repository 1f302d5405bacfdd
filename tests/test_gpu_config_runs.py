"""Each measured config's stated workload on the HIP path against the CPU restatement's run of the same
workload (tests/golden/config_runs.json, written by tests/golden/make_config_runs.py): C2 a 40-token prompt
+ 256 greedy steps, C3 a 2032-token prompt in the reference's 16-row chunks (compiler/frontend/export.py:
69-72) + 16 steps up to T = 2048, C4 512 + 256, C5 64 + 256 (top-8 MoE, routing on the device). Bit-exact:
the prefill's last logits, every decode step's logits and greedy token, and the int8 KV cache; then the
same decode as one HIP graph of device-side greedy steps (the bench's form) ends on the same token and
cache."""
import hashlib
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
F = np.float32


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def runs():
    return json.load(open(os.path.join(HERE, "golden", "config_runs.json")))["runs"]


@pytest.mark.parametrize("name", ["c2-smollm2-135m", "c3-qwen3-0.6b", "c4-llama3.2-1b", "c5-granite-1b-a400m"])
def test_config_workload_vs_oracle(name):
    import torch
    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    rec = runs().get(name)
    if rec is None:
        pytest.skip(f"{name}: no fixture in config_runs.json")
    cfg = C.get(name)
    prompt = cfg.prompt()
    assert sha(np.array(prompt, np.int64)) == rec["prompt_sha"]
    P = len(prompt)
    chunked = P > 512                               # C3: the reference's 16-row chunk schedule
    rm = ResidentModel(W.QuantModel(cfg), max_rows=16 if chunked else P)
    print(f"{name}: prompt {P} ({'16-row chunks' if chunked else 'one call'}), "
          f"{len(rec['step_logits_sha'])} decode steps", flush=True)

    def prefill():
        rm.reset()
        return rm.prefill_chunks(prompt, M=16) if chunked else rm.prefill(prompt)

    lg = prefill().cpu().numpy()
    assert sha(lg) == rec["prefill_logits_sha"] and int(np.argmax(lg)) == rec["prefill_argmax"]
    tok, steps = rec["tokens"][0], len(rec["step_logits_sha"])
    for i in range(steps):
        lg = rm.decode(tok, P + i).cpu().numpy()
        assert sha(lg) == rec["step_logits_sha"][i], f"{name} step {i} (position {P + i})"
        tok = int(rm.next.item())
        assert tok == rec["step_argmax"][i] == int(np.argmax(lg))
    n = P + steps
    assert sha(rm.kc[:, :n].cpu().numpy(), rm.vc[:, :n].cpu().numpy()) == rec["kv_sha"]

    # the same decode as one HIP graph of device-side greedy steps
    prefill()
    rm.tok.copy_(rm.next)
    rm.pos.fill_(P)
    torch.cuda.synchronize()
    g = rm.capture_decode(steps)
    g.replay()
    torch.cuda.synchronize()
    assert int(rm.tok.item()) == rec["tokens"][-1] and int(rm.pos.item()) == n
    assert sha(rm.kc[:, :n].cpu().numpy(), rm.vc[:, :n].cpu().numpy()) == rec["kv_sha"]
    assert rm.status() == 0
    rm.close()
