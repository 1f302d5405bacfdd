#!/usr/bin/env python3
"""Writes tests/golden/config_runs.json: each measured config's stated workload (C2 a
40-token prompt + 256 decode steps, C3 2032 + 16 (the decode at T -> 2048), C4 512 + 256, C5 64 + 256;
C1's 32 + 128 run is the reference's own fixture, model_golden.json) run through the CPU restatement
(oracle/): the prompt prefilled, then greedy decode (first maximal index, no stop token).

Per config: the prompt, the generated tokens, sha256 of the prefill's last-row logits and of every decode
step's logits (fp32 bits), each step's argmax, and sha256 of the int8 KV cache rows written. The GPU test
(tests/test_gpu_config_runs.py) replays the same workload on the HIP path and compares all of them.

    python3 tests/golden/make_config_runs.py [--only c2 c3 c4 c5]
"""
import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
F = np.float32

RUNS = {"c2": "c2-smollm2-135m", "c3": "c3-qwen3-0.6b", "c4": "c4-llama3.2-1b", "c5": "c5-granite-1b-a400m"}


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def run(name):
    import t2r_amd.config as C
    from oracle import OracleModel
    from t2r_amd import weights as W
    cfg = C.get(name)
    t0 = time.time()
    qm = W.QuantModel(cfg)
    om = OracleModel(qm)
    prompt = cfg.prompt()
    P, steps = len(prompt), cfg.decode_steps
    # the prompt in chunks of at most 512 rows (each row a decode step at its position, so the chunking
    # changes nothing; it bounds the oracle's memory)
    lg = None
    for s in range(0, P, 512):
        lg = om.prefill(prompt[s:s + 512], start=s)
    rec = {"config": name, "prompt_len": P, "decode_steps": steps, "prompt_sha": sha(np.array(prompt, np.int64)),
           "prefill_logits_sha": sha(np.asarray(lg, F)), "prefill_argmax": int(np.argmax(lg))}
    print(f"{name}: prefill of {P} rows in {time.time() - t0:.0f} s", flush=True)
    tok = int(np.argmax(lg))
    gen, shas, arg = [tok], [], []
    for i in range(steps):
        pos = P + i
        if pos >= cfg.seq_len:
            break
        lg = np.asarray(om.forward(tok, pos), F)
        shas.append(sha(lg))
        tok = int(np.argmax(lg))
        arg.append(tok)
        gen.append(tok)
        if (i + 1) % 32 == 0:
            print(f"  {name}: {i + 1} decode steps, {time.time() - t0:.0f} s", flush=True)
    n = P + len(shas)
    rec.update({"tokens": gen, "step_logits_sha": shas, "step_argmax": arg,
                "kv_sha": sha(om.kc[:, :n], om.vc[:, :n]), "seconds": round(time.time() - t0, 1)})
    print(f"{name}: {len(shas)} decode steps, {rec['seconds']} s", flush=True)
    return rec


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--only", nargs="*")
    args = ap.parse_args()
    path = os.path.join(HERE, "config_runs.json")
    out = json.load(open(path)) if os.path.exists(path) else {"generator": "tests/golden/make_config_runs.py",
                                                                "runs": {}}
    for key in (args.only or list(RUNS)):
        out["runs"][RUNS[key]] = run(RUNS[key])
        json.dump(out, open(path, "w"), indent=0)


if __name__ == "__main__":
    main()
