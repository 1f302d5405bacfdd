"""Batched decode (t2r_decode_batch) against the CPU restatement, row by row: each slot's cache holds the
oracle's prefill of a prompt of its own length, one batched step runs every slot at its position, and
every row's logits and new KV row equal OracleModel.forward on that slot's cache. The shapes reach every
instantiation of the grouped-query attention kernel (k_attn_gqa<hd/16, OPT, GW>): head dims 64 and 128,
groups of 2, 3 and 4 query heads (four-head groups take two heads per workgroup), with and without the HF
options, K and V per channel among them."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def shape(name):
    import t2r_amd.config as C
    # hd 128 with four-head groups (no measured config has it): C3's shape with 4 KV heads, 4 layers
    g4 = C.C3.with_(name="c3-g4", kv_heads=4, layers=4, prompt_len=64)
    table = {
        "c4-llama3.2-1b": C.C4,                                            # hd 64, G 4: <4, false, 2>
        "c2-smollm2-135m": C.C2,                                           # hd 64, G 3: <4, false, 1>
        "c3-qwen3-0.6b": C.C3,                                             # hd 128, G 2: <8, false, 1>
        "c3-g4": g4,                                                       # hd 128, G 4: <8, false, 2>
        "c4-llama3.2-1b-hf": C.hf_options(C.C4),                           # <4, true, 2>: qsum, K per channel
        "c3-g4-hf": C.hf_options(g4),                                      # <8, true, 2>
        "c2-kv": C.C2.with_(name="c2-kv", kv_channel="kv", layers=6),      # <4, true, 1>: K and V per channel
        "c4-v": C.C4.with_(name="c4-v", kv_channel="v", attn_norm="qsum", layers=4),   # <4, true, 2>: V per channel
    }
    return table[name]


@pytest.mark.parametrize("name,lens", [("c4-llama3.2-1b", [5, 37, 70, 100]), ("c2-smollm2-135m", [3, 40, 66]),
                                       ("c3-qwen3-0.6b", [9, 50]), ("c3-g4", [7, 33, 64]),
                                       ("c4-llama3.2-1b-hf", [6, 45]), ("c3-g4-hf", [12, 40]),
                                       ("c2-kv", [4, 31, 57]), ("c4-v", [8, 65])])
def test_decode_batch_rows_vs_oracle(name, lens):
    import torch
    from oracle import OracleModel
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    import t2r_amd.config as C
    cfg = shape(name)
    # the measured configs' recorded KV scales; the others calibrated on 32 prompt tokens (per channel
    # where the config says)
    kv = None if cfg.name in C.CONFIGS else W.calibrate_kv(cfg, tokens=cfg.prompt()[:32])
    qm = W.QuantModel(cfg, kv_scales=kv)
    om = OracleModel(qm)
    B = len(lens)
    rng = np.random.default_rng(31)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in lens]
    nxt = [int(rng.integers(0, cfg.vocab)) for _ in lens]
    rm = ResidentModel(qm, max_rows=B)
    kc, vc = rm.batch_caches(B)
    want, rows = [], []
    for b, p in enumerate(prompts):
        om.reset()
        om.prefill(p)
        kc[b].copy_(torch.from_numpy(om.kc))
        vc[b].copy_(torch.from_numpy(om.vc))
        want.append(om.forward(nxt[b], lens[b]))
        rows.append((om.kc[:, lens[b]].copy(), om.vc[:, lens[b]].copy()))
    print(f"{name}: B = {B} at positions {lens}", flush=True)
    got = rm.decode_batch(nxt, lens, kc, vc).cpu().numpy()
    for b in range(B):
        assert np.array_equal(got[b].view(np.uint32), want[b].view(np.uint32)), f"{name} row {b} at {lens[b]}"
        assert np.array_equal(kc[b, :, lens[b]].cpu().numpy(), rows[b][0]), f"K row {b}"
        assert np.array_equal(vc[b, :, lens[b]].cpu().numpy(), rows[b][1]), f"V row {b}"
    rm.close()
