"""Batched decode (t2r_decode_batch, BatchLlamaDevice): every live row is bit-identical to the same
token of its sequence decoded alone, logits and KV rows (the reference's L5b check,
llm/test_l5b.py:67-98: sequence b starts at step b, dummy BOS rows at pos 0 before that)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


# The full-size shapes run the grouped-query attention kernel (one workgroup per row and KV head):
# head dims 64 and 128, groups of 2, 3 and 4 query heads, QK-norm and MoE.
@pytest.mark.parametrize("name,B", [("tiny", 4), ("tiny-gqa", 3), ("tiny-qwen", 4), ("tiny-moe", 4),
                                    ("c1-stories15m", 8), ("c2-smollm2-135m", 4), ("c3-qwen3-0.6b", 3),
                                    ("c4-llama3.2-1b", 4), ("c5-granite-1b-a400m", 4),
                                    ("tiny-gqa", 40), ("c2-smollm2-135m", 36)])   # (33..64 rows: two row groups)
def test_decode_batch_equals_single(name, B):
    import torch
    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = W.QuantModel(cfg)
    rm = ResidentModel(qm, max_rows=B)
    rng = np.random.default_rng(5)
    steps = min(cfg.seq_len, 12)
    seqs = [rng.integers(0, cfg.vocab, steps + B).tolist() for _ in range(B)]
    kc, vc = rm.batch_caches(B)
    nxt = torch.zeros(B, dtype=torch.int32, device=rm.device)
    got = [[] for _ in range(B)]
    snap = [None] * B                                   # each slot's caches after its last live step
    print(f"{name}: B = {B}, {steps} positions per sequence", flush=True)
    for s in range(steps + B - 1):
        poses = [s - b if 0 <= s - b < steps else 0 for b in range(B)]
        live = [0 <= s - b < steps for b in range(B)]
        toks = [seqs[b][poses[b]] if live[b] else 1 for b in range(B)]
        lg = rm.decode_batch(toks, poses, kc, vc, next_tokens=nxt).cpu().numpy()
        nx = nxt.cpu().numpy()
        for b in range(B):
            if live[b]:
                got[b].append(lg[b].copy())
                assert nx[b] == int(np.argmax(lg[b]))
                if poses[b] == steps - 1:                 # (later dummy rows rewrite row 0 of the slot)
                    snap[b] = (kc[b, :, :steps].cpu().numpy(), vc[b, :, :steps].cpu().numpy())
    # each sequence alone through the single-row decode path (the model's own cache)
    for b in range(B):
        rm.reset()
        for p in range(steps):
            want = rm.decode(seqs[b][p], p).cpu().numpy()
            assert np.array_equal(got[b][p].view(np.uint32), want.view(np.uint32)), f"sequence {b} pos {p}"
        assert np.array_equal(snap[b][0], rm.kc[:, :steps].cpu().numpy())
        assert np.array_equal(snap[b][1], rm.vc[:, :steps].cpu().numpy())
    with pytest.raises(ValueError):
        rm.decode_batch([1] * (B + 1), [0] * (B + 1), kc, vc)
    rm.close()


def test_batch_llamadevice_generate():
    """BatchLlamaDevice.generate (staggered starts) gives each prompt the tokens LlamaDevice.generate
    gives it alone (greedy, BOS not stopping either)."""
    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.runtime import BatchLlamaDevice, LlamaDevice
    cfg = C.get("tiny-qwen")
    qm = W.QuantModel(cfg)
    prompts = [[1, 5, 9], [1, 7], [1, 3, 4, 5, 6], [1]]
    bd = BatchLlamaDevice(qm, slots=4)
    out = bd.generate(prompts, steps=14, stagger=2)
    one = LlamaDevice(qm)
    for p, o in zip(prompts, out):
        want = [p[0]] + [t for t, _ in one.generate(p, steps=14, stop_at_bos=False)]
        assert o == want[:14]
    seen = []
    bd.generate(prompts[:2], steps=3, on_logits=lambda b, pos, lg: seen.append((b, pos, lg.shape)))
    assert sorted((b, p) for b, p, _ in seen) == [(0, 0), (0, 1), (0, 2), (1, 0), (1, 1), (1, 2)]
    assert all(s == (cfg.vocab,) for _, _, s in seen)
    bd.close()
    one.close()


@pytest.mark.parametrize("name,lens", [("c4-llama3.2-1b", [40, 700, 1100]), ("c3-qwen3-0.6b", [33, 1500])])
def test_decode_batch_long_context(name, lens):
    """Sequences at positions past several 32-key tiles and past one 1024-key pass of the grouped
    attention: each slot's cache holds a prefilled prompt of its own length; one batched step equals
    each sequence's single decode at that position (logits and the new KV row)."""
    import torch
    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = W.QuantModel(cfg)
    B = len(lens)
    rm = ResidentModel(qm, max_rows=max(lens))
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in lens]
    nxt = [int(rng.integers(0, cfg.vocab)) for _ in lens]
    kc, vc = rm.batch_caches(B)
    for b, p in enumerate(prompts):
        rm.reset()
        rm.prefill(p, logits=False)
        kc[b].copy_(rm.kc)
        vc[b].copy_(rm.vc)
    print(f"{name}: positions {lens}", flush=True)
    got = rm.decode_batch(nxt, lens, kc, vc).cpu().numpy()
    for b, p in enumerate(prompts):
        rm.reset()
        rm.prefill(p, logits=False)
        want = rm.decode(nxt[b], lens[b]).cpu().numpy()
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), f"sequence {b} at {lens[b]}"
        assert torch.equal(kc[b, :, lens[b]], rm.kc[:, lens[b]])
        assert torch.equal(vc[b, :, lens[b]], rm.vc[:, lens[b]])
    rm.close()
