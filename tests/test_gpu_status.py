"""The device status word and the reference's failure contract at the Python boundary, and the split
decode attention's carried state.

- llm/runtime.py:118-119 raises RuntimeError(f"pos {pos}: list failed, status {s:#x}") when a list ends
  with a non-zero status, and BatchLlamaDevice.step (:202-203) RuntimeError(f"step failed, status ...").
  Here the status word is the model's (t2r_model_status): bit 0 a token outside the vocabulary reached the
  embedding, bit 2 a row's position was outside the cache. Both conditions are forced from the host through
  the raw C-ABI (the Python wrappers refuse them), and every kernel still ends normally: the embedding reads
  row 0 instead, the attention kernels end at once.
- The split decode attention (head dim 128, caches over 512 rows) keeps per-head counters and, for layers
  with the HF options, int32 sums from launch to launch; a model whose layers mix both forms (per-layer and
  per-channel KV scales, qsum off) is checked against the oracle past 512 positions.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = np.float32


def c3_small(**kw):
    """A C3-shaped model small enough for the oracle: head dim 128 with QK-norm, a 640-row cache (so the
    batch-1 decode attention splits each head's keys over workgroups), 2 layers."""
    import t2r_amd.config as C
    base = dict(name="c3-small", dim=256, hidden=256, layers=2, heads=4, kv_heads=2, vocab=512, seq_len=640,
                seed_w=901, seed_p=902, prompt_len=520, weight_std=None, gain_std=0.1, emb_scale=4.0)
    base.update(kw)
    return C.C3.with_(**base)


def test_forward_raises_on_status_then_recovers():
    import t2r_amd.config as C
    from t2r_amd.runtime import LlamaDevice
    dev = LlamaDevice(C.TINY)
    m = dev.m
    assert m.status() == 0
    # a raw step with a token outside the vocabulary: embedded as row 0, status bit 0, no fault
    m.tok.fill_(C.TINY.vocab + 5)
    m.pos.fill_(0)
    m.step()
    print("forward after an out-of-vocab raw step", flush=True)
    with pytest.raises(RuntimeError, match=r"pos 0: list failed, status 0x1"):
        dev.forward(3)
    # the word was cleared with the report: the next positions run clean and match a fresh device
    ref = LlamaDevice(C.TINY)
    dev.reset()
    for t in (3, 9, 1):
        a, b = dev.forward(t), ref.forward(t)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert m.status() == 0
    dev.close()
    ref.close()


def test_position_outside_cache_sets_bit2():
    import t2r_amd.config as C
    from t2r_amd.runtime import LlamaDevice
    cfg = C.TINY
    dev = LlamaDevice(cfg)
    m = dev.m
    m.tok.fill_(3)
    m.pos.fill_(cfg.seq_len)              # one past the cache: the attention kernels write nothing
    m.step()
    assert m.status(clear=False) == 4
    assert not m.kc.any().item() and not m.vc.any().item()     # nothing written anywhere
    dev.pos = 2
    print("forward after a raw step past the cache", flush=True)
    with pytest.raises(RuntimeError, match=r"pos 2: list failed, status 0x4"):
        dev.forward(5)
    assert m.status() == 0
    dev.close()


def test_batch_step_raises_on_status():
    import t2r_amd.config as C
    from t2r_amd import abi
    from t2r_amd.runtime import BatchLlamaDevice
    cfg = C.TINY_GQA
    bd = BatchLlamaDevice(cfg, slots=4)
    m = bd.m
    torch = m.torch
    toks = torch.tensor([3, cfg.vocab, 5, 7], dtype=torch.int32, device=m.device)   # row 1 out of range
    poses = torch.zeros(4, dtype=torch.int32, device=m.device)
    out = torch.empty((4, cfg.vocab), dtype=torch.float32, device=m.device)
    abi.check("t2r_decode_batch", m.lib.t2r_decode_batch(
        m.handle, abi.ptr(toks), abi.ptr(poses), 4, abi.ptr(bd.kc), abi.ptr(bd.vc), bd.kc[0].numel(),
        abi.ptr(out), None, abi.stream_ptr()))
    print("batched step after an out-of-vocab raw batch", flush=True)
    with pytest.raises(RuntimeError, match=r"step failed, status 0x1"):
        bd.step([0, 0, 0, 0], [3, 4, 5, 7])
    bd.step([1, 1, 1, 1], [3, 4, 5, 7])   # clean again
    bd.close()


def test_split_attention_mixed_kv_forms_against_oracle():
    """Layer 0 with per-layer KV scales (the split's sums handed to Wo), layer 1 with K and V per channel
    (the HF instantiation, its sums met by device atomics): decode at positions 520.. against the oracle."""
    from oracle import OracleModel
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = c3_small(kv_channel="kv")
    kv = W.calibrate_kv(cfg)                                  # (L, 2, kv_dim)
    kv[0] = kv[0].max(-1, keepdims=True)                      # layer 0: one value per row -> per layer
    qm = W.QuantModel(cfg, kv_scales=kv)
    assert list(qm.kv_flags) == [0, 3]
    rm = ResidentModel(qm, max_rows=64)
    om = OracleModel(qm)
    toks = cfg.prompt()
    print(f"{cfg.name}: prefill {len(toks)} rows", flush=True)
    got = rm.prefill(toks).cpu().numpy()
    want = om.prefill(toks)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    nxt = int(np.argmax(want))
    for p in range(len(toks), len(toks) + 4):
        print(f"{cfg.name}: decode pos {p}", flush=True)
        got = rm.decode(nxt, p).cpu().numpy()
        want = om.forward(nxt, p)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"pos {p}"
        nxt = int(np.argmax(want))
    n = len(toks) + 4
    assert np.array_equal(rm.kc[:, :n].cpu().numpy(), om.kc[:, :n])
    assert np.array_equal(rm.vc[:, :n].cpu().numpy(), om.vc[:, :n])
    assert rm.status() == 0
    rm.close()
