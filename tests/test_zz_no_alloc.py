"""t2r_model_create_static: a model whose workspace is the library's static device array (nothing
allocated by the call or by the caller beyond inputs and outputs) gives the results of the same model on a
caller-allocated workspace (t2r_model_create), bit for bit: two calls in a row, the second smaller, each
checked on logits and KV cache; and the entry point's rejections (a workspace given, max_rows beyond the
array)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def run(rm, toks, steps):
    """Prefill of toks, then `steps` greedy decode steps: (logits of each call, greedy tokens)."""
    rm.reset()
    out = [rm.prefill(toks).cpu().numpy().copy()]
    nxt = int(np.argmax(out[-1]))
    fed = []
    for p in range(len(toks), len(toks) + steps):
        fed.append(nxt)
        out.append(rm.decode(nxt, p).cpu().numpy().copy())
        nxt = int(np.argmax(out[-1]))
    return out, fed


@pytest.mark.parametrize("name,rows", [("tiny-qwen", 32), ("c4-llama3.2-1b", 64)])
def test_static_workspace_equals_allocated(name, rows):
    import t2r_amd.config as C
    from t2r_amd import abi
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = C.get(name)
    qm = W.QuantModel(cfg)
    ref = ResidentModel(qm, max_rows=rows)
    st = ResidentModel(qm, max_rows=rows, static_workspace=True)
    assert st.workspace is None and ref.workspace is not None
    rng = np.random.default_rng(17)
    for M in (rows, rows // 4):                       # two calls in a row, the second with a smaller input
        toks = rng.integers(0, cfg.vocab, M).tolist()
        print(f"{name}: prefill {M} rows + 3 decode steps", flush=True)
        want, fed_w = run(ref, toks, 3)
        got, fed_g = run(st, toks, 3)
        assert fed_w == fed_g
        for a, b in zip(got, want):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        n = M + 3
        assert np.array_equal(st.kc[:, :n].cpu().numpy(), ref.kc[:, :n].cpu().numpy())
        assert np.array_equal(st.vc[:, :n].cpu().numpy(), ref.vc[:, :n].cpu().numpy())
    st.close()
    ref.close()


def test_static_workspace_batched_and_rejections():
    import torch
    import t2r_amd.config as C
    from t2r_amd import abi
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = C.get("tiny-gqa")
    qm = W.QuantModel(cfg)
    ref = ResidentModel(qm, max_rows=4)
    st = ResidentModel(qm, max_rows=4, static_workspace=True)
    for B in (4, 2):
        kc, vc = st.batch_caches(B)
        kr, vr = ref.batch_caches(B)
        toks, poses = [3, 9, 11, 5][:B], [0] * B
        a = st.decode_batch(toks, poses, kc, vc).cpu().numpy()
        b = ref.decode_batch(toks, poses, kr, vr).cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert torch.equal(kc, kr) and torch.equal(vc, vr)
    # a workspace given: EINVAL; max_rows needing more than the array: ENOMEM
    lib = abi.load()
    d = abi.ModelDesc.from_buffer_copy(bytes(ref.desc))
    h = ctypes.c_void_p()
    assert lib.t2r_model_create_static(ctypes.byref(d), ctypes.byref(h)) == abi.T2R_EINVAL
    d.workspace, d.workspace_bytes = None, 0
    big = C.get("c4-llama3.2-1b")
    rows = 512
    d2 = abi.ModelDesc.from_buffer_copy(bytes(d))
    d2.dim, d2.hidden, d2.layers, d2.heads, d2.kv_heads, d2.head_dim = big.dim, big.hidden, 1, big.heads, \
        big.kv_heads, big.head_dim
    d2.vocab, d2.max_rows = big.vocab, rows
    assert lib.t2r_model_workspace_bytes(ctypes.byref(d2), rows) > abi.T2R_STATIC_WORKSPACE_BYTES
    assert lib.t2r_model_create_static(ctypes.byref(d2), ctypes.byref(h)) == abi.T2R_ENOMEM
    st.close()
    ref.close()


def c3_small():
    """C3's attention shape (head dim 128, QK-norm) with a 640-row cache, so that batch-1 decode splits
    each head's keys over workgroups and carries counters from call to call; small elsewhere."""
    import t2r_amd.config as C
    return C.C3.with_(name="c3-small", dim=256, hidden=256, layers=2, heads=4, kv_heads=2, vocab=512, seq_len=640,
                      seed_w=911, seed_p=912, prompt_len=530, weight_std=None, gain_std=0.1, emb_scale=4.0)


def test_two_static_models_interleaved():
    """Two static models of different max_rows alive at once (each handle keeps its carried state, the
    status word and the split attention's counters, in its own part of the array; the rest is shared
    scratch), their calls interleaved: prefills in their own chunk sizes, then decode steps in turn, each
    equal bit for bit to an allocated model doing the same; no status bit set."""
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = c3_small()
    qm = W.QuantModel(cfg)
    rng = np.random.default_rng(5)
    prompts = [cfg.prompt(), rng.integers(0, cfg.vocab, 522).tolist()]
    rows = (64, 16)
    st = [ResidentModel(qm, max_rows=r, static_workspace=True) for r in rows]
    ref = [ResidentModel(qm, max_rows=r) for r in rows]
    outs = {0: [], 1: []}
    for k in (0, 1):
        print(f"static model {k} (max_rows {rows[k]}): prefill {len(prompts[k])} rows", flush=True)
        a = st[k].prefill(prompts[k]).cpu().numpy().copy()
        b = ref[k].prefill(prompts[k]).cpu().numpy().copy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        outs[k].append(int(np.argmax(b)))
    for i in range(3):
        for k in (0, 1):
            p = len(prompts[k]) + i
            print(f"static model {k}: decode pos {p}", flush=True)
            a = st[k].decode(outs[k][-1], p).cpu().numpy().copy()
            b = ref[k].decode(outs[k][-1], p).cpu().numpy().copy()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"model {k} pos {p}"
            outs[k].append(int(np.argmax(b)))
    for k in (0, 1):
        n = len(prompts[k]) + 3
        assert np.array_equal(st[k].kc[:, :n].cpu().numpy(), ref[k].kc[:, :n].cpu().numpy())
        assert st[k].status() == 0 and ref[k].status() == 0
    for m in st + ref:
        m.close()


def test_static_create_allocates_nothing():
    """t2r_model_create_static leaves the device's free memory unchanged (after one warm-up creation, which
    may set up the runtime's own state)."""
    import torch
    import t2r_amd.config as C
    from t2r_amd import abi
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    qm = W.QuantModel(C.get("tiny-qwen"))
    ref = ResidentModel(qm, max_rows=8)
    lib = abi.load()
    d = abi.ModelDesc.from_buffer_copy(bytes(ref.desc))
    d.workspace, d.workspace_bytes = None, 0
    for i in range(2):
        h = ctypes.c_void_p()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        abi.check("t2r_model_create_static", lib.t2r_model_create_static(ctypes.byref(d), ctypes.byref(h)))
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        lib.t2r_model_destroy(h)
        if i == 1:
            assert free1 == free0, f"creation took {free0 - free1} bytes of device memory"
    ref.close()
