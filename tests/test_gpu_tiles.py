"""The prefill GEMM's tile shapes on ragged sizes: the 256-row SwiGLU / GeGLU tiles (M >= 256) and the
128-row tiles, with rows past M and gate columns past F in the last tiles (F = 16 mod 64). Logits and
every KV byte are checked against the CPU restatement, bit for bit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _cfg(hidden, act):
    import t2r_amd.config as C
    # dim 128: K % 128 == 0 sends Wqkv, Wo and W1 / W3 to the direct-to-LDS kernel; W2 (K = hidden)
    # takes the 64-byte slabs or the register-staged kernel
    return C.ModelConfig(f"tiny-tiles-{hidden}-{act}", dim=128, hidden=hidden, layers=2, heads=4, kv_heads=2,
                         head_dim=32, vocab=96, seq_len=512, theta=1e4, eps=1e-5, weight_std=None, gain_std=0.1,
                         emb_scale=4.0, seed_w=91 + hidden, seed_p=92, prompt_len=64, act=act).validate()


@pytest.mark.parametrize("M,hidden,act", [(300, 208, "silu"), (256, 144, "silu"), (257, 64, "gelu_tanh"),
                                          (200, 208, "silu"), (511, 336, "gelu_tanh")])
def test_prefill_ragged_tiles_vs_oracle(M, hidden, act):
    from oracle import OracleModel
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = _cfg(hidden, act)
    qm = W.QuantModel(cfg)
    rng = np.random.default_rng(M + hidden)
    toks = rng.integers(0, cfg.vocab, M).tolist()
    om = OracleModel(qm)
    want = om.prefill(toks)
    rm = ResidentModel(qm, max_rows=512)
    print(f"{cfg.name}: prefill {M} rows", flush=True)
    got = rm.prefill(toks).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(rm.kc[:, :M].cpu().numpy(), om.kc[:, :M])
    assert np.array_equal(rm.vc[:, :M].cpu().numpy(), om.vc[:, :M])
    rm.close()
