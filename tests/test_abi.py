"""The C-ABI library without a GPU: it loads, exports every function include/t2r.h declares,
rejects bad arguments with the documented codes before touching a device, and sizes workspaces.
Also the host-side model data (configs, weights, KV constants)."""
import ctypes
import os
import re

import numpy as np
import pytest

import t2r_amd.config as C
from t2r_amd import abi
from t2r_amd import weights as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "t2r.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(t2r_\w+)\s*\(", text)))


def test_library_exports_header():
    lib = abi.load()
    names = header_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(abi.EXPORTS) == names
    assert lib.t2r_abi_version() == abi.T2R_ABI_VERSION


def test_strerror_codes():
    lib = abi.load()
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert lib.t2r_strerror(code)
    assert b"XERR_SHAPE" in lib.t2r_strerror(abi.T2R_ESHAPE)


def test_argument_validation_before_launch():
    """Shape and pointer checks return before any HIP call (SaError's XERR_SHAPE / XERR_RANGE,
    llm/sa_funcsim.py:26-31), so they are testable without a device."""
    lib = abi.load()
    p = ctypes.c_void_p(16)
    assert lib.t2r_gemv_w8a8(None, p, p, p, 16, 16, p, None, None, None) == abi.T2R_EINVAL
    assert lib.t2r_gemv_w8a8(p, p, p, p, 16, 24, p, None, None, None) == abi.T2R_ESHAPE     # K % 16
    assert lib.t2r_gemv_w8a8(p, p, p, p, 16, 16384, p, None, None, None) == abi.T2R_ESHAPE  # K > 8192
    assert lib.t2r_gemm_w8a8(p, p, p, p, 0, 16, 16, p, None, None, None) == abi.T2R_ESHAPE
    assert lib.t2r_quant_act(p, 1, 20, p, p, None) == abi.T2R_ESHAPE
    assert lib.t2r_rmsnorm(p, p, 1, 64, 1e-5, 4, p, None) == abi.T2R_ESHAPE                 # D
    assert lib.t2r_rope(p, p, p, p, 1, 30, 8, 16, None) == abi.T2R_ESHAPE
    assert lib.t2r_moe_route(p, 1, 32, 9, 16, p, p, None) == abi.T2R_ESHAPE                  # k > 8
    assert lib.t2r_requant(p, 4, 1, 40, 0, 0, 1, p, None) == abi.T2R_ERANGE                 # shift
    assert lib.t2r_sfu(7, p, p, 4, None) == abi.T2R_EINVAL
    assert lib.t2r_model_create(None, ctypes.byref(ctypes.c_void_p())) == abi.T2R_EINVAL
    d = abi.ModelDesc()
    d.abi_version = 99
    assert lib.t2r_model_create(ctypes.byref(d), ctypes.byref(ctypes.c_void_p())) == abi.T2R_EINVAL
    with pytest.raises(ValueError):
        abi.check("t2r_gemv_w8a8", abi.T2R_ESHAPE)
    with pytest.raises(RuntimeError):
        abi.check("t2r_decode_step", abi.T2R_EHIP)


def _desc(cfg, max_rows):
    d = abi.ModelDesc()
    d.abi_version = abi.T2R_ABI_VERSION
    d.dim, d.hidden, d.layers, d.heads, d.kv_heads = cfg.dim, cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads
    d.head_dim, d.vocab, d.seq_len, d.n_experts, d.top_k = cfg.head_dim, cfg.vocab, cfg.seq_len, cfg.n_experts, cfg.top_k
    d.D, d.max_rows = cfg.D, max_rows
    return d


def test_workspace_bytes_scale_with_rows():
    lib = abi.load()
    for cfg in C.CONFIGS.values():
        one = lib.t2r_model_workspace_bytes(ctypes.byref(_desc(cfg, 1)), 1)
        many = lib.t2r_model_workspace_bytes(ctypes.byref(_desc(cfg, 512)), 512)
        assert one > 4 * cfg.vocab and many > one
        # x, qkv, att, u rows in fp32 plus int8 rows: at least 512 * 4 * (dim + q + 2 kv + q + F) bytes
        ffn = cfg.top_k * cfg.hidden if cfg.moe else cfg.hidden
        assert many >= 512 * 4 * (cfg.dim + 2 * cfg.q_dim + 2 * cfg.kv_dim + ffn)


def test_config_shapes():
    assert C.C4.weight_bytes_per_token() == 1_235_746_816
    assert round(C.C3.weight_bytes_per_token() / 1e6, 2) == 595.98
    assert round(C.C5.weight_bytes_per_token() / 1e6, 2) == 428.61
    assert C.C3.q_dim == 2048 and C.C3.dim == 1024
    with pytest.raises(ValueError):
        C.C1.with_(kv_heads=4)                                             # 6 heads, 4 KV heads
    with pytest.raises(KeyError):
        C.get("c9")


def test_weights_deterministic_and_quantised():
    cfg = C.TINY_QWEN
    a, b = W.fp32_tensor(cfg, "wq", 1), W.fp32_tensor(cfg, "wq", 1)
    assert np.array_equal(a, b) and not np.array_equal(a, W.fp32_tensor(cfg, "wq", 0))
    q, s = W.quantize_rows(a)
    assert q.dtype == np.int8 and np.abs(q).max() == 127
    assert np.array_equal(np.abs(q).max(axis=1), np.full(a.shape[0], 127))
    with np.errstate(all="ignore"):
        assert np.all(np.abs(q.astype(np.float32) * s[:, None] - a) <= s[:, None] * 0.5 + 1e-9)
    z, sz = W.quantize_rows(np.zeros((2, 16), np.float32))                  # an all-zero row: s = 0, q = 0
    assert not z.any() and not sz.any()


def test_kv_scales_recorded_for_every_config():
    for cfg in C.CONFIGS.values():
        kv = W.stored_kv_scales(cfg)
        assert kv.shape == (cfg.layers, 2) and np.all(kv > 0) and np.all(np.isfinite(kv))
    kvc = W.kv_constants(C.C4, W.stored_kv_scales(C.C4))
    sk, sv = W.stored_kv_scales(C.C4)[0]
    assert kvc[0, 2] == np.float32(float(sk) / 8.0) and kvc[0, 3] == np.float32(float(sv) / 127.0)


def test_hf_option_validation_before_launch():
    """The HF-path options: bad flags / activations are refused before any HIP call; the ABI-2 model
    descriptor's option fields are validated before the device is touched (a valid descriptor only then
    fails, here, at device initialisation: no GPU), and an ABI-1 descriptor's bytes past max_rows are
    ignored (read with the options off)."""
    import numpy as np
    lib = abi.load()
    p = ctypes.c_void_p(16)
    assert lib.t2r_attn_decode_opt(p, p, p, p, 1, 4, 2, 16, 32, 0.1, 0.1, 16, 2, None, None, p, None) == abi.T2R_EINVAL
    assert lib.t2r_gated_ffn_w8a8(2, p, p, p, p, p, p, 64, 64, p, p, p, None) == abi.T2R_EINVAL
    assert lib.t2r_gated_ffn_w8a8(1, p, p, p, p, p, p, 24, 64, p, p, p, None) == abi.T2R_ESHAPE     # F % 16
    assert lib.t2r_kv_append_ch(p, p, 1.0, 1.0, None, None, p, p, p, 0, 64, 16, None) == abi.T2R_ESHAPE
    import torch
    if torch.cuda.device_count() > 0:                      # (counting devices does not initialise them)
        pytest.skip("the descriptor cases rely on device initialisation failing: no GPU may be visible")
    cfg = C.TINY_QWEN
    flags = np.zeros(cfg.layers, np.int32)

    def full(version, **opt):
        d = _desc(cfg, 4)
        d.abi_version = version
        d.qk_norm, d.eps = 1, 1e-6
        for n in ("emb_q", "emb_s", "cls_q", "cls_s", "rms_att", "rms_ffn", "rms_final", "q_norm", "k_norm", "wqkv",
                  "s_wqkv", "wo", "s_wo", "w1", "s_w1", "w3", "s_w3", "w2", "s_w2", "rope_cos", "rope_sin",
                  "kv_consts", "k_cache", "v_cache", "workspace"):
            setattr(d, n, 16)
        d.workspace_bytes = 1 << 40
        for k, v in opt.items():
            setattr(d, k, v)
        return lib.t2r_model_create(ctypes.byref(d), ctypes.byref(ctypes.c_void_p()))
    assert full(2) == abi.T2R_EHIP                                          # valid: only the device is missing
    assert full(2, attn_qsum=2) == abi.T2R_EINVAL
    assert full(2, ffn_act=3) == abi.T2R_EINVAL
    flags[1] = 4
    assert full(2, kv_channel=16, kv_channel_flags=flags.ctypes.data) == abi.T2R_EINVAL   # unknown flag bit
    flags[1] = 1
    assert full(2, kv_channel_flags=flags.ctypes.data) == abi.T2R_EINVAL                  # per channel, no table
    assert full(2, kv_channel=16, kv_channel_flags=flags.ctypes.data) == abi.T2R_EHIP
    assert full(1, attn_qsum=7, ffn_act=9, kv_channel_flags=16) == abi.T2R_EHIP           # ABI 1: options off
    v1 = _desc(cfg, 4)
    v1.abi_version = 1
    v1.attn_qsum = 7
    assert lib.t2r_model_workspace_bytes(ctypes.byref(v1), 4) == lib.t2r_model_workspace_bytes(
        ctypes.byref(_desc(cfg, 4)), 4)
