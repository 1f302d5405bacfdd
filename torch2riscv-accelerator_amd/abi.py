"""ctypes binding of libt2r.so (include/t2r.h).

The library is built in-tree by t2r_amd.build (hipcc, gfx950). Loading it never falls back to
anything else: a missing or stale library raises here, and every call's status code becomes a
T2RError (ValueError for shape / range problems, RuntimeError for HIP errors), the exception
types the reference's runtime uses for the same conditions (llm/runtime.py:110-119).
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libt2r.so")

T2R_ABI_VERSION = 2
T2R_OK, T2R_EINVAL, T2R_ESHAPE, T2R_ERANGE, T2R_EHIP, T2R_ENOMEM, T2R_ESTATE = 0, -1, -2, -3, -4, -5, -6
T2R_ADVANCE_POS = 1
T2R_ATTN_QSUM = 1
T2R_STATIC_WORKSPACE_BYTES = 16 * 1024 * 1024
T2R_STATIC_STATE_BYTES = 512 * 1024

c_int, c_int64, c_uint64, c_float, c_void_p = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p
P = c_void_p    # every tensor argument is a raw device pointer


class T2RError(RuntimeError):
    def __init__(self, fn, code, msg):
        super().__init__(f"{fn}: {msg} (code {code})")
        self.code = code


class T2RShapeError(T2RError, ValueError):
    pass


class ModelDesc(ctypes.Structure):
    """t2r_model_desc (include/t2r.h); field order is the ABI."""
    _fields_ = [("abi_version", ctypes.c_int32)] + \
        [(n, ctypes.c_int32) for n in ("dim", "hidden", "layers", "heads", "kv_heads", "head_dim", "vocab", "seq_len",
                                       "n_experts", "top_k", "qk_norm", "D")] + \
        [("eps", c_float)] + \
        [(n, c_void_p) for n in ("emb_q", "emb_s", "cls_q", "cls_s", "rms_att", "rms_ffn", "rms_final", "q_norm",
                                 "k_norm", "wqkv", "s_wqkv", "wo", "s_wo", "w1", "s_w1", "w3", "s_w3", "w2", "s_w2",
                                 "router", "s_router", "wg", "s_wg", "wu", "s_wu", "wd", "s_wd", "rope_cos",
                                 "rope_sin", "kv_consts", "k_cache", "v_cache", "workspace")] + \
        [("workspace_bytes", c_int64), ("max_rows", ctypes.c_int32)] + \
        [("attn_qsum", ctypes.c_int32), ("ffn_act", ctypes.c_int32), ("kv_channel", c_void_p),
         ("kv_channel_flags", c_void_p)]


# name: (restype, argtypes)
_SIGS = {
    "t2r_abi_version": (c_int, []),
    "t2r_strerror": (ctypes.c_char_p, [c_int]),
    "t2r_init": (c_int, []),
    "t2r_sfu_tables": (c_int, [P]),
    "t2r_sfu": (c_int, [c_int, P, P, c_int64, P]),
    "t2r_sfu_check": (c_int, [c_int, c_uint64, c_uint64, P, P]),
    "t2r_fp32_op": (c_int, [c_int, P, P, P, c_int64, P]),
    "t2r_requant": (c_int, [P, c_int64, c_int, c_int, c_int, c_int, c_int, P, P]),
    "t2r_embed": (c_int, [P, P, P, c_int, c_int, c_int, P, P, P]),
    "t2r_rmsnorm": (c_int, [P, P, c_int, c_int, c_float, c_int, P, P]),
    "t2r_quant_act": (c_int, [P, c_int, c_int, P, P, P]),
    "t2r_gemv_w8a8": (c_int, [P, P, P, P, c_int, c_int, P, P, P, P]),
    "t2r_gemm_w8a8": (c_int, [P, P, P, P, c_int, c_int, c_int, P, P, P, P]),
    "t2r_rope": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, P]),
    "t2r_kv_append": (c_int, [P, P, c_float, c_float, P, P, P, c_int, c_int, c_int, P]),
    "t2r_kv_append_ch": (c_int, [P, P, c_float, c_float, P, P, P, P, P, c_int, c_int, c_int, P]),
    "t2r_attn_decode": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, c_float, c_int, P, P]),
    "t2r_attn_decode_opt": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, c_float, c_int, c_int, P, P,
                                    P, P]),
    "t2r_attn_prefill": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, c_float, c_int, c_int, P, P,
                                 P, P]),
    "t2r_swiglu_w8a8": (c_int, [P, P, P, P, P, P, c_int, c_int, P, P, P, P]),
    "t2r_gated_ffn_w8a8": (c_int, [c_int, P, P, P, P, P, P, c_int, c_int, P, P, P, P]),
    "t2r_moe_route": (c_int, [P, c_int, c_int, c_int, c_int, P, P, P]),
    "t2r_argmax": (c_int, [P, c_int, c_int, P, P]),
    "t2r_model_workspace_bytes": (c_int64, [ctypes.POINTER(ModelDesc), c_int]),
    "t2r_model_create": (c_int, [ctypes.POINTER(ModelDesc), ctypes.POINTER(c_void_p)]),
    "t2r_model_create_static": (c_int, [ctypes.POINTER(ModelDesc), ctypes.POINTER(c_void_p)]),
    "t2r_model_destroy": (None, [c_void_p]),
    "t2r_decode_step": (c_int, [c_void_p, P, P, P, P, c_int, P]),
    "t2r_prefill": (c_int, [c_void_p, P, P, c_int, P, P, P]),
    "t2r_prefill_at": (c_int, [c_void_p, P, c_int, c_int, P, P, P]),
    "t2r_decode_batch": (c_int, [c_void_p, P, P, c_int, P, P, c_int64, P, P, P]),
    "t2r_model_status": (c_int, [c_void_p, P, c_int]),
    "t2r_model_profile": (c_int, [c_void_p, c_int, c_int]),
    "t2r_model_profile_read": (c_int, [c_void_p, P, P, c_int]),
}
PROF_KINDS = ("qkv", "attn", "wo", "ffn_up", "ffn_down", "cls", "route", "other")
EXPORTS = tuple(_SIGS)

_lib = None


def load(path=LIB_PATH):
    """The library (loaded once). Raises if it is missing or its ABI version differs."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise OSError(f"{path} not built: run `python -m t2r_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if lib.t2r_abi_version() != T2R_ABI_VERSION:
        raise OSError(f"{path}: ABI version {lib.t2r_abi_version()}, expected {T2R_ABI_VERSION}")
    _lib = lib
    return lib


def check(fn, code):
    if code == T2R_OK:
        return
    msg = load().t2r_strerror(code).decode()
    if code in (T2R_ESHAPE, T2R_ERANGE, T2R_EINVAL):
        raise T2RShapeError(fn, code, msg)
    raise T2RError(fn, code, msg)


def call(name, *args):
    check(name, getattr(load(), name)(*args))


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else c_void_p(t.data_ptr())


def stream_ptr(stream=None):
    import torch
    s = torch.cuda.current_stream() if stream is None else stream
    return c_void_p(s.cuda_stream)
