"""ctypes binding of libattnnn.so (declarations in include/attnnn.h).

The library is required: if it is missing or fails to load, every entry
point raises -- there is no CPU fallback on the product path.
"""

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libattnnn.so")

ANN_OK = 0
ANN_E_ARG = -1
ANN_E_STATE = -2
ANN_E_CAPACITY = -3
ANN_E_HIP = -4
ANN_MAX_LONG_LAYERS = 8
DTYPE_F32 = 0
DTYPE_BF16 = 1


class AnnConfig(ctypes.Structure):
    _fields_ = [("d", ctypes.c_int32), ("L", ctypes.c_int32), ("H", ctypes.c_int32),
                ("V", ctypes.c_int32), ("V_sample", ctypes.c_int32), ("window", ctypes.c_int32),
                ("n_long", ctypes.c_int32),
                ("long_layers", ctypes.c_int32 * ANN_MAX_LONG_LAYERS),
                ("attn_scale", ctypes.c_float), ("rope_base", ctypes.c_float),
                ("rms_eps", ctypes.c_float), ("max_batch", ctypes.c_int32),
                ("max_ctx", ctypes.c_int32), ("max_tokens", ctypes.c_int32)]


class AnnParamsF32(ctypes.Structure):
    _fields_ = [(k, ctypes.c_void_p) for k in (
        "embed", "lm_head", "attn_bank", "fc_bank", "proj_bank",
        "resid_lambdas", "post_lambdas", "x0_lambdas", "sa_lambdas")]


class AnnSampling(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32),
                ("seed", ctypes.c_uint64), ("step", ctypes.c_uint64)]


_P = ctypes.c_void_p
_I = ctypes.c_int32
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); every symbol include/attnnn.h declares.
SIGNATURES = {
    "ann_last_error": (ctypes.c_char_p, []),
    "ann_version": (ctypes.c_int, []),
    "ann_create": (ctypes.c_int, [ctypes.POINTER(AnnConfig), ctypes.POINTER(_P)]),
    "ann_destroy": (None, [_P]),
    "ann_weight_bytes": (_SZ, [ctypes.POINTER(AnnConfig)]),
    "ann_kv_bytes": (_SZ, [ctypes.POINTER(AnnConfig)]),
    "ann_workspace_bytes": (_SZ, [ctypes.POINTER(AnnConfig)]),
    "ann_pack_weights": (ctypes.c_int, [_P, ctypes.POINTER(AnnParamsF32), _P, _SZ, _P]),
    "ann_bind": (ctypes.c_int, [_P, _P, _SZ, _P, _SZ, _P, _SZ]),
    "ann_reset": (ctypes.c_int, [_P]),
    "ann_forward_logits": (ctypes.c_int, [_P, _P, _I, _I, _P, _P]),
    "ann_forward_loss": (ctypes.c_int, [_P, _P, _P, _I, _I, _P, _P, _P]),
    "ann_prefill": (ctypes.c_int, [_P, _P, _I, _I, ctypes.POINTER(AnnSampling), _P, _P, _P]),
    "ann_decode_step": (ctypes.c_int, [_P, _P, _I, ctypes.POINTER(AnnSampling), _P, _P, _P]),
    "ann_context_length": (ctypes.c_int, [_P]),
    "ann_op_relu2": (ctypes.c_int, [_P, _P, _SZ, _I, _P]),
    "ann_op_rope_ht": (ctypes.c_int, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "ann_op_rope_tables": (ctypes.c_int, [_P, _P, _I, _I, ctypes.c_float, _P]),
    "ann_op_rms_norm": (ctypes.c_int, [_P, _P, _I, _I, ctypes.c_float, _I, _P]),
    "ann_op_adam_step": (ctypes.c_int, [_P, _P, _P, _P, _SZ, _F, _F, _F, _F, _F, _P, _P, _P, _P]),
    "ann_op_muon_momentum": (ctypes.c_int, [_P, _P, _SZ, _F, _P, _P, _P]),
    "ann_op_muon_apply": (ctypes.c_int, [_P, _P, _SZ, _F, _F, _P, _P]),
    "ann_op_polar_express_ws_bytes": (ctypes.c_size_t, [_I, _I, _I]),
    "ann_op_polar_express": (ctypes.c_int, [_P, _I, _I, _I, _P, _P, _SZ, _P]),
    "ann_op_normuon_ws_bytes": (ctypes.c_size_t, [_I, _I, _I]),
    "ann_op_normuon": (ctypes.c_int, [_P, _P, _I, _I, _I, _F, _P, _P, _SZ, _P]),
    "ann_op_normuon_noalloc_max_bytes": (ctypes.c_size_t, []),
    "ann_op_normuon_noalloc": (ctypes.c_int, [_P, _P, _I, _I, _I, _F, _P, _P]),
    "ann_profile_enable": (ctypes.c_int, [_P, _I, _I]),
    "ann_profile_read": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(_I)]),
    "ann_check_device": (ctypes.c_int, [_P, _P]),
}

PROF_KINDS = {"lm_head": 0, "qkv": 1, "o": 2, "fc": 3, "proj": 4, "attn": 5, "step": 6}

_lib = None


class AnnError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class AnnArgError(AnnError, ValueError):
    pass


def lib():
    """Load libattnnn.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: build it with `python -m attention_nn_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != ANN_OK:
        msg = lib().ann_last_error().decode(errors="replace")
        if rc in (ANN_E_ARG, ANN_E_CAPACITY):
            raise AnnArgError(rc, msg)
        raise AnnError(rc, msg)
    return rc


def make_config(cfg, max_batch, max_ctx, max_tokens, v_sample=50257):
    c = AnnConfig()
    c.d, c.L, c.H = cfg.model_dim, cfg.num_layers, cfg.num_heads
    c.V = cfg.vocab_size
    c.V_sample = min(v_sample, cfg.vocab_size)
    c.window = cfg.window
    longs = sorted(set(int(l) for l in cfg.long_layers))
    if len(longs) > ANN_MAX_LONG_LAYERS:
        raise ValueError(f"at most {ANN_MAX_LONG_LAYERS} long layers")
    c.n_long = len(longs)
    for i, l in enumerate(longs):
        c.long_layers[i] = l
    c.attn_scale = cfg.attn_scale
    c.rope_base = cfg.rope_base
    c.rms_eps = 1e-6
    c.max_batch, c.max_ctx, c.max_tokens = max_batch, max_ctx, max_tokens
    return c
