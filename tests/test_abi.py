"""Host-only checks of the C ABI: the library loads, exports every declared
symbol, and rejects bad configurations / calls before touching the GPU."""

import ctypes
import os
import re

import pytest

from attention_nn_amd import _lib
from attention_nn_amd.config import GPTConfig, cfg_155m

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "attnnn.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(ann_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        from attention_nn_amd.build import build
        build()
    return _lib.lib()


def test_exports_every_declared_symbol(L):
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(L, n), f"{n} declared in attnnn.h but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"


def _cfg(**kw):
    c = _lib.make_config(cfg_155m(), 1, 1024, 1024)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def _create(L, c):
    ctx = ctypes.c_void_p()
    rc = L.ann_create(ctypes.byref(c), ctypes.byref(ctx))
    return rc, ctx


@pytest.mark.parametrize("field,value,msg", [
    ("H", 7, "divisible"),
    ("H", 3, "head_dim"),           # 768/3 = 256
    ("V_sample", 60000, "V_sample"),
    ("window", 0, "window"),
    ("n_long", 9, "n_long"),
    ("max_tokens", 0, "positive"),
])
def test_create_rejects_bad_config(L, field, value, msg):
    rc, ctx = _create(L, _cfg(**{field: value}))
    assert rc == _lib.ANN_E_ARG
    assert msg in L.ann_last_error().decode()
    assert not ctx.value


def test_create_rejects_long_layer_out_of_range(L):
    c = _cfg()
    c.long_layers[1] = 11
    rc, _ = _create(L, c)
    assert rc == _lib.ANN_E_ARG and "long layer" in L.ann_last_error().decode()


def test_sizes(L):
    c = _cfg()
    wb = L.ann_weight_bytes(ctypes.byref(c))
    # bf16 weights of the 155M model (embed + lm_head + 12 d^2 per layer) plus tables
    d, V, Lr = 768, 50304, 11
    assert wb >= 2 * (2 * V * d + 12 * d * d * Lr)
    assert wb < 2 * (2 * V * d + 12 * d * d * Lr) + 4 * 1024 * 1024
    assert L.ann_kv_bytes(ctypes.byref(c)) == 2 * Lr * 1 * 1024 * d * 2
    assert L.ann_workspace_bytes(ctypes.byref(c)) > 0
    bad = _cfg(H=7)
    assert L.ann_weight_bytes(ctypes.byref(bad)) == 0


def test_sampling_needs_vocab_multiple_of_8(L):
    """Sampled calls (temperature > 0) are refused on the host for a vocabulary
    that is not a multiple of 8 (the samplers read z rows in 16-byte chunks)."""
    c = _cfg(V=50257, V_sample=50257)
    rc, ctx = _create(L, c)
    assert rc == 0
    try:
        fake = ctypes.c_void_p(1 << 40)
        wb = L.ann_weight_bytes(ctypes.byref(c))
        kb = L.ann_kv_bytes(ctypes.byref(c))
        sb = L.ann_workspace_bytes(ctypes.byref(c))
        assert L.ann_bind(ctx, fake, wb, fake, kb, fake, sb) == 0
        tok = ctypes.c_void_p(0x1000)
        s = _lib.AnnSampling(0.8, 50, 1, 0)
        assert L.ann_prefill(ctx, tok, 1, 4, ctypes.byref(s), tok, None, None) == _lib.ANN_E_ARG
        assert "multiple of 8" in L.ann_last_error().decode()
    finally:
        L.ann_destroy(ctx)


def test_call_order_and_capacity_errors(L):
    c = _cfg()
    rc, ctx = _create(L, c)
    assert rc == 0
    try:
        s = _lib.AnnSampling(0.0, 0, 0, 0)
        tok = ctypes.c_void_p(0x1000)
        # not bound yet
        assert L.ann_prefill(ctx, tok, 1, 4, ctypes.byref(s), tok, None, None) == _lib.ANN_E_STATE
        assert L.ann_check_device(ctx, None) == _lib.ANN_E_STATE
        assert L.ann_check_device(None, None) == _lib.ANN_E_ARG
        # bind with fake (never dereferenced) aligned pointers; sizes checked first
        wb = L.ann_weight_bytes(ctypes.byref(c))
        kb = L.ann_kv_bytes(ctypes.byref(c))
        sb = L.ann_workspace_bytes(ctypes.byref(c))
        fake = ctypes.c_void_p(1 << 40)
        assert L.ann_bind(ctx, fake, wb - 1, fake, kb, fake, sb) == _lib.ANN_E_CAPACITY
        assert L.ann_bind(ctx, fake, wb, fake, kb - 1, fake, sb) == _lib.ANN_E_CAPACITY
        assert L.ann_bind(ctx, fake, wb, fake, kb, fake, sb - 1) == _lib.ANN_E_CAPACITY
        assert L.ann_bind(ctx, ctypes.c_void_p((1 << 40) + 8), wb, fake, kb, fake, sb) == _lib.ANN_E_ARG
        assert L.ann_bind(ctx, fake, wb, fake, kb, fake, sb) == 0
        # shape / capacity errors are caught on the host before any launch
        assert L.ann_prefill(ctx, tok, 2, 4, ctypes.byref(s), tok, None, None) == _lib.ANN_E_CAPACITY
        assert L.ann_prefill(ctx, tok, 1, 1025, ctypes.byref(s), tok, None, None) == _lib.ANN_E_CAPACITY
        assert L.ann_prefill(ctx, tok, 0, 4, ctypes.byref(s), tok, None, None) == _lib.ANN_E_ARG
        bad_t = _lib.AnnSampling(-1.0, 0, 0, 0)
        assert L.ann_prefill(ctx, tok, 1, 4, ctypes.byref(bad_t), tok, None, None) == _lib.ANN_E_ARG
        # decode before any prefill
        assert L.ann_decode_step(ctx, tok, 1, ctypes.byref(s), tok, None, None) == _lib.ANN_E_STATE
        assert L.ann_context_length(ctx) == 0
        assert L.ann_forward_logits(ctx, tok, 1, 4, None, None) == _lib.ANN_E_ARG
    finally:
        L.ann_destroy(ctx)


def test_operator_argument_errors(L):
    p = ctypes.c_void_p(1 << 40)
    assert L.ann_op_relu2(p, p, 16, 7, None) == _lib.ANN_E_ARG
    assert L.ann_op_rope_ht(p, p, p, p, 1, 1, 1, 6, 0, 0, 0, None) == _lib.ANN_E_ARG   # D % 4
    assert L.ann_op_rope_tables(p, p, 0, 64, 1024.0, None) == _lib.ANN_E_ARG
    assert L.ann_op_rms_norm(None, p, 1, 8, 1e-6, 0, None) == _lib.ANN_E_ARG
    assert L.ann_create(None, None) == _lib.ANN_E_ARG


def test_python_errors_map_to_exceptions(L):
    with pytest.raises(ValueError):
        _lib.check(_lib.ANN_E_ARG)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ANN_E_STATE)


def test_engine_refuses_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from attention_nn_amd.engine import Engine
    from attention_nn_amd.weights import init_params
    cfg = GPTConfig(vocab_size=512, num_layers=2, num_heads=2, model_dim=128, seq_len=32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Engine(cfg, init_params(cfg))
