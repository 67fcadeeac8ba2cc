"""ann_op_normuon_noalloc: NorMuon with its scratch in the library's fixed
device array (no allocation), through the C ABI, against ann_op_normuon with a
caller workspace -- the same kernels, so outputs and second moments must be
bitwise equal -- on two calls in a row, the second smaller (the array keeps
the first call's contents)."""

import ctypes

import numpy as np
import pytest
import torch

from attention_nn_amd import _lib


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def test_noalloc_rejects_oversize_before_any_launch():
    """Host-side: a shape whose scratch exceeds the fixed array is refused
    with a capacity error (no GPU needed: nothing is dereferenced or launched)."""
    L = _lib.lib()
    cap = L.ann_op_normuon_noalloc_max_bytes()
    assert cap == 4 << 20
    dummy = ctypes.c_void_p(256)
    R = cap // 8 + 1                       # one line past what fits
    rc = L.ann_op_normuon_noalloc(dummy, dummy, 1, R, 64, ctypes.c_float(0.9), dummy, None)
    assert rc == _lib.ANN_E_CAPACITY
    assert "fixed array" in L.ann_last_error().decode()
    rc = L.ann_op_normuon_noalloc(dummy, dummy, 0, 64, 64, ctypes.c_float(0.9), dummy, None)
    assert rc == _lib.ANN_E_ARG


def _with_workspace(v, sm, beta2):
    L = _lib.lib()
    batch, M, N = v.shape
    out = torch.empty(v.shape, dtype=torch.float32, device="cuda")
    sm = sm.clone()
    nws = L.ann_op_normuon_ws_bytes(batch, M, N)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    _lib.check(L.ann_op_normuon(_p(v), _p(sm), batch, M, N, ctypes.c_float(beta2), _p(out),
                                _p(ws), nws, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    return out, sm


def _no_alloc(v, sm, beta2):
    L = _lib.lib()
    batch, M, N = v.shape
    out = torch.empty(v.shape, dtype=torch.float32, device="cuda")
    sm = sm.clone()
    _lib.check(L.ann_op_normuon_noalloc(_p(v), _p(sm), batch, M, N, ctypes.c_float(beta2),
                                        _p(out),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    return out, sm


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_point_twice():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    g = torch.Generator().manual_seed(7)
    # first: a proj-bank-like stack (rows reduced over 3072-long lines);
    # second, smaller: 256-wide columns (the other reduction direction)
    for shape in [(11, 3072, 768), (3, 64, 256), (2, 96, 64)]:
        batch, M, N = shape
        print(f"case normuon_noalloc {shape}", flush=True)
        v = (torch.randn(shape, generator=g) * 0.02).to(torch.bfloat16).cuda()
        R = M if M >= N else N
        sm = (torch.rand(batch * R, generator=g) * 1e-4).cuda()
        ref_out, ref_sm = _with_workspace(v, sm, 0.9)
        out, sm2 = _no_alloc(v, sm, 0.9)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), shape
        assert torch.equal(sm2, ref_sm), shape
        assert torch.isfinite(out).all()
