"""Operator API mirroring the reference's hot-path Metal kernels.

    relu2(x)                        metal_kernels.py:37-47,62-68
    rope_ht(x, cs, sn, pos0=0)      metal_kernels.py:87-134
    make_rope_tables(T, D, base)    metal_kernels.py:144-150
    rms(x)                          model.py:48-49

Inputs are torch tensors on the GPU (fp32 or bf16); outputs keep the input
dtype, computed in fp32 inside the HIP kernels.  ``rope_ht`` takes the
position of row 0 explicitly (the reference derives it from the row index
within the tensor, i.e. pos0 = 0).
"""

import ctypes

import torch

from . import _lib


def _dt(x):
    if x.dtype == torch.float32:
        return _lib.DTYPE_F32
    if x.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    raise TypeError(f"unsupported dtype {x.dtype} (float32 or bfloat16)")


def _gpu(x):
    if not (isinstance(x, torch.Tensor) and x.is_cuda):
        raise ValueError("expected a GPU tensor")
    return x.contiguous()


def _s():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def relu2(x):
    x = _gpu(x)
    y = torch.empty_like(x)
    _lib.check(_lib.lib().ann_op_relu2(_p(x), _p(y), x.numel(), _dt(x), _s()))
    return y


def rope_ht(x, cs, sn, pos0=0, inverse=False):
    x = _gpu(x)
    cs, sn = _gpu(cs).float(), _gpu(sn).float()
    if x.dim() != 4:
        raise ValueError("x must be (B, T, H, D)")
    B, T, H, D = x.shape
    if cs.shape[-1] != D // 4 or cs.shape[0] < pos0 + T or sn.shape != cs.shape:
        raise ValueError("tables must be (>= pos0 + T, D/4)")
    y = torch.empty_like(x)
    _lib.check(_lib.lib().ann_op_rope_ht(_p(x), _p(y), _p(cs), _p(sn), B, T, H, D, pos0,
                                         int(bool(inverse)), _dt(x), _s()))
    return y


def make_rope_tables(seq_len, head_dim, base=1024.0, device="cuda"):
    cs = torch.empty((seq_len, head_dim // 4), dtype=torch.float32, device=device)
    sn = torch.empty_like(cs)
    _lib.check(_lib.lib().ann_op_rope_tables(_p(cs), _p(sn), seq_len, head_dim, float(base), _s()))
    return cs, sn


def rms(x, eps=1e-6):
    x = _gpu(x)
    y = torch.empty_like(x)
    dim = x.shape[-1]
    _lib.check(_lib.lib().ann_op_rms_norm(_p(x), _p(y), x.numel() // dim, dim, float(eps),
                                          _dt(x), _s()))
    return y
