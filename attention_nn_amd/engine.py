"""Device-side engine: owns the torch buffers, drives libattnnn.so.

PyTorch only provides device memory and the stream; every computation runs
in the library's HIP kernels.  Requires a ROCm GPU: constructing an Engine
without one raises.
"""

import ctypes

import numpy as np
import torch

from . import _lib
from .config import V_SAMPLE
from .weights import check_params

PARAM_ORDER = ("embed", "lm_head", "attn_bank", "fc_bank", "proj_bank",
               "resid_lambdas", "post_lambdas", "x0_lambdas", "sa_lambdas")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Engine:
    """One model bound to KV-cache / workspace capacities on one GPU.

    max_batch  sequences per call;  max_ctx  tokens per sequence (also the
    RoPE table length, so it may exceed cfg.seq_len);  max_tokens  rows of the
    largest prefill (B*T).
    """

    def __init__(self, cfg, params, max_batch=1, max_ctx=None, max_tokens=None,
                 device="cuda"):
        if not torch.cuda.is_available():
            raise RuntimeError("attention_nn_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
        cfg.validate()
        check_params(cfg, params)
        self.cfg = cfg
        self.device = torch.device(device)
        self.max_batch = int(max_batch)
        self.max_ctx = int(max_ctx or cfg.seq_len)
        self.max_tokens = int(max_tokens or self.max_batch * self.max_ctx)
        L = _lib.lib()
        self._c = _lib.make_config(cfg, self.max_batch, self.max_ctx, self.max_tokens, V_SAMPLE)
        ctx = ctypes.c_void_p()
        _lib.check(L.ann_create(ctypes.byref(self._c), ctypes.byref(ctx)))
        self._ctx = ctx
        wb = L.ann_weight_bytes(ctypes.byref(self._c))
        kb = L.ann_kv_bytes(ctypes.byref(self._c))
        sb = L.ann_workspace_bytes(ctypes.byref(self._c))
        self.wbuf = torch.empty(wb, dtype=torch.uint8, device=self.device)
        self.kv = torch.empty(kb, dtype=torch.uint8, device=self.device)
        self.ws = torch.zeros(sb, dtype=torch.uint8, device=self.device)
        self._pack(params)
        _lib.check(L.ann_bind(self._ctx, _ptr(self.wbuf), wb, _ptr(self.kv), kb,
                              _ptr(self.ws), sb))
        self.batch = 0

    def _pack(self, params):
        src = {k: torch.as_tensor(np.ascontiguousarray(params[k], dtype=np.float32)).to(self.device)
               for k in PARAM_ORDER}
        p = _lib.AnnParamsF32(**{k: src[k].data_ptr() for k in PARAM_ORDER})
        _lib.check(_lib.lib().ann_pack_weights(self._ctx, ctypes.byref(p), _ptr(self.wbuf),
                                               self.wbuf.numel(), _stream()))
        torch.cuda.current_stream().synchronize()
        del src

    def __del__(self):
        ctx = getattr(self, "_ctx", None)
        if ctx is not None and _lib._lib is not None:
            _lib.lib().ann_destroy(ctx)
            self._ctx = None

    # -- helpers -------------------------------------------------------------
    def _tokens(self, tokens, ndim):
        if isinstance(tokens, torch.Tensor) and tokens.is_cuda:
            t = tokens.to(torch.int32).contiguous()
        else:
            a = np.asarray(tokens)
            if a.size and (a.min() < 0 or a.max() >= self.cfg.vocab_size):
                raise ValueError(f"token ids must lie in [0, {self.cfg.vocab_size})")
            t = torch.as_tensor(a.astype(np.int32)).to(self.device)
        if t.dim() != ndim:
            raise ValueError(f"tokens must have {ndim} dims, got shape {tuple(t.shape)}")
        return t

    @staticmethod
    def _sampling(temperature, top_k, seed, step):
        return _lib.AnnSampling(float(temperature), int(top_k or 0), int(seed) & (2**64 - 1),
                                int(step) & (2**64 - 1))

    @property
    def length(self):
        return _lib.lib().ann_context_length(self._ctx)

    def profile(self, kind, max_launches=4096):
        """Bracket every launch of one kernel class ('lm_head', 'qkv', 'o',
        'fc', 'proj', 'attn', or 'step' = the persistent batch-1 decode
        kernel) with HIP events; None disables."""
        k = -1 if kind is None else _lib.PROF_KINDS[kind]
        _lib.check(_lib.lib().ann_profile_enable(self._ctx, k, int(max_launches)))

    def profile_read(self):
        """(summed ms, launches) since the last read."""
        ms = ctypes.c_float()
        n = ctypes.c_int32()
        _lib.check(_lib.lib().ann_profile_read(self._ctx, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def check_device(self):
        """Raise if a bounded cross-work-group wait of the persistent decode
        step timed out since the last check (synchronises the stream)."""
        _lib.check(_lib.lib().ann_check_device(self._ctx, _stream()))

    def reset(self):
        _lib.check(_lib.lib().ann_reset(self._ctx))
        self.batch = 0

    # -- entry points --------------------------------------------------------
    def forward_logits(self, tokens):
        """GPT.logits: (B, T) ids -> (B, T, V) softcapped fp32 on the device."""
        t = self._tokens(tokens, 2)
        B, T = t.shape
        out = torch.empty((B, T, self.cfg.vocab_size), dtype=torch.float32, device=self.device)
        _lib.check(_lib.lib().ann_forward_logits(self._ctx, _ptr(t), B, T, _ptr(out), _stream()))
        self.batch = B
        return out

    def forward_loss(self, tokens, targets, rows=False):
        """GPT.__call__ (model.py:180-221): mean softcapped CE of (B, T) ids
        against (B, T) targets as a 0-d fp32 device tensor; with ``rows`` also
        the (B*T,) per-row losses."""
        t = self._tokens(tokens, 2)
        g = self._tokens(targets, 2)
        if tuple(g.shape) != tuple(t.shape):
            raise ValueError(f"targets {tuple(g.shape)} must match tokens {tuple(t.shape)}")
        B, T = t.shape
        mean = torch.empty((), dtype=torch.float32, device=self.device)
        per = torch.empty((B * T,), dtype=torch.float32, device=self.device) if rows else None
        _lib.check(_lib.lib().ann_forward_loss(self._ctx, _ptr(t), _ptr(g), B, T, _ptr(mean),
                                               _ptr(per) if rows else None, _stream()))
        self.batch = B
        return (mean, per) if rows else mean

    def prefill(self, tokens, temperature=0.0, top_k=0, seed=0, step=0, want_logits=False):
        """Prefill (B, T) prompts; returns (next ids (B,) int32, logits (B,V) or None)."""
        t = self._tokens(tokens, 2)
        B, T = t.shape
        nxt = torch.empty((B,), dtype=torch.int32, device=self.device)
        lg = torch.empty((B, self.cfg.vocab_size), dtype=torch.float32, device=self.device) \
            if want_logits else None
        s = self._sampling(temperature, top_k, seed, step)
        _lib.check(_lib.lib().ann_prefill(self._ctx, _ptr(t), B, T, ctypes.byref(s), _ptr(nxt),
                                          _ptr(lg) if lg is not None else None, _stream()))
        self.batch = B
        return nxt, lg

    def decode(self, tokens, temperature=0.0, top_k=0, seed=0, step=0, want_logits=False,
               out=None):
        """One decode step for (B,) ids; returns (next ids (B,), logits or None)."""
        t = self._tokens(tokens, 1)
        B = t.shape[0]
        nxt = out if out is not None else torch.empty((B,), dtype=torch.int32, device=self.device)
        lg = torch.empty((B, self.cfg.vocab_size), dtype=torch.float32, device=self.device) \
            if want_logits else None
        s = self._sampling(temperature, top_k, seed, step)
        _lib.check(_lib.lib().ann_decode_step(self._ctx, _ptr(t), B, ctypes.byref(s), _ptr(nxt),
                                              _ptr(lg) if lg is not None else None, _stream()))
        return nxt, lg
