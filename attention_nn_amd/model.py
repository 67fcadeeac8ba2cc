"""``GPT(cfg).logits(params, tokens)`` and ``GPT(cfg)(params, tokens,
targets)`` on the MI355X engine.

Same call shapes as the reference (``model.py:138-153,180-263``): ``params``
is the flat fp32 dict (numpy arrays or tensors), ``tokens`` / ``targets`` are
(B, T) int with T <= seq_len.  ``logits`` returns (B, T, V) fp32 softcapped
logits, the call returns the mean softcapped cross-entropy (a 0-d fp32
tensor; forward only -- there is no backward here).  Both are GPU tensors.
The packed bf16 weights of a params dict are cached per GPT object so
repeated calls with the same dict do not re-pack.
"""

import numpy as np

from .config import GPTConfig
from .engine import Engine


class GPT:
    def __init__(self, cfg: GPTConfig):
        self.cfg = cfg.validate()
        self._engine = None
        self._key = None

    def engine(self, params, max_batch=1, max_tokens=None):
        key = (id(params), max_batch, max_tokens)
        if self._engine is None or self._key != key:
            self._engine = Engine(self.cfg, params, max_batch=max_batch,
                                  max_ctx=self.cfg.seq_len,
                                  max_tokens=max_tokens or max_batch * self.cfg.seq_len)
            self._key = key
        return self._engine

    def logits(self, params, tokens):
        tokens = np.asarray(tokens.cpu() if hasattr(tokens, "cpu") else tokens)
        if tokens.ndim != 2:
            raise ValueError("tokens must be (B, T)")
        B, T = tokens.shape
        if T > self.cfg.seq_len:
            raise ValueError(f"T={T} exceeds seq_len={self.cfg.seq_len}")
        eng = self.engine(params, max_batch=max(B, 1), max_tokens=max(B * T, B))
        return eng.forward_logits(tokens)

    def _shape(self, tokens):
        tokens = np.asarray(tokens.cpu() if hasattr(tokens, "cpu") else tokens)
        if tokens.ndim != 2:
            raise ValueError("tokens must be (B, T)")
        B, T = tokens.shape
        if T > self.cfg.seq_len:
            raise ValueError(f"T={T} exceeds seq_len={self.cfg.seq_len}")
        return tokens, B, T

    def __call__(self, params, tokens, targets):
        """Training forward: mean loss over the B*T rows (model.py:180-221)."""
        tokens, B, T = self._shape(tokens)
        targets = np.asarray(targets.cpu() if hasattr(targets, "cpu") else targets)
        eng = self.engine(params, max_batch=max(B, 1), max_tokens=max(B * T, B))
        return eng.forward_loss(tokens, targets)
