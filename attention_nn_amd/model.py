"""``GPT(cfg).logits(params, tokens)`` and ``GPT(cfg)(params, tokens,
targets)`` on the MI355X engine.

Same call shapes as the reference (``model.py:138-153,180-263``): ``params``
is the flat fp32 dict (numpy arrays or tensors), ``tokens`` / ``targets`` are
(B, T) int with T <= seq_len.  ``logits`` returns (B, T, V) fp32 softcapped
logits, the call returns the mean softcapped cross-entropy (a 0-d fp32
tensor; forward only -- there is no backward here).  Both are GPU tensors.

The packed bf16 weights are cached per GPT object.  The cache is keyed on the
identity of every array in the dict (the dict itself may be reused or
updated): replacing any entry, as an optimizer step or ``params.update`` does,
re-packs on the next call.  The reference's arrays are immutable (MLX), so an
array is never changed in place there; code that does write into an array in
place must call ``GPT.refresh()``.  The engine is sized to ``seq_len`` tokens
per sequence once, so calls with a growing T (the reference's sampling loop,
``sample.py:42-44``) reuse it; a larger batch re-sizes it.
"""

import numpy as np

from .config import GPTConfig
from .engine import PARAM_ORDER, Engine


def param_key(params):
    """Identity key of a parameter dict: (name, array object, shape) per entry.
    Holding the arrays keeps their ids from being reused while cached."""
    return tuple((k, params[k], tuple(np.shape(params[k]))) for k in PARAM_ORDER)


def same_key(a, b):
    return a is not None and b is not None and len(a) == len(b) and all(
        x[0] == y[0] and x[1] is y[1] and x[2] == y[2] for x, y in zip(a, b))


class GPT:
    def __init__(self, cfg: GPTConfig):
        self.cfg = cfg.validate()
        self._engine = None
        self._key = None
        self._batch = 0
        self.packs = 0      # how many times weights were packed (observable for tests)

    def refresh(self):
        """Drop the packed weights: the next call re-packs (after an in-place
        write into one of the parameter arrays)."""
        self._engine = None
        self._key = None

    def engine(self, params, batch=1):
        key = param_key(params)
        if self._engine is None or not same_key(self._key, key) or batch > self._batch:
            self._engine = None     # free the old buffers before allocating new ones
            B = max(batch, self._batch if same_key(self._key, key) else 0, 1)
            self._engine = Engine(self.cfg, params, max_batch=B, max_ctx=self.cfg.seq_len,
                                  max_tokens=B * self.cfg.seq_len)
            self._key = key
            self._batch = B
            self.packs += 1
        return self._engine

    def _shape(self, tokens):
        tokens = np.asarray(tokens.cpu() if hasattr(tokens, "cpu") else tokens)
        if tokens.ndim != 2:
            raise ValueError("tokens must be (B, T)")
        B, T = tokens.shape
        if T > self.cfg.seq_len:
            raise ValueError(f"T={T} exceeds seq_len={self.cfg.seq_len}")
        return tokens, B, T

    def logits(self, params, tokens):
        tokens, B, T = self._shape(tokens)
        return self.engine(params, batch=B).forward_logits(tokens)

    def __call__(self, params, tokens, targets):
        """Training forward: mean loss over the B*T rows (model.py:180-221)."""
        tokens, B, T = self._shape(tokens)
        targets = np.asarray(targets.cpu() if hasattr(targets, "cpu") else targets)
        return self.engine(params, batch=B).forward_loss(tokens, targets)
