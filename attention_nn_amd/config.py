"""Model hyper-parameters for the decode/prefill token loop.

Mirrors ``GPTConfig`` of the reference (``model.py:30-45``): same field names,
same defaults, same ``head_dim`` property, so a config built for the reference
builds here unchanged.  ``sample.py:31-33`` of the reference derives
``long_layers = (L//2 - 1, L - 1)`` from ``--layers``; :func:`sample_config`
does the same.
"""

from dataclasses import dataclass, field

# Number of vocabulary rows that sampling considers (GPT-2's 50257 tokens);
# the remaining rows of the padded 50304 vocabulary are never sampled
# (reference ``sample.py:45``).
V_SAMPLE = 50257


@dataclass
class GPTConfig:
    vocab_size: int = 50304        # GPT-2 50257 padded to a multiple of 128
    num_layers: int = 8
    num_heads: int = 8
    model_dim: int = 512
    seq_len: int = 1024
    window: int = 384              # sliding window of the short layers
    long_layers: tuple = (3, 7)    # layers with full causal attention
    attn_scale: float = 0.1
    rope_base: float = 1024.0
    ce_chunk: int = 2048           # kept for field parity; unused at inference

    @property
    def head_dim(self):
        return self.model_dim // self.num_heads

    def validate(self):
        d, H = self.model_dim, self.num_heads
        if d % H:
            raise ValueError(f"model_dim {d} not divisible by num_heads {H}")
        if self.head_dim % 4:
            raise ValueError(f"head_dim {self.head_dim} must be a multiple of 4 (half-truncated RoPE pairs)")
        for l in self.long_layers:
            if not 0 <= l < self.num_layers:
                raise ValueError(f"long layer {l} outside [0, {self.num_layers})")
        if self.window < 1:
            raise ValueError("window must be >= 1")
        return self


def sample_config(dim=512, layers=8, heads=8, **kw):
    """Config exactly as the reference CLI builds it (``sample.py:31-33``)."""
    return GPTConfig(num_layers=layers, num_heads=heads, model_dim=dim,
                     long_layers=(layers // 2 - 1, layers - 1), **kw)


# Named workloads of the benchmark (the model shapes of the five configs).
def cfg_small_h4():
    """76.7M: d=512, 8 layers, 4 heads x 128 (head_dim 128), long {3,7}."""
    return sample_config(dim=512, layers=8, heads=4)


def cfg_155m(seq_len=1024):
    """155M: d=768, 11 layers, 6 heads x 128, long {4,10}."""
    return sample_config(dim=768, layers=11, heads=6, seq_len=seq_len)


def cfg_834m(seq_len=2048):
    """Scaled variant: d=1536, 24 layers, 12 heads x 128, long {11,23}."""
    return sample_config(dim=1536, layers=24, heads=12, seq_len=seq_len)
