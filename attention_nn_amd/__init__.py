"""attention_nn's token loop (sample.py x model.py) on one MI355X (gfx950).

Hand-written HIP kernels behind a C ABI (include/attnnn.h, libattnnn.so);
this package is the host side: config, checkpoint format, ctypes binding,
``GPT.logits`` and ``sample``.
"""

from .config import GPTConfig, sample_config, V_SAMPLE  # noqa: F401
from .weights import (init_params, load_params, save_params, param_count,  # noqa: F401
                      checkpoint_path)


def __getattr__(name):
    # torch-dependent pieces load lazily so the config / checkpoint helpers
    # import without a GPU stack.
    if name == "Engine":
        from .engine import Engine
        return Engine
    if name == "GPT":
        from .model import GPT
        return GPT
    raise AttributeError(name)
