"""The flat fp32 parameter dict: synthetic init, checkpoint read/write.

Keys, shapes and dtype follow the reference exactly (``model.py:52-77``):

    embed          (V, d)        lm_head     (d, V)
    attn_bank      (L, 4, d, d)  [q, k, v, o], each stored (in, out)
    fc_bank        (L, d, 4d)    proj_bank   (L, 4d, d)
    resid_lambdas  (L, 2)        post_lambdas (L, 2)
    x0_lambdas     (L,)          sa_lambdas  (L, 2)

Checkpoints are ``*.params.safetensors`` files holding that dict as F32
(written by the reference at ``train.py:182``, read at ``sample.py:35-38``).

The reference draws its init with MLX's RNG, which is not available here, so
:func:`init_params` uses numpy's seeded PCG64 with the same distributions:
inputs ~ U(+-sqrt(3)*0.5/sqrt(d)), head ~ N(0, 0.005^2), embed = head.T,
Wo = proj = 0, resid = sqrt(1.1), post = 1, x0 = 0, sa = [0.5, 1.0].
``dense=True`` additionally draws Wo and proj from the input distribution:
with Wo = proj = x0 = 0 every layer is an identity on the residual stream and
a parity test could not see attention or MLP mistakes.
"""

import os

import numpy as np

PARAM_KEYS = ("embed", "lm_head", "attn_bank", "fc_bank", "proj_bank",
              "resid_lambdas", "post_lambdas", "x0_lambdas", "sa_lambdas")


def param_shapes(cfg):
    d, L, V = cfg.model_dim, cfg.num_layers, cfg.vocab_size
    return {
        "embed": (V, d), "lm_head": (d, V), "attn_bank": (L, 4, d, d),
        "fc_bank": (L, d, 4 * d), "proj_bank": (L, 4 * d, d),
        "resid_lambdas": (L, 2), "post_lambdas": (L, 2),
        "x0_lambdas": (L,), "sa_lambdas": (L, 2),
    }


def param_count(cfg):
    return sum(int(np.prod(s)) for s in param_shapes(cfg).values())


def init_params(cfg, seed=0, dense=False):
    """Synthetic fp32 master weights with the distributions of ``model.py:52-77``."""
    rng = np.random.default_rng(seed)
    d, L, V = cfg.model_dim, cfg.num_layers, cfg.vocab_size
    bound = np.float32((3 ** 0.5) * 0.5 * d ** -0.5)

    def u(*shape):
        return (rng.random(shape, dtype=np.float32) * np.float32(2) - np.float32(1)) * bound

    head = rng.standard_normal((d, V), dtype=np.float32) * np.float32(0.005)
    attn = np.zeros((L, 4, d, d), np.float32)
    for l in range(L):
        for j in range(3):
            attn[l, j] = u(d, d)
        if dense:
            attn[l, 3] = u(d, d)
    fc = np.stack([u(d, 4 * d) for _ in range(L)])
    proj = np.stack([u(4 * d, d) for _ in range(L)]) if dense else np.zeros((L, 4 * d, d), np.float32)
    return {
        "embed": np.ascontiguousarray(head.T),
        "lm_head": head,
        "attn_bank": attn,
        "fc_bank": fc,
        "proj_bank": proj,
        "resid_lambdas": np.full((L, 2), 1.1 ** 0.5, np.float32),
        "post_lambdas": np.ones((L, 2), np.float32),
        "x0_lambdas": np.zeros((L,), np.float32),
        "sa_lambdas": np.tile(np.array([0.5, 1.0], np.float32), (L, 1)),
    }


def perturb_lambdas(params, seed=1):
    """Move the per-layer lambdas off their init values (x0 != 0, sa != 0.5/1),
    so the residual-mix and weight-scale paths are exercised by parity tests."""
    rng = np.random.default_rng(seed)
    out = dict(params)
    for k, lo, hi in (("resid_lambdas", 0.8, 1.2), ("post_lambdas", 0.5, 1.5),
                      ("x0_lambdas", -0.3, 0.3), ("sa_lambdas", 0.3, 1.3)):
        out[k] = rng.uniform(lo, hi, params[k].shape).astype(np.float32)
    return out


def check_params(cfg, params):
    """Raise ValueError unless ``params`` has exactly the reference keys/shapes."""
    shapes = param_shapes(cfg)
    missing = [k for k in shapes if k not in params]
    if missing:
        raise ValueError(f"checkpoint lacks parameters {missing}")
    for k, s in shapes.items():
        got = tuple(params[k].shape)
        if got != s:
            raise ValueError(f"parameter {k}: shape {got}, config expects {s}")


def checkpoint_path(path):
    """``sample.py:35-37``: append ``.params.safetensors`` unless already a safetensors path."""
    return path if path.endswith(".safetensors") else f"{path}.params.safetensors"


def save_params(path, params):
    """Write the flat dict as F32 safetensors (the layout of ``train.py:182``)."""
    from safetensors.numpy import save_file
    save_file({k: np.ascontiguousarray(np.asarray(v, dtype=np.float32)) for k, v in params.items()},
              checkpoint_path(path))


def load_params(path):
    """Read a ``*.params.safetensors`` file into a dict of fp32 numpy arrays."""
    from safetensors.numpy import load_file
    p = checkpoint_path(path)
    if not os.path.exists(p):
        raise FileNotFoundError(p)
    return {k: np.asarray(v, dtype=np.float32) for k, v in load_file(p).items()}
