"""Training checkpoints in the reference's on-disk format.

A checkpoint named ``save`` is three files (``train.py:135-148,178-185``):

    save.params.safetensors   the flat fp32 parameter dict (``weights.save_params``)
    save.opt.safetensors      optimizer state, one tensor per (parameter, state
                              key) under the flat key "name|key" (``muon.py:146-149``)
    save.meta.json            {"step": int, "config": {...}}, written with
                              ``default=str`` (``train.py:183-184``)

Loading follows the reference's checks: every parameter of the running model
must be present with the same shape (``train.py:142-145``), and every
optimizer entry must name a known (parameter, key) pair of the same shape
(``muon.py:151-157``).  A resume starts from ``meta["step"]`` when the meta
file exists and from step 0 otherwise (``train.py:137-141``).  Violations
raise ValueError.  Tensors are numpy arrays; their dtype is kept.
"""

import json
import os

import numpy as np

from .weights import load_params, save_params


def paths(save):
    """The three file names of checkpoint ``save``."""
    return (f"{save}.params.safetensors", f"{save}.opt.safetensors", f"{save}.meta.json")


def flatten_opt_state(state):
    """{name: {key: array}} -> {"name|key": array} (``muon.py:146-149``)."""
    flat = {}
    for name, st in state.items():
        for k, v in st.items():
            if "|" in k:
                raise ValueError(f"optimizer state key {k!r} of {name!r} contains '|'")
            # order="C" keeps 0-d arrays 0-d (the step counter "_step|t" is a
            # 0-d array in the reference's files); ascontiguousarray would not
            flat[f"{name}|{k}"] = np.asarray(v, order="C")
    return flat


def unflatten_opt_state(flat, like=None):
    """Inverse of :func:`flatten_opt_state`, splitting each key at its last '|'.

    With ``like`` (the running optimizer's state), every entry must name an
    existing (parameter, key) pair of the same shape (``muon.py:151-157``)."""
    out = {}
    for key, v in flat.items():
        if "|" not in key:
            raise ValueError(f"optimizer state key {key!r} has no '|'")
        name, k = key.rsplit("|", 1)
        if like is not None:
            if name not in like or k not in like[name]:
                raise ValueError(f"unknown optimizer state {key}")
            want = tuple(np.shape(like[name][k]))
            if tuple(v.shape) != want:
                raise ValueError(f"shape mismatch for {key}: {tuple(v.shape)} vs {want}")
        out.setdefault(name, {})[k] = v
    return out


def save_checkpoint(save, params, opt_state, step, config):
    """Write the three files of checkpoint ``save`` (``train.py:178-185``)."""
    from safetensors.numpy import save_file
    p_path, o_path, m_path = paths(save)
    save_params(p_path, params)
    save_file(flatten_opt_state(opt_state or {}), o_path)
    with open(m_path, "w") as f:
        json.dump({"step": int(step), "config": dict(config)}, f, default=str)


def resume_step(save):
    """``train.py:137-141``: the saved step if ``save.meta.json`` exists, else 0."""
    m_path = paths(save)[2]
    if not os.path.exists(m_path):
        return 0
    with open(m_path) as f:
        return int(json.load(f)["step"])


def load_checkpoint(save, params_like=None, opt_like=None):
    """Read checkpoint ``save`` -> (params, opt_state, meta).

    ``params_like`` (the running model's dict) requires every one of its
    parameters in the file with the same shape; ``opt_like`` checks the
    optimizer entries the same way."""
    from safetensors.numpy import load_file
    p_path, o_path, m_path = paths(save)
    with open(m_path) as f:
        meta = json.load(f)
    params = load_params(p_path)
    if params_like is not None:
        for k, v in params_like.items():
            if k not in params:
                raise ValueError(f"checkpoint lacks parameter {k}")
            if tuple(params[k].shape) != tuple(np.shape(v)):
                raise ValueError(f"parameter {k}: shape {tuple(params[k].shape)}, "
                                 f"model has {tuple(np.shape(v))}")
    opt = unflatten_opt_state(load_file(o_path), opt_like) if os.path.exists(o_path) else {}
    return params, opt, meta
