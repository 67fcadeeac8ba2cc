"""Host logic of the drop-in GPT API (no GPU): the packed-weight cache key.
CPU only."""

import numpy as np

from attention_nn_amd.model import param_key, same_key
from attention_nn_amd.weights import init_params


def test_cache_key_follows_the_arrays_not_the_dict(tiny_cfg):
    p = init_params(tiny_cfg, 0)
    k0 = param_key(p)
    assert same_key(k0, param_key(p))
    assert same_key(k0, param_key(dict(p)))             # a copy of the dict, same arrays
    q = dict(p)
    q["fc_bank"] = p["fc_bank"].copy()                  # one entry replaced
    assert not same_key(k0, param_key(q))
    p["x0_lambdas"] = np.full_like(p["x0_lambdas"], 0.5)    # updated in the same dict
    assert not same_key(k0, param_key(p))
    r = init_params(tiny_cfg, 0)                        # equal values, other arrays
    assert not same_key(param_key(r), param_key(init_params(tiny_cfg, 0)))


def test_cache_key_keeps_arrays_alive(tiny_cfg):
    """The key holds the arrays, so a freed array's id cannot come back and
    match a stale key."""
    p = init_params(tiny_cfg, 0)
    k0 = param_key(p)
    ids = [id(e[1]) for e in k0]
    del p
    assert [id(e[1]) for e in k0] == ids and all(e[1] is not None for e in k0)
