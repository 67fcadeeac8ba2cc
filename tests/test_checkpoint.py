"""Training checkpoints in the reference's format (train.py:135-148,178-185,
muon.py:146-157).  CPU only."""

import json

import numpy as np
import pytest

from attention_nn_amd import checkpoint as C
from attention_nn_amd.config import GPTConfig
from attention_nn_amd.weights import init_params, load_params


@pytest.fixture
def small():
    cfg = GPTConfig(vocab_size=96, num_layers=2, num_heads=2, model_dim=32, seq_len=16,
                    window=8, long_layers=(1,))
    p = init_params(cfg, 4, dense=True)
    rng = np.random.default_rng(5)
    opt = {k: {"m": rng.standard_normal(v.shape).astype(np.float32),
               "v": rng.random(v.shape).astype(np.float32)} for k, v in p.items()}
    opt["attn_bank"]["step"] = np.array([7], dtype=np.int32)
    return cfg, p, opt


def test_round_trip_and_file_layout(tmp_path, small):
    cfg, p, opt = small
    save = str(tmp_path / "ckpt")
    C.save_checkpoint(save, p, opt, 123, {"batch": 8, "lr": 0.02, "path": tmp_path})
    pp, op, mp = C.paths(save)
    # the params file is what sample.py reads (sample.py:35-38)
    q = load_params(save)
    assert set(q) == set(p) and all(np.array_equal(q[k], p[k]) for k in p)
    # optimizer keys are "name|key" (muon.py:146-149); the meta file is plain json
    from safetensors.numpy import load_file
    flat = load_file(op)
    assert "attn_bank|m" in flat and "embed|v" in flat and flat["attn_bank|step"].dtype == np.int32
    meta = json.load(open(mp))
    assert meta["step"] == 123 and meta["config"]["batch"] == 8
    assert meta["config"]["path"] == str(tmp_path)          # default=str (train.py:184)
    params, state, meta2 = C.load_checkpoint(save, p, opt)
    assert meta2 == meta
    assert all(np.array_equal(params[k], p[k]) for k in p)
    assert all(np.array_equal(state[n][k], opt[n][k]) for n in opt for k in opt[n])
    assert C.resume_step(save) == 123


def test_resume_without_meta_starts_at_zero(tmp_path):
    assert C.resume_step(str(tmp_path / "none")) == 0       # train.py:138


def test_key_split_at_last_bar():
    flat = {"a|b|m": np.zeros(2), "x|v": np.ones(3)}
    st = C.unflatten_opt_state(flat)
    assert set(st) == {"a|b", "x"} and set(st["a|b"]) == {"m"}
    with pytest.raises(ValueError):
        C.flatten_opt_state({"p": {"bad|key": np.zeros(1)}})


def test_shape_and_name_checks(tmp_path, small):
    cfg, p, opt = small
    save = str(tmp_path / "c")
    C.save_checkpoint(save, p, opt, 1, {})
    bigger = dict(p)
    bigger["embed"] = np.zeros((97, 32), np.float32)
    with pytest.raises(ValueError, match="embed"):               # train.py:143-144
        C.load_checkpoint(save, bigger, None)
    extra = dict(p)
    extra["new_param"] = np.zeros(3, np.float32)
    with pytest.raises(ValueError, match="new_param"):
        C.load_checkpoint(save, extra, None)
    fewer = {k: dict(v) for k, v in opt.items()}
    del fewer["embed"]["m"]
    with pytest.raises(ValueError, match="unknown optimizer state embed|m"):   # muon.py:155
        C.load_checkpoint(save, p, fewer)
    wrong = {k: dict(v) for k, v in opt.items()}
    wrong["fc_bank"]["v"] = np.zeros((1,), np.float32)
    with pytest.raises(ValueError, match="shape mismatch for fc_bank"):       # muon.py:156
        C.load_checkpoint(save, p, wrong)


def test_zero_d_state_keeps_its_shape(tmp_path):
    """The optimizer's step counter is a 0-d array ("_step|t", muon.py:143):
    written and read back it stays 0-d, as a reference file holds it."""
    from safetensors.numpy import load_file, save_file
    st = {"_step": {"t": np.array(3.0, dtype=np.float32)},
          "embed": {"m": np.zeros((2, 3), np.float32)[:, ::2]}}     # non-contiguous too
    flat = C.flatten_opt_state(st)
    assert flat["_step|t"].shape == ()
    assert flat["embed|m"].flags.c_contiguous and flat["embed|m"].shape == (2, 2)
    path = str(tmp_path / "s.opt.safetensors")
    save_file(flat, path)
    back = C.unflatten_opt_state(load_file(path), st)
    assert back["_step"]["t"].shape == () and float(back["_step"]["t"]) == 3.0
