"""Pins the CPU oracle (oracle/) against the reference's own known-answer
tests and against what the mathematics fixes.  CPU only."""

import math

import numpy as np
import pytest
import torch

import oracle.ref_model as R
import oracle.ref_sample as S
from attention_nn_amd.config import GPTConfig, cfg_155m, cfg_small_h4, sample_config
from attention_nn_amd.weights import init_params, param_count, perturb_lambdas


def _golden():
    """Known-answer values from outside this code base (tests/golden)."""
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "reference_golden.json")) as f:
        return json.load(f)


# ---- kernels: the reference self-tests (metal_kernels.py:334-407) ----------

def test_relu2_kat():
    # metal_kernels.py:339-343: default_rng(0) normal (64, 33), vs max(x,0)**2, atol 1e-6
    rng = np.random.default_rng(0)
    x = rng.standard_normal((64, 33)).astype(np.float32)
    y = R.relu2_f32(torch.from_numpy(x)).numpy()
    assert np.allclose(y, np.maximum(x, 0) ** 2, atol=1e-6)
    # bf16 storage rounds the fp32 result once
    yb = R.relu2(torch.from_numpy(x))
    assert torch.equal(yb, torch.from_numpy(np.maximum(x, 0) ** 2).to(torch.bfloat16).float())


def _rope_reference_loop(xn, csn, snn):
    """The reference's explicit pair loop (metal_kernels.py:356-362)."""
    D = xn.shape[-1]
    refn = xn.copy()
    for d2 in range(D // 4):
        c = csn[:, d2][None, :, None]
        s = snn[:, d2][None, :, None]
        x0, x1 = xn[..., 2 * d2], xn[..., 2 * d2 + 1]
        refn[..., 2 * d2] = c * x0 + s * x1
        refn[..., 2 * d2 + 1] = c * x1 - s * x0
    return refn


def test_rope_kat():
    # metal_kernels.py:349-363: (B,T,H,D)=(2,16,3,64), default_rng(0), atol 1e-5
    rng = np.random.default_rng(0)
    B, T, H, D = 2, 16, 3, 64
    cs, sn = R.rope_tables(T, D)
    x = rng.standard_normal((B, T, H, D)).astype(np.float32)
    out = R.rope_ht_f32(torch.from_numpy(x), cs, sn, torch.arange(T)).numpy()
    ref = _rope_reference_loop(x, cs.numpy(), sn.numpy())
    assert np.allclose(out, ref, atol=1e-5)
    # half-truncation: the second half of each head passes through untouched
    assert np.array_equal(out[..., D // 2:], x[..., D // 2:])


def test_rope_tables_closed_form():
    # metal_kernels.py:144-150: freqs = (1/base)**linspace(0,1,D/4), theta = t*freq
    cs, sn = R.rope_tables(1024, 128, 1024.0)
    assert cs.shape == (1024, 32)
    d4 = 32
    freqs = (1.0 / 1024.0) ** (np.arange(d4) / (d4 - 1))
    th = np.arange(1024)[:, None] * freqs[None, :]
    assert np.allclose(cs.numpy(), np.cos(th), atol=2e-4)
    assert np.allclose(sn.numpy(), np.sin(th), atol=2e-4)
    assert torch.all(cs[0] == 1) and torch.all(sn[0] == 0)
    assert math.isclose(math.atan2(sn[1, -1].item(), cs[1, -1].item()), 1 / 1024, rel_tol=1e-5)
    assert math.isclose(math.atan2(sn[1, 0].item(), cs[1, 0].item()), 1.0, rel_tol=1e-6)


def test_rope_is_rotation():
    # rotation preserves the norm of each pair; inverse rotation undoes it
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.standard_normal((1, 8, 2, 128)).astype(np.float32))
    cs, sn = R.rope_tables(8, 128)
    y = R.rope_ht_f32(x, cs, sn, torch.arange(8))
    n_x = x[..., :64].reshape(1, 8, 2, 32, 2).norm(dim=-1)
    n_y = y[..., :64].reshape(1, 8, 2, 32, 2).norm(dim=-1)
    assert torch.allclose(n_x, n_y, atol=1e-5)
    back = R.rope_ht_f32(y, cs, -sn, torch.arange(8))
    assert torch.allclose(back, x, atol=1e-5)


def test_rms_textbook():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 768)).astype(np.float32) * 3
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.allclose(R.rms_f32(torch.from_numpy(x)).numpy(), ref, atol=1e-5)
    y = R.rms_f32(torch.from_numpy(x)).double()
    assert torch.allclose((y * y).mean(-1), torch.ones(5, dtype=torch.float64), atol=1e-5)
    # scale invariance (eps aside)
    assert torch.allclose(R.rms_f32(torch.from_numpy(x * 7)), R.rms_f32(torch.from_numpy(x)),
                          atol=1e-5)


def test_softcap_closed_form():
    z = torch.linspace(-200, 200, 4001)
    c = R.softcap(z)
    assert torch.all(c >= 0) and torch.all(c <= 23)
    assert torch.all(c[1:] >= c[:-1])
    assert R.softcap(torch.tensor([-5.0])).item() == 11.5
    # the reference CE's pure-MLX restatement (model.py:107) uses the same form
    zz = torch.tensor([0.3, -1.2, 4.0])
    assert torch.allclose(R.softcap(zz), 23 / (1 + torch.exp(-(zz + 5) / 7.5)))


# ---- attention: fp64 brute force (pattern of old.mm:2277-2348) --------------

def _attn_brute(q, k, v, scale, window, long_layer):
    B, H, T, D = q.shape
    out = np.zeros((B, H, T, D))
    for b in range(B):
        for h in range(H):
            for i in range(T):
                js = [j for j in range(T) if j <= i and (long_layer or i - j < window)]
                s = np.array([scale * float(np.dot(q[b, h, i], k[b, h, j])) for j in js])
                p = np.exp(s - s.max())
                p /= p.sum()
                for pj, j in zip(p, js):
                    out[b, h, i] += pj * v[b, h, j]
    return out


@pytest.mark.parametrize("long_layer", [False, True])
def test_attention_brute_force(long_layer):
    rng = np.random.default_rng(123)
    B, H, T, D, W = 2, 3, 7, 16, 3
    q, k, v = (rng.normal(0, 0.5, (B, H, T, D)).astype(np.float32) for _ in range(3))
    keep = R.keep_mask(torch.arange(T), torch.arange(T), long_layer, W)
    got = R.attention(*(torch.from_numpy(a) for a in (q, k, v)), keep, 0.1)
    ref = _attn_brute(q, k, v, 0.1, W, long_layer)
    # output rounded once to bf16: |err| <= half an ulp of values below 2
    assert np.abs(got.numpy() - ref).max() < 4e-3


def test_window_equals_full_below_window():
    rng = np.random.default_rng(5)
    q, k, v = (torch.from_numpy(rng.normal(0, 1, (1, 2, 12, 16)).astype(np.float32))
               for _ in range(3))
    t = torch.arange(12)
    a = R.attention(q, k, v, R.keep_mask(t, t, False, 12), 0.1)
    b = R.attention(q, k, v, R.keep_mask(t, t, True, 12), 0.1)
    c = R.attention(q, k, v, R.keep_mask(t, t, False, 4), 0.1)
    assert torch.equal(a, b)
    assert not torch.equal(a, c)


# ---- whole forward ------------------------------------------------------------

def test_param_counts():
    # totals computed from the model.py:52-77 shapes (fixture), and the rounded
    # figures the reference README states: "76.7M params" (README.md:41) and
    # "155M params" (README.md:64)
    g = _golden()["param_counts"]
    assert param_count(cfg_small_h4()) == g["default_d512_L8"]
    assert param_count(cfg_155m()) == g["d768_L11_H6"]
    assert param_count(GPTConfig()) == g["default_d512_L8"]
    assert round(g["default_d512_L8"] / 1e6, 1) == 76.7
    assert round(g["d768_L11_H6"] / 1e6) == 155


def test_sample_config_long_layers():
    # sample.py:31-33
    assert sample_config(768, 11, 6).long_layers == (4, 10)
    assert sample_config(512, 8, 4).long_layers == (3, 7)
    assert sample_config(1536, 24, 12).long_layers == (11, 23)


def test_degenerate_init_known_answer(tiny_cfg):
    p = init_params(tiny_cfg, 0)
    tok = np.random.default_rng(0).integers(0, 512, (2, 32))
    got = R.logits(tiny_cfg, p, tok)
    assert torch.equal(got, R.degenerate_known_answer(tiny_cfg, p, tok))
    # logits of a row depend only on that row's token
    tok2 = tok.copy()
    tok2[:, :-1] = np.random.default_rng(9).integers(0, 512, (2, 31))
    got2 = R.logits(tiny_cfg, p, tok2)
    assert torch.equal(got[:, -1], got2[:, -1])
    # embed = head.T => greedy repeats the last token
    assert np.array_equal(got[:, -1].argmax(-1).numpy(), tok[:, -1])


def _drop(key):
    def f(q):
        if key == "wo":
            ab = q["attn_bank"].copy()
            ab[:, 3] = 0
            q["attn_bank"] = ab
        elif key == "sa_lambdas":
            q[key] = np.ones_like(q[key])
        else:
            q[key] = np.zeros_like(q[key])
    return f


def test_forward_close_to_fp64(tiny_cfg):
    p = perturb_lambdas(init_params(tiny_cfg, 3, dense=True))
    tok = np.random.default_rng(4).integers(0, 512, (2, 32))
    a = R.logits(tiny_cfg, p, tok).double()
    b = R.forward_fp64(tiny_cfg, p, tok)
    assert (a - b).abs().max().item() < 5e-3
    assert (a - b).abs().mean().item() < 4e-4
    # each plausible mistake (a dropped term, a lambda ignored) lands well outside
    for key in ("x0_lambdas", "wo", "proj_bank", "sa_lambdas"):
        q = dict(p)
        _drop(key)(q)
        c = R.logits(tiny_cfg, q, tok).double()
        assert (c - b).abs().mean().item() > 8e-4, key


def test_mlx_sdpa_reading_within_tolerance(tiny_cfg):
    p = init_params(tiny_cfg, 3, dense=True)
    tok = np.random.default_rng(4).integers(0, 512, (2, 32))
    a = R.logits(tiny_cfg, p, tok)
    b = R.logits(tiny_cfg, p, tok, mlx_fallback_attn=True)
    assert (a - b).abs().max().item() < 2e-2


def test_kv_cache_decode_equals_full_recompute(tiny_cfg):
    p = perturb_lambdas(init_params(tiny_cfg, 7, dense=True))
    tok = np.random.default_rng(8).integers(0, 512, (2, 32))
    full = R.logits(tiny_cfg, p, tok)
    prep = R.Prepared(tiny_cfg, p)
    cache = R.KVCache(tiny_cfg.num_layers)
    outs = [R.forward(prep, tok[:, :5], cache)]
    for t in range(5, 32):
        outs.append(R.forward(prep, tok[:, t:t + 1], cache))
    assert (torch.cat(outs, 1) - full).abs().max().item() < 1e-3


# ---- training forward: softcapped CE (metal_kernels.py:153-193) -------------

def test_softcap_ce_matches_torch_cross_entropy():
    """The fused CE restatement against torch's own cross_entropy applied to
    the softcapped logits (an independent library routine)."""
    g = torch.Generator().manual_seed(3)
    z = R.bf(torch.randn(37, 1000, generator=g) * 6)
    tg = torch.randint(0, 1000, (37,), generator=g)
    rows, lse = R.softcap_ce(z, tg)
    ref = torch.nn.functional.cross_entropy(R.softcap(z).double(), tg, reduction="none")
    assert (rows.double() - ref).abs().max().item() < 1e-5
    assert (lse.double() - torch.logsumexp(R.softcap(z).double(), -1)).abs().max().item() < 1e-5
    # a target off by one lands far away
    bad, _ = R.softcap_ce(z, (tg + 1) % 1000)
    assert (bad.double() - ref).abs().max().item() > 0.1


def test_softcap_ce_uniform_is_log_v():
    """Equal logits give every class the same softcapped value: loss = log V."""
    for c in (-30.0, 0.0, 7.5):
        z = torch.full((3, 50304), c)
        rows, _ = R.softcap_ce(z, torch.tensor([0, 17, 50303]))
        assert torch.allclose(rows.double(), torch.full((3,), math.log(50304), dtype=torch.float64),
                              atol=2e-5)


@pytest.mark.parametrize("long_layer", [False, True])
def test_banded_bf16_attention_brute_force(long_layer):
    """The training attention reading (bf16 scores and probabilities) stays
    within bf16 rounding of the fp64 brute force; dropping the scale does not."""
    rng = np.random.default_rng(321)
    B, H, T, D, W = 2, 2, 9, 16, 4
    q, k, v = (rng.normal(0, 0.5, (B, H, T, D)).astype(np.float32) for _ in range(3))
    q, k, v = (R.bf(torch.from_numpy(a)) for a in (q, k, v))
    keep = R.keep_mask(torch.arange(T), torch.arange(T), long_layer, W)
    ref = _attn_brute(q.numpy(), k.numpy(), v.numpy(), 0.1, W, long_layer)
    got = R.attention(q, k, v, keep, 0.1, banded_bf16=True)
    assert np.abs(got.numpy() - ref).max() < 1.5e-2
    unscaled = R.attention(q, k, v, keep, 1.0, banded_bf16=True)
    assert np.abs(unscaled.numpy() - ref).max() > 5e-2


def test_loss_is_torch_cross_entropy_of_the_logits(tiny_cfg):
    """GPT.__call__'s loss = mean CE of the softcapped logits over every row
    and all V columns (torch cross_entropy over the pinned logits), and the
    training attention reading moves it by far less than the tolerance."""
    p = perturb_lambdas(init_params(tiny_cfg, 13, dense=True))
    rng = np.random.default_rng(14)
    tok = rng.integers(0, 512, (2, 24))
    tgt = rng.integers(0, 512, (2, 24))
    mean, rows = R.loss(tiny_cfg, p, tok, tgt, banded_bf16=False)
    lg = R.logits(tiny_cfg, p, tok).reshape(-1, 512).double()
    ref = torch.nn.functional.cross_entropy(lg, torch.from_numpy(tgt).reshape(-1), reduction="none")
    assert (rows.double() - ref).abs().max().item() < 1e-5
    assert abs(mean.item() - ref.mean().item()) < 1e-5
    mb, _ = R.loss(tiny_cfg, p, tok, tgt, banded_bf16=True)
    assert abs(mb.item() - mean.item()) < 1e-2


# ---- sampler ----------------------------------------------------------------

def test_philox_random123_kat():
    # Random123 known-answer vectors for philox4x32-10 (tests/golden)
    vecs = _golden()["philox4x32_10"]["vectors"]
    assert len(vecs) == 3
    for v in vecs:
        ctr, key, out = (tuple(int(x, 16) for x in v[k]) for k in ("ctr", "key", "out"))
        assert S.philox4x32_10(ctr, key) == out


def test_greedy_lowest_index_on_ties():
    z = np.zeros(50304, np.float32)
    z[[10, 7, 50300]] = 3.0
    assert S.sample_row(z, 0.0, 50, 0.5) == 7      # 50300 is outside the 50257 rows


def test_topk_keeps_ties_at_threshold():
    z = np.arange(60, dtype=np.float32)
    z[:20] = 5.0          # 20 entries tied at the k-th value
    _, keep = S.kept_set(np.pad(z, (0, 50257 - 60), constant_values=-1.0), 1.0, 50)
    # the top 40 distinct + all 20 ties at value 5 (the 50th largest)
    assert set(keep.tolist()) == set(range(60)) - set() and len(keep) == 60


def test_categorical_frequencies_chi_square():
    rng = np.random.default_rng(0)
    z = np.full(50304, -1.0, np.float32)
    z[:8] = rng.uniform(10, 12, 8)
    p = S.probabilities(z, 0.8, 5)
    n = 4000
    draws = [S.sample_row(z, 0.8, 5, S.uniform(123, i, 0)) for i in range(n)]
    counts = np.bincount(draws, minlength=50257)[:8]
    expect = p[:8] * n
    mask = expect > 0
    chi2 = (((counts - expect) ** 2)[mask] / expect[mask]).sum()
    assert counts[~mask].sum() == 0          # nothing outside the top-5 set
    assert chi2 < 20.5                       # 4 dof, p ~ 4e-4
