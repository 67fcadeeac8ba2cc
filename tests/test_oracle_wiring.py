"""Pins the wiring of the oracle's dense forward (reference ``model.py:236-263``)
with closed-form special cases computed in numpy from the equations, never
through the oracle's own forward.  CPU only.

Three weight settings make the forward solvable by hand:

* ``Wq = Wk = 0`` and ``fc = 0``: q and k are zero after QK-norm
  (rms(0) = 0), every kept score is 0, so attention is the plain mean of the
  kept v rows; the MLP branch is exactly 0.  Pins the mask (window / full),
  the v slice of ``qkv_w``, ``sa[l,0]``, ``sa[l,1]``, ``resid[l,0]``,
  ``post[l,0]``, ``x0_lambdas`` and ``resid[l,1]``.
* ``Wv = 0``: the attention output is exactly 0 whatever q and k are; the MLP
  is dense.  Pins ``resid[l,1]``, ``post[l,1]``, where relu^2 sits, and again
  ``resid[l,0]`` / ``x0_lambdas``.

Every lambda slot and layer gets a distinct value, so an index swap changes
the answer.  Each planted mistake (on the CPU, in the oracle) must then move
the oracle away from the closed form by far more than the rounding slack.

The comparison is on the normalised final hidden state rms(x_L) (what the
lm_head multiplies), in bf16 ulps, and on the softcapped logits.  Swapping
``sa[l,0]`` and ``sa[l,1]`` is not a detectable mistake: q and k are
RMS-normalised, so ``sa[l,0]`` scales only v and ``sa[l,1]`` only Wo, and the
output depends on their product alone (up to rounding).
"""

import numpy as np
import pytest
import torch

import oracle.ref_model as R
from attention_nn_amd.config import GPTConfig
from attention_nn_amd.weights import init_params


# ---- numpy bf16 arithmetic (own rounding, independent of torch) --------------

def bf(a):
    """Round fp32 values to bf16 (round to nearest, ties to even), as fp32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def rms_bf(x):
    x64 = x.astype(np.float64)
    return bf((x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6)).astype(np.float32))


def mm_bf(a, b):
    """bf16 matmul: exact products, fp64 accumulation, one rounding."""
    return bf((a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32))


def softcap(z):
    return (23.0 / (1.0 + np.exp(-(z.astype(np.float64) + 5.0) / 7.5))).astype(np.float32)


CFG = GPTConfig(vocab_size=512, num_layers=3, num_heads=2, model_dim=64, seq_len=32, window=5,
                long_layers=(1,))


def _params(seed, zero):
    """Dense init with distinct lambdas per slot and layer, and the named
    weight blocks zeroed ('q', 'k', 'v', 'fc')."""
    p = init_params(CFG, seed, dense=True)
    L = CFG.num_layers
    lay = np.arange(L, dtype=np.float32)[:, None]
    p["resid_lambdas"] = (np.array([[1.25, 0.8125]], np.float32) + 0.0625 * lay).astype(np.float32)
    p["post_lambdas"] = (np.array([[0.625, 1.375]], np.float32) - 0.03125 * lay).astype(np.float32)
    p["x0_lambdas"] = (0.375 + 0.125 * np.arange(L)).astype(np.float32)
    p["sa_lambdas"] = (np.array([[0.75, 1.5]], np.float32) + 0.09375 * lay).astype(np.float32)
    ab = p["attn_bank"].copy()
    for name, slot in (("q", 0), ("k", 1), ("v", 2)):
        if name in zero:
            ab[:, slot] = 0
    p["attn_bank"] = ab
    if "fc" in zero:
        p["fc_bank"] = np.zeros_like(p["fc_bank"])
    return p


def _embed(p, tok):
    return rms_bf(bf(p["embed"])[tok])


def _head(p, x):
    h = rms_bf(x)
    return h, softcap(mm_bf(h, bf(p["lm_head"])))


def closed_form_uniform_attention(p, tok):
    """Wq = Wk = 0, fc = 0: attention = mean of the kept v rows, MLP = 0."""
    B, T = tok.shape
    d, H = CFG.model_dim, CFG.num_heads
    Dh = d // H
    res, post, x0l, sal = (bf(p[k]) for k in ("resid_lambdas", "post_lambdas", "x0_lambdas",
                                               "sa_lambdas"))
    x = _embed(p, tok)
    x0 = x
    for l in range(CFG.num_layers):
        wv = bf(bf(p["attn_bank"][l, 2]) * sal[l, 0])
        wo = bf(bf(p["attn_bank"][l, 3]) * sal[l, 1])
        v = mm_bf(rms_bf(x), wv).reshape(B, T, H, Dh)
        # mean over the kept keys via prefix sums (fp64), rounded once
        cs = np.concatenate([np.zeros((B, 1, H, Dh)), np.cumsum(v.astype(np.float64), 1)], 1)
        y = np.empty((B, T, H, Dh), np.float32)
        for i in range(T):
            lo = 0 if l in CFG.long_layers else max(0, i - CFG.window + 1)
            y[:, i] = ((cs[:, i + 1] - cs[:, lo]) / (i + 1 - lo)).astype(np.float32)
        o = mm_bf(bf(y).reshape(B, T, d), wo)
        x = bf(bf(bf(res[l, 0] * x) + bf(post[l, 0] * o)) + bf(x0l[l] * x0))
        x = bf(res[l, 1] * x)                      # + post * 0 adds nothing
    return _head(p, x)


def closed_form_zero_v(p, tok):
    """Wv = 0: the attention output is 0; the MLP is dense."""
    res, post, x0l = (bf(p[k]) for k in ("resid_lambdas", "post_lambdas", "x0_lambdas"))
    x = _embed(p, tok)
    x0 = x
    for l in range(CFG.num_layers):
        x = bf(bf(res[l, 0] * x) + bf(x0l[l] * x0))      # post * 0 adds nothing
        u = mm_bf(rms_bf(x), bf(p["fc_bank"][l]))
        a = bf(np.maximum(u, 0).astype(np.float32) ** 2)
        y = mm_bf(a, bf(p["proj_bank"][l]))
        x = bf(bf(res[l, 1] * x) + bf(post[l, 1] * y))
    return _head(p, x)


def _tokens():
    return np.random.default_rng(17).integers(0, CFG.vocab_size, (2, 14))


def _oracle(p, tok, cfg=CFG):
    out, _, hfin = R.forward(R.Prepared(cfg, p), tok, return_hidden=True)
    return hfin.numpy(), out.numpy()


def _gap(got, want):
    """(largest gap of rms(x_L) in units of the bf16 spacing at 1.0 -- its rows
    have unit RMS --, fraction of its elements off by more than that spacing,
    largest logit gap)."""
    u = np.abs(got[0].astype(np.float64) - want[0]) / 2.0 ** -7
    return u.max(), (u > 1.0).mean(), np.abs(got[1].astype(np.float64) - want[1]).max()


def _matches(g):
    # accumulation order (fp32 vs fp64 sums) may flip a bf16 rounding: an
    # element of the hidden state may sit an ulp or two off
    umax, frac, lmax = g
    return umax <= 4 and frac < 0.02 and lmax < 2e-3


def _differs(g):
    return g[1] > 0.05


CASES = {
    "uniform_attention": (("q", "k", "fc"), closed_form_uniform_attention),
    "zero_v": (("v",), closed_form_zero_v),
}


@pytest.mark.parametrize("case", list(CASES))
def test_oracle_equals_closed_form(case):
    zero, fn = CASES[case]
    p = _params(3, zero)
    tok = _tokens()
    g = _gap(_oracle(p, tok), fn(p, tok))
    assert _matches(g), g


def test_window_matters_in_the_uniform_case():
    """The closed form's mask is not vacuous: with every layer full-causal
    (or the window wider than the context) the answer moves."""
    p = _params(3, ("q", "k", "fc"))
    tok = _tokens()
    full = GPTConfig(**{**CFG.__dict__, "long_layers": (0, 1, 2)})
    g = _gap(_oracle(p, tok, full), closed_form_uniform_attention(p, tok))
    assert _differs(g), g


def _swap_cols(key):
    def f(p):
        q = dict(p)
        q[key] = np.ascontiguousarray(p[key][:, ::-1])
        return q
    return f


def _swap_slots(a, b):
    def f(p):
        q = dict(p)
        ab = p["attn_bank"].copy()
        ab[:, [a, b]] = ab[:, [b, a]]
        q["attn_bank"] = ab
        return q
    return f


def _reverse_layers(key):
    def f(p):
        q = dict(p)
        q[key] = np.ascontiguousarray(p[key][::-1])
        return q
    return f


# planted mistakes expressible as a transformed input to the unchanged oracle:
# the oracle reading index j where the reference reads index i
PARAM_MUTATIONS = {
    "resid[l,0]<->resid[l,1]": _swap_cols("resid_lambdas"),
    "post[l,0]<->post[l,1]": _swap_cols("post_lambdas"),
    "k<->v slice": _swap_slots(1, 2),
    "q<->v slice": _swap_slots(0, 2),
    "x0_lambdas layer order": _reverse_layers("x0_lambdas"),
    "resid layer order": _reverse_layers("resid_lambdas"),
}


@pytest.mark.parametrize("mut", list(PARAM_MUTATIONS))
def test_planted_index_mistakes_fail(mut):
    """A mistake whose slot is inert in one case (post[l,1] times a zero MLP)
    must be caught by the other; every planted mistake by at least one."""
    tok = _tokens()
    caught = []
    for case, (zero, fn) in CASES.items():
        p = _params(3, zero)
        if _differs(_gap(_oracle(PARAM_MUTATIONS[mut](p), tok), fn(p, tok))):
            caught.append(case)
    assert caught, f"no closed-form case detects the planted mistake {mut}"


# planted mistakes in the oracle's code: replace one of its wiring functions
def _x0_in_mlp_mix(monkeypatch):
    monkeypatch.setattr(R, "mix_attn", lambda x, y, x0, r0, p0, xl: R.bf(R.bf(r0 * x) + R.bf(p0 * y)))
    monkeypatch.setattr(R, "mix_mlp", lambda x, y, x0, r1, p1, xl:
                        R.bf(R.bf(R.bf(r1 * x) + R.bf(p1 * y)) + R.bf(xl * x0)))


def _relu2_after_proj(monkeypatch):
    monkeypatch.setattr(R, "mlp_branch", lambda h, fc, proj: R.relu2(R.bf(R.bf(h @ fc) @ proj)))


def _relu_not_squared(monkeypatch):
    monkeypatch.setattr(R, "mlp_branch",
                        lambda h, fc, proj: R.bf(R.bf(torch.clamp_min(R.bf(h @ fc), 0)) @ proj))


def _mix_order(monkeypatch):
    monkeypatch.setattr(R, "mix_attn", lambda x, y, x0, r0, p0, xl:
                        R.bf(R.bf(r0 * x) + R.bf(R.bf(p0 * y) + R.bf(xl * x0))))


def _no_x0(monkeypatch):
    monkeypatch.setattr(R, "mix_attn", lambda x, y, x0, r0, p0, xl: R.bf(R.bf(r0 * x) + R.bf(p0 * y)))


CODE_MUTATIONS = {
    "x0 moved into the MLP mix": (_x0_in_mlp_mix, "uniform_attention"),
    "x0 dropped": (_no_x0, "zero_v"),
    "relu2 after proj": (_relu2_after_proj, "zero_v"),
    "relu not squared": (_relu_not_squared, "zero_v"),
}


@pytest.mark.parametrize("mut", list(CODE_MUTATIONS))
def test_planted_code_mistakes_fail(mut, monkeypatch):
    plant, case = CODE_MUTATIONS[mut]
    zero, fn = CASES[case]
    p = _params(3, zero)
    tok = _tokens()
    want = fn(p, tok)
    plant(monkeypatch)
    g = _gap(_oracle(p, tok), want)
    assert _differs(g), (mut, g)


def test_mix_order_is_below_resolution_but_documented(monkeypatch):
    """Regrouping the three-term sum of model.py:256 changes only roundings:
    the closed forms cannot separate it (both groupings stay within the
    slack), which is why the oracle follows MLX's left-to-right evaluation
    as written rather than as tested."""
    p = _params(3, ("q", "k", "fc"))
    tok = _tokens()
    want = closed_form_uniform_attention(p, tok)
    _mix_order(monkeypatch)
    g = _gap(_oracle(p, tok), want)
    assert not _differs(g), g


# ---- the composed q / k path: QK-norm, RoPE at each row's position, 0.1 scale ----
#
# One layer with fc = 0, so the MLP adds nothing and the output is fixed by
# attention alone (model.py:242-256): q = rope(rms(q)), k = rope(rms(k)) at
# each row's own position, scores 0.1 q.k over the causal keys, a plain
# softmax, P.V.  The brute force below builds the RoPE tables and applies the
# pair rotation with its own loop (the reference's known-answer loop,
# metal_kernels.py:356-362: pairs (2 p, 2 p + 1) for p < D/4 take
# y0 = c x0 + s x1, y1 = c x1 - s x0, the rest pass through) and computes the
# softmax in fp64 -- nothing goes through the oracle's attention or RoPE.

QK_CFG = GPTConfig(vocab_size=512, num_layers=1, num_heads=2, model_dim=128, seq_len=32,
                   window=16, long_layers=(0,))


def _qk_params(seed):
    p = init_params(QK_CFG, seed, dense=True)
    p["resid_lambdas"] = np.array([[0.5, 1.125]], np.float32)
    p["post_lambdas"] = np.array([[1.5, 0.75]], np.float32)
    p["x0_lambdas"] = np.array([0.25], np.float32)
    p["sa_lambdas"] = np.array([[0.875, 1.25]], np.float32)
    p["fc_bank"] = np.zeros_like(p["fc_bank"])
    return p


def _rope_pairs(x, t, base=1024.0):
    """x (H, D) of the row at position t: the pair loop with its own tables."""
    D = x.shape[-1]
    d4 = D // 4
    freqs = np.power(np.float32(1.0 / base), np.linspace(0.0, 1.0, d4, dtype=np.float32))
    theta = (np.float32(t) * freqs).astype(np.float32)
    c, s = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    y = x.astype(np.float32).copy()
    for p2 in range(d4):
        x0, x1 = x[:, 2 * p2].astype(np.float32), x[:, 2 * p2 + 1].astype(np.float32)
        y[:, 2 * p2] = c[p2] * x0 + s[p2] * x1
        y[:, 2 * p2 + 1] = c[p2] * x1 - s[p2] * x0
    return bf(y)


def closed_form_qk_path(p, tok):
    """Brute force of one full-causal layer with fc = 0 (B, T tokens from
    position 0): returns (rms(x_L), softcapped logits)."""
    B, T = tok.shape
    d, H = QK_CFG.model_dim, QK_CFG.num_heads
    Dh = d // H
    res, post, x0l, sal = (bf(p[k]) for k in ("resid_lambdas", "post_lambdas", "x0_lambdas",
                                               "sa_lambdas"))
    ab = p["attn_bank"][0]
    wqkv = bf(np.concatenate([bf(ab[0]), bf(ab[1]), bf(ab[2])], -1) * sal[0, 0])
    wo = bf(bf(ab[3]) * sal[0, 1])
    x = _embed(p, tok)
    x0 = x
    qkv = mm_bf(rms_bf(x), wqkv).reshape(B, T, 3, H, Dh)
    y = np.zeros((B, T, H, Dh), np.float32)
    for b in range(B):
        q = [_rope_pairs(rms_bf(qkv[b, t, 0]), t) for t in range(T)]
        k = [_rope_pairs(rms_bf(qkv[b, t, 1]), t) for t in range(T)]
        v = qkv[b, :, 2].astype(np.float64)
        for i in range(T):
            for h in range(H):
                s = np.array([0.1 * np.dot(q[i][h].astype(np.float64), k[j][h].astype(np.float64))
                              for j in range(i + 1)])
                w = np.exp(s - s.max())
                w /= w.sum()
                y[b, i, h] = (w[:, None] * v[:i + 1, h]).sum(0)
    o = mm_bf(bf(y).reshape(B, T, d), wo)
    x = bf(bf(bf(res[0, 0] * x) + bf(post[0, 0] * o)) + bf(x0l[0] * x0))
    x = bf(res[0, 1] * x)                      # + post * 0 adds nothing
    return _head(p, x)


def _qk_tokens(T):
    return np.random.default_rng(29).integers(0, QK_CFG.vocab_size, (3, T))


@pytest.mark.parametrize("T", [3, 12])
def test_oracle_qk_path_equals_brute_force(T):
    p = _qk_params(7)
    tok = _qk_tokens(T)
    g = _gap(_oracle(p, tok, QK_CFG), closed_form_qk_path(p, tok))
    assert _matches(g), g


def test_oracle_qk_path_decode_equals_brute_force():
    """The same path through the oracle's KV cache: a 1-token prefill, then one
    token per step, every row at its own position (q rotated at t, the cached
    keys at theirs)."""
    p = _qk_params(8)
    tok = _qk_tokens(6)
    want = closed_form_qk_path(p, tok)
    prep = R.Prepared(QK_CFG, p)
    cache = R.KVCache(1)
    rows = [R.forward(prep, tok[:, i:i + 1], cache, return_hidden=True) for i in range(6)]
    got = (torch.cat([r[2] for r in rows], 1).numpy(), torch.cat([r[0] for r in rows], 1).numpy())
    assert _matches(_gap(got, want))


def _plant_scale(monkeypatch):
    f = R.attention
    monkeypatch.setattr(R, "attention", lambda q, k, v, keep, scale, *a, **kw:
                        f(q, k, v, keep, 1.0 / np.sqrt(q.shape[-1]), *a, **kw))


def _plant_rope_q_only(monkeypatch):
    f, calls = R.rope_ht, [0]

    def g(x, cs, sn, pos):
        calls[0] += 1
        return f(x, cs, sn, pos) if calls[0] % 2 == 1 else x   # forward rotates q, then k
    monkeypatch.setattr(R, "rope_ht", g)


def _plant_qk_swap(monkeypatch):
    f = R.attention
    monkeypatch.setattr(R, "attention", lambda q, k, v, *a, **kw: f(k, q, v, *a, **kw))


def _plant_k_at_q_position(monkeypatch):
    # scoring q_i against k_j rotated at position i instead of j: the same
    # rotation on both sides cancels in the dot product, which is the
    # forward with no rotation at all
    monkeypatch.setattr(R, "rope_ht", lambda x, cs, sn, pos: x)


def _plant_inverse_rotation(monkeypatch):
    f = R.rope_ht
    monkeypatch.setattr(R, "rope_ht", lambda x, cs, sn, pos: f(x, cs, -sn, pos))


def _plant_no_qk_norm(monkeypatch):
    f = R.rms
    monkeypatch.setattr(R, "rms", lambda x, eps=1e-6: R.bf(x) if x.dim() == 4 else f(x, eps))


QK_MUTATIONS = {
    "scale 1/sqrt(Dh)": _plant_scale,
    "RoPE on q only": _plant_rope_q_only,
    "q<->k swapped": _plant_qk_swap,
    "k rotated at q's position": _plant_k_at_q_position,
    "inverse rotation": _plant_inverse_rotation,
    "no QK-norm": _plant_no_qk_norm,
}


@pytest.mark.parametrize("mut", list(QK_MUTATIONS))
def test_planted_qk_path_mistakes_fail(mut, monkeypatch):
    p = _qk_params(7)
    tok = _qk_tokens(12)
    want = closed_form_qk_path(p, tok)
    QK_MUTATIONS[mut](monkeypatch)
    g = _gap(_oracle(p, tok, QK_CFG), want)
    assert _differs(g), (mut, g)
