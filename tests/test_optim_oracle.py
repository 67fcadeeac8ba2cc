"""Pins the optimizer oracle (oracle/ref_optim.py).  CPU only."""

import math

import numpy as np
import pytest
import torch

import oracle.ref_optim as O


def _selftest_inputs():
    """The draw sequence of the reference self-test (metal_kernels.py:335-389):
    relu2 x, rope xq, rope ct, then the optimizer arrays."""
    rng = np.random.default_rng(0)
    rng.standard_normal((64, 33))
    rng.standard_normal((2, 16, 3, 64))
    rng.standard_normal((2, 16, 3, 64))
    p = rng.standard_normal(1000).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    buf = rng.standard_normal(512).astype(np.float32)
    gg = rng.standard_normal(512).astype(np.float32)
    return [torch.from_numpy(a) for a in (p, g, buf, gg)]


def test_reference_selftests_adam_momentum_apply():
    """metal_kernels.py:373-398, expectations as the reference states them."""
    p, g, buf, gg = _selftest_inputs()
    pn, mn, vn = O.adam_step(p, g, torch.zeros(1000), torch.zeros(1000), 0.9, 0.99, 1e-10, 0.01,
                             0.05)
    m_ref, v_ref = 0.1 * g, 0.01 * g * g
    u_ref = m_ref / (torch.sqrt(v_ref) + 1e-10) * 0.01
    u_ref = u_ref + p * ((u_ref * p) > 0) * 0.05
    assert torch.allclose(pn, p - u_ref, atol=1e-6)
    geff, bnew = O.muon_momentum(gg, buf, 0.95)
    bref = buf + 0.05 * (gg - buf)
    assert torch.allclose(bnew, bref, atol=1e-6)
    assert torch.allclose(geff, gg + 0.95 * (bref - gg), atol=1e-6)
    pn = O.muon_apply(p, g, 0.02, 1.2)
    assert torch.allclose(pn, p - p * ((g * p) >= 0) * 1.2 * 0.02 - g * 0.02, atol=1e-6)


def test_adam_path_is_torch_adam_without_decay():
    """With adam_wd = 0 the Adam rule of MuonAdam is torch.optim.Adam (same
    bias correction; eps moves inside the sqrt scaling, negligible at 1e-10)."""
    torch.manual_seed(0)
    p0 = torch.randn(64, 32)
    opt = O.MuonAdam({"embed": p0}, {"embed": {"optim": "adam", "adam_betas": (0.5, 0.95)}},
                     adam_lr=0.01, adam_wd=0.0)
    tp = p0.clone().requires_grad_(True)
    ta = torch.optim.Adam([tp], lr=0.01, betas=(0.5, 0.95), eps=1e-10)
    p = {"embed": p0.clone()}
    for _ in range(4):
        g = torch.randn(64, 32)
        p = opt(p, {"embed": g})
        tp.grad = g.clone()
        ta.step()
    assert torch.allclose(p["embed"], tp.detach(), atol=2e-6)


@pytest.mark.parametrize("shape", [(2, 64, 64), (2, 64, 192), (1, 192, 64)])
def test_polar_express_orthogonalizes(shape):
    """Singular values land near 1 (the Polar Express contract), the result is
    close to the exact polar factor U V^T of an SVD, and the bf16 chain stays
    close to the unrounded fp64 iteration."""
    torch.manual_seed(1)
    g = torch.randn(shape)
    x = O.polar_express(g)
    # five iterations with these coefficients leave the singular values in
    # about [0.86, 1.14] (fp64 measured); bf16 widens that a little
    s = torch.linalg.svdvals(x.double())
    assert s.min().item() > 0.78 and s.max().item() < 1.2
    U, _, Vh = torch.linalg.svd(g.double(), full_matrices=False)
    polar = U @ Vh
    assert ((x.double() - polar).norm() / polar.norm()).item() < 0.15     # measured 0.10
    x64 = O.polar_express_fp64(g)
    assert ((x.double() - x64).norm() / x64.norm()).item() < 0.12        # measured 0.08
    # the raw input is far from orthogonal: the check has teeth
    gn = g.double() / g.double().norm(dim=(-2, -1), keepdim=True)
    assert ((gn - polar).norm() / polar.norm()).item() > 0.5
    # unrounded coefficients: the same to bf16 noise
    xr = O.polar_express(g, round_coeffs=False)
    assert ((x - xr).norm() / xr.norm()).item() < 0.12


def test_polar_express_scale_and_transpose():
    torch.manual_seed(2)
    g = torch.randn(1, 64, 128)
    x = O.polar_express(g)
    assert ((O.polar_express(g * 37.0) - x).norm() / x.norm()).item() < 0.02
    xt = O.polar_express(g.transpose(-2, -1).contiguous())
    assert ((xt.transpose(-2, -1) - x).norm() / x.norm()).item() < 0.02
    # a dropped coefficient (c = 0) lands far away
    good = O.polar_express_fp64(g)
    coeffs = O.POLAR_EXPRESS_COEFFS
    O.POLAR_EXPRESS_COEFFS = [(a, b, 0.0) for a, b, _ in coeffs]
    try:
        bad = O.polar_express_fp64(g)
    finally:
        O.POLAR_EXPRESS_COEFFS = coeffs
    assert ((bad - good).norm() / good.norm()).item() > 0.05


@pytest.mark.parametrize("shape", [(3, 96, 64), (2, 64, 160)])
def test_normuon_first_step_closed_form(shape):
    """From zero second moments: every line (row if M >= N, else column) gets
    the same norm ||v||_F / sqrt(lines) and the Frobenius norm is kept."""
    torch.manual_seed(3)
    v = torch.randn(shape) * torch.rand(shape[0], shape[1], 1)
    M, N = shape[-2], shape[-1]
    red = -1 if M >= N else -2
    sm0 = torch.zeros([s if i != (len(shape) + red) else 1 for i, s in enumerate(shape)])
    out, sm = O.normuon_rescale(v, sm0, 0.9)
    lines = out.norm(dim=red)
    fro = v.norm(dim=(-2, -1))
    nl = M if M >= N else N
    assert torch.allclose(lines, (fro / math.sqrt(nl))[:, None].expand_as(lines), rtol=1e-4)
    assert torch.allclose(out.norm(dim=(-2, -1)), fro, rtol=1e-4)
    assert torch.allclose(sm, 0.1 * (v * v).mean(dim=red, keepdim=True), rtol=1e-6)


# ---- first-step closed forms with weight decay on (muon.py:104-137) --------

def test_adam_first_step_closed_form_with_decay():
    """From zero state, step t = 1: m = (1-b1) g, v = (1-b2) g^2, the bias
    corrections cancel them, so the step is lr * sign(g) (eps aside); the
    cautious decay subtracts lr^2 * adam_wd * wd_mul * p where sign(g) =
    sign(p).  Pins lr_mul, wd_mul and the lr^2 form of the decay."""
    torch.manual_seed(5)
    p0 = torch.randn(40, 24)
    g = torch.randn(40, 24)
    table = {"embed": {"optim": "adam", "adam_betas": (0.5, 0.95), "wd_mul": 150.0},
             "x0_lambdas": {"optim": "adam", "adam_betas": (0.9, 0.95), "lr_mul": 5.0,
                            "wd_mul": 0.0}}
    lr, wd = 0.008, 0.005
    opt = O.MuonAdam({"embed": p0, "x0_lambdas": p0}, table, adam_lr=lr, adam_wd=wd)
    out = opt({"embed": p0.clone(), "x0_lambdas": p0.clone()},
              {"embed": g.clone(), "x0_lambdas": g.clone()}, lr_scale=0.5)
    lr_e = lr * 0.5
    same = (torch.sign(g) == torch.sign(p0)).float()
    want_e = p0 - lr_e * torch.sign(g) - same * (lr_e * lr_e * wd * 150.0) * p0
    assert torch.allclose(out["embed"], want_e, atol=1e-6)
    lr_l = lr * 5.0 * 0.5
    want_l = p0 - lr_l * torch.sign(g)                     # wd_mul = 0: no decay
    assert torch.allclose(out["x0_lambdas"], want_l, atol=1e-6)
    # the decay term has teeth: its size here against the tolerance
    assert (same * (lr_e * lr_e * wd * 150.0) * p0).abs().max().item() > 1e-5


def test_adam_second_step_bias_correction():
    """t = 2 with a constant gradient: m = (1 - b1^2) g, v = (1 - b2^2) g^2 after
    two steps, and the bias corrections (1 - b^2) cancel them again: the
    second step is lr * sign(g) as well."""
    p0 = torch.linspace(-1, 1, 50)
    g = torch.linspace(0.5, -0.7, 50)
    opt = O.MuonAdam({"embed": p0}, {"embed": {"optim": "adam", "adam_betas": (0.5, 0.95)}},
                     adam_lr=0.01, adam_wd=0.0)
    p1 = opt({"embed": p0}, {"embed": g})["embed"]
    p2 = opt({"embed": p1}, {"embed": g})["embed"]
    assert torch.allclose(p2, p0 - 2 * 0.01 * torch.sign(g), atol=1e-6)


@pytest.mark.parametrize("shape,shape_mul", [((2, 64, 64), 1.0), ((2, 128, 64), 2 ** 0.5),
                                             ((1, 256, 64), 2.0), ((1, 64, 192), 1.0)])
def test_muon_first_step_closed_form(shape, shape_mul):
    """From zero state: g_eff = (1 - mu^2) g (Nesterov momentum from an empty
    buffer); Polar Express is scale invariant, so u = PE(g); NorMuon's first
    step keeps ||u||_F.  With p = 0 there is no decay and the update is
    -lr * shape_mul * lr_scale * NorMuon(PE(g)): its norm is
    lr * shape_mul * lr_scale * ||PE(g)||_F, tall banks sqrt(M/N) larger."""
    torch.manual_seed(6)
    g = torch.randn(shape)
    lr, lrs = 0.023, 0.7
    opt = O.MuonAdam({"b": torch.zeros(shape)}, {"b": {"optim": "muon"}}, muon_lr=lr)
    d = opt({"b": torch.zeros(shape)}, {"b": g}, lr_scale=lrs)["b"]
    # g_eff from the momentum kernel the reference's own self-test pins; it is
    # (1 - mu^2) g up to fp32 rounding, and PE is sensitive at the ulp level
    g_eff, _ = O.muon_momentum(g, torch.zeros(shape), 0.95)
    assert torch.allclose(g_eff, (1 - 0.95 ** 2) * g, rtol=1e-5, atol=1e-7)
    u = O.polar_express(g_eff).float()
    want = lr * shape_mul * lrs * u.norm(dim=(-2, -1))
    assert torch.allclose(d.norm(dim=(-2, -1)), want, rtol=1e-4)
    assert opt.table["b"]["shape_mul"] == pytest.approx(shape_mul)
    # direction: -NorMuon(PE(g_eff)) from a zero second moment
    nm, _ = O.normuon_rescale(u, torch.zeros_like(opt.state["b"]["second_mom"]), 0.9)
    assert torch.allclose(d, -lr * shape_mul * lrs * nm, atol=1e-7)


def test_muon_cautious_decay_closed_form():
    """p != 0: where u * p >= 0 the parameter also shrinks by the factor
    (1 - muon_wd * muon_lr * lr_scale * lr_eff), lr_eff = muon_lr * shape_mul *
    lr_scale; elsewhere only -lr_eff * u."""
    torch.manual_seed(7)
    shape = (1, 128, 64)
    g = torch.randn(shape)
    p0 = torch.randn(shape) * 0.1
    mlr, mwd, lrs = 0.023, 1.2, 0.9
    opt = O.MuonAdam({"b": p0}, {"b": {"optim": "muon"}}, muon_lr=mlr, muon_wd=mwd)
    p1 = opt({"b": p0}, {"b": g}, lr_scale=lrs)["b"]
    lr_eff = mlr * 2 ** 0.5 * lrs
    # a fresh optimizer from p = 0 gives the first-step u (closed form above)
    fresh = O.MuonAdam({"b": p0}, {"b": {"optim": "muon"}}, muon_lr=mlr, muon_wd=mwd)
    u = -fresh({"b": torch.zeros(shape)}, {"b": g}, lr_scale=lrs)["b"] / lr_eff
    keep = ((u * p0) >= 0).float()
    decay = mwd * mlr * lrs * lr_eff
    want = p0 - keep * decay * p0 - lr_eff * u
    assert torch.allclose(p1, want, atol=1e-6)
    assert (keep * decay * p0).abs().max().item() > 1e-5
