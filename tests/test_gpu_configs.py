"""GPU parity at the model shapes of the benchmark's larger configurations
(reference ``sample.py:42-51`` running ``model.py:223-263``), through the C ABI.

Each test runs the whole batch on the GPU -- so the kernels and tile shapes
those workloads use are the ones exercised -- and checks a few rows against
the oracle's KV-cache forward (batch rows are independent; the oracle
computes the lm_head of the last row only).  Sampled tokens are checked for
every row against the oracle sampler applied to the engine's own logits of
that step (the draws use Philox with counter (step, row)).

Tolerances: the north star's 2e-2 max-abs on softcapped logits; draws equal.
"""

import numpy as np
import pytest
import torch

import oracle.ref_model as R
import oracle.ref_sample as S
from attention_nn_amd.config import GPTConfig, cfg_small_h4
from attention_nn_amd.weights import init_params, perturb_lambdas
from tests.test_gpu_parity import LOGIT_TOL, _greedy_gpu, _sample_small

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import attention_nn_amd._lib as L
    L.lib()


def _engine(cfg, params, B, ctx, tokens):
    from attention_nn_amd.engine import Engine
    return Engine(cfg, params, max_batch=B, max_ctx=ctx, max_tokens=tokens)


def _run_case(cfg, params, B, T0, steps, rows, temp, k, seed, ctx):
    """Prefill B prompts of T0 tokens, then `steps` teacher-forced decode
    steps, all with (temp, k) sampling and logits; returns the worst logit
    gap over the checked rows and the number of draws checked."""
    rng = np.random.default_rng(B * 7 + T0)
    tok = rng.integers(0, min(50257, cfg.vocab_size), (B, T0 + steps))
    eng = _engine(cfg, params, B, ctx, B * T0)
    prep = R.Prepared(cfg, params)
    cache = R.KVCache(cfg.num_layers)
    print(f"  prefill B={B} T={T0}", flush=True)
    nxt, lg = eng.prefill(tok[:, :T0], temp, k, seed=seed, step=0, want_logits=True)
    ref = R.forward(prep, tok[rows, :T0], cache, last_only=True)[:, -1]
    lg_rows = lg[rows].cpu()
    worst = (lg_rows - ref).abs().max().item()
    draws = _check_draws(nxt, lg, temp, k, seed, 0, cfg.vocab_size)
    for i in range(steps - 1):
        t = tok[:, T0 + i]
        print(f"  decode step {i} at position {T0 + i}", flush=True)
        nxt, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), temp, k, seed=seed,
                             step=i + 1, want_logits=True)
        ref = R.forward(prep, t[rows, None], cache, last_only=True)[:, -1]
        worst = max(worst, (lg[rows].cpu() - ref).abs().max().item())
        draws += _check_draws(nxt, lg, temp, k, seed, i + 1, cfg.vocab_size)
    eng.check_device()
    return worst, draws


def _check_draws(nxt, lg, temp, k, seed, step, V):
    if temp == 0.0:
        want = lg[:, :min(50257, V)].argmax(-1).to(torch.int32)
        assert torch.equal(nxt, want), step
        return nxt.numel()
    lg = lg.cpu().numpy()
    got = nxt.cpu().numpy()
    for b in range(lg.shape[0]):
        z = lg[b, :min(50257, V)]
        assert int(got[b]) == _sample_small(z, temp, k, S.uniform(seed, step, b)), (step, b)
    return lg.shape[0]


def test_cfg3_shape_b64_prefill512_topk50():
    """cfg3's shapes: d768 H6 x 128 at the full vocabulary (V = 50304, sampled
    over 50257), 64 sequences, a 512-token prefill (one 512-query block), then
    decode steps at 64 rows -- the skinny MFMA decode GEMMs at K = 768 and
    33-64 rows, the decode attention at 64 x 6 heads, the top-k sampler over
    the real vocabulary (1024 threads x 56 keys, partial last thread) at
    T = 0.8, k = 50.  Three layers, layer 1 full-causal."""
    cfg = GPTConfig(num_layers=3, num_heads=6, model_dim=768, seq_len=1024, window=384,
                    long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 51, dense=True))
    print("case cfg3 shape: d768 L3 V50304 B=64 T0=512, T=0.8 top-k 50", flush=True)
    worst, draws = _run_case(cfg, p, 64, 512, 4, [0, 29, 63], 0.8, 50, 2024, 1024)
    assert worst < LOGIT_TOL, worst
    assert draws == 64 * 4


@pytest.mark.parametrize("route", ["candidates", "z", "persistent"])
@pytest.mark.parametrize("case", ["period600", "levels"])
def test_sampler_tied_logits_full_vocab(case, route, monkeypatch):
    """The top-k sampler over the real vocabulary with tied logits (k = 50,
    T = 0.8).  period600: lm_head columns repeat with period 600, so each
    logit value has ~84 copies, at most one per thread's 56 entries; the top
    value's copies are all kept and fill the candidate list.  levels: every
    column is one of three multiples of one vector (30, 2000 and the rest of
    the columns), so 2030 or ~48,000 keys reach the per-thread-maxima bound
    and the sampler falls back to its block-wide bisection from that bound.
    Each sampler input: the lm_head's top-k candidates at 8 rows (levels:
    every tile holds more tied keys than its 8 candidates, so each row is
    recomputed), z (ANN_TOPK_CAND=0), and at 2 rows the persistent step's
    candidates with its z as the fallback.  Draws against the oracle sampler
    on the engine's own logits."""
    monkeypatch.setenv("ANN_TOPK_CAND", "0" if route == "z" else "1")
    cfg = GPTConfig(num_layers=2, num_heads=2, model_dim=256, seq_len=128, window=16,
                    long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 61, dense=True))
    V = cfg.vocab_size
    h = p["lm_head"]
    if case == "period600":
        p["lm_head"] = np.ascontiguousarray(h[:, np.arange(V) % 600] * 40)
    else:
        level = np.full(V, 2)
        perm = np.random.default_rng(5).permutation(V)
        level[perm[:30]], level[perm[30:2030]] = 0, 1
        alpha = np.array([3.0, 2.0, 1.0], dtype=np.float32)
        p["lm_head"] = np.ascontiguousarray(h[:, :1] * 40 * alpha[level][None, :])
    B, T0, temp, k, seed = 2 if route == "persistent" else 8, 16, 0.8, 50, 99
    print(f"case sampler ties {case} {route}: d256 L2 V50304 B={B}, T=0.8 top-k 50", flush=True)
    tok = np.random.default_rng(7).integers(0, 50257, (B, T0 + 3))
    eng = _engine(cfg, p, B, 64, B * T0)
    nxt, lg = eng.prefill(tok[:, :T0], temp, k, seed=seed, step=0, want_logits=True)
    edge = 0
    for step in range(3):
        if step:
            t = torch.from_numpy(tok[:, T0 + step - 1].astype(np.int32)).cuda()
            nxt, lg = eng.decode(t, temp, k, seed=seed, step=step, want_logits=True)
        z, got = lg.cpu().numpy(), nxt.cpu().numpy()
        for b in range(B):
            r = _draw_position(int(got[b]), z[b, :50257], temp, k, S.uniform(seed, step, b))
            assert r is not None, (case, step, b)
            edge += r
    eng.check_device()
    # with ~48,000 tied maxima u * total keeps ~8 fraction bits in fp32
    assert edge <= 2, edge


def _draw_position(got, z, temp, k, u):
    """0 if `got` is the oracle's draw; 1 if it is the neighbouring kept entry
    across a cumulative boundary within 1e-5 of the total from u * total (the
    device sums fp32 weights and forms u * total in fp32); None otherwise."""
    zt = z.astype(np.float32) / np.float32(temp)
    kth = np.sort(zt)[-k]
    keep = np.nonzero(zt >= kth)[0]
    c = np.cumsum(np.exp(zt[keep].astype(np.float64) - zt[keep].max()))
    t = u * c[-1]
    i = min(int(np.searchsorted(c, t, side="right")), keep.size - 1)
    if keep[i] == got:
        return 0
    j = int(np.searchsorted(keep, got))
    if j >= keep.size or keep[j] != got or abs(j - i) != 1:
        return None
    return 1 if abs(c[min(i, j)] - t) <= 1e-5 * c[-1] else None


@pytest.mark.parametrize("d, H, B", [(256, 2, 16), (256, 2, 80), (768, 6, 64), (1536, 12, 128)])
def test_topk_candidates_recompute_bitwise(d, H, B, monkeypatch):
    """The candidate sampler's recomputation of lm_head tiles is bit-identical
    to the GEMM: with ANN_TOPK_VERIFY=1 every tile of every row is recomputed
    and its 9 largest (key, column) words compared with the GEMM epilogue's
    (a difference fails check_device), and the draws -- now made over the
    recomputed rows -- equal the oracle sampler's on the engine's logits.
    16 and 64 rows run the 64-row lm_head tiles, 80 and 128 the 128-row ones;
    K = 256, 768 (cfg3's dims) and 1536 (cfg5's)."""
    monkeypatch.setenv("ANN_TOPK_VERIFY", "1")
    cfg = GPTConfig(num_layers=1 if d > 768 else 2, num_heads=H, model_dim=d, seq_len=128,
                    window=16, long_layers=(0,) if d > 768 else (1,))
    p = perturb_lambdas(init_params(cfg, 67, dense=True))
    p["lm_head"] = p["lm_head"] * 4
    print(f"case candidate recompute check: d{d} V50304 B={B}, T=0.8 top-k 50", flush=True)
    worst, draws = _run_case(cfg, p, B, 12, 3, [0, B - 1], 0.8, 50, 31, 64)
    assert worst < LOGIT_TOL, worst
    assert draws == B * 3


@pytest.mark.parametrize("V, B", [(50304, 4), (50304, 70), (40000, 4)])
def test_topk_candidates_draws_match_oracle_full_vocab(V, B):
    """Draws over a full vocabulary at the rows the candidate lm_head takes
    (4: 64-row tiles, 70: 128-row tiles; V = 40000 leaves a last tile of 64
    columns and samples over every column), for temperatures 0.5 / 0.8 / 2
    and top_k 1, 2, 5, 50 and 256 (the candidate route's limit), 257 and 0
    (every entry kept: z), plus greedy: each row's draw equals the oracle
    sampler's on the engine's logits (Philox counter (step, row))."""
    cfg = GPTConfig(vocab_size=V, num_layers=2, num_heads=2, model_dim=256, seq_len=64,
                    window=16, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 74, dense=True))
    p["lm_head"] = p["lm_head"] * 8
    print(f"case candidate draws: d256 L2 V{V} B={B}", flush=True)
    tok = np.random.default_rng(75).integers(0, min(V, 50257), (B, 10))
    eng = _engine(cfg, p, B, 64, B * 64)
    cases = [(0.8, 50), (0.5, 1), (2.0, 2), (0.8, 5), (1.0, 256), (0.8, 257), (0.8, 0), (0.0, 0)]
    for step, (temp, k) in enumerate(cases):
        nxt, lg = eng.prefill(tok, temp, k, seed=9, step=step, want_logits=True)
        _check_draws(nxt, lg, temp, k, 9, step, V)
        nxt, lg = eng.decode(nxt, temp, k, seed=9, step=100 + step, want_logits=True)
        _check_draws(nxt, lg, temp, k, 9, 100 + step, V)
    eng.check_device()


def test_topk_candidates_clustered_tile_falls_back():
    """Top keys clustered in one lm_head tile: columns 1000-1039 (tile 7)
    are pairs +-12 u_j, so every row has 11-19 of its 50 largest logits in
    that tile (oracle logits), more than its 8 candidates; the sampler
    recomputes that tile (the other tiles' keys beyond their candidates lie
    below the threshold) and draws over the whole row.  The check repeats at
    top-k 200, and at top-k 5, where the tile's candidates hold its 4-5 kept
    keys and the sampler stays on the candidates.  Draws against the oracle
    sampler on the engine's logits."""
    cfg = GPTConfig(num_layers=2, num_heads=2, model_dim=256, seq_len=128, window=16,
                    long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 68, dense=True))
    h = p["lm_head"] * 2
    # columns 1000 + 2j and 1001 + 2j are +-12 u_j: one of each pair is large
    # and positive for any row
    u = h[:, 1000:1020].copy()
    h[:, 1000:1040:2] = 12 * u
    h[:, 1001:1040:2] = -12 * u
    p["lm_head"] = np.ascontiguousarray(h)
    print("case clustered tile: d256 L2 V50304 B=8", flush=True)
    B, T0 = 8, 12
    tok = np.random.default_rng(69).integers(0, 50257, (B, T0 + 2))
    eng = _engine(cfg, p, B, 64, B * T0)
    for k in (50, 5, 200):
        nxt, lg = eng.prefill(tok[:, :T0], 0.8, k, seed=41, step=k, want_logits=True)
        top = lg[:, :50257].topk(k, dim=-1).indices.cpu().numpy()
        assert ((top >= 1000) & (top < 1040)).sum(axis=1).min() >= min(k - 1, 9), k
        _check_draws(nxt, lg, 0.8, k, 41, k, cfg.vocab_size)
        nxt, lg = eng.decode(torch.from_numpy(tok[:, T0].astype(np.int32)).cuda(), 0.8, k,
                             seed=41, step=k + 1, want_logits=True)
        _check_draws(nxt, lg, 0.8, k, 41, k + 1, cfg.vocab_size)
    eng.check_device()


@pytest.mark.parametrize("B", [1, 3])
def test_persistent_sampled_155m_dims_topk_candidates(B):
    """Sampled decode (T = 0.8, top-k 50) on the persistent step at the 155M
    dims (d768 H6 x 128, V = 50304, two layers): each work-group leaves its
    slice's 8 largest keys and the next one, and the sampler draws from those
    (z only when they cannot prove the kept set).  Logits against the
    oracle's KV-cache forward, every draw against the oracle sampler on the
    engine's logits."""
    cfg = GPTConfig(num_layers=2, num_heads=6, model_dim=768, seq_len=256, window=64,
                    long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 73, dense=True))
    print(f"case persistent sampled 155M dims: L2 B={B}", flush=True)
    worst, draws = _run_case(cfg, p, B, 16, 8, list(range(B)), 0.8, 50, 5, 64)
    assert worst < LOGIT_TOL, worst
    assert draws == B * 8


def test_cfg4_shape_ctx8192_b16():
    """cfg4's shapes: the 155M dims at max_ctx 8192, 16 sequences, a
    7680-token prefill (15 query blocks of 512; the windowed layers read 896
    keys per block, the full layer all of them), then decode steps past 7680
    where the full-causal layer reads every cached key.  Greedy."""
    cfg = GPTConfig(num_layers=3, num_heads=6, model_dim=768, seq_len=8192, window=384,
                    long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 53, dense=True))
    print("case cfg4 shape: d768 L3 ctx8192 B=16 T0=7680 greedy", flush=True)
    worst, draws = _run_case(cfg, p, 16, 7680, 3, [0, 15], 0.0, 0, 0, 8192)
    assert worst < LOGIT_TOL, worst


def test_cfg5_shape_d1536_b128_topk50():
    """cfg5's shapes: d1536 H12 x 128 at the full vocabulary, 128 sequences:
    decode qkv / fc on the 64 x 64 MFMA tiles after the row norm, o / proj
    on the LDS-staged skinny GEMM (proj K = 6144), the lm_head on the
    128-row tiles, top-k 50 at T = 0.8 over 128 rows.  Three layers, layer 1
    full-causal."""
    cfg = GPTConfig(num_layers=3, num_heads=12, model_dim=1536, seq_len=256, window=384,
                    long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 55, dense=True))
    print("case cfg5 shape: d1536 L3 V50304 B=128 T0=64, T=0.8 top-k 50", flush=True)
    worst, draws = _run_case(cfg, p, 128, 64, 4, [0, 77, 127], 0.8, 50, 99, 256)
    assert worst < LOGIT_TOL, worst
    assert draws == 128 * 4


def test_cfg5_full_prompts_d1536_b128_prefill1024_topk50():
    """cfg5 at its own prompt length: d1536 H12 x 128 at the full vocabulary,
    128 sequences of 1024-token prompts -- a 131,072-row prefill (QKV with its
    fused epilogue on the 256 x 256 GEMM, two 512-query blocks per (row, head)
    in the prefill attention) -- then decode steps at positions 1024..1026
    (past the first 1024 keys on the full-causal layer) with T = 0.8, top-k
    50.  Three layers, layer 1 full-causal; rows 0, 77 and 127 against the
    oracle, every row's draw against the oracle sampler."""
    cfg = GPTConfig(num_layers=3, num_heads=12, model_dim=1536, seq_len=1040, window=384,
                    long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 57, dense=True))
    print("case cfg5 full prompts: d1536 L3 V50304 B=128 T0=1024, T=0.8 top-k 50", flush=True)
    worst, draws = _run_case(cfg, p, 128, 1024, 4, [0, 77, 127], 0.8, 50, 7, 1040)
    assert worst < LOGIT_TOL, worst
    assert draws == 128 * 4


def test_cfg1_degenerate_64_greedy_steps():
    """cfg1 as specified (76.7M, model.py init: Wo = proj = x0 = 0), 16-token
    prompt, all 64 greedy steps: every step repeats the last prompt token and
    the logits equal the oracle's closed form."""
    cfg = cfg_small_h4()
    p = init_params(cfg, 0)
    prompt = np.random.default_rng(1).integers(0, 50257, 16)
    print("case cfg1: 76.7M degenerate init, 64 greedy steps", flush=True)
    eng = _engine(cfg, p, 1, 128, 128)
    got, glog = _greedy_gpu(eng, prompt, 64)
    eng.check_device()
    assert got == [int(prompt[-1])] * 64
    ka = R.degenerate_known_answer(cfg, p, prompt[None, -1:])[0, -1]
    assert max((g - ka).abs().max().item() for g in glog) < LOGIT_TOL


def test_cfg1_dense_64_greedy_steps_match_oracle():
    """cfg1's model with the dense init (Wo, proj drawn): 64 greedy steps
    identical to the oracle's greedy decode, logits within tolerance."""
    from tests.test_gpu_parity import _greedy_oracle
    cfg = cfg_small_h4()
    p = perturb_lambdas(init_params(cfg, 0, dense=True))
    prompt = np.random.default_rng(1).integers(0, 50257, 16)
    print("case cfg1 dense: 76.7M, 64 greedy steps vs oracle", flush=True)
    eng = _engine(cfg, p, 1, 128, 128)
    got, glog = _greedy_gpu(eng, prompt, 64)
    eng.check_device()
    ref, rlog = _greedy_oracle(cfg, p, prompt, 64)
    n_same = next((i for i, (a, b) in enumerate(zip(got, ref)) if a != b), 64)
    worst = max((g - r).abs().max().item() for g, r in zip(glog[:n_same], rlog[:n_same]))
    assert worst < LOGIT_TOL, worst
    assert got == ref, f"first divergence at step {n_same}"


# ---- the drop-in API --------------------------------------------------------

def test_sample_api_64_tokens_equals_engine_loop():
    """sample() (ids kept on the device, streamed through pinned memory)
    returns exactly what a plain prefill + decode loop on the engine draws,
    for 64 top-k tokens of a batch of 3, and hands every step to on_token
    in order."""
    from attention_nn_amd.engine import Engine
    from attention_nn_amd.sample import sample
    cfg = GPTConfig(vocab_size=1000, num_layers=2, num_heads=2, model_dim=256, seq_len=96,
                    window=16, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 61, dense=True))
    p["lm_head"] = p["lm_head"] * 40
    prompt = np.random.default_rng(62).integers(0, cfg.vocab_size, (3, 9))
    seen = []
    got = sample(prompt, 64, 0.9, 20, seed=7, params=p, cfg=cfg, on_token=seen.append)
    eng = Engine(cfg, p, max_batch=3, max_ctx=96, max_tokens=3 * 96)
    nxt, _ = eng.prefill(prompt, 0.9, 20, 7, 0)
    want = [nxt.cpu().numpy()]
    for i in range(1, 64):
        nxt, _ = eng.decode(nxt, 0.9, 20, 7, i, out=nxt)
        want.append(nxt.cpu().numpy())
    want = np.stack(want, 1)
    assert np.array_equal(np.asarray(got), want)
    assert len(seen) == 64 and np.array_equal(np.stack(seen, 1), want)
    # batch 1: the persistent step; a single prompt returns a list
    one = sample(list(prompt[0]), 64, 0.0, 0, params=p, cfg=cfg)
    eng1 = Engine(cfg, p, max_batch=1, max_ctx=96, max_tokens=96)
    nxt, _ = eng1.prefill(prompt[:1])
    ref = [int(nxt.item())]
    for i in range(1, 64):
        nxt, _ = eng1.decode(nxt, out=nxt)
        ref.append(int(nxt.item()))
    eng1.check_device()
    assert one == ref


def test_gpt_cache_repacks_on_new_params_not_on_growing_T():
    """GPT.logits re-packs when an entry of the params dict is replaced and
    not when the reference's loop calls it with a growing T."""
    from attention_nn_amd.model import GPT
    cfg = GPTConfig(vocab_size=512, num_layers=2, num_heads=2, model_dim=128, seq_len=64,
                    window=16, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 63, dense=True))
    tok = np.random.default_rng(64).integers(0, 512, (2, 40))
    gpt = GPT(cfg)
    for T in range(1, 40, 7):
        a = gpt.logits(p, tok[:, :T])
    assert gpt.packs == 1
    ref = R.logits(cfg, p, tok[:, :T])
    assert (a.cpu() - ref).abs().max().item() < LOGIT_TOL
    p["lm_head"] = p["lm_head"] * 3          # same dict, new array
    b = gpt.logits(p, tok[:, :T])
    assert gpt.packs == 2
    ref = R.logits(cfg, p, tok[:, :T])
    assert (b.cpu() - ref).abs().max().item() < LOGIT_TOL
    assert (a - b).abs().max().item() > 0.1
    gpt.logits(p, tok[:1, :T])               # a smaller batch reuses the engine
    assert gpt.packs == 2


def test_sampling_state_greedy_after_sampled_and_more_rows():
    """The device sampling state follows each call: a greedy call after a
    sampled one at 12 rows (greedy then runs in the sampler kernel, which
    reads the temperature from the device) returns the argmax; a sampled
    call with more rows than the previous one draws every row with its own
    (step, row) counter."""
    cfg = GPTConfig(vocab_size=1000, num_layers=2, num_heads=2, model_dim=256, seq_len=64,
                    window=16, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 65, dense=True))
    p["lm_head"] = p["lm_head"] * 40
    tok = np.random.default_rng(66).integers(0, cfg.vocab_size, (12, 7))
    eng = _engine(cfg, p, 12, 64, 12 * 64)
    print("case sampling state: 12 rows sampled -> greedy -> 4 rows -> 12 rows", flush=True)
    nxt, lg = eng.prefill(tok, 0.8, 50, seed=3, step=0, want_logits=True)
    _check_draws(nxt, lg, 0.8, 50, 3, 0, cfg.vocab_size)
    nxt, lg = eng.prefill(tok, 0.0, 0, want_logits=True)
    _check_draws(nxt, lg, 0.0, 0, 0, 0, cfg.vocab_size)
    nxt, lg = eng.prefill(tok[:4], 0.9, 10, seed=4, step=5, want_logits=True)
    _check_draws(nxt, lg, 0.9, 10, 4, 5, cfg.vocab_size)
    nxt, lg = eng.prefill(tok, 0.9, 10, seed=4, step=6, want_logits=True)
    _check_draws(nxt, lg, 0.9, 10, 4, 6, cfg.vocab_size)
    for i in range(3):
        nxt, lg = eng.decode(nxt, 0.9, 10, seed=4, step=7 + i, want_logits=True)
        _check_draws(nxt, lg, 0.9, 10, 4, 7 + i, cfg.vocab_size)


def test_decode_graph_and_direct_launch_bitwise(monkeypatch):
    """The per-kernel decode path at 16 rows, replayed as a captured graph
    (ANN_DECODE_GRAPH=1), launched directly (=0, the default from 16 rows)
    and with the default: the same tokens and bitwise-equal logits over
    sampled steps (T = 0.8, top-k 50), so both launch forms stay covered."""
    cfg = GPTConfig(num_layers=2, num_heads=2, model_dim=256, seq_len=128, window=16,
                    long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 71, dense=True))
    B, T0, steps = 16, 24, 5
    tok = np.random.default_rng(9).integers(0, 50257, (B, T0))
    print("case decode launch forms: d256 L2 B=16, graph / direct / default", flush=True)
    runs = {}
    for mode in ("1", "0", None):
        if mode is None:
            monkeypatch.delenv("ANN_DECODE_GRAPH", raising=False)
        else:
            monkeypatch.setenv("ANN_DECODE_GRAPH", mode)
        eng = _engine(cfg, p, B, 64, B * T0)
        nxt, lg = eng.prefill(tok, 0.8, 50, seed=5, step=0, want_logits=True)
        toks, lgs = [nxt.cpu()], [lg.cpu()]
        for i in range(steps):
            nxt, lg = eng.decode(nxt, 0.8, 50, seed=5, step=i + 1, want_logits=True)
            toks.append(nxt.cpu())
            lgs.append(lg.cpu())
        eng.check_device()
        runs[mode] = (torch.stack(toks), torch.stack(lgs))
        del eng
    for mode in ("0", None):
        assert torch.equal(runs[mode][0], runs["1"][0]), mode
        assert torch.equal(runs[mode][1], runs["1"][1]), mode
