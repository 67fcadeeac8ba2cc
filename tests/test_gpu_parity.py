"""Parity of the HIP path (through the C ABI) against the CPU oracle.

Bars (the north star's): softcapped logits within 2e-2 max-abs of the oracle,
greedy token sequences identical (64 steps on the 155M model); kernels
against the reference's own known-answer tests at their tolerances.
"""

import numpy as np
import pytest
import torch

import oracle.ref_model as R
import oracle.ref_sample as S
from attention_nn_amd.config import GPTConfig, cfg_155m, cfg_small_h4
from attention_nn_amd.weights import init_params, perturb_lambdas

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import attention_nn_amd._lib as L
    L.lib()   # the native library must load; no fallback exists


def small_cfgs():
    return {
        "dh64": GPTConfig(vocab_size=512, num_layers=2, num_heads=2, model_dim=128, seq_len=64,
                          window=16, long_layers=(1,)),
        "dh128": GPTConfig(vocab_size=1000, num_layers=3, num_heads=2, model_dim=256, seq_len=96,
                           window=8, long_layers=(0, 2)),
    }


def _engine(cfg, params, B, ctx=None, tokens=None):
    from attention_nn_amd.engine import Engine
    ctx = ctx or cfg.seq_len
    return Engine(cfg, params, max_batch=B, max_ctx=ctx, max_tokens=tokens or B * ctx)


# ---- operators: the reference self-tests on the HIP kernels ----------------

def test_relu2_kernel_kat():
    from attention_nn_amd import kernels as K
    rng = np.random.default_rng(0)
    x = rng.standard_normal((64, 33)).astype(np.float32)
    y = K.relu2(torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.allclose(y, np.maximum(x, 0) ** 2, atol=1e-6)          # metal_kernels.py:342
    xb = torch.from_numpy(rng.standard_normal((128, 128)).astype(np.float32)).cuda().bfloat16()
    yb = K.relu2(xb)
    assert yb.dtype == torch.bfloat16                                  # metal_kernels.py:403
    assert torch.equal(yb.float().cpu(), R.relu2(xb.float().cpu()))


def test_rope_kernel_kat():
    from attention_nn_amd import kernels as K
    rng = np.random.default_rng(0)
    B, T, H, D = 2, 16, 3, 64
    cs, sn = K.make_rope_tables(T, D)
    csr, snr = R.rope_tables(T, D)
    assert torch.allclose(cs.cpu(), csr, atol=1e-6) and torch.allclose(sn.cpu(), snr, atol=1e-6)
    x = rng.standard_normal((B, T, H, D)).astype(np.float32)
    out = K.rope_ht(torch.from_numpy(x).cuda(), cs, sn).cpu().numpy()
    from tests.test_oracle import _rope_reference_loop
    ref = _rope_reference_loop(x, cs.cpu().numpy(), sn.cpu().numpy())
    assert np.allclose(out, ref, atol=1e-5)                            # metal_kernels.py:363
    back = K.rope_ht(torch.from_numpy(out).cuda(), cs, sn, inverse=True).cpu().numpy()
    assert np.allclose(back, x, atol=1e-5)
    # explicit position offset == rows of a longer sequence
    cs2, sn2 = K.make_rope_tables(64, D)
    a = K.rope_ht(torch.from_numpy(x).cuda(), cs2, sn2, pos0=20).cpu().numpy()
    r = _rope_reference_loop(x, cs2.cpu().numpy()[20:36], sn2.cpu().numpy()[20:36])
    assert np.allclose(a, r, atol=1e-5)
    xb = torch.from_numpy(x).cuda().bfloat16()
    yb = K.rope_ht(xb, cs, sn)
    assert yb.dtype == torch.bfloat16
    rb = _rope_reference_loop(xb.float().cpu().numpy(), cs.cpu().numpy(), sn.cpu().numpy())
    rb = torch.from_numpy(rb).bfloat16().float().numpy()   # the fp32 rotation rounded once
    assert np.allclose(yb.float().cpu().numpy(), rb, rtol=2 ** -7, atol=1e-6)
    # buffers one element off a pair boundary: the element-wise path of the kernel
    big = torch.zeros(x.size + 1, dtype=torch.float32, device="cuda")
    xo = big[1:].view(x.shape)
    xo.copy_(torch.from_numpy(x).cuda())
    assert np.allclose(K.rope_ht(xo, cs, sn).cpu().numpy(), ref, atol=1e-5)


def test_rope_tables_long():
    from attention_nn_amd import kernels as K
    cs, sn = K.make_rope_tables(8192, 128)
    csr, snr = R.rope_tables(8192, 128)
    # theta up to 8191 rad: fp32 argument rounding dominates
    assert (cs.cpu() - csr).abs().max().item() < 2e-3
    assert (sn.cpu() - snr).abs().max().item() < 2e-3


def test_rms_kernel():
    from attention_nn_amd import kernels as K
    rng = np.random.default_rng(2)
    x = rng.standard_normal((7, 768)).astype(np.float32) * 3
    y = K.rms(torch.from_numpy(x).cuda()).cpu()
    assert torch.allclose(y, R.rms_f32(torch.from_numpy(x)), atol=1e-5)
    xb = torch.from_numpy(x).cuda().bfloat16()
    yb = K.rms(xb).float().cpu()
    ref = R.rms(xb.float().cpu())
    assert (yb - ref).abs().max().item() <= 2 ** -7 * ref.abs().max().item()


# ---- whole forward -------------------------------------------------------------

@pytest.mark.parametrize("name", ["dh64", "dh128"])
@pytest.mark.parametrize("B,T", [(1, 5), (2, 40), (3, 1), (3, 12)])
def test_forward_logits_parity(name, B, T):
    cfg = small_cfgs()[name]
    p = perturb_lambdas(init_params(cfg, 11, dense=True))
    tok = np.random.default_rng(B * 100 + T).integers(0, cfg.vocab_size, (B, T))
    print(f"case {name} B={B} T={T}", flush=True)
    eng = _engine(cfg, p, B)
    got = eng.forward_logits(tok).cpu()
    ref = R.logits(cfg, p, tok)
    err = (got - ref).abs().max().item()
    assert err < LOGIT_TOL, err
    assert torch.all((got > 0) & (got < 23))


@pytest.mark.parametrize("dh,window", [(64, 70), (128, 100)])
def test_prefill_logits_every_position_long_prompt(dh, window):
    """Prefill of 300 tokens (three 128-query blocks, 64-key tiles): logits at
    every position match the oracle.  The windows are not multiples of the key
    tile, so the prefill attention meets tiles it evaluates unmasked, tiles
    crossing the diagonal or the window edge, and tiles a wave skips."""
    cfg = GPTConfig(vocab_size=700, num_layers=2, num_heads=2, model_dim=2 * dh, seq_len=320,
                    window=window, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 23, dense=True))
    tok = np.random.default_rng(dh + window).integers(0, cfg.vocab_size, (2, 300))
    print(f"case dh={dh} window={window} B=2 T=300", flush=True)
    eng = _engine(cfg, p, 2)
    got = eng.forward_logits(tok).cpu()
    ref = R.logits(cfg, p, tok)
    err = (got - ref).abs().max().item()
    assert err < LOGIT_TOL, err


@pytest.mark.parametrize("dh,window", [(64, 70), (128, 100)])
def test_prefill_bf16_p_within_both_oracle_readings(dh, window):
    """The prefill attention rounds the softmax weights to bf16 before P.V.
    Its logits at every position of a 300-token prompt stay within the 2e-2
    bar of both oracle readings of model.py:251-254's attention: fp32 scores,
    softmax and P.V (the default), and MLX's decomposed form (q pre-scaled in
    bf16, bf16 scores and probabilities, bf16 P.V)."""
    cfg = GPTConfig(vocab_size=700, num_layers=3, num_heads=2, model_dim=2 * dh, seq_len=320,
                    window=window, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 29, dense=True))
    tok = np.random.default_rng(dh * 3 + window).integers(0, cfg.vocab_size, (2, 300))
    print(f"case dh={dh} window={window} B=2 T=300, both attention readings", flush=True)
    eng = _engine(cfg, p, 2)
    got = eng.forward_logits(tok).cpu()
    for mlx in (False, True):
        ref = R.logits(cfg, p, tok, mlx_fallback_attn=mlx)
        err = (got - ref).abs().max().item()
        assert err < LOGIT_TOL, (mlx, err)


@pytest.mark.parametrize("d,B,T", [(512, 2, 300), (768, 3, 200)])
def test_prefill_wide_tiles(d, B, T):
    """Prefill shapes on the large-tile GEMMs: M = B*T >= 512 rows, not a
    multiple of the 256-row tile, so the QKV / fc projections run on the
    256 x 128 tiles and o / proj on the 128 x 256 tiles, each with a ragged
    last row block and a tile count that is not a multiple of the 8 XCDs;
    logits at every position against the oracle."""
    cfg = GPTConfig(vocab_size=1000, num_layers=2, num_heads=d // 128, model_dim=d, seq_len=320,
                    window=100, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 31, dense=True))
    tok = np.random.default_rng(d + T).integers(0, cfg.vocab_size, (B, T))
    print(f"case d={d} B={B} T={T}", flush=True)
    eng = _engine(cfg, p, B)
    got = eng.forward_logits(tok).cpu()
    ref = R.logits(cfg, p, tok)
    err = (got - ref).abs().max().item()
    assert err < LOGIT_TOL, err


# ---- training forward: GPT.__call__ with the fused softcap CE ---------------

@pytest.mark.parametrize("dh,V,B,T", [(64, 512, 1, 40), (128, 1000, 2, 40), (128, 700, 2, 300)])
def test_forward_loss_matches_oracle(dh, V, B, T):
    """GPT.__call__ (model.py:180-221): per-row softcapped CE and the mean
    against the oracle's training forward (bf16 attention reading) and its
    fp32 reading.  V = 1000 and 700 leave a partial last 128-column tile;
    targets include 0 and V - 1."""
    cfg = GPTConfig(vocab_size=V, num_layers=2, num_heads=2, model_dim=2 * dh, seq_len=320,
                    window=70, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 29, dense=True))
    rng = np.random.default_rng(dh + V + T)
    tok = rng.integers(0, V, (B, T))
    tgt = rng.integers(0, V, (B, T))
    tgt[0, 0], tgt[-1, -1] = 0, V - 1
    print(f"case dh={dh} V={V} B={B} T={T}", flush=True)
    eng = _engine(cfg, p, B)
    mean, rows = eng.forward_loss(tok, tgt, rows=True)
    rows = rows.cpu().double()
    # measured: rows within 1.4e-3, means within 6e-5 (both readings)
    for banded in (True, False):
        rm, rr = R.loss(cfg, p, tok, tgt, banded_bf16=banded)
        assert (rows - rr.double()).abs().max().item() < 1e-2, banded
        assert abs(mean.item() - rm.item()) < 5e-4, banded
    assert abs(mean.item() - rows.mean().item()) < 1e-5


@pytest.mark.parametrize("V", [50304, 16384])
def test_forward_loss_large_vocab_equals_cross_entropy_of_own_logits(V):
    """The fused CE epilogue at the model's vocabulary (393 column tiles of 128,
    the last partial) and at 1024 rows, against torch cross_entropy over the
    same engine's softcapped logits."""
    cfg = GPTConfig(vocab_size=V, num_layers=2, num_heads=2, model_dim=256, seq_len=512,
                    window=100, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 41, dense=True))
    rng = np.random.default_rng(V)
    B, T = 2, 512
    tok = rng.integers(0, V, (B, T))
    tgt = rng.integers(0, V, (B, T))
    tgt[0, 0], tgt[-1, -1] = 0, V - 1
    print(f"case V={V} B={B} T={T}", flush=True)
    eng = _engine(cfg, p, B)
    lg = eng.forward_logits(tok).double()
    ref = torch.nn.functional.cross_entropy(lg.reshape(-1, V),
                                            torch.from_numpy(tgt).reshape(-1).cuda(),
                                            reduction="none")
    del lg
    mean, rows = eng.forward_loss(tok, tgt, rows=True)
    assert (rows.double() - ref).abs().max().item() < 1e-4
    assert abs(mean.item() - ref.mean().item()) < 1e-5


def test_forward_loss_equals_cross_entropy_of_own_logits():
    """Without the oracle: the fused CE epilogue equals torch cross_entropy
    over the same engine's (B, T, V) softcapped logits (same z, only the
    summation order of the log-sum-exp differs)."""
    cfg = small_cfgs()["dh128"]
    p = perturb_lambdas(init_params(cfg, 37, dense=True))
    rng = np.random.default_rng(38)
    tok = rng.integers(0, cfg.vocab_size, (3, 50))
    tgt = rng.integers(0, cfg.vocab_size, (3, 50))
    eng = _engine(cfg, p, 3)
    lg = eng.forward_logits(tok).double()
    ref = torch.nn.functional.cross_entropy(lg.reshape(-1, cfg.vocab_size),
                                            torch.from_numpy(tgt).reshape(-1).cuda(),
                                            reduction="none")
    mean, rows = eng.forward_loss(tok, tgt, rows=True)
    assert (rows.double() - ref).abs().max().item() < 1e-4
    assert abs(mean.item() - ref.mean().item()) < 1e-5


@pytest.mark.parametrize("name,B", [("dh64", 2), ("dh128", 2), ("dh128", 4), ("dh128", 8),
                                    ("dh128", 12)])
def test_decode_teacher_forced_past_window(name, B, monkeypatch):
    """Decode logits at every position (well past the window) match the
    oracle's KV-cache forward on the same tokens, on the per-kernel path
    (ANN_PERSIST=0: two rows take the GEMV with the fused greedy keys; 4, 8
    and 12 rows the skinny MFMA GEMMs, the logits GEMM and the sampler kernel,
    and the split-combine attention)."""
    cfg = small_cfgs()[name]
    p = perturb_lambdas(init_params(cfg, 5, dense=True))
    T0, steps = 7, cfg.seq_len - 7
    tok = np.random.default_rng(1).integers(0, cfg.vocab_size, (B, T0 + steps))
    monkeypatch.setenv("ANN_PERSIST", "0")
    eng = _engine(cfg, p, B)
    monkeypatch.delenv("ANN_PERSIST")
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :T0], want_logits=True)
    ref = R.forward(prep, tok[:, :T0], cache)[:, -1]
    worst = (lg.cpu() - ref).abs().max().item()
    for i in range(steps - 1):
        t = tok[:, T0 + i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    assert worst < LOGIT_TOL, worst


@pytest.mark.parametrize("B,persist", [(3, True), (4, True), (4, False), (8, False)])
def test_decode_small_batch_sampled_matches_oracle(B, persist, monkeypatch):
    """Sampled decode (T = 0.9, top-k 20) at 3, 4 and 8 rows -- 3 and 4 rows on
    the persistent step (its z rows, then the sampler kernel; 4 rows through
    ANN_PERSIST_MAX_B), 4 and 8 rows on the per-kernel path: the logits match
    the oracle at every step and every row's draw equals the oracle sampler's
    draw (Philox counter (step, row)) from the engine's own logits."""
    cfg = small_cfgs()["dh128"]
    p = perturb_lambdas(init_params(cfg, 25, dense=True))
    T0, steps, temp, k, seed = 7, 30, 0.9, 20, 77
    tok = np.random.default_rng(3 + B).integers(0, cfg.vocab_size, (B, T0 + steps))
    monkeypatch.setenv("ANN_PERSIST_MAX_B", "4")
    if not persist:
        monkeypatch.setenv("ANN_PERSIST", "0")
    eng = _engine(cfg, p, B)
    monkeypatch.delenv("ANN_PERSIST", raising=False)
    monkeypatch.delenv("ANN_PERSIST_MAX_B")
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    nxt, lg = eng.prefill(tok[:, :T0], temp, k, seed=seed, step=0, want_logits=True)
    worst = (lg.cpu() - R.forward(prep, tok[:, :T0], cache)[:, -1]).abs().max().item()
    draws = [(nxt, lg, 0)]
    for i in range(steps - 1):
        t = tok[:, T0 + i]
        nxt, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), temp, k, seed=seed,
                             step=i + 1, want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
        draws.append((nxt, lg, i + 1))
    eng.check_device()
    assert worst < LOGIT_TOL, worst
    for nxt, lg, step in draws:
        got, z = nxt.cpu().numpy(), lg.cpu().numpy()
        for b in range(B):
            want = _sample_small(z[b, :min(50257, cfg.vocab_size)], temp, k, S.uniform(seed, step, b))
            assert int(got[b]) == want, (step, b)


@pytest.mark.parametrize("persist", [False, True])
def test_one_token_prompts_then_decode_match_oracle(persist, monkeypatch):
    """Prompts of one token at 4 rows: the prefill's attention is then the
    decode kernel itself, with 8 key splits on the full-causal layers (ticket
    counters and tagged partials), so the decode steps after it continue from
    the counters it left (per-kernel path, ANN_PERSIST=0) or start the
    persistent step from the exchange area it cleared.  Logits match the
    oracle's KV-cache forward at every step, and no bounded wait timed out."""
    cfg = GPTConfig(vocab_size=1000, num_layers=3, num_heads=2, model_dim=256, seq_len=512,
                    window=8, long_layers=(0, 2))
    p = perturb_lambdas(init_params(cfg, 31, dense=True))
    B, steps = 4, 24
    tok = np.random.default_rng(31).integers(0, cfg.vocab_size, (B, 1 + steps))
    monkeypatch.setenv("ANN_PERSIST_MAX_B", "4")
    if not persist:
        monkeypatch.setenv("ANN_PERSIST", "0")
    eng = _engine(cfg, p, B, ctx=512, tokens=4 * B)
    monkeypatch.delenv("ANN_PERSIST", raising=False)
    monkeypatch.delenv("ANN_PERSIST_MAX_B")
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :1], want_logits=True)
    worst = (lg.cpu() - R.forward(prep, tok[:, :1], cache)[:, -1]).abs().max().item()
    for i in range(steps):
        t = tok[:, 1 + i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    eng.check_device()
    assert worst < LOGIT_TOL, worst


@pytest.mark.parametrize("name", ["dh64", "dh128"])
def test_persistent_decode_matches_oracle(name):
    """Batch-1 decode runs as the single persistent kernel (tagged exchanges
    between work-groups); its logits at every position, past the window, match
    the oracle, and no bounded wait timed out."""
    cfg = small_cfgs()[name]
    p = perturb_lambdas(init_params(cfg, 15, dense=True))
    T0, steps = 5, cfg.seq_len - 5
    tok = np.random.default_rng(11).integers(0, cfg.vocab_size, (1, T0 + steps))
    eng = _engine(cfg, p, 1)
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :T0], want_logits=True)
    ref = R.forward(prep, tok[:, :T0], cache)[:, -1]
    worst = (lg.cpu() - ref).abs().max().item()
    for i in range(steps - 1):
        t = tok[:, T0 + i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    eng.check_device()
    assert worst < LOGIT_TOL, worst


@pytest.mark.parametrize("name,B", [("dh64", 2), ("dh128", 3), ("dh128", 4)])
def test_persistent_rows_decode_matches_oracle(name, B, monkeypatch):
    """The persistent step at 2-4 rows (every projection row's weights applied
    to the rows held in LDS, one attention work-group per (row, head, split);
    4 rows through ANN_PERSIST_MAX_B): teacher-forced logits of every row at
    every position, past the window, match the oracle, and no bounded wait
    timed out."""
    cfg = small_cfgs()[name]
    p = perturb_lambdas(init_params(cfg, 17, dense=True))
    T0, steps = 5, cfg.seq_len - 5
    tok = np.random.default_rng(19 + B).integers(0, cfg.vocab_size, (B, T0 + steps))
    monkeypatch.setenv("ANN_PERSIST_MAX_B", "4")
    eng = _engine(cfg, p, B)
    monkeypatch.delenv("ANN_PERSIST_MAX_B")
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :T0], want_logits=True)
    worst = (lg.cpu() - R.forward(prep, tok[:, :T0], cache)[:, -1]).abs().max().item()
    for i in range(steps - 1):
        t = tok[:, T0 + i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    eng.check_device()
    assert worst < LOGIT_TOL, worst


def test_persistent_rows_match_kernel_path(monkeypatch):
    """3 rows: the persistent step and the per-kernel step (ANN_PERSIST=0)
    give identical greedy tokens in every row over 60 steps and logits within
    the oracle tolerance (they sum in different orders); seeded top-k draws
    of the persistent step equal the oracle sampler's draws from the step's
    own logits."""
    cfg = small_cfgs()["dh128"]
    p = perturb_lambdas(init_params(cfg, 27, dense=True))
    prompt = np.random.default_rng(14).integers(0, cfg.vocab_size, (3, 6))

    def run(persist, temp, k):
        if not persist:
            monkeypatch.setenv("ANN_PERSIST", "0")
        eng = _engine(cfg, p, 3)
        monkeypatch.delenv("ANN_PERSIST", raising=False)
        nxt, _ = eng.prefill(prompt, temp, k, seed=9, step=0)
        toks, lgs = [nxt.cpu().numpy().copy()], []
        for i in range(60):
            nxt, lg = eng.decode(nxt, temp, k, seed=9, step=i + 1, want_logits=True)
            toks.append(nxt.cpu().numpy().copy())
            lgs.append(lg.cpu())
        eng.check_device()
        return np.stack(toks), torch.stack(lgs)

    ta, la = run(True, 0.0, 0)
    tb, lb = run(False, 0.0, 0)
    assert np.array_equal(ta, tb)
    assert (la - lb).abs().max().item() < LOGIT_TOL
    temp, k = 0.9, 20
    sa, ls = run(True, temp, k)
    for i in range(60):
        for b in range(3):
            z = ls[i, b].numpy()[:min(50257, cfg.vocab_size)]
            assert sa[i + 1, b] == _sample_small(z, temp, k, S.uniform(9, i + 1, b)), (i, b)


def test_persistent_cooperative_launch(monkeypatch):
    """ANN_PERSIST_COOP=1 launches the same step kernel cooperatively (the
    runtime guarantees residency); logits still match the oracle."""
    monkeypatch.setenv("ANN_PERSIST_COOP", "1")
    cfg = small_cfgs()["dh64"]
    p = perturb_lambdas(init_params(cfg, 16, dense=True))
    tok = np.random.default_rng(13).integers(0, cfg.vocab_size, (1, 30))
    eng = _engine(cfg, p, 1)
    monkeypatch.delenv("ANN_PERSIST_COOP")
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :5], want_logits=True)
    R.forward(prep, tok[:, :5], cache)
    worst = 0.0
    for i in range(5, 29):
        t = tok[:, i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    eng.check_device()
    assert worst < LOGIT_TOL, worst


def test_persistent_matches_kernel_path(monkeypatch):
    """The persistent batch-1 step and the per-kernel step (ANN_PERSIST=0)
    agree: greedy tokens identical over 60 steps and logits within the oracle
    tolerance (the two sum the projections in different orders, so z can
    differ by one bf16 ulp).  Seeded top-k draws of the persistent step equal
    the oracle sampler's draws from that step's own logits."""
    cfg = small_cfgs()["dh128"]
    p = perturb_lambdas(init_params(cfg, 21, dense=True))
    prompt = np.random.default_rng(12).integers(0, cfg.vocab_size, (1, 6))

    def run(persist, temp, k):
        if not persist:
            monkeypatch.setenv("ANN_PERSIST", "0")
        eng = _engine(cfg, p, 1)
        monkeypatch.delenv("ANN_PERSIST", raising=False)
        nxt, _ = eng.prefill(prompt, temp, k, seed=5, step=0)
        toks, lgs = [int(nxt[0])], []
        for i in range(60):
            nxt, lg = eng.decode(nxt, temp, k, seed=5, step=i + 1, want_logits=True)
            toks.append(int(nxt[0]))
            lgs.append(lg.cpu())
        eng.check_device()
        return toks, torch.stack(lgs)

    ta, la = run(True, 0.0, 0)
    tb, lb = run(False, 0.0, 0)
    assert ta == tb
    assert (la - lb).abs().max().item() < LOGIT_TOL
    temp, k = 0.9, 20
    sa, ls = run(True, temp, k)
    for i in range(60):
        z = ls[i, 0].numpy()[:min(50257, cfg.vocab_size)]
        assert sa[i + 1] == _sample_small(z, temp, k, S.uniform(5, i + 1, 0)), i


@pytest.mark.parametrize("B", [40, 80])
def test_decode_wide_batch_skinny_tiles(B):
    """Decode at 40 and 80 rows: the skinny MFMA GEMM with 32x32 work-group
    tiles for N >= 2048 above 32 rows (fc at 40 rows) and with 16x16 tiles
    above 64 rows where the 32x32 grid would hold under 128 work-groups (o /
    proj at d = 512, 80 rows), against the oracle."""
    cfg = GPTConfig(vocab_size=600, num_layers=2, num_heads=4, model_dim=512, seq_len=32,
                    window=8, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 41, dense=True))
    tok = np.random.default_rng(42).integers(0, cfg.vocab_size, (B, 12))
    eng = _engine(cfg, p, B)
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :9], want_logits=True)
    worst = (lg.cpu() - R.forward(prep, tok[:, :9], cache)[:, -1]).abs().max().item()
    for i in range(9, 11):
        t = tok[:, i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    assert worst < LOGIT_TOL, worst


def test_decode_deep_load_rings():
    """Decode at 72 rows of a d = 768 model: the qkv / fc projections on
    64 x 64 MFMA tiles with four K tiles in flight, the o / proj projections
    (K = 768 / 3072) on the LDS-staged skinny GEMM with 16 x 16 tiles (a
    32 x 32 grid would hold 72 work-groups), and (vocabulary above 8 d) the
    lm_head on the 128-row MFMA tiles; logits against the oracle.  The 32 x 32
    tiles with three rounds in flight run in the cfg5-shape test."""
    cfg = GPTConfig(vocab_size=8192, num_layers=2, num_heads=6, model_dim=768, seq_len=16,
                    window=8, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 47, dense=True))
    B = 72
    tok = np.random.default_rng(48).integers(0, cfg.vocab_size, (B, 12))
    print(f"case d=768 B={B} V=8192", flush=True)
    eng = _engine(cfg, p, B)
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :9], want_logits=True)
    worst = (lg.cpu() - R.forward(prep, tok[:, :9], cache)[:, -1]).abs().max().item()
    for i in range(9, 12):
        t = tok[:, i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    eng.check_device()
    assert worst < LOGIT_TOL, worst


def test_decode_weight_prefetch_bitwise(monkeypatch):
    """From 16 rows the decode attention launch carries extra work-groups that
    read the next projections' weights ahead (this layer's o / fc / proj and
    the next layer's qkv; the last layer's o / fc / proj).  They change no
    result: logits are bitwise equal with the prefetch off and on (fixed and
    byte-sized work-group counts), and within tolerance of the oracle."""
    cfg = GPTConfig(vocab_size=704, num_layers=3, num_heads=2, model_dim=256, seq_len=32,
                    window=8, long_layers=(2,))
    p = perturb_lambdas(init_params(cfg, 45, dense=True))
    B = 16
    tok = np.random.default_rng(46).integers(0, cfg.vocab_size, (B, 14))

    def run(pf):
        if pf is None:
            monkeypatch.delenv("ANN_PREFETCH_WG", raising=False)
        else:
            monkeypatch.setenv("ANN_PREFETCH_WG", str(pf))
        eng = _engine(cfg, p, B)
        _, lg = eng.prefill(tok[:, :10], want_logits=True)
        out = [lg.cpu()]
        for i in range(10, 13):
            _, lg = eng.decode(torch.from_numpy(tok[:, i].astype(np.int32)).cuda(),
                               want_logits=True)
            out.append(lg.cpu())
        eng.check_device()
        return torch.stack(out)

    off, fixed, sized = run(0), run(7), run(None)
    assert torch.equal(off, fixed) and torch.equal(off, sized)
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    ref = [R.forward(prep, tok[:, :10], cache)[:, -1]]
    for i in range(10, 13):
        ref.append(R.forward(prep, tok[:, i:i + 1], cache)[:, -1])
    worst = (sized - torch.stack(ref)).abs().max().item()
    assert worst < LOGIT_TOL, worst


def test_decode_attention_ring_forms_bitwise(monkeypatch):
    """The decode attention has a three-chunk K/V ring (two work-groups per
    CU) and a two-chunk one held to three waves per SIMD, taken by default when
    the grid has more than two work-groups per CU.  Both walk each wave's key
    chunks in the same order: logits are bitwise equal under either form, with
    one and with two key splits, and within tolerance of the oracle."""
    cfg = GPTConfig(vocab_size=704, num_layers=3, num_heads=2, model_dim=256, seq_len=48,
                    window=8, long_layers=(2,))
    p = perturb_lambdas(init_params(cfg, 51, dense=True))
    B = 12
    tok = np.random.default_rng(52).integers(0, cfg.vocab_size, (B, 30))

    def run(ring, splits):
        monkeypatch.setenv("ANN_ATTN_RING", str(ring))
        monkeypatch.setenv("ANN_DEC_SPLITS", str(splits))
        print(f"case attention ring {ring} splits {splits}", flush=True)
        eng = _engine(cfg, p, B)
        _, lg = eng.prefill(tok[:, :20], want_logits=True)
        out = [lg.cpu()]
        for i in range(20, 29):
            _, lg = eng.decode(torch.from_numpy(tok[:, i].astype(np.int32)).cuda(),
                               want_logits=True)
            out.append(lg.cpu())
        eng.check_device()
        return torch.stack(out)

    for splits in (1, 2):
        r3, r2 = run(3, splits), run(2, splits)
        assert torch.equal(r3, r2), splits
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    ref = [R.forward(prep, tok[:, :20], cache)[:, -1]]
    for i in range(20, 29):
        ref.append(R.forward(prep, tok[:, i:i + 1], cache)[:, -1])
    worst = (r2 - torch.stack(ref)).abs().max().item()
    assert worst < LOGIT_TOL, worst


def test_wide_lm_head_64_row_tile():
    """A vocabulary wider than 8 d at 12 rows takes the large-tile MFMA GEMM
    with its 64-row work-group tile for the lm_head."""
    cfg = GPTConfig(vocab_size=4096, num_layers=1, num_heads=2, model_dim=128, seq_len=32,
                    window=8, long_layers=(0,))
    p = perturb_lambdas(init_params(cfg, 43, dense=True))
    tok = np.random.default_rng(44).integers(0, cfg.vocab_size, (12, 6))
    eng = _engine(cfg, p, 12)
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :5], want_logits=True)
    worst = (lg.cpu() - R.forward(prep, tok[:, :5], cache)[:, -1]).abs().max().item()
    t = tok[:, 5]
    _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
    worst = max(worst, (lg.cpu() - R.forward(prep, t[:, None], cache)[:, -1]).abs().max().item())
    assert worst < LOGIT_TOL, worst


def test_long_context_decode():
    """Decode at positions up to 2100 on a full-causal layer (the split count
    caps at 32, several 64-key chunks per split) and a windowed layer."""
    cfg = GPTConfig(vocab_size=600, num_layers=2, num_heads=2, model_dim=256, seq_len=2112,
                    window=384, long_layers=(1,))
    p = perturb_lambdas(init_params(cfg, 31, dense=True))
    tok = np.random.default_rng(32).integers(0, cfg.vocab_size, (1, 2100))
    eng = _engine(cfg, p, 1)
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    _, lg = eng.prefill(tok[:, :2090], want_logits=True)
    ref = R.forward(prep, tok[:, :2090], cache)[:, -1]
    worst = (lg.cpu() - ref).abs().max().item()
    for i in range(2090, 2099):
        t = tok[:, i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    assert worst < LOGIT_TOL, worst


def test_batch_rows_independent():
    cfg = small_cfgs()["dh128"]
    p = perturb_lambdas(init_params(cfg, 2, dense=True))
    tok = np.random.default_rng(3).integers(0, cfg.vocab_size, (3, 12))
    eng3 = _engine(cfg, p, 3)
    eng1 = _engine(cfg, p, 1)
    a = eng3.forward_logits(tok).cpu()
    for b in range(3):
        c = eng1.forward_logits(tok[b:b + 1]).cpu()
        assert (a[b] - c[0]).abs().max().item() < LOGIT_TOL


def _greedy_oracle(cfg, params, prompt, steps):
    prep = R.Prepared(cfg, params)
    cache = R.KVCache(cfg.num_layers)
    lg = R.forward(prep, prompt[None, :], cache)[0, -1]
    out, logits = [], []
    for _ in range(steps):
        nxt = int(np.argmax(lg[:50257].numpy()))
        out.append(nxt)
        logits.append(lg)
        lg = R.forward(prep, [[nxt]], cache)[0, -1]
    return out, logits


def _greedy_gpu(eng, prompt, steps):
    nxt, lg = eng.prefill(prompt[None, :], want_logits=True)
    out, logits = [int(nxt.item())], [lg[0].cpu()]
    for _ in range(steps - 1):
        nxt, lg = eng.decode(nxt, want_logits=True, out=nxt)
        out.append(int(nxt.item()))
        logits.append(lg[0].cpu())
    return out, logits


def test_greedy_155m_identical_64_steps():
    """North-star gate: 155M (d768 L11 H6x128), dense random init, 32-token
    prompt, 64 greedy steps identical to the oracle; per-step logits <= 2e-2.
    A second run without fp32 logits (the persistent step's greedy-only
    instance, the one the bench runs) gives the same 64 tokens."""
    cfg = cfg_155m()
    p = init_params(cfg, 0, dense=True)
    prompt = np.random.default_rng(0).integers(0, 50257, 32)
    eng = _engine(cfg, p, 1, ctx=1024, tokens=1024)
    got, glog = _greedy_gpu(eng, prompt, 64)
    ref, rlog = _greedy_oracle(cfg, p, prompt, 64)
    n_same = next((i for i, (a, b) in enumerate(zip(got, ref)) if a != b), 64)
    worst = max((g - r).abs().max().item() for g, r in zip(glog[:n_same], rlog[:n_same]))
    assert worst < LOGIT_TOL, worst
    assert got == ref, f"first divergence at step {n_same}"
    eng2 = _engine(cfg, p, 1, ctx=1024, tokens=1024)
    nxt, _ = eng2.prefill(prompt[None, :])
    plain = [int(nxt.item())]
    for _ in range(63):
        nxt, _ = eng2.decode(nxt, out=nxt)
        plain.append(int(nxt.item()))
    eng2.check_device()
    assert plain == ref


@pytest.mark.parametrize("B,temp", [(1, 0.8), (3, 0.0), (4, 0.8)])
def test_155m_mode_instances_draws(B, temp, monkeypatch):
    """The 155M persistent step without fp32 logits runs instances with the
    mode (greedy or sampled) at compile time (the bench's batch-1 lines, and
    2-4 rows): 48 steps after 32-token prompts, greedy or T = 0.8 / top-k 50,
    the same tokens in every row as the generic kernel (ANN_PD_SPECIALIZE=0)
    and as the instance that also returns the logits, whose tokens and draws
    the oracle tests check."""
    cfg = cfg_155m()
    p = init_params(cfg, 2, dense=True)
    prompt = np.random.default_rng(22 + B).integers(0, 50257, (B, 32))
    k = 50 if temp > 0 else 0

    def run(spec, want_logits):
        monkeypatch.setenv("ANN_PD_SPECIALIZE", spec)
        monkeypatch.setenv("ANN_PERSIST_MAX_B", "4")
        eng = _engine(cfg, p, B, ctx=1024, tokens=B * 32)
        monkeypatch.delenv("ANN_PD_SPECIALIZE")
        monkeypatch.delenv("ANN_PERSIST_MAX_B")
        print(f"case 155M {B} rows, T={temp}, ANN_PD_SPECIALIZE={spec}, logits={want_logits}",
              flush=True)
        nxt, _ = eng.prefill(prompt, temp, k, 9, 0, want_logits=want_logits)
        toks = [nxt.cpu().numpy().copy()]
        for i in range(47):
            nxt, _ = eng.decode(nxt, temp, k, 9, i + 1, want_logits=want_logits, out=nxt)
            toks.append(nxt.cpu().numpy().copy())
        eng.check_device()
        return np.stack(toks)

    inst = run("1", False)
    assert np.array_equal(inst, run("0", False))
    assert np.array_equal(inst, run("1", True))
    if temp > 0:   # the draws are not one repeated token (greedy at this init can be)
        assert len(set(inst[:, 0].tolist())) > 8


@pytest.mark.parametrize("B", [3, 4])
def test_greedy_155m_rows_identical_to_oracle(B, monkeypatch):
    """The 155M model, three and four independent sequences on the
    persistent step (four through ANN_PERSIST_MAX_B): 32-token prompts, 32
    greedy steps, every row's tokens identical to the oracle's greedy decode
    of that row and its logits within 2e-2."""
    cfg = cfg_155m()
    p = init_params(cfg, 4, dense=True)
    prompts = np.random.default_rng(44).integers(0, 50257, (B, 32))
    monkeypatch.setenv("ANN_PERSIST_MAX_B", "4")
    eng = _engine(cfg, p, B, ctx=1024, tokens=B * 32)
    monkeypatch.delenv("ANN_PERSIST_MAX_B")
    print(f"case 155M, {B} rows, 32 greedy steps", flush=True)
    nxt, lg = eng.prefill(prompts, want_logits=True)
    got, glog = [nxt.cpu().numpy().copy()], [lg.cpu()]
    for _ in range(31):
        nxt, lg = eng.decode(nxt, want_logits=True, out=nxt)
        got.append(nxt.cpu().numpy().copy())
        glog.append(lg.cpu())
    eng.check_device()
    got = np.stack(got)
    for b in range(B):
        ref, rlog = _greedy_oracle(cfg, p, prompts[b], 32)
        n_same = next((i for i, (a, r) in enumerate(zip(got[:, b], ref)) if a != r), 32)
        worst = max((glog[i][b] - rlog[i]).abs().max().item() for i in range(n_same))
        assert worst < LOGIT_TOL, (b, worst)
        assert list(got[:, b]) == ref, f"row {b}: first divergence at step {n_same}"


def test_persistent_155m_late_positions_match_oracle():
    """The 155M model at batch 1 near the end of cfg2's context: a 1000-token
    prefill, then teacher-forced decode steps on the persistent kernel at
    positions 1000..1022 -- the windowed layers read keys [p - 383, p] over
    three 128-key splits with lo > 0, the full-causal layers all p + 1 keys
    over eight.  Logits within 2e-2 of the oracle at every step."""
    cfg = cfg_155m()
    p = perturb_lambdas(init_params(cfg, 9, dense=True))
    tok = np.random.default_rng(91).integers(0, 50257, (1, 1024))
    eng = _engine(cfg, p, 1, ctx=1024, tokens=1024)
    prep = R.Prepared(cfg, p)
    cache = R.KVCache(cfg.num_layers)
    print("case 155M batch 1: prefill 1000, decode at positions 1000..1022", flush=True)
    _, lg = eng.prefill(tok[:, :1000], want_logits=True)
    worst = (lg.cpu() - R.forward(prep, tok[:, :1000], cache, last_only=True)[:, -1]).abs().max().item()
    for i in range(1000, 1023):
        t = tok[:, i]
        _, lg = eng.decode(torch.from_numpy(t.astype(np.int32)).cuda(), want_logits=True)
        ref = R.forward(prep, t[:, None], cache, last_only=True)[:, -1]
        worst = max(worst, (lg.cpu() - ref).abs().max().item())
    eng.check_device()
    assert eng.length == 1023
    assert worst < LOGIT_TOL, worst


@pytest.mark.parametrize("var,B,va,vb", [("ANN_PD_XCD", 1, "1", "0"),
                                         ("ANN_PD_SPECIALIZE", 1, "1", "0"),
                                         ("ANN_PD_SPECIALIZE", 2, "1", "0"),
                                         ("ANN_PD_ON", 1, "96", "112"),
                                         ("ANN_PD_REP", 1, "8", "4"),
                                         ("ANN_PERSIST_G", 1, "192", "128")])
def test_persistent_155m_variants_bitwise(var, B, va, vb, monkeypatch):
    """The persistent step at 155M against its variants, teacher-forced
    decode steps after a 500-token prefill (windowed layers over three splits,
    full-causal over eight at one row), logits bitwise equal:
    ANN_PD_XCD=0 splits the qkv rows contiguously over all work-groups
    instead of each head's rows and attention splits on XCD h (the default
    where the shares divide: 192 work-groups, 8 row pairs each);
    ANN_PD_SPECIALIZE=0 runs the generic kernel instead of the instance with
    the 155M model's d and H as compile-time constants (one and two rows);
    ANN_PD_ON=112 spreads the 384 o-projection row pairs over 112 work-groups
    instead of 96 (unequal shares); ANN_PD_REP=4 writes 4 copies of x' / x
    instead of 8; ANN_PERSIST_G=128 runs the step on 128 work-groups instead
    of 192 (other row shares, the contiguous qkv layout).  Every row and
    attention unit is computed the same way in each pair."""
    cfg = cfg_155m()
    p = perturb_lambdas(init_params(cfg, 13, dense=True))
    tok = np.random.default_rng(131).integers(0, 50257, (B, 520))

    def run(val):
        monkeypatch.setenv(var, val)
        eng = _engine(cfg, p, B, ctx=1024, tokens=B * 512)
        monkeypatch.delenv(var)
        print(f"case 155M {B} rows, {var}={val}: prefill 500, 20 decode steps", flush=True)
        eng.prefill(tok[:, :500])
        lgs = []
        for i in range(500, 520):
            t = torch.from_numpy(tok[:, i].astype(np.int32)).cuda()
            _, lg = eng.decode(t, want_logits=True)
            lgs.append(lg.cpu())
        eng.check_device()
        return torch.stack(lgs)

    a, b = run(va), run(vb)
    assert torch.equal(a, b), (a - b).abs().max().item()


@pytest.mark.parametrize("B", [16, 33, 64])
def test_fused_qkv_attention_bitwise(B, monkeypatch):
    """Decode steps of 16..64 rows (155M) with the qkv projection and the
    attention in one launch (tagged q / k / v words) against the two separate
    launches (ANN_QKV_ATTN=0): teacher-forced steps after a 300-token prefill,
    windowed and full-causal layers, logits bitwise equal."""
    cfg = cfg_155m()
    p = perturb_lambdas(init_params(cfg, 17, dense=True))
    tok = np.random.default_rng(170 + B).integers(0, 50257, (B, 312))

    def run(val):
        monkeypatch.setenv("ANN_QKV_ATTN", val)
        eng = _engine(cfg, p, B, ctx=1024, tokens=B * 300)
        monkeypatch.delenv("ANN_QKV_ATTN")
        print(f"case 155M {B} rows, ANN_QKV_ATTN={val}: prefill 300, 12 decode steps", flush=True)
        eng.prefill(tok[:, :300])
        lgs = []
        for i in range(300, 312):
            t = torch.from_numpy(tok[:, i].astype(np.int32)).cuda()
            _, lg = eng.decode(t, want_logits=True)
            lgs.append(lg.cpu())
        eng.check_device()
        return torch.stack(lgs)

    a, b = run("1"), run("0")
    assert torch.equal(a, b), (a - b).abs().max().item()


def test_degenerate_init_repeats_last_token():
    """cfg1 as specified (model.py init: Wo = proj = x0 = 0): greedy repeats
    the last prompt token; logits equal the oracle's closed form."""
    cfg = cfg_small_h4()
    p = init_params(cfg, 0)
    prompt = np.random.default_rng(1).integers(0, 50257, 16)
    eng = _engine(cfg, p, 1, ctx=128, tokens=128)
    got, glog = _greedy_gpu(eng, prompt, 16)
    assert got == [int(prompt[-1])] * 16
    ka = R.degenerate_known_answer(cfg, p, prompt[None, -1:])[0, -1]
    assert (glog[0] - ka).abs().max().item() < LOGIT_TOL


# ---- sampling ---------------------------------------------------------------

def test_sampling_matches_oracle_draws():
    cfg = small_cfgs()["dh128"]
    p = init_params(cfg, 9, dense=True)
    p["lm_head"] = p["lm_head"] * 60    # spread the logits so top-k matters
    B = 4
    tok = np.random.default_rng(6).integers(0, cfg.vocab_size, (B, 10))
    eng = _engine(cfg, p, B)
    for step, (temp, k) in enumerate([(0.8, 50), (1.0, 5), (0.5, 0), (2.0, 1), (0.8, 2000)]):
        nxt, lg = eng.prefill(tok, temp, k, seed=1234, step=step, want_logits=True)
        lg = lg.cpu().numpy()
        for b in range(B):
            z = lg[b, :min(50257, cfg.vocab_size)]
            want = _sample_small(z, temp, k, S.uniform(1234, step, b))
            assert int(nxt[b]) == want, (step, b)


def _sample_small(z, temp, k, u):
    zt = z.astype(np.float32) / np.float32(temp)
    if k and k < zt.size:
        kth = np.sort(zt)[-k]
        keep = np.nonzero(zt >= kth)[0]
    else:
        keep = np.arange(zt.size)
    w = np.exp(zt[keep].astype(np.float64) - zt[keep].max())
    c = np.cumsum(w)
    i = int(np.searchsorted(c, u * c[-1], side="right"))
    return int(keep[min(i, keep.size - 1)])


def test_sampling_chi_square():
    cfg = small_cfgs()["dh64"]
    p = init_params(cfg, 4, dense=True)
    p["lm_head"] = p["lm_head"] * 300
    tok = np.random.default_rng(2).integers(0, cfg.vocab_size, (1, 6))
    eng = _engine(cfg, p, 1)
    _, lg = eng.prefill(tok, want_logits=True)
    z = lg[0].cpu().numpy()
    temp, k, n = 1.0, 8, 3000
    zt = z.astype(np.float32) / np.float32(temp)
    kth = np.sort(zt)[-k]
    keep = zt >= kth
    w = np.where(keep, np.exp(zt.astype(np.float64) - zt.max()), 0.0)
    prob = w / w.sum()
    draws = [int(eng.prefill(tok, temp, k, seed=77, step=i)[0].item()) for i in range(n)]
    counts = np.bincount(draws, minlength=z.size)
    assert counts[~keep].sum() == 0
    m = prob * n > 5
    chi2 = (((counts - prob * n) ** 2)[m] / (prob * n)[m]).sum()
    assert chi2 < 30.0, chi2      # <= 7 dof


def test_sample_api_slides_window_like_reference():
    """sample() past seq_len re-encodes ids[-seq_len:] from position 0
    (sample.py:43), exactly like the reference's recompute loop."""
    from attention_nn_amd.sample import sample
    cfg = small_cfgs()["dh64"]
    p = perturb_lambdas(init_params(cfg, 8, dense=True))
    prompt = list(np.random.default_rng(4).integers(0, cfg.vocab_size, 50))
    got = sample(prompt, 30, temperature=0.0, params=p, cfg=cfg)
    ids = list(prompt)
    for _ in range(30):
        ctx = np.array(ids[-cfg.seq_len:])[None, :]
        lg = R.logits(cfg, p, ctx)[0, -1]
        ids.append(int(np.argmax(lg.numpy())))
    assert got == ids[50:]


# ---- the 256 x 256 prefill GEMM (gemm_big.hip) -------------------------------

def _big_cfg(dh):
    return GPTConfig(vocab_size=4096, num_layers=2, num_heads=768 // dh if dh == 128 else 8,
                     model_dim=768 if dh == 128 else 512, seq_len=512, window=100,
                     long_layers=(1,))


@pytest.mark.parametrize("dh", [128, 64])
def test_big_gemm_prefill_every_position(dh, monkeypatch):
    """A prefill of 16 x 500 tokens (8000 rows: a ragged last 256-row tile)
    puts the QKV (fused QK-norm / RoPE / cache epilogue), fc (relu^2) and, at
    d = 768, the o / proj (residual mixes) projections on the 256 x 256 GEMM;
    logits at every position against the oracle, and against the same
    forward on the previous tiles (ANN_GEMM_BIG=0)."""
    cfg = _big_cfg(dh)
    p = perturb_lambdas(init_params(cfg, 71, dense=True))
    tok = np.random.default_rng(72).integers(0, cfg.vocab_size, (16, 500))
    print(f"case big gemm dh={dh} B=16 T=500", flush=True)
    eng = _engine(cfg, p, 16)
    monkeypatch.setenv("ANN_GEMM_BIG", "2")    # every epilogue the kernel takes
    got = eng.forward_logits(tok).cpu()
    monkeypatch.setenv("ANN_GEMM_BIG", "1")    # the routed ones (fc, o-proj)
    routed = eng.forward_logits(tok).cpu()
    monkeypatch.setenv("ANN_GEMM_BIG", "0")
    old = eng.forward_logits(tok).cpu()
    monkeypatch.delenv("ANN_GEMM_BIG")
    # same products in the same k order: equal up to the order of the K tiles'
    # accumulation inside an MFMA (measured bitwise equal)
    assert (got - old).abs().max().item() < 2e-3
    assert (routed - old).abs().max().item() < 2e-3
    ref = R.logits(cfg, p, tok)
    err = max((got - ref).abs().max().item(), (routed - ref).abs().max().item())
    assert err < LOGIT_TOL, err


def test_big_gemm_training_forward():
    """GPT.__call__ on 16 x 500 tokens (the body's projections on the 256 x
    256 GEMM, the lm_head's CE epilogue on the previous tiles): per-row losses
    against the oracle."""
    cfg = _big_cfg(128)
    p = perturb_lambdas(init_params(cfg, 73, dense=True))
    rng = np.random.default_rng(74)
    tok = rng.integers(0, cfg.vocab_size, (16, 500))
    tgt = rng.integers(0, cfg.vocab_size, (16, 500))
    print("case big gemm training forward", flush=True)
    eng = _engine(cfg, p, 16)
    mean, rows = eng.forward_loss(tok, tgt, rows=True)
    rm, rr = R.loss(cfg, p, tok, tgt, banded_bf16=True)
    assert (rows.cpu().double() - rr.double()).abs().max().item() < 1e-2
    assert abs(mean.item() - rm.item()) < 5e-4
