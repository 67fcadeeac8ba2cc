"""Decode benchmark of the token loop on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]

Workload: 155M model (d768, 11 layers, 6 heads x
128, long layers {4,10}, window 384, vocab 50304), random-init bf16 weights
(model.py distributions, Wo/proj drawn dense), batch 1, 32-token random
prompt, greedy decode to context 1024.  A "step" is one whole generation of
that workload: the prefill of the 32-token prompt (which samples the first
token) and 991 decode steps, 992 generated tokens at positions 32..1023.  K
steps are timed between two device synchronisations with HIP events on the
stream the kernels run on, after W untimed ones.  value = generated tokens /
s over the K steps (prefill included); the median over the K generations and
the decode-only rate are reported beside it.

roofline: the dominant kernel -- at batch 1 the whole decode step is one
persistent kernel (k_decode_persist: embed, every layer, lm_head + softcap,
greedy argmax in one launch), launched directly once per token.  The decode
part of a timed generation is nothing but its 991 back-to-back launches
(positions 32..1022), so the mean launch duration is the median decode time
of the timed pass / 991 (an upper bound: it includes the launch gaps);
achieved = the mean algorithmic bytes of a step (bf16 weights once, K/V rows
read and appended, embedding row) / that duration, against the 8 TB/s peak.
One more generation brackets every launch with a HIP event pair on its
stream; its mean is reported beside it (the pairs add ~1%).

Every pass ends with the device check of the persistent step's bounded waits
(a step that gave up would end early and inflate the rate); the run exits
non-zero if one did.

secondary: the same batch-1 generation sampled at sample.py's defaults
(T = 0.8, top-k 50; median of 3); each of the following the median of 5
repetitions: batch-64 decode (configs[2]:
512-token prompts, temperature 0.8, top-k 50) against HBM and its prefill
against the bf16 MFMA peak; the training forward; one optimizer step;
configs[3] (B=16 at context 8192) and configs[4] (d1536, B=128).

cpu_baseline: the CPU oracle (PyTorch restatement of model.py's forward)
with sample.py's semantics -- a full forward over the whole context for every
token -- timed best-of-3 at 24 context lengths spanning 32..1023 and integrated over the
loop; threads = the host cores this process may use.
"""

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_BF16_TFLOPS = 2500.0
METRIC = "decode tok/s (155M, batch 1 & 64) + % of HBM/MFMA roofline on 1 MI355X"


def step_bytes(cfg, B, pos):
    """Algorithmic HBM bytes of one decode step at position pos (0-based)."""
    d, L, V = cfg.model_dim, cfg.num_layers, cfg.vocab_size
    w = 2 * (12 * d * d * L + d * V)
    kv = 0
    for l in range(L):
        n = pos + 1 if l in cfg.long_layers else min(pos + 1, cfg.window)
        kv += 4 * d * n
    return w + B * kv + B * L * 4 * d + B * 2 * d


def step_flops(cfg, B, pos):
    d, L, V = cfg.model_dim, cfg.num_layers, cfg.vocab_size
    f = 2 * (12 * d * d * L + d * V)
    for l in range(L):
        n = pos + 1 if l in cfg.long_layers else min(pos + 1, cfg.window)
        f += 4 * d * n
    return B * f


def prefill_flops(cfg, B, T):
    d, L, V = cfg.model_dim, cfg.num_layers, cfg.vocab_size
    f = 2 * 12 * d * d * L * B * T + 2 * d * V * B
    for l in range(L):
        for i in range(T):
            n = i + 1 if l in cfg.long_layers else min(i + 1, cfg.window)
            f += B * 4 * d * n
    return f


def train_fwd_flops(cfg, B, T):
    """GPT.__call__: the prefill body plus the lm_head over every row."""
    d, V = cfg.model_dim, cfg.vocab_size
    return prefill_flops(cfg, B, T) - 2 * d * V * B + 2 * d * V * B * T


def step_traffic():
    """HBM bytes per launch of the persistent decode kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by a known-size copy),
    or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "decode_persist_b1_hbm_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return int((t["fetch_kib"] * t["fetch_scale"] + t["write_kib"] * t["write_scale"]) * 1024)
    except (OSError, KeyError, ValueError):
        return None


def check(eng, what):
    """Raise if a bounded wait of the persistent step gave up during `what`."""
    try:
        eng.check_device()
    except Exception as e:
        raise SystemExit(f"bench: device check failed after {what}: {e}")


def generate(eng, prompt, n_decode, temperature, top_k, seed):
    """One generation: prefill (samples the first token), then n_decode
    decode steps.  Enqueued only; returns the last token tensor."""
    nxt, _ = eng.prefill(prompt, temperature, top_k, seed, 0)
    for i in range(n_decode):
        nxt, _ = eng.decode(nxt, temperature, top_k, seed, i + 1, out=nxt)
    return nxt


def timed_generations(eng, prompt, n_decode, reps, warmup, temperature, top_k, seed):
    """`reps` generations between two synchronisations, HIP events on the
    launch stream around each generation and around its decode part.
    Returns (total ms, [per-generation ms], [per-generation decode ms])."""
    import torch
    for _ in range(warmup):
        generate(eng, prompt, n_decode, temperature, top_k, seed)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(reps)]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for r in range(reps):
        ev[r][0].record(st)
        nxt, _ = eng.prefill(prompt, temperature, top_k, seed, 0)
        ev[r][1].record(st)
        for i in range(n_decode):
            nxt, _ = eng.decode(nxt, temperature, top_k, seed, i + 1, out=nxt)
        ev[r][2].record(st)
    e1.record(st)
    torch.cuda.synchronize()
    total = e0.elapsed_time(e1)
    gen = [a.elapsed_time(c) for a, _, c in ev]
    dec = [b.elapsed_time(c) for _, b, c in ev]
    return total, gen, dec


def step_kernel_times(eng, prompt, n_decode):
    """One generation launched eagerly with an event pair around every launch
    of the persistent step kernel: (summed ms, launches)."""
    import torch
    eng.profile("step", max_launches=n_decode + 8)
    generate(eng, prompt, n_decode, 0.0, 0, 0)
    torch.cuda.synchronize()
    k = eng.profile_read()
    eng.profile(None)
    return k


def cpu_baseline(cfg, params, prompt_len, ctx_end, budget_s=20.0):
    """sample.py semantics on the CPU oracle: full recompute per token."""
    import torch
    import oracle.ref_model as R
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    prep = R.Prepared(cfg, params)
    rng = np.random.default_rng(1)
    ctxs = np.linspace(prompt_len, ctx_end, 24).astype(int)
    times = []
    t_start = time.perf_counter()
    for T in ctxs:
        tok = rng.integers(0, 50257, (1, int(T)))
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            with torch.no_grad():
                R.forward(prep, tok)
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        times.append(best)
        if time.perf_counter() - t_start > budget_s:
            break
    ctxs = ctxs[:len(times)]
    # per-step time as a function of context, integrated over every step
    all_ctx = np.arange(prompt_len, ctx_end)
    per_step = np.interp(all_ctx, ctxs, times)
    total = float(per_step.sum())
    full_s = time.perf_counter() - t_start
    return {
        "value": round(len(all_ctx) / total, 3),
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle full-recompute forward (sample.py semantics, no KV cache), best of 3 "
                   f"at {len(ctxs)} contexts {int(ctxs[0])}..{int(ctxs[-1])}, interpolated and "
                   f"summed over the {len(all_ctx)} steps {prompt_len}..{ctx_end - 1} "
                   f"({full_s:.1f} s of CPU work)"),
        "kv_cache_variant": cpu_kv_cache(prep, prompt_len, ctx_end, cores),
    }


def cpu_kv_cache(prep, prompt_len, ctx_end, cores, budget_s=8.0):
    """The same oracle with a KV cache (one token per step, as the GPU path
    decodes): a fairer CPU comparison than sample.py's full recompute.
    Greedy steps from position prompt_len until the budget or ctx_end."""
    import torch
    import oracle.ref_model as R
    tok = np.random.default_rng(1).integers(0, min(50257, prep.cfg.vocab_size), (1, prompt_len))
    cache = R.KVCache(prep.cfg.num_layers)
    with torch.no_grad():
        nxt = R.forward(prep, tok, cache)[:, -1].argmax(-1).numpy()
        t0 = time.perf_counter()
        n = 0
        while prompt_len + n < ctx_end and time.perf_counter() - t0 < budget_s:
            nxt = R.forward(prep, nxt[:, None], cache)[:, -1].argmax(-1).numpy()
            n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": (f"oracle with a KV cache, batch 1, greedy steps at positions "
                       f"{prompt_len}..{prompt_len + n - 1} ({dt:.1f} s)")}


def _events_ms(fn, reps):
    """Median and mean of `reps` calls of fn, each bracketed by HIP events."""
    import torch
    fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    t = [a.elapsed_time(b) for a, b in ev]
    return float(np.median(t)), float(np.mean(t))


REPS = 5


def decode_section(cfg, params, B, P, S, temp, k, seed, eng=None):
    """Prefill B prompts of P tokens and decode S steps, REPS times: the
    median decode time against HBM and the median prefill against MFMA."""
    import torch
    from attention_nn_amd.engine import Engine
    own = eng is None
    if own:
        eng = Engine(cfg, params, max_batch=B, max_ctx=P + S, max_tokens=B * P)
    pr = np.random.default_rng(P + B).integers(0, 50257, (B, P))
    pmed, _ = _events_ms(lambda: eng.prefill(pr, temp, k, seed, 0), REPS)
    _, gen, dec = timed_generations(eng, pr, S, REPS, 1, temp, k, seed)
    check(eng, f"B={B} decode")
    dms = float(np.median(dec))
    byts = float(np.mean([step_bytes(cfg, B, P + i) for i in range(S)]))
    gbs = byts / (dms / S / 1e3) / 1e9
    pf = prefill_flops(cfg, B, P)
    tf = pf / (pmed / 1e3) / 1e12
    out = {"decode_tok_s": round(B * S / (dms / 1e3), 1),
           "decode_ms_per_step": round(dms / S, 4),
           "decode_achieved_GBs": round(gbs, 1), "decode_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "decode_step_bytes": int(byts),
           "decode_ms_per_step_reps": [round(x / S, 4) for x in dec],
           "prefill_ms": round(pmed, 3), "prefill_tok_s": round(B * P / (pmed / 1e3), 1),
           "prefill_tflops": round(tf, 2), "prefill_mfma_frac": round(tf / MFMA_BF16_TFLOPS, 4),
           "prefill_flops": pf, "reps": REPS, "statistic": "median"}
    if own:
        del eng
        torch.cuda.empty_cache()
    return out


def secondary_b64(cfg, params):
    """B=64, 512-token prompts: prefill vs MFMA, 512 decode steps
    at T=0.8 / top-k 50 vs HBM; and the training forward on the same tokens."""
    import torch
    from attention_nn_amd.engine import Engine
    B, P, S = 64, 512, 512
    eng = Engine(cfg, params, max_batch=B, max_ctx=P + S, max_tokens=B * P)
    sec = decode_section(cfg, params, B, P, S, 0.8, 50, 7, eng)
    sec["workload"] = "cfg3: B=64, 512-token prompts, 512 decode steps, T=0.8, top-k 50"
    # training forward (GPT.__call__): same tokens, targets = the next ids
    pr = np.random.default_rng(P + B).integers(0, 50257, (B, P))
    tg = np.roll(pr, -1, axis=1)
    tmed, _ = _events_ms(lambda: eng.forward_loss(pr, tg), REPS)
    loss = eng.forward_loss(pr, tg)
    tfl = train_fwd_flops(cfg, B, P)
    del eng
    torch.cuda.empty_cache()
    return {
        "b64": sec,
        "b64_train_fwd": {"ms": round(tmed, 3), "tok_s": round(B * P / (tmed / 1e3), 1),
                          "tflops": round(tfl / (tmed / 1e3) / 1e12, 2),
                          "mfma_frac": round(tfl / (tmed / 1e3) / 1e12 / MFMA_BF16_TFLOPS, 4),
                          "flops": tfl, "loss": round(float(loss.item()), 4),
                          "reps": REPS, "statistic": "median",
                          "workload": "GPT.__call__ on the cfg3 prompts (64 x 512), "
                                      "targets = next ids, loss only"},
    }


def polar_express_flops(shape):
    """Five iterations of A = x x^T (or x^T x), A A, B x (or x B) per matrix."""
    *lead, M, N = shape
    batch = int(np.prod(lead)) if lead else 1
    S, L = min(M, N), max(M, N)
    return 5 * batch * (4 * S * S * L + 2 * S ** 3)


def secondary_optim(cfg, params):
    """One MuonAdam step (muon.py:66-137) over the 155M parameter dict with
    random gradients; Polar Express timed alone against the MFMA peak."""
    import torch
    from attention_nn_amd import optim as G
    p = {k: torch.from_numpy(v).cuda() for k, v in params.items()}
    rng = torch.Generator(device="cuda").manual_seed(5)
    grads = {k: torch.randn(v.shape, device="cuda", generator=rng) * 1e-3 for k, v in p.items()}
    opt = G.MuonAdam(p, G.optimizer_table())
    p = opt(p, grads)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 3
    e0.record()
    for _ in range(reps):
        p = opt(p, grads)
    e1.record()
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / reps
    banks = [grads[k] for k in ("attn_bank", "fc_bank", "proj_bank")]
    for g in banks:
        G.polar_express(g)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        for g in banks:
            G.polar_express(g)
    e1.record()
    torch.cuda.synchronize()
    pe_ms = e0.elapsed_time(e1) / reps
    pe_fl = sum(polar_express_flops(tuple(g.shape)) for g in banks)
    tf = pe_fl / (pe_ms / 1e3) / 1e12
    del p, grads, opt
    torch.cuda.empty_cache()
    return {"optimizer_step": {
        "ms": round(step_ms, 3), "polar_express_ms": round(pe_ms, 3),
        "polar_express_tflops": round(tf, 2), "mfma_frac": round(tf / MFMA_BF16_TFLOPS, 4),
        "polar_express_flops": pe_fl,
        "workload": "MuonAdam step over the 155M parameter dict (attn/fc/proj banks on "
                    "NorMuon + Polar Express, embeddings and lambdas on Adam), random grads"}}


def extra_config(name):
    """prefill then decode, medians of REPS."""
    from attention_nn_amd.config import cfg_155m, cfg_834m
    from attention_nn_amd.weights import init_params
    if name == "cfg4":
        cfg, B, P, S = cfg_155m(seq_len=8192), 16, 7680, 512
        desc = "cfg4: 155M, B=16, 7680-token prompts + 512 decode steps (ctx 8192), greedy"
        temp, k = 0.0, 0
    else:
        cfg, B, P, S = cfg_834m(seq_len=2048), 128, 1024, 1024
        desc = "cfg5: d1536 L24 H12x128, B=128, 1024-token prompts + 1024 steps, softcap + top-k 50"
        temp, k = 0.8, 50
    params = init_params(cfg, seed=0, dense=True)
    out = decode_section(cfg, params, B, P, S, temp, k, 11)
    out["workload"] = desc
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5,
                    help="timed steps; a step is one whole generation (prefill 32 + 991 decode)")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", type=str, default="", choices=["", "b64", "optim", "cfg4", "cfg5"],
                    help="run only one secondary section and print its JSON (for profiling)")
    ap.add_argument("--trace-run", action="store_true",
                    help="run only the batch-1 workload (one generation, graph-replayed decode "
                         "steps, no event instrumentation) for rocprofv3 traces and counters")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first copy 512 MiB device-to-device (a known-size kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the decode path runs on a single MI355X "
              "(multi-GPU sharding is a design note, not built)", file=sys.stderr)
        return 2
    if args.steps < 1:
        print("--steps must be >= 1", file=sys.stderr)
        return 2

    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from attention_nn_amd.config import cfg_155m
    from attention_nn_amd.engine import Engine
    from attention_nn_amd.weights import init_params

    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.ones(512 * 2**20 // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    cfg = cfg_155m(seq_len=1024)
    params = init_params(cfg, seed=0, dense=True)
    prompt_len, ctx_end = 32, 1024
    n_decode = ctx_end - prompt_len - 1          # 991 decode steps after the prefill's token
    prompt = np.random.default_rng(0).integers(0, 50257, (1, prompt_len))
    if args.only == "b64":
        print(json.dumps(secondary_b64(cfg, params)), flush=True)
        return 0
    if args.only == "optim":
        print(json.dumps(secondary_optim(cfg, params)), flush=True)
        return 0
    if args.only in ("cfg4", "cfg5"):
        print(json.dumps({args.only: extra_config(args.only)}, default=float), flush=True)
        return 0
    eng = Engine(cfg, params, max_batch=1, max_ctx=ctx_end, max_tokens=ctx_end)
    if args.trace_run:
        generate(eng, prompt, n_decode, 0.0, 0, 0)
        torch.cuda.synchronize()
        check(eng, "trace run")
        print(f"trace run: prefill {prompt_len} + {n_decode} greedy decode steps", flush=True)
        return 0
    # timed: K whole generations; each decode step is one launch of the
    # persistent step kernel
    total_ms, gen, dec = timed_generations(eng, prompt, n_decode, args.steps, args.warmup,
                                           0.0, 0, 0)
    check(eng, "the timed generations")
    # roofline: one more generation, every step kernel launch bracketed by
    # events on its stream
    k_ms, k_n = step_kernel_times(eng, prompt, n_decode)
    check(eng, "the roofline generation")
    # the reference's default sampling (sample.py:18-19: T = 0.8, top-k 50),
    # same prompt and length: persistent step + top-k candidate sampler
    s_total, s_gen, s_dec = timed_generations(eng, prompt, n_decode, 3, 1, 0.8, 50, 1)
    check(eng, "the sampled generations")
    gen_tokens = n_decode + 1
    value = args.steps * gen_tokens / (total_ms / 1e3)
    avg_bytes = float(np.mean([step_bytes(cfg, 1, prompt_len + i) for i in range(n_decode)]))
    dec_med = float(np.median(dec))
    k_avg_ms = dec_med / n_decode                # timed pass: back-to-back step launches
    achieved = avg_bytes / (k_avg_ms / 1e3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights (model.py distributions, Wo/proj dense), random prompt ids",
        "config": {"workload": "cfg2: 155M (d768 L11 H6x128), batch 1, 32-token prompt, greedy decode "
                               "to context 1024",
                   "step": f"one whole generation: prefill {prompt_len} tokens + {n_decode} decode "
                           f"steps = {gen_tokens} tokens at positions {prompt_len}..{ctx_end - 1}",
                   "global_batch": 1, "seq_len": ctx_end, "parallelism": "single GPU"},
        "median_tok_s": round(gen_tokens / (float(np.median(gen)) / 1e3), 2),
        "decode_only_tok_s": round(n_decode / (dec_med / 1e3), 2),
        "decode_ms_per_token": round(dec_med / n_decode, 5),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": step_traffic(),
                     "traffic_source": "profiles/decode_persist_b1_hbm_traffic.md (rocprofv3 "
                                       "FETCH_SIZE/WRITE_SIZE)",
                     "kernel": "k_decode_persist<128,1,2,768,6,1> (the 155M greedy instance of the "
                               "whole batch-1 decode step: embed, 11 layers, lm_head + softcap, "
                               "greedy argmax)",
                     "bytes_per_launch": int(avg_bytes), "avg_launch_us": round(k_avg_ms * 1e3, 3),
                     "avg_launch_source": "median decode segment of the timed generations / "
                                          f"{n_decode} back-to-back launches",
                     "event_bracketed_us": round(k_ms / max(k_n, 1) * 1e3, 3),
                     "launches": n_decode, "positions": f"{prompt_len}..{prompt_len + n_decode - 1}"},
    }
    step_gbs = avg_bytes / (dec_med / n_decode / 1e3) / 1e9
    s_dec_med = float(np.median(s_dec))
    sec = {"b1_step": {"avg_alg_bytes": int(avg_bytes), "achieved_GBs": round(step_gbs, 1),
                       "hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
                       "generation_ms_reps": [round(x, 3) for x in gen]},
           "b1_sampled": {"tok_s": round(gen_tokens / (float(np.median(s_gen)) / 1e3), 2),
                          "decode_ms_per_token": round(s_dec_med / n_decode, 5),
                          "generation_ms_reps": [round(x, 3) for x in s_gen],
                          "reps": 3, "statistic": "median",
                          "workload": "cfg2 shape, batch 1, T = 0.8 / top-k 50 (sample.py "
                                      "defaults), seed 1, same prompt and length"}}
    del eng
    torch.cuda.empty_cache()

    if not args.no_secondary:
        sec.update(secondary_b64(cfg, params))
        sec.update(secondary_optim(cfg, params))
        for name in ("cfg4", "cfg5"):
            sec[name] = extra_config(name)
    out["secondary"] = sec
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, params, prompt_len, ctx_end)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
