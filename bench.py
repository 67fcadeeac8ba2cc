"""Decode benchmark of the token loop on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]

Workload: 155M model (d768, 11 layers, 6 heads x
128, long layers {4,10}, window 384, vocab 50304), random-init bf16 weights
(model.py distributions, Wo/proj drawn dense), batch 1, 32-token random
prompt, greedy decode to context 1024: a "step" is one decode step of the
whole model for the batch.  K steps (default 992 = positions 32..1023) are
timed with HIP events on the stream the kernels run on, after W warm-up steps
and a fresh prefill.  value = decoded tokens / s.

roofline: the dominant kernel -- at batch 1 the whole decode step is one
persistent kernel (k_decode_persist: embed, every layer, lm_head + softcap,
greedy argmax in one cooperative launch).  The timed pass replays it from a
HIP graph, where events cannot bracket it, so a second pass over the
identical workload launches it eagerly with a HIP event pair around every
launch on the stream it runs on; achieved = algorithmic bytes of the step
(bf16 weights once, K/V rows read and appended, embedding row) / mean
launch time, against the 8 TB/s peak.

secondary: the step's wall rate, batch-64 decode
(configs[2]: 512-token prompts, temperature 0.8, top-k 50) and its prefill
against the bf16 MFMA peak.

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


def run_decode(eng, prompt, steps, warmup, temperature, top_k, seed, prof=None):
    import torch
    B = prompt.shape[0]
    if warmup:
        nxt, _ = eng.prefill(prompt, temperature, top_k, seed, 0)
        for i in range(warmup):
            nxt, _ = eng.decode(nxt, temperature, top_k, seed, i + 1, out=nxt)
    torch.cuda.synchronize()
    nxt, _ = eng.prefill(prompt, temperature, top_k, seed, 0)
    torch.cuda.synchronize()
    if prof:
        eng.profile(prof, max_launches=steps + 8)
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(st)
    for i in range(steps):
        nxt, _ = eng.decode(nxt, temperature, top_k, seed, i + 1, out=nxt)
    e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1)
    kern = eng.profile_read() if prof else (0.0, 0)
    eng.profile(None)
    return ms, wall, kern, B * steps


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


def secondary_b64(cfg, params):
    """B=64, 512-token prompts: prefill vs MFMA, 512 decode steps vs HBM."""
    import torch
    from attention_nn_amd.engine import Engine
    B, P, S = 64, 512, 512
    eng = Engine(cfg, params, max_batch=B, max_ctx=1024, max_tokens=B * P)
    pr = np.random.default_rng(2).integers(0, 50257, (B, P))
    eng.prefill(pr, 0.8, 50, 7, 0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 3
    e0.record()
    for _ in range(reps):
        eng.prefill(pr, 0.8, 50, 7, 0)
    e1.record()
    torch.cuda.synchronize()
    pms = e0.elapsed_time(e1) / reps
    pf = prefill_flops(cfg, B, P)
    # training forward (GPT.__call__): same tokens, targets = the next ids
    tg = np.roll(pr, -1, axis=1)
    loss = eng.forward_loss(pr, tg)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        loss = eng.forward_loss(pr, tg)
    e1.record()
    torch.cuda.synchronize()
    tms = e0.elapsed_time(e1) / reps
    tfl = train_fwd_flops(cfg, B, P)
    ms64, _, _, toks64 = run_decode(eng, pr, S, 8, 0.8, 50, 7)
    b64_bytes = np.mean([step_bytes(cfg, B, P + i) for i in range(S)])
    b64_gbs = b64_bytes / (ms64 / S / 1e3) / 1e9
    tf = pf / (pms / 1e3) / 1e12
    del eng
    torch.cuda.empty_cache()
    return {
        "b64_decode": {"tok_s": round(toks64 / (ms64 / 1e3), 1), "ms_per_step": round(ms64 / S, 4),
                       "achieved_GBs": round(b64_gbs, 1), "hbm_frac": round(b64_gbs / HBM_PEAK_GBS, 4),
                       "workload": "cfg3: B=64, 512-token prompts, 512 steps, T=0.8, top-k 50"},
        "b64_prefill": {"ms": round(pms, 3), "tok_s": round(B * P / (pms / 1e3), 1),
                        "tflops": round(tf, 2), "mfma_frac": round(tf / MFMA_BF16_TFLOPS, 4),
                        "flops": pf},
        "b64_train_fwd": {"ms": round(tms, 3), "tok_s": round(B * P / (tms / 1e3), 1),
                          "tflops": round(tfl / (tms / 1e3) / 1e12, 2),
                          "mfma_frac": round(tfl / (tms / 1e3) / 1e12 / MFMA_BF16_TFLOPS, 4),
                          "flops": tfl, "loss": round(float(loss.item()), 4),
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
    """prefill then decode, reported as secondary lines."""
    import torch
    from attention_nn_amd.config import cfg_155m, cfg_834m
    from attention_nn_amd.engine import Engine
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
    eng = Engine(cfg, params, max_batch=B, max_ctx=P + S, max_tokens=B * P)
    pr = np.random.default_rng(3).integers(0, 50257, (B, P))
    # one untimed prefill first: the first launch of each kernel also loads
    # its code object (a cold call measured ~15 ms slower at cfg4)
    eng.prefill(pr, temp, k, 11, 0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 2
    e0.record()
    for _ in range(reps):
        nxt, _ = eng.prefill(pr, temp, k, 11, 0)
    e1.record()
    torch.cuda.synchronize()
    pms = e0.elapsed_time(e1) / reps
    ms, _, _, toks = run_decode(eng, pr, S, 0, temp, k, 11)
    byts = np.mean([step_bytes(cfg, B, P + i) for i in range(S)])
    gbs = byts / (ms / S / 1e3) / 1e9
    pf = prefill_flops(cfg, B, P)
    del eng
    torch.cuda.empty_cache()
    return {"workload": desc,
            "decode_tok_s": round(toks / (ms / 1e3), 1), "decode_ms_per_step": round(ms / S, 4),
            "decode_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "prefill_ms": round(pms, 2), "prefill_tflops": round(pf / (pms / 1e3) / 1e12, 2),
            "prefill_mfma_frac": round(pf / (pms / 1e3) / 1e12 / MFMA_BF16_TFLOPS, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=992)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-b64", action="store_true",
                    help="run only the batch-64 prefill/decode section (for profiling)")
    ap.add_argument("--only", type=str, default="", choices=["", "b64", "optim", "cfg4", "cfg5"],
                    help="run only one secondary section and print its JSON (for profiling)")
    ap.add_argument("--configs", type=str, default="",
                    help="comma list of extra workloads to add as secondary lines: cfg4,cfg5")
    ap.add_argument("--trace-run", action="store_true",
                    help="run only the batch-1 workload (prefill + K graph-replayed decode "
                         "steps, no event instrumentation) for rocprofv3 traces and counters")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first copy 512 MiB device-to-device (a known-size kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the decode path runs on a single MI355X "
              "(multi-GPU sharding is described in DESIGN.md, not built)", file=sys.stderr)
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
    prompt_len = 32
    steps = min(args.steps, 1024 - prompt_len)
    prompt = np.random.default_rng(0).integers(0, 50257, (1, prompt_len))
    if args.only_b64 or args.only == "b64":
        print(json.dumps(secondary_b64(cfg, params)), flush=True)
        return 0
    if args.only == "optim":
        print(json.dumps(secondary_optim(cfg, params)), flush=True)
        return 0
    if args.only in ("cfg4", "cfg5"):
        print(json.dumps({args.only: extra_config(args.only)}, default=float), flush=True)
        return 0
    eng = Engine(cfg, params, max_batch=1, max_ctx=1024, max_tokens=1024)
    if args.trace_run:
        nxt, _ = eng.prefill(prompt, 0.0, 0, 0, 0)
        for i in range(steps):
            nxt, _ = eng.decode(nxt, 0.0, 0, 0, i + 1, out=nxt)
        torch.cuda.synchronize()
        eng.check_device()
        print(f"trace run: prefill {prompt_len} + {steps} greedy decode steps", flush=True)
        return 0
    # timed pass: the decode step replays as one captured HIP graph (one
    # cooperative launch of the persistent step kernel per token)
    ms, wall, _, toks = run_decode(eng, prompt, steps, args.warmup, 0.0, 0, 0)
    # roofline pass: same workload launched eagerly with a HIP event pair on
    # the call's stream around every launch of the step kernel (events cannot
    # sit inside the replayed graph)
    _, _, (k_ms, k_n), _ = run_decode(eng, prompt, steps, 0, 0.0, 0, 0, prof="step")
    value = toks / (ms / 1e3)
    avg_bytes = np.mean([step_bytes(cfg, 1, prompt_len + i) for i in range(steps)])
    k_avg_ms = k_ms / max(k_n, 1)
    achieved = avg_bytes / (k_avg_ms / 1e3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights (model.py distributions, Wo/proj dense), random prompt ids",
        "config": {"workload": "cfg2: 155M (d768 L11 H6x128), batch 1, 32-token prompt, greedy decode "
                               "to context 1024", "global_batch": 1, "seq_len": 1024,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": step_traffic(),
                     "traffic_source": "profiles/decode_persist_b1_hbm_traffic.md (rocprofv3 "
                                       "FETCH_SIZE/WRITE_SIZE)",
                     "kernel": "k_decode_persist<128,1,2> (whole batch-1 decode step: embed, 11 "
                               "layers, lm_head + softcap, greedy argmax)",
                     "bytes_per_launch": int(avg_bytes), "avg_launch_us": round(k_avg_ms * 1e3, 3),
                     "launches": k_n},
    }
    step_gbs = avg_bytes / (ms / steps / 1e3) / 1e9
    sec = {"b1_step": {"avg_alg_bytes": int(avg_bytes), "achieved_GBs": round(step_gbs, 1),
                       "hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
                       "wall_tok_s": round(toks / wall, 2)}}
    del eng
    torch.cuda.empty_cache()

    if not args.no_secondary:
        sec.update(secondary_b64(cfg, params))
        sec.update(secondary_optim(cfg, params))
    for name in [c for c in args.configs.split(",") if c]:
        sec[name] = extra_config(name)
    out["secondary"] = sec
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, params, prompt_len, 1024)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
