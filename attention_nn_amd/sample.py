"""Autoregressive sampling on the MI355X engine -- drop-in for the reference
``sample.py`` (``/root/reference/sample.py:13-56``).

    python -m attention_nn_amd.sample --ckpt gpt2_ckpt --dim 768 --layers 11 --heads 6 \
        --prompt "The history of" --tokens 120

Semantics per generated token (sample.py:42-50): the logits of the last
position over the context ``ids[-seq_len:]`` (positions re-encoded from 0),
sliced to the first 50257 rows, divided by the temperature, every value below
the k-th largest dropped, one categorical draw.  Here the context lives in a
KV cache: one prefill, then one decode step per token.  When the context would
grow past seq_len the window slides exactly as in the reference, by
re-prefilling the last seq_len ids.  ``temperature=0`` means greedy (argmax,
lowest index on ties), which the reference leaves undefined (division by 0).
Draws come from Philox4x32-10 keyed by ``seed`` with counter (token index,
batch row); the reference's draws (unseeded MLX) cannot be reproduced.
"""

import argparse
import sys

import numpy as np
import torch

from .config import sample_config
from .engine import Engine
from .weights import init_params, load_params


def _encode(prompt):
    if isinstance(prompt, str):
        try:
            import tiktoken
        except ImportError as e:
            raise SystemExit("text prompts need tiktoken (pass token ids instead)") from e
        return tiktoken.get_encoding("gpt2").encode(prompt)
    return [int(t) for t in prompt]


def sample(prompt, steps, temperature=0.8, top_k=50, seed=None, *, params=None, cfg=None,
           engine=None, batch=None, on_token=None):
    """Generate ``steps`` tokens after ``prompt``.

    prompt: str (tiktoken GPT-2), a list of ids, or a (B, T) array of ids.
    Returns the generated ids: a list for a single prompt, (B, steps) array
    for a batch.  ``engine`` may be passed to reuse packed weights / buffers.

    The sampled ids stay on the device: each step feeds the next one there,
    and a device record of every step is copied to the host once at the end.
    ``on_token`` (called with each step's (B,) ids, in order) receives them
    through a pinned host buffer and one event per step, as they complete,
    without stopping the device queue.  The host waits on the device only
    when the context slides past seq_len (the re-prefill needs the ids) and
    at the end, where the persistent step's bounded waits are also checked.
    """
    ids = np.asarray(_encode(prompt) if not hasattr(prompt, "shape") else prompt)
    single = ids.ndim == 1
    ids = np.atleast_2d(ids).astype(np.int64)
    if batch and single:
        ids = np.repeat(ids, batch, axis=0)
    B, T0 = ids.shape
    if T0 < 1:
        raise ValueError("empty prompt")
    if steps < 0:
        raise ValueError("steps must be >= 0")
    if engine is None:
        if params is None or cfg is None:
            raise ValueError("pass params and cfg, or an engine")
        engine = Engine(cfg, params, max_batch=B, max_ctx=cfg.seq_len,
                        max_tokens=B * cfg.seq_len)
    cfg = engine.cfg
    seq_len = min(cfg.seq_len, engine.max_ctx)
    seed = int(np.random.SeedSequence().entropy % (2**63)) if seed is None else int(seed)
    if steps == 0:
        return [] if single else np.empty((B, 0), np.int64)

    dev = engine.device
    rec = torch.empty((steps, B), dtype=torch.int32, device=dev)     # every step's ids
    host = torch.empty((steps, B), dtype=torch.int32, pin_memory=True)
    pending = []            # (step, event) of host copies not yet handed to on_token

    def emit(block):
        while pending and (block or pending[0][1].query()):
            i, ev = pending.pop(0)
            ev.synchronize()
            on_token(host[i].numpy().astype(np.int64))

    hist = ids.copy()       # host ids up to the last slide
    n_hist = 0              # generated ids already appended to hist
    cur = None
    for i in range(steps):
        if i == 0 or engine.length + 1 > seq_len:
            if i > 0:       # the window slides (sample.py:43): bring the new ids to the host
                hist = np.concatenate([hist, rec[n_hist:i].cpu().numpy().T.astype(np.int64)], 1)
                n_hist = i
            cur, _ = engine.prefill(hist[:, -seq_len:], temperature, top_k, seed, i)
        else:
            cur, _ = engine.decode(cur, temperature, top_k, seed, i, out=cur)
        rec[i].copy_(cur)
        if on_token is not None:
            host[i].copy_(rec[i], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            pending.append((i, ev))
            emit(False)
    out = rec.cpu().numpy().T.astype(np.int64)
    if on_token is not None:
        emit(True)
    engine.check_device()
    return list(out[0]) if single else out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--ckpt", type=str, default="checkpoint.safetensors")
    ap.add_argument("--prompt", type=str, default="The")
    ap.add_argument("--prompt-ids", type=str, default=None,
                    help="comma-separated token ids (instead of --prompt)")
    ap.add_argument("--tokens", type=int, default=100)
    ap.add_argument("--temp", type=float, default=0.8)
    ap.add_argument("--top-k", type=int, default=50)
    ap.add_argument("--dim", type=int, default=512)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--seq-len", type=int, default=1024)
    ap.add_argument("--window", type=int, default=384)
    ap.add_argument("--synthetic", action="store_true",
                    help="random-init weights (model.py distributions) instead of --ckpt")
    args = ap.parse_args(argv)

    cfg = sample_config(dim=args.dim, layers=args.layers, heads=args.heads,
                        seq_len=args.seq_len, window=args.window)
    params = init_params(cfg, seed=0, dense=True) if args.synthetic else load_params(args.ckpt)
    prompt = [int(t) for t in args.prompt_ids.split(",")] if args.prompt_ids else args.prompt
    dec = None
    if not args.prompt_ids:
        try:
            import tiktoken
            dec = tiktoken.get_encoding("gpt2")
        except ImportError:
            raise SystemExit("pip3 install tiktoken (or pass --prompt-ids)")
        print(args.prompt, end="", flush=True)

    def show(nxt):
        if args.batch == 1:
            t = int(nxt[0])
            print(dec.decode([t]) if dec else f"{t} ", end="", flush=True)

    res = sample(prompt, args.tokens, args.temp, args.top_k, args.seed, params=params, cfg=cfg,
                 batch=args.batch if args.batch > 1 else None, on_token=show)
    print()
    if args.batch > 1:
        for row in np.asarray(res):
            print(" ".join(str(int(t)) for t in row))
    return 0


if __name__ == "__main__":
    sys.exit(main())
