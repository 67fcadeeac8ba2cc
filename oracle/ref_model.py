"""ORACLE -- test infrastructure only.

A CPU (PyTorch fp32) restatement of the reference inference forward
``GPT.logits`` (``/root/reference/model.py:223-263``), of the two custom
Metal kernels it calls (``metal_kernels.py:37-47`` relu2,
``metal_kernels.py:87-134,144-150`` half-truncated RoPE), and of the
training forward's loss ``GPT.__call__`` (``model.py:180-221``) with its
fused softcapped cross-entropy (``metal_kernels.py:153-193``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import
this module, and only as the checker or the timed CPU baseline; the product
path (``attention_nn_amd``) never calls it.

Rounding model ("fp32 masters, bf16 compute", eager MLX):
  * fp32 weights are cast to bf16 (round to nearest even);
  * every matmul accumulates bf16 inputs in fp32 and rounds once to bf16;
  * rms, relu2, RoPE and the attention softmax compute in fp32 and round
    once to bf16 at their output;
  * every elementwise product / sum of the residual mixes rounds to bf16, in
    the left-to-right order of ``model.py:256,260``;
  * z = bf16(rms(x) @ lm_head) is widened to fp32 before the softcap
    ``23 * sigmoid((z + 5) / 7.5)`` (``model.py:262-263``).

The SDPA rounding inside MLX (``mx.fast.scaled_dot_product_attention``) is not
part of the reference source; the default here keeps scores, softmax and P.V
in fp32 and rounds the output once.  ``mlx_fallback_attn=True`` switches to
the decomposed variant (q pre-scaled in bf16, bf16 scores and probabilities)
so tests can bound how far the two readings differ.

Parity status per function (what pins each one; checked in tests/):
  rope_tables / rope_ht : reference KAT loop (metal_kernels.py:349-363)
  relu2                 : closed form KAT (metal_kernels.py:339-343)
  rms                   : fp64 textbook formula + invariants
  attention             : fp64 brute force (pattern of old.mm:2277-2348),
                          window == full while pos < window
  softcap               : closed form, bounds (0, 23), monotonicity
  logits (whole)        : closed-form known answer of the degenerate init
                          (Wo = proj = x0 = 0 => x_L is a scaled x0);
                          the dense wiring (mix_attn, mix_mlp, mlp_branch,
                          the q/k/v slices, mask, every lambda slot) by
                          closed forms in numpy -- Wq = Wk = 0 with fc = 0
                          (uniform attention over the kept keys, zero MLP)
                          and Wv = 0 (zero attention, dense MLP) -- with
                          distinct lambdas, where each planted index or
                          wiring mistake fails (tests/test_oracle_wiring.py);
                          KV-cache decode == full recompute, fp64 forward
  softcap_ce            : torch.nn.functional.cross_entropy on the softcapped
                          logits; uniform z => loss = log V exactly
  attention(banded_bf16): within bf16 rounding of the fp64 brute force
  loss (whole)          : composition of the pinned parts; equals the mean
                          of softcap_ce over the rows of the pinned logits
"""

import math

import torch

F32 = torch.float32


def bf(x):
    """Round an fp32 tensor to bf16 (RNE) and widen back to fp32."""
    return x.to(torch.bfloat16).to(F32)


# -- metal_kernels.py:144-150 -------------------------------------------------
def rope_tables(seq_len, head_dim, base=1024.0):
    """cos/sin tables (seq_len, head_dim/4) fp32: freqs = (1/base)**linspace(0,1,D/4)."""
    d4 = head_dim // 4
    lin = torch.linspace(0.0, 1.0, d4, dtype=F32)
    freqs = torch.pow(torch.tensor(1.0 / base, dtype=F32), lin)
    t = torch.arange(seq_len, dtype=F32)
    theta = t[:, None] * freqs[None, :]
    return torch.cos(theta), torch.sin(theta)


# -- model.py:48-49 -------------------------------------------------------------
def rms_f32(x, eps=1e-6):
    """Weight-free RMSNorm over the last axis in fp32."""
    x = x.to(F32)
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)


def rms(x, eps=1e-6):
    """rms_f32 rounded to bf16 (MLX's bf16 rms_norm output)."""
    return bf(rms_f32(x, eps))


# -- metal_kernels.py:37-47 ------------------------------------------------------
def relu2_f32(x):
    r = torch.clamp_min(x.to(F32), 0.0)
    return r * r


def relu2(x):
    return bf(relu2_f32(x))


# -- metal_kernels.py:87-113 -----------------------------------------------------
def rope_ht(x, cs, sn, positions):
    """rope_ht_f32 rounded to bf16."""
    return bf(rope_ht_f32(x, cs, sn, positions))


def rope_ht_f32(x, cs, sn, positions):
    """x (B,T,H,D); rotate adjacent pairs (2p, 2p+1) for p < D/4 with the
    angle of ``positions`` (T,), pass the other dims through.  fp32 output."""
    D = x.shape[-1]
    d4 = D // 4
    c = cs[positions][None, :, None, :]   # (1,T,1,D/4)
    s = sn[positions][None, :, None, :]
    x = x.to(F32)
    x0 = x[..., 0:2 * d4:2]
    x1 = x[..., 1:2 * d4:2]
    y = x.clone()
    y[..., 0:2 * d4:2] = c * x0 + s * x1
    y[..., 1:2 * d4:2] = c * x1 - s * x0
    return y


# -- model.py:263 -----------------------------------------------------------------
def softcap(z):
    return 23.0 * torch.sigmoid((z.to(F32) + 5.0) / 7.5)


def keep_mask(q_pos, k_pos, long_layer, window):
    """model.py:248-250: keep <=> j <= i and (long layer or i - j < window)."""
    i = q_pos[:, None]
    j = k_pos[None, :]
    keep = i >= j
    if not long_layer:
        keep = keep & (i - j < window)
    return keep


def attention(q, k, v, keep, scale, mlx_fallback_attn=False, banded_bf16=False):
    """q (B,H,Tq,Dh), k/v (B,H,Tk,Dh) bf16-valued fp32; keep (Tq,Tk) bool.

    ``banded_bf16`` restates the training forward's block-banded attention
    (model.py:171-178): the scores come out of a bf16 matmul and are scaled in
    bf16, the -30000 additive mask zeroes the dropped keys exactly (exp
    underflows in fp32), softmax(precise=True) runs in fp32 and returns bf16,
    and P.V is a bf16 matmul.  The 512-query bands (model.py:155-169) never
    drop an allowed key (ks = max(0, qs - W) <= i - W + 1), so the band
    structure itself changes nothing and is not restated.

    Long inputs are processed in blocks of query rows, each against the key
    columns its rows keep (softmax is per row and a dropped key contributes an
    exact zero), which bounds the memory of the score matrix."""
    Tq, Tk = keep.shape
    if Tq * Tk <= (1 << 22):
        return _attention_block(q, k, v, keep, scale, mlx_fallback_attn, banded_bf16)
    outs = []
    for qs in range(0, Tq, 512):
        qe = min(qs + 512, Tq)
        cols = torch.nonzero(keep[qs:qe].any(0)).flatten()
        ks, ke = (int(cols[0]), int(cols[-1]) + 1) if cols.numel() else (0, 1)
        outs.append(_attention_block(q[:, :, qs:qe], k[:, :, ks:ke], v[:, :, ks:ke],
                                     keep[qs:qe, ks:ke], scale, mlx_fallback_attn, banded_bf16))
    return torch.cat(outs, dim=2)


def _attention_block(q, k, v, keep, scale, mlx_fallback_attn, banded_bf16):
    if banded_bf16:
        s = bf(bf(q @ k.transpose(-1, -2)) * scale)
        s = s.masked_fill(~keep, float("-inf"))
        p = bf(torch.softmax(s, dim=-1))
        return bf(p @ v)
    if mlx_fallback_attn:
        s = bf(bf(q * scale) @ k.transpose(-1, -2))
        s = s.masked_fill(~keep, float("-inf"))
        p = bf(torch.softmax(s, dim=-1))
        return bf(p @ v)
    s = (q @ k.transpose(-1, -2)) * scale
    s = s.masked_fill(~keep, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return bf(p @ v)


# -- model.py:255-260: the two residual mixes and the MLP branch ----------------
def mix_attn(x, y, x0, r0, p0, xl):
    """model.py:256, eager bf16 left to right: (r0*x + p0*y) + xl*x0."""
    return bf(bf(bf(r0 * x) + bf(p0 * y)) + bf(xl * x0))


def mix_mlp(x, y, x0, r1, p1, xl):
    """model.py:260: r1*x + p1*y (the embedding stream x0 does not enter)."""
    return bf(bf(r1 * x) + bf(p1 * y))


def mlp_branch(h, fc, proj):
    """model.py:258-259: bf16(relu2(bf16(h @ fc)) @ proj)."""
    return bf(relu2(bf(h @ fc)) @ proj)


class Prepared:
    """bf16-rounded, lambda-folded weights (model.py:229-241, 258-259, 262)."""

    def __init__(self, cfg, params):
        self.cfg = cfg
        t = {k: torch.as_tensor(v, dtype=F32) for k, v in params.items()}
        L = cfg.num_layers
        self.resid = bf(t["resid_lambdas"])
        self.post = bf(t["post_lambdas"])
        self.x0l = bf(t["x0_lambdas"])
        sal = bf(t["sa_lambdas"])
        self.embed = bf(t["embed"])
        self.lm_head = bf(t["lm_head"])
        self.qkv_w, self.wo, self.fc, self.proj = [], [], [], []
        for l in range(L):
            wl = bf(t["attn_bank"][l])
            self.qkv_w.append(bf(torch.cat([wl[0], wl[1], wl[2]], dim=-1) * sal[l, 0]))
            self.wo.append(bf(wl[3] * sal[l, 1]))
            self.fc.append(bf(t["fc_bank"][l]))
            self.proj.append(bf(t["proj_bank"][l]))
        self.cs, self.sn = rope_tables(cfg.seq_len, cfg.head_dim, cfg.rope_base)


class KVCache:
    """Per-layer K/V (B,H,T,Dh) bf16-valued fp32, grown by forward()."""

    def __init__(self, L):
        self.k = [None] * L
        self.v = [None] * L

    @property
    def length(self):
        return 0 if self.k[0] is None else self.k[0].shape[2]


def forward(prep, tokens, cache=None, mlx_fallback_attn=False, return_hidden=False,
            banded_bf16=False, last_only=False):
    """Forward of ``tokens`` (B,T) placed at positions [start, start+T) where
    start = cache.length (0 without a cache).  Returns softcapped fp32 logits
    (B,T,V).  With ``cache`` the new K/V are appended (KV-cache decode);
    without it this is exactly ``GPT.logits`` (model.py:223-263).
    ``last_only`` computes the lm_head for the last row only (B,1,V): the
    rows of the lm_head product are independent, so that row is unchanged.""" 
    cfg = prep.cfg
    tokens = torch.as_tensor(tokens, dtype=torch.long)
    B, T = tokens.shape
    H, Dh, d = cfg.num_heads, cfg.head_dim, cfg.model_dim
    start = 0 if cache is None else cache.length
    pos = torch.arange(start, start + T)
    kpos = torch.arange(0, start + T)
    if start + T > cfg.seq_len:
        raise ValueError("context exceeds seq_len (RoPE table length)")

    x = rms(prep.embed[tokens])                                     # model.py:236
    x0 = x
    for l in range(cfg.num_layers):
        h = rms(x)                                                  # :242
        qkv = bf(h @ prep.qkv_w[l]).reshape(B, T, 3, H, Dh)         # :243
        q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
        q, k = rms(q), rms(k)                                       # :245
        q = rope_ht(q, prep.cs, prep.sn, pos)                       # :246
        k = rope_ht(k, prep.cs, prep.sn, pos)                       # :247
        q, k, v = (t.transpose(1, 2) for t in (q, k, v))            # (B,H,T,Dh)
        if cache is not None:
            if cache.k[l] is not None:
                k = torch.cat([cache.k[l], k], dim=2)
                v = torch.cat([cache.v[l], v], dim=2)
            cache.k[l], cache.v[l] = k, v
        keep = keep_mask(pos, kpos, l in cfg.long_layers, cfg.window)   # :248-250
        y = attention(q, k, v, keep, cfg.attn_scale, mlx_fallback_attn,  # :251-254
                      banded_bf16)
        y = bf(y.transpose(1, 2).reshape(B, T, d) @ prep.wo[l])        # :255
        x = mix_attn(x, y, x0, prep.resid[l, 0], prep.post[l, 0], prep.x0l[l])   # :256
        h = rms(x)                                                  # :257
        y = mlp_branch(h, prep.fc[l], prep.proj[l])                 # :258-259
        x = mix_mlp(x, y, x0, prep.resid[l, 1], prep.post[l, 1], prep.x0l[l])    # :260
    if last_only:
        x = x[:, -1:]
    hfin = rms(x)
    z = bf(hfin @ prep.lm_head)                                     # :262
    out = softcap(z)                                                # :263
    if return_hidden:
        return out, z, hfin
    return out


def softcap_ce(z, targets):
    """Fused softcapped cross-entropy of ``ce_softcap_fwd`` (metal_kernels.py:
    153-193; pure-MLX form model.py:104-110): per row of z (N, V), in fp32,
    zc = 23 sigmoid((z + 5) / 7.5), lse = log sum exp(zc) over all V columns,
    loss = lse - zc[target].  Returns (loss (N,), lse (N,))."""
    zc = softcap(z)
    lse = torch.logsumexp(zc, dim=-1)
    tl = zc.gather(-1, torch.as_tensor(targets, dtype=torch.long)[:, None]).squeeze(-1)
    return lse - tl, lse


def loss(cfg, params, tokens, targets, banded_bf16=True):
    """``GPT.__call__`` (model.py:180-221): the forward with the training
    attention, z = bf16(rms(x) @ lm_head) for every row (B*T, V) and the mean
    softcapped CE.  Returns (mean fp32 scalar, per-row losses (B*T,))."""
    prep = Prepared(cfg, params)
    _, z, _ = forward(prep, tokens, None, return_hidden=True, banded_bf16=banded_bf16)
    rows, _ = softcap_ce(z.reshape(-1, cfg.vocab_size),
                         torch.as_tensor(targets, dtype=torch.long).reshape(-1))
    return rows.mean(), rows


def logits(cfg, params, tokens, mlx_fallback_attn=False):
    """``GPT(cfg).logits(params, tokens)`` restated: (B,T) -> (B,T,V) fp32."""
    return forward(Prepared(cfg, params), tokens, None, mlx_fallback_attn)


def forward_fp64(cfg, params, tokens):
    """Same graph with no bf16 rounding anywhere, in fp64 (for tolerance checks)."""
    t = {k: torch.as_tensor(v, dtype=torch.float64) for k, v in params.items()}
    tokens = torch.as_tensor(tokens, dtype=torch.long)
    B, T = tokens.shape
    H, Dh, d = cfg.num_heads, cfg.head_dim, cfg.model_dim

    def r(x):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6)

    cs, sn = (a.double() for a in rope_tables(cfg.seq_len, Dh, cfg.rope_base))
    pos = torch.arange(T)

    def rope(x):
        d4 = Dh // 4
        c, s = cs[pos][None, :, None, :], sn[pos][None, :, None, :]
        y = x.clone()
        x0, x1 = x[..., 0:2 * d4:2], x[..., 1:2 * d4:2]
        y[..., 0:2 * d4:2] = c * x0 + s * x1
        y[..., 1:2 * d4:2] = c * x1 - s * x0
        return y

    x = r(t["embed"][tokens])
    x0 = x
    for l in range(cfg.num_layers):
        wl = t["attn_bank"][l]
        sal = t["sa_lambdas"][l]
        qkv = (r(x) @ (torch.cat([wl[0], wl[1], wl[2]], -1) * sal[0])).reshape(B, T, 3, H, Dh)
        q, k, v = r(qkv[:, :, 0]), r(qkv[:, :, 1]), qkv[:, :, 2]
        q, k = rope(q), rope(k)
        q, k, v = (a.transpose(1, 2) for a in (q, k, v))
        keep = keep_mask(pos, pos, l in cfg.long_layers, cfg.window)
        s = (q @ k.transpose(-1, -2)) * cfg.attn_scale
        p = torch.softmax(s.masked_fill(~keep, float("-inf")), -1)
        y = (p @ v).transpose(1, 2).reshape(B, T, d) @ (wl[3] * sal[1])
        x = t["resid_lambdas"][l, 0] * x + t["post_lambdas"][l, 0] * y + t["x0_lambdas"][l] * x0
        m = torch.clamp_min(r(x) @ t["fc_bank"][l], 0.0) ** 2
        x = t["resid_lambdas"][l, 1] * x + t["post_lambdas"][l, 1] * (m @ t["proj_bank"][l])
    z = r(x) @ t["lm_head"]
    return 23.0 * torch.sigmoid((z + 5.0) / 7.5)


def degenerate_known_answer(cfg, params, tokens):
    """Closed form of the forward under the model.py init (Wo = proj = x0 = 0).

    Every layer then maps x -> bf16(bf16(r1 * bf16(bf16(r0*x) + 0)) + 0) with
    r = bf16(resid), so x_L is a per-element bf16 chain of x0 = rms(embed[tok])
    and the logits of a row depend only on that row's token.  Returned: (B,T,V).
    """
    t = {k: torch.as_tensor(v, dtype=F32) for k, v in params.items()}
    for k in ("x0_lambdas",):
        if torch.any(t[k] != 0):
            raise ValueError("known answer needs x0_lambdas == 0")
    if torch.any(t["attn_bank"][:, 3] != 0) or torch.any(t["proj_bank"] != 0):
        raise ValueError("known answer needs Wo == 0 and proj == 0")
    tokens = torch.as_tensor(tokens, dtype=torch.long)
    x = rms(bf(t["embed"])[tokens])
    res = bf(t["resid_lambdas"])
    post = bf(t["post_lambdas"])
    for l in range(cfg.num_layers):
        x = bf(bf(res[l, 0] * x) + bf(post[l, 0] * 0.0))
        x = bf(bf(res[l, 1] * x) + bf(post[l, 1] * 0.0))
    z = bf(rms(x) @ bf(t["lm_head"]))
    return softcap(z)
