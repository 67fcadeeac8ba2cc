"""ORACLE -- test infrastructure only.

Restatement of the reference sampling step (``/root/reference/sample.py:42-51``)
for a row of softcapped logits, plus the counter-based generator the build
uses for its draws.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may use it.

sample.py per token:  z = logits[0,-1][:50257] / temp
                      kth = sort(z)[-top_k];  z = where(z < kth, -1e9, z)
                      nxt = categorical(z)
  * every value >= kth is kept (ties at the threshold included);
  * temp = 0 divides by zero in the reference, so greedy is defined here as
    argmax over the first 50257 entries with the lowest index winning ties;
  * the reference never seeds MLX's generator, so its draws cannot be
    reproduced; the build draws u ~ U[0,1) from Philox4x32-10 with
    counter (step, row, 0, 0) and key (seed_lo, seed_hi), and picks the first
    kept index whose running sum of exp((z_i - z_max)) exceeds u * total
    (inverse CDF over the kept set in index order).

Parity status: greedy and the kept set are pinned by closed forms (argmax,
sort threshold); the draw distribution by a chi-square test; Philox4x32-10 by
the Random123 known-answer vectors (Salmon et al., SC'11).
"""

import numpy as np

V_SAMPLE = 50257

_M0, _M1 = 0xD2511F53, 0xCD9E8D57
_W0, _W1 = 0x9E3779B9, 0xBB67AE85
_MASK = 0xFFFFFFFF


def philox4x32_10(ctr, key):
    """Philox4x32 with 10 rounds (Salmon, Moraes, Dror, Shaw, SC'11)."""
    c0, c1, c2, c3 = (int(c) & _MASK for c in ctr)
    k0, k1 = (int(k) & _MASK for k in key)
    for _ in range(10):
        p0 = _M0 * c0
        p1 = _M1 * c2
        hi0, lo0 = p0 >> 32, p0 & _MASK
        hi1, lo1 = p1 >> 32, p1 & _MASK
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        k0 = (k0 + _W0) & _MASK
        k1 = (k1 + _W1) & _MASK
    return (c0, c1, c2, c3)


def uniform(seed, step, row):
    """u in [0,1): top 24 bits of the first Philox word."""
    w = philox4x32_10((step & _MASK, row & _MASK, (step >> 32) & _MASK, 0),
                      (seed & _MASK, (seed >> 32) & _MASK))[0]
    return (w >> 8) * (1.0 / 16777216.0)


def kept_set(z, temperature, top_k):
    """Indices sample.py:45-48 keeps (all >= the k-th largest of z/temp)."""
    zt = np.asarray(z[:V_SAMPLE], dtype=np.float32) / np.float32(temperature)
    if top_k and top_k < zt.size:
        kth = np.sort(zt)[-top_k]
        return zt, np.nonzero(zt >= kth)[0]
    return zt, np.arange(zt.size)


def sample_row(z, temperature, top_k, u):
    """One draw for one row of softcapped logits z (V,) fp32."""
    z = np.asarray(z, dtype=np.float32)
    if temperature == 0.0:
        return int(np.argmax(z[:V_SAMPLE]))          # first maximal index
    zt, keep = kept_set(z, temperature, top_k)
    vals = zt[keep].astype(np.float64)
    w = np.exp(vals - vals.max())
    c = np.cumsum(w)
    i = int(np.searchsorted(c, u * c[-1], side="right"))
    return int(keep[min(i, keep.size - 1)])


def probabilities(z, temperature, top_k):
    """The categorical distribution sample.py:49 draws from (V_SAMPLE,)."""
    zt, keep = kept_set(z, temperature, top_k)
    p = np.zeros(zt.size)
    w = np.exp(zt[keep].astype(np.float64) - zt[keep].max())
    p[keep] = w / w.sum()
    return p
