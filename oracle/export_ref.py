"""CPU restatement of the reference's tau-export reductions (numpy).

TEST INFRASTRUCTURE ONLY: the checker for ``bozo_amd/export.py`` and its
HIP reductions, and the CPU baseline ``bench.py`` times; nothing in the
product imports it.

Follows (reference ``ts_bridge/``):
* ``head_stats``      <- ``head_filter.py:98-130`` (``profile_heads``: batch
  mean, then per head: mean, ``np.quantile(.., 0.99)``, mean arg-max over w,
  mean max over w; the quantile restated in ``quantile99_f32``) and, with
  ``valid_only``, ``corpus_profile.py:58-98``
  (cells with t + w < W zeroed first; no mean there, computed anyway);
* ``classify``        <- ``head_filter.py:74-90`` (thresholds 0.40, 0.35,
  0.7 W, 0.3 W);
* ``aggregate``       <- ``export.py:185-200`` (stack of local layers, batch
  mean, mean over the selected (layer, head) pairs; all pairs when none);
* ``concentration``   <- ``export.py:202-218`` (Gini over the valid pairs
  t - (W - w) >= 0 and their mean);
* ``edges``           <- ``export.py:225-268`` (pairs with s >= 0 and weight
  >= threshold, in t then w order; own pull = row mean over all w).
"""
from __future__ import annotations

import numpy as np

MAX_TAU_FLOOR = 0.40
CONCENTRATION = 0.35


def quantile99_f32(vals) -> float:
    """``np.quantile(vals, 0.99)`` of float32 values as numpy >= 2 computes
    it (the reference's call at head_filter.py:113; requirements.txt pins
    only numpy>=1.24): a Python-float q is cast to the array's dtype, so q,
    the rank g = (n - 1) q, its fractional part t and the linear
    interpolation a + (b - a) t (b - (b - a)(1 - t) for t >= 0.5) are each
    rounded to float32 -- g = 2034.45007 for n = 2056, not 2034.45.  numpy
    1.x formed the rank in float64; the two differ by about 1e-4 of the gap
    between the two order statistics."""
    s = np.sort(np.asarray(vals, dtype=np.float32).ravel())
    n = s.size
    g = np.float32(n - 1) * np.float32(0.99)
    k = int(np.floor(g))
    t = np.float32(g - np.float32(k))
    a, b = s[k], s[min(k + 1, n - 1)]
    d = np.float32(b - a)
    if t >= 0.5:
        return float(np.float32(b - np.float32(d * np.float32(np.float32(1) - t))))
    return float(np.float32(a + np.float32(d * t)))


def head_stats(taus, valid_only: bool = False) -> np.ndarray:
    """taus: list of L arrays [B,T,H,W].  Returns [L,H,4] = mean, p99,
    peak_pos, concentration."""
    out = []
    for tau in taus:
        t = np.asarray(tau, dtype=np.float32).mean(axis=0)       # T H W
        T, H, W = t.shape
        if valid_only:
            valid = (np.arange(T)[:, None] + np.arange(W)[None, :]) >= W
            t = t * valid[:, None, :]
        rows = []
        for h in range(H):
            vals = t[:, h, :]
            rows.append([float(vals.mean()), quantile99_f32(vals),
                         float(vals.argmax(axis=-1).mean()), float(vals.max(axis=-1).mean())])
        out.append(rows)
    return np.asarray(out, dtype=np.float64)


def classify(mean_tau, max_tau, peak_pos, concentration, W) -> str:
    if max_tau < MAX_TAU_FLOOR:
        return "inactive"
    if concentration < CONCENTRATION:
        return "diffuse"
    if peak_pos > W * 0.7:
        return "syntactic"
    if peak_pos < W * 0.3:
        return "long_range"
    return "mid_range"


def aggregate(taus, head_mask) -> np.ndarray:
    """Mean over the selected (layer, head) pairs of the batch-mean tau: [T, W]."""
    tau = np.stack([np.asarray(t, dtype=np.float32).mean(axis=0) for t in taus])  # L T H W
    L, T, H, W = tau.shape
    lh = tau.transpose(1, 3, 0, 2).reshape(T, W, L * H)
    m = np.asarray(head_mask, dtype=bool).reshape(-1)
    return lh[:, :, m].mean(axis=-1) if m.any() else lh.mean(axis=-1)


def valid_mask(T: int, W: int) -> np.ndarray:
    return (np.arange(T)[:, None] - (W - np.arange(W)[None, :])) >= 0


def concentration(agg) -> tuple:
    """(Gini, mean) over the valid pairs of the aggregated matrix."""
    T, W = agg.shape
    vals = agg[valid_mask(T, W)]
    if vals.size > 1 and vals.sum() > 1e-9:
        s = np.sort(vals)
        n = s.size
        cum = np.cumsum(s)
        gini = float((n + 1 - 2 * cum.sum() / cum[-1]) / n)
    else:
        gini = 0.0
    return gini, (float(vals.mean()) if vals.size else 0.0)


def edges(agg, threshold: float):
    """[(t, s, weight)] in emission order, and the per-query own pull [T]."""
    T, W = agg.shape
    out = []
    for t in range(T):
        for w in range(W):
            s = t - (W - w)
            if s < 0:
                continue
            if float(agg[t, w]) < threshold:
                continue
            out.append((t, s, float(agg[t, w])))
    return out, agg.mean(axis=-1)
