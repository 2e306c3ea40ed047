"""CPU restatement of the reference's graph-bias builder (pure Python).

TEST INFRASTRUCTURE ONLY: the checker for ``bozo_amd/bias.py`` and the CPU
baseline ``bench.py`` times; nothing in the product imports it.

Follows ``ts_bridge/bias.py``: ``local_bias`` <- 141-187 (bias[b, t, w] =
alpha * weight(content[t - (W - w)] -> content[t]) when that weight > 0 and
the key is inside the context), ``global_bias`` <- 189-233 (bias[b, t, s]
for s < t), both with the (hits, max, mean) statistics; weights come from a
(src_content, dst_content) -> weight map.
"""
from __future__ import annotations

import numpy as np


def _fill(edge_map, alpha, contents, pairs, shape, batch, dtype):
    bias = np.zeros((batch,) + shape, dtype=np.float64)
    hits, total, mx = 0, 0.0, 0.0
    for (t, j, s) in pairs:
        weight = edge_map.get((contents[s], contents[t]), 0.0)
        if weight <= 0.0:
            continue
        bias[:, t, j] = alpha * weight
        hits += 1
        total += weight
        mx = max(mx, weight)
    return bias.astype(np.float32).astype(dtype) if dtype != np.float64 else bias, \
        (hits, mx, total / hits if hits else 0.0)


def local_bias(edge_map, alpha, contents, W, batch=1, dtype=np.float32):
    T = len(contents)
    pairs = [(t, w, t - (W - w)) for t in range(T) for w in range(W) if t - (W - w) >= 0]
    return _fill(edge_map, alpha, contents, pairs, (T, W), batch, dtype)


def global_bias(edge_map, alpha, contents, batch=1, dtype=np.float32):
    T = len(contents)
    pairs = [(t, s, s) for t in range(T) for s in range(t)]
    return _fill(edge_map, alpha, contents, pairs, (T, T), batch, dtype)
