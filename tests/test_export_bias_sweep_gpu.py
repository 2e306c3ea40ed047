"""Seeded sweeps of the tau-export reductions and of the graph-bias builder.

Head statistics (16 cases): layers, batch, length, heads, W, tau dtype and
the valid-only mask, drawn so that both the register-resident selection
(batch 1, W dividing 512, T * W <= 65536) and the general streaming path
run; against oracle/export_ref.py with the tolerances of
test_export_gpu.py (the 0.99 quantile to 1e-7: the kernel forms it in
float32 as np.quantile does on float32 data).  Head-masked aggregate (10 cases): random masks,
including all-off (the reference then averages every head).  Graph bias
(12 cases): local [B, T, W] and global [B, T, T] tables over random edge
maps (weights <= 0 included, repeated and unknown tokens), every output
dtype, bit-exact against the reference loops of oracle/bias_ref.py.
"""
import numpy as np
import pytest
import torch

from bozo_amd import export as E
from bozo_amd.bias import GraphBias
from oracle import bias_ref as R
from oracle import export_ref as X
from tests.test_bias_gpu import Tok as BiasTok
from tests.test_bias_gpu import make as make_edges

pytestmark = pytest.mark.gpu

_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32, "f64": torch.float64}


def _taus(seed, L, B, T, H, W, dtype):
    g = torch.Generator().manual_seed(seed)
    return [(torch.rand(B, T, H, W, generator=g, dtype=torch.float64) ** (1 + 3 * (l % 4))).to(dtype)
            for l in range(L)]


def _draw_stats(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        W = int(rng.choice([1, 3, 8, 16, 64, 100]))
        T = int(rng.choice([1, 2, 63, 257, 1024] + ([2048] if W <= 64 else [])))
        cases.append((i, int(rng.choice([1, 3, 9])), int(rng.choice([1, 1, 2, 3])), T, int(rng.choice([1, 5, 12])),
                      W, str(rng.choice(["f32", "bf16", "f16"])), bool(rng.integers(2))))
    return cases


STATS = _draw_stats(16, 2032)


@pytest.mark.parametrize("case", STATS, ids=[f"{c[0]}-L{c[1]}B{c[2]}T{c[3]}H{c[4]}W{c[5]}-{c[6]}"
                                             f"{'-valid' if c[7] else ''}" for c in STATS])
def test_head_stats_sweep(dev, case):
    i, L, B, T, H, W, dt, valid_only = case
    taus = _taus(1300 + i, L, B, T, H, W, _DT[dt])
    fast = B == 1 and W <= 64 and 512 % W == 0 and T * W <= 65536
    print(f"[head stats sweep {case}] {'register-resident' if fast else 'streaming'} select", flush=True)
    got = E.head_stats([t.to(dev) for t in taus], valid_only).cpu().numpy()
    ref = X.head_stats([t.float().numpy() for t in taus], valid_only)
    assert got.shape == ref.shape == (L, H, 4)
    assert np.allclose(got[..., [0, 2, 3]], ref[..., [0, 2, 3]], rtol=1e-5, atol=1e-6)
    assert np.max(np.abs(got[..., 1] - ref[..., 1])) <= 1e-7


def _draw_agg(n, seed):
    rng = np.random.default_rng(seed)
    return [(i, int(rng.choice([1, 2, 4, 9])), int(rng.choice([1, 2])), int(rng.choice([1, 17, 130, 600])),
             int(rng.choice([1, 6, 12, 64])), int(rng.choice([1, 5, 16, 64])), str(rng.choice(["f32", "bf16"])),
             float(rng.choice([0.0, 0.3, 0.7, 1.0]))) for i in range(n)]


AGG = _draw_agg(10, 2033)


@pytest.mark.parametrize("case", AGG, ids=[f"{c[0]}-L{c[1]}B{c[2]}T{c[3]}H{c[4]}W{c[5]}-{c[6]}-on{c[7]}" for c in AGG])
def test_aggregate_sweep(dev, case):
    i, L, B, T, H, W, dt, frac_on = case
    taus = _taus(1400 + i, L, B, T, H, W, _DT[dt])
    mask = torch.rand(L, H, generator=torch.Generator().manual_seed(1500 + i)) < frac_on
    print(f"[aggregate sweep {case}] heads on: {int(mask.sum())}", flush=True)
    got = E.aggregate_tau([t.to(dev) for t in taus], mask).cpu().numpy()
    ref = X.aggregate([t.float().numpy() for t in taus], mask.numpy())
    assert got.shape == ref.shape == (T, W)
    assert np.allclose(got, ref, atol=1e-6)


def _draw_bias(n, seed):
    rng = np.random.default_rng(seed)
    return [(i, bool(rng.integers(2)), int(rng.choice([0, 10, 500, 4000])), int(rng.choice([1, 9, 128, 300])),
             int(rng.choice([1, 3, 16, 64])), int(rng.choice([1, 2])), str(rng.choice(["f32", "bf16", "f16", "f64"])),
             float(rng.choice([0.25, 0.6, 1.5]))) for i in range(n)]


BIAS = _draw_bias(12, 2034)


@pytest.mark.parametrize("case", BIAS, ids=[f"{c[0]}-{'global' if c[1] else 'local'}-E{c[2]}T{c[3]}W{c[4]}b{c[5]}"
                                            f"-{c[6]}" for c in BIAS])
def test_bias_sweep(dev, case):
    i, glob, n_edges, T, W, batch, dt, alpha = case
    dtype = _DT[dt]
    edge_map, ids = make_edges(1600 + i, 97, n_edges, T)
    gb = GraphBias(edge_map, alpha=alpha)
    tok = BiasTok()
    contents = [tok.id_to_token(t) or f"<{t}>" for t in ids]
    print(f"[bias sweep {case}]", flush=True)
    if glob:
        bias, st = gb.global_bias(ids, tok, batch=batch, device=dev, dtype=dtype)
        ref, (hits, mx, mean) = R.global_bias(edge_map, alpha, contents, batch, dtype=np.float64)
        shape = (batch, T, T)
    else:
        bias, st = gb.local_bias(ids, tok, window=W, batch=batch, device=dev, dtype=dtype)
        ref, (hits, mx, mean) = R.local_bias(edge_map, alpha, contents, W, batch, dtype=np.float64)
        shape = (batch, T, W)
    ref_t = torch.from_numpy(ref)
    if dtype != torch.float64:
        ref_t = ref_t.float().to(dtype)
    assert bias.shape == shape and bias.dtype == dtype
    assert torch.equal(bias.cpu(), ref_t)
    assert st.nonzero_pairs == hits and st.max_weight == mx
    assert abs(st.mean_weight - mean) <= 1e-12 * max(1.0, mean)
