"""Input generation and comparison helpers shared by the tests.

Inputs follow the benchmark recipe: CPU ``torch.Generator`` seeds, drawn as
float32 in the order Q, K, V, dOut (then dTau), RoPE (base 10000, positions
0..T-1, half-split) applied to Q and K in float32 before the cast, so values
are device independent.  The oracle consumes the cast values upcast to
float64.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import tension_oracle as O


def make_inputs(B, T, H, D, *, seed, std=1.0, rope=True, dtype=torch.float32, W=None,
                dtau_std=None, bias_std=None, bias_shape=None):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, T, H, D, generator=g) * std
    K = torch.randn(B, T, H, D, generator=g) * std
    V = torch.randn(B, T, H, D, generator=g) * std
    dO = torch.randn(B, T, H, D, generator=g)
    dTau = torch.randn(B, T, H, W, generator=g) * dtau_std if dtau_std else None
    bias = torch.randn(*bias_shape, generator=g) * bias_std if bias_std else None
    if rope:
        cos, sin = O.rope_tables(T, D)
        Q = torch.from_numpy(O.rope_apply(Q.numpy(), cos, sin).astype(np.float32))
        K = torch.from_numpy(O.rope_apply(K.numpy(), cos, sin).astype(np.float32))
    cast = lambda t: None if t is None else t.to(dtype)  # noqa: E731
    return dict(Q=cast(Q), K=cast(K), V=cast(V), dO=cast(dO), dTau=cast(dTau), bias=bias)


def f64(t):
    return None if t is None else t.detach().to(torch.float64).cpu().numpy()


def max_abs(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b))) if a.size else 0.0


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a - b))


def scale_of(D):
    return math.sqrt(D)


def device_cus(dev=0):
    """Compute units of the GPU the kernels run on (the host launch code
    queries the same attribute); 256 on MI355X, also assumed without a GPU."""
    if torch.cuda.is_available():
        return int(torch.cuda.get_device_properties(dev).multi_processor_count)
    return 256


def fused_geometry(B, H, T, tile=64, cus=None):
    """Launch geometry of the bf16 W <= 64 band kernels, restated from their
    host dispatch (bozo_amd/csrc/mfma.hip ``launch_mfma``: forward chunks while
    the grid keeps >= 3 workgroups per CU, backward runs aimed at 2 per CU;
    the fast forward with tau caps its tiles per workgroup at 2,
    mfma_fwd.hip ``go``), for a device with ``cus`` compute units (default:
    the current GPU's).

    Returns (fwd_tiles_per_workgroup, bwd_runs_per_sequence,
    longest_bwd_run_in_tiles).  A backward run of r tiles takes r own steps
    plus one recomputed halo step; runs longer than one tile hand dTau rows
    and the previous key block's partial dK/dV from step to step."""
    if cus is None:
        cus = device_cus()
    ntiles = -(-T // tile)
    bh = B * H
    chunk = 1
    while chunk < 4 and bh * (-(-ntiles // (2 * chunk))) >= 3 * cus:
        chunk *= 2
    runs = min(max(1, (2 * cus + bh // 2) // bh), ntiles)
    longest = max((r + 1) * ntiles // runs - r * ntiles // runs for r in range(runs))
    return chunk, runs, longest
