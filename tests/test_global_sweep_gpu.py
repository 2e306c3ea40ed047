"""Seeded sweep of the global (full causal, diagonal included) block against
the float64 oracle (model.py:217-238).

Twenty-four configurations drawn once from a fixed generator: batch and
head counts, ragged T around the 64-row tiles, head dims 64 (the MFMA
kernels for bfloat16) and 32 (the exact kernels), bfloat16 and float32,
with and without the [B, T, T] bias, and the tau_local output with its
gradient at several widths.  Tolerances as in test_global_gpu.py: float32
max-abs 1e-5, bfloat16 2e-2 relative L2, tau_local elementwise.
"""
import numpy as np
import pytest
import torch

from tests._util import f64, make_inputs, max_abs, rel_l2
from tests.test_global_gpu import hip_run, oracle_run

pytestmark = pytest.mark.gpu


def _draw(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B = int(rng.choice([1, 2, 3]))
        H = int(rng.choice([1, 2, 3, 4]))
        T = int(rng.choice([1, 2, 31, 63, 64, 65, 128, 129, 200, 257]))
        D = int(rng.choice([64, 64, 32]))
        dtype = str(rng.choice(["bf16", "f32"]))
        bias = bool(rng.integers(2))
        wl = [None, 1, 16, 64][int(rng.integers(4))]
        if wl is not None and wl > T:
            wl = T
        cases.append((i, B, H, T, D, dtype, bias, wl))
    return cases


CASES = _draw(24, 2028)


def _id(c):
    i, B, H, T, D, dtype, bias, wl = c
    return f"{i}-B{B}H{H}T{T}D{D}-{dtype}{'-bias' if bias else ''}{f'-tl{wl}' if wl else ''}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_global_sweep(dev, case):
    i, B, H, T, D, dtype, bias, wl = case
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    inp = make_inputs(B, T, H, D, seed=500 + i, std=0.5, dtype=dt, W=wl or 1, dtau_std=0.1 if wl else None,
                      bias_std=0.5 if bias else None, bias_shape=(B, T, T) if bias else None)
    scale = float(np.sqrt(D))
    print(f"[global sweep {_id(case)}]", flush=True)
    out, tl, grads = hip_run(inp, scale, dev, W_local=wl, use_bias=bias, use_dtl=wl is not None)
    rout, rtl, rgrads = oracle_run(inp, scale, W_local=wl, use_bias=bias, use_dtl=wl is not None)
    # T = 1: the one query sees only itself, out = v_0 whatever the score, so
    # without a tau_local gradient dQ and dK vanish in exact arithmetic and
    # are held to max-abs 1e-5 (a relative error of rounding noise is
    # meaningless)
    zero_qk = T == 1 and wl is None
    for what, got, want in zip(("out", "dQ", "dK", "dV"), (out,) + tuple(grads), (rout,) + tuple(rgrads)):
        if dt == torch.float32 or (zero_qk and what in ("dQ", "dK")):
            err, lim = max_abs(f64(got), want), 1e-5
        else:
            err, lim = rel_l2(f64(got), want), 2e-2
        print(f"  {what}: err {err:.3e} (limit {lim:.0e})", flush=True)
        assert err <= lim, f"{what}: err {err:.3e} > {lim:.0e}"
    if wl:
        err = max_abs(f64(tl), rtl)
        lim = 1e-5 if dt == torch.float32 else 4e-3
        print(f"  tau_local: max abs err {err:.3e}", flush=True)
        assert err <= lim, f"tau_local: max abs err {err:.3e} > {lim:.0e}"
