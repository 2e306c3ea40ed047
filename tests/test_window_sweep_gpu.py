"""Seeded sweep of the local-window op against the float64 oracle.

Forty-eight configurations drawn once from a fixed generator cover the
space the targeted tests in test_window_gpu.py sample by hand: batch and
head counts that change the launch geometry, ragged T around the 64-row
tiles, windows below, at and above 64 (the fused single-pass backward, the
split backward), head dims 64 and 32, bfloat16 and float32 (the
float32 flow: the split kernels with every operand as three bf16 terms),
every normalisation, with and without the bias, with and without tau and
its gradient.  Sixteen more run the split-operand kernels of the
reference's autocast flow (float32 Q / K, bfloat16 V) at head dims 32 and
64 and windows up to 300, and twelve float16 throughout.  Tolerances are
the ones of test_window_gpu.py (float32 max-abs 1e-5 absolute, raw sums
included; bfloat16 2e-2 relative L2; tau elementwise) and of
test_float16_flow_gpu.py (float16 1e-3 relative L2, tau 2^-11), checked
against the same oracle functions.
"""
import numpy as np
import pytest
import torch

from tests._util import f64, make_inputs, max_abs
from tests.test_float16_flow_gpu import check as check_f16
from tests.test_window_gpu import check_bf16, check_mixed, hip_run, mixed_inputs, oracle_run

pytestmark = pytest.mark.gpu


def _draw(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B = int(rng.choice([1, 2, 3]))
        H = int(rng.choice([1, 2, 3, 5]))
        T = int(rng.choice([1, 2, 17, 63, 64, 65, 127, 128, 129, 200, 256, 320]))
        W = int(rng.choice([1, 3, 16, 31, 32, 63, 64, 65, 100, 128]))
        D = int(rng.choice([64, 64, 64, 32]))
        dtype = str(rng.choice(["bf16", "f32"]))
        norm = [None, "mass", "count"][int(rng.integers(3))]
        bias = bool(rng.integers(2))
        tau = bool(rng.integers(2))
        cases.append((i, B, H, T, W, D, dtype, norm, bias, tau))
    return cases


CASES = _draw(48, 2026)


def _id(c):
    i, B, H, T, W, D, dtype, norm, bias, tau = c
    return f"{i}-B{B}H{H}T{T}W{W}D{D}-{dtype}-{norm}{'-bias' if bias else ''}{'-tau' if tau else ''}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_window_sweep(dev, case):
    i, B, H, T, W, D, dtype, norm, bias, tau = case
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    inp = make_inputs(B, T, H, D, seed=100 + i, std=0.5, dtype=dt, W=W, dtau_std=0.1 if tau else None,
                      bias_std=0.5 if bias else None, bias_shape=(B, T, W) if bias else None)
    scale = float(np.sqrt(D))
    print(f"[sweep {_id(case)}]", flush=True)
    out, tau_h, grads = hip_run(inp, W, scale, dev, normalize=norm, return_tau=tau, use_bias=bias, use_dtau=tau)
    rout, rtau, rgrads = oracle_run(inp, W, scale, normalize=norm, use_bias=bias, use_dtau=tau)
    # W = 1 under tau-mass: out_t = v_{t-1} whatever the score, so dQ and dK
    # vanish in exact arithmetic (the oracle's are float64 rounding noise) and
    # a relative error is meaningless; they are held to max-abs 1e-5 instead
    zero_qk = norm == "mass" and W == 1 and not tau
    for what, got, want in zip(("out", "dQ", "dK", "dV"), (out,) + tuple(grads), (rout,) + tuple(rgrads)):
        if zero_qk and what in ("dQ", "dK"):
            err = max_abs(f64(got), want)
            print(f"  {what}: max abs err {err:.3e} (identically zero)", flush=True)
            assert err <= 1e-5, f"{what}: max abs err {err:.3e} > 1e-5"
            continue
        if dt == torch.bfloat16:
            check_bf16(got, want, what)
            continue
        lim = 1e-5
        err = max_abs(f64(got), want)
        print(f"  {what}: max abs err {err:.3e} (limit {lim:.2e})", flush=True)
        assert err <= lim, f"{what}: max abs err {err:.3e} > {lim:.2e}"
    if tau:
        err = max_abs(f64(tau_h), rtau)
        lim = 1e-5 if dt == torch.float32 else 4e-3
        print(f"  tau: max abs err {err:.3e}", flush=True)
        assert err <= lim, f"tau: max abs err {err:.3e} > {lim:.1e}"


def _draw_mixed(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B = int(rng.choice([1, 2, 3]))
        H = int(rng.choice([1, 2, 3]))
        T = int(rng.choice([1, 17, 64, 65, 129, 200, 256, 320]))
        W = int(rng.choice([1, 16, 33, 63, 64, 65, 128, 200, 256, 300]))
        D = int(rng.choice([32, 64]))
        norm = [None, "mass", "count"][int(rng.integers(3))]
        bias = bool(rng.integers(2))
        tau = bool(rng.integers(2))
        cases.append((i, B, H, T, W, D, norm, bias, tau))
    return cases


MIXED = _draw_mixed(16, 2027)


@pytest.mark.parametrize("case", MIXED, ids=[f"{c[0]}-B{c[1]}H{c[2]}T{c[3]}W{c[4]}D{c[5]}-{c[6]}"
                                             f"{'-bias' if c[7] else ''}{'-tau' if c[8] else ''}" for c in MIXED])
def test_window_sweep_mixed(dev, case):
    i, B, H, T, W, D, norm, bias, tau = case
    inp = mixed_inputs(B, T, H, seed=300 + i, W=W, dtau_std=0.1 if tau else None,
                       bias_std=0.5 if bias else None, D=D)
    scale = float(np.sqrt(D))
    print(f"[sweep mixed {case}]", flush=True)
    hip = hip_run(inp, W, scale, dev, normalize=norm, return_tau=tau, use_bias=bias, use_dtau=tau)
    ref = oracle_run(inp, W, scale, normalize=norm, use_bias=bias, use_dtau=tau)
    check_mixed(hip, ref, tau)


F16 = _draw_mixed(12, 2028)


@pytest.mark.parametrize("case", F16, ids=[f"{c[0]}-B{c[1]}H{c[2]}T{c[3]}W{c[4]}D{c[5]}-{c[6]}"
                                           f"{'-bias' if c[7] else ''}{'-tau' if c[8] else ''}" for c in F16])
def test_window_sweep_f16(dev, case):
    i, B, H, T, W, D, norm, bias, tau = case
    inp = make_inputs(B, T, H, D, seed=400 + i, std=0.5, dtype=torch.float16, W=W,
                      dtau_std=0.1 if tau else None, bias_std=0.5 if bias else None,
                      bias_shape=(B, T, W) if bias else None)
    scale = float(np.sqrt(D))
    print(f"[sweep f16 {case}]", flush=True)
    hip = hip_run(inp, W, scale, dev, normalize=norm, return_tau=tau, use_bias=bias, use_dtau=tau)
    ref = oracle_run(inp, W, scale, normalize=norm, use_bias=bias, use_dtau=tau)
    check_f16(hip, ref, tau)
