"""Golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle still reproduces every fixture (guards against oracle drift).
GPU: the HIP kernels reproduce the fixtures' expected outputs.
"""
import math
import os

import numpy as np
import pytest

from oracle import tension_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


def near(a, b, tol):
    """Absolute max-abs bound (raw sums included)."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    err = float(np.max(np.abs(a - b))) if a.size else 0.0
    assert err <= tol, f"max abs err {err:.3e} > {tol:.1e} (|ref| max {float(np.max(np.abs(b))):.3g})"


# ------------------------------------------------------------------ CPU

@pytest.mark.parametrize("name", ["window_f32_small.npz", "window_bf16_d64.npz"])
def test_oracle_reproduces_window_fixture(name):
    g = load(name)
    W, sc = int(g["W"]), float(g["scale"])
    msg, tau = O.window_forward(g["Q"], g["K"], g["V"], W, sc, g["bias"])
    near(msg, g["msg"], 1e-6)
    near(tau, g["tau"], 1e-6)
    out, mass = O.normalize_mass(msg, tau)
    near(out, g["out_mass"], 1e-6)
    gr = O.window_backward_normalized(g["Q"], g["K"], g["V"], W, sc, g["dO"], g["dTau"], g["bias"])
    for got, key in zip(gr, ("dQ_mass", "dK_mass", "dV_mass")):
        near(got, g[key], 1e-6)


@pytest.mark.parametrize("name", ["global_f32_small.npz", "global_bf16_d64.npz"])
def test_oracle_reproduces_global_fixture(name):
    g = load(name)
    out, mass, tl = O.global_forward(g["Q"], g["K"], g["V"], float(g["scale"]), g["bias"], int(g["Wl"]))
    near(out, g["out"], 1e-6)
    near(tl, g["tau_local"], 1e-6)
    gr = O.global_backward(g["Q"], g["K"], g["V"], float(g["scale"]), g["dO"], g["bias"], g["dTl"])
    for got, key in zip(gr, ("dQ", "dK", "dV")):
        near(got, g[key], 1e-6)


def test_oracle_reproduces_rope_fixture():
    g = load("rope_small.npz")
    near(O.rope_apply(g["x"], g["cos"], g["sin"], int(g["off"])), g["y"], 1e-6)
    near(O.rope_apply_adjoint(g["dy"], g["cos"], g["sin"], int(g["off"])), g["dx"], 1e-6)


# ------------------------------------------------------------------ GPU

def _t(x, dev, dtype):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=dev, dtype=dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("name,dtype_name,tol", [("window_f32_small.npz", "float32", 1e-5),
                                                 ("window_bf16_d64.npz", "bfloat16", 2e-2)])
@pytest.mark.parametrize("normalize", [None, "mass"])
def test_hip_matches_window_fixture(dev, name, dtype_name, tol, normalize):
    import torch

    from bozo_amd import causal_tension
    dtype = getattr(torch, dtype_name)
    g = load(name)
    W, sc = int(g["W"]), float(g["scale"])
    Q, K, V = (_t(g[n], dev, dtype).requires_grad_(True) for n in "QKV")
    out, tau = causal_tension(Q, K, V, W, sc, return_tau=True, bias=_t(g["bias"], dev, torch.float32),
                              normalize=normalize)
    ((out.float() * _t(g["dO"], dev, torch.float32)).sum()
     + (tau.float() * _t(g["dTau"], dev, torch.float32)).sum()).backward()
    suffix = "mass" if normalize else "raw"
    want_out = g["out_mass"] if normalize else g["msg"]
    pairs = [(out, want_out), (Q.grad, g["dQ_" + suffix]), (K.grad, g["dK_" + suffix]),
             (V.grad, g["dV_" + suffix])]
    for got, want in pairs:
        got = got.detach().double().cpu().numpy()
        if dtype == torch.float32:
            near(got, want, tol)
        else:
            assert np.linalg.norm(got - want) <= tol * np.linalg.norm(want)
    near(tau.detach().double().cpu().numpy(), g["tau"], 1e-5 if dtype == torch.float32 else 4e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("name,dtype_name,tol", [("global_f32_small.npz", "float32", 1e-5),
                                                 ("global_bf16_d64.npz", "bfloat16", 2e-2)])
def test_hip_matches_global_fixture(dev, name, dtype_name, tol):
    import torch

    from bozo_amd import global_tension
    dtype = getattr(torch, dtype_name)
    g = load(name)
    Q, K, V = (_t(g[n], dev, dtype).requires_grad_(True) for n in "QKV")
    out, tl = global_tension(Q, K, V, float(g["scale"]), bias=_t(g["bias"], dev, torch.float32),
                             W_local=int(g["Wl"]))
    ((out.float() * _t(g["dO"], dev, torch.float32)).sum()
     + (tl.float() * _t(g["dTl"], dev, torch.float32)).sum()).backward()
    for got, key in ((out, "out"), (Q.grad, "dQ"), (K.grad, "dK"), (V.grad, "dV")):
        got = got.detach().double().cpu().numpy()
        if dtype == torch.float32:
            near(got, g[key], tol)
        else:
            assert np.linalg.norm(got - g[key]) <= tol * np.linalg.norm(g[key])


@pytest.mark.gpu
def test_hip_matches_decode_fixture(dev):
    import torch

    from bozo_amd import TensionDecodeCache
    g = load("decode_bf16_d64.npz")
    q, k, v = g["q"], g["k"], g["v"]
    N, L, H, D = q.shape
    W, pre = int(g["W"]), int(g["prefill"])
    cache = TensionDecodeCache(N, H, D, W, dtype=torch.bfloat16, device=dev)
    bf = lambda x: _t(x, dev, torch.bfloat16)  # noqa: E731
    for t in range(L):
        out, tau = cache.step(bf(q[:, t]), bf(k[:, t]), bf(v[:, t]), return_tau=True)
        if t >= pre:
            want = g["out"][:, t - pre]
            got = out.double().cpu().numpy()
            assert np.linalg.norm(got - want) <= 2e-2 * np.linalg.norm(want)
            near(tau.double().cpu().numpy(), g["tau"][:, t - pre], 4e-3)


@pytest.mark.gpu
def test_hip_matches_rope_fixture(dev):
    import torch

    from bozo_amd import rope
    g = load("rope_small.npz")
    x = _t(g["x"], dev, torch.float32).requires_grad_(True)
    y = rope(x, _t(g["cos"], dev, torch.float32), _t(g["sin"], dev, torch.float32), int(g["off"]))
    (y * _t(g["dy"], dev, torch.float32)).sum().backward()
    near(y.detach().double().cpu().numpy(), g["y"], 1e-6)
    near(x.grad.double().cpu().numpy(), g["dx"], 1e-6)
