"""Regenerate the golden fixtures in this directory from the float64 oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors (all its kernel tests draw CUDA
``torch.randn`` at run time), so these fixtures are produced by the oracle
(``oracle/tension_oracle.py``), whose own pins live in ``tests/test_oracle.py``.
They freeze small, device-independent input/output pairs: the CPU suite checks
the oracle still reproduces them, the GPU suite checks the HIP kernels
against them.  Inputs are float32 (or bf16-rounded float32) arrays drawn from
numpy's PCG64 with fixed seeds.
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import tension_oracle as O  # noqa: E402


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round to nearest even), kept as float32."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def f32(**arrs):
    """Expected outputs are stored as float32: their rounding (<= 6e-8
    relative) is far below every tolerance that reads them."""
    return {k: (np.asarray(v, np.float32) if np.asarray(v).dtype == np.float64 and np.asarray(v).ndim
                else v) for k, v in arrs.items()}


def draw(seed, *shape, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def window_case(name, B, T, H, D, W, seed, std=1.0, bf16=False):
    r = lambda k, *s, sd=std: draw(seed * 10 + k, *s, std=sd)  # noqa: E731
    Q, K, V = r(1, B, T, H, D), r(2, B, T, H, D), r(3, B, T, H, D)
    if bf16:
        Q, K, V = bf16_round(Q), bf16_round(K), bf16_round(V)
    dO = r(4, B, T, H, D, sd=1.0)
    dTau = r(5, B, T, H, W, sd=0.1)
    bias = r(6, B, T, W, sd=0.5)
    scale = math.sqrt(D)
    msg, tau = O.window_forward(Q, K, V, W, scale, bias)
    out, mass = O.normalize_mass(msg, tau)
    g_raw = O.window_backward(Q, K, V, W, scale, dO, dTau, bias)
    g_mass = O.window_backward_normalized(Q, K, V, W, scale, dO, dTau, bias)
    np.savez_compressed(
        os.path.join(HERE, name), **f32(Q=Q, K=K, V=V, dO=dO, dTau=dTau, bias=bias,
        W=np.int64(W), scale=np.float64(scale), msg=msg, tau=tau, out_mass=out, mass=mass,
        dQ_raw=g_raw[0], dK_raw=g_raw[1], dV_raw=g_raw[2],
        dQ_mass=g_mass[0], dK_mass=g_mass[1], dV_mass=g_mass[2]))


def global_case(name, B, T, H, D, Wl, seed, bf16=False):
    r = lambda k, *s, sd=0.5: draw(seed * 10 + k, *s, std=sd)  # noqa: E731
    Q, K, V = r(1, B, T, H, D), r(2, B, T, H, D), r(3, B, T, H, D)
    if bf16:
        Q, K, V = bf16_round(Q), bf16_round(K), bf16_round(V)
    dO = r(4, B, T, H, D, sd=1.0)
    dTl = r(5, B, T, H, Wl, sd=0.1)
    bias = r(6, B, T, T, sd=0.5)
    scale = math.sqrt(D)
    out, mass, tl = O.global_forward(Q, K, V, scale, bias, Wl)
    g = O.global_backward(Q, K, V, scale, dO, bias, dTl)
    np.savez_compressed(
        os.path.join(HERE, name), **f32(Q=Q, K=K, V=V, dO=dO, dTl=dTl, bias=bias, Wl=np.int64(Wl),
        scale=np.float64(scale), out=out, mass=mass, tau_local=tl, dQ=g[0], dK=g[1], dV=g[2]))


def decode_case(name, N, H, D, W, prefill, steps, seed, bf16=False):
    L = prefill + steps
    r = lambda k, *s: draw(seed * 10 + k, *s, std=0.5)  # noqa: E731
    q, k, v = r(1, N, L, H, D), r(2, N, L, H, D), r(3, N, L, H, D)
    if bf16:
        q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
    kc, vc = np.zeros((N, H, W, D)), np.zeros((N, H, W, D))
    pos = np.zeros(N, np.int64)
    outs, taus = [], []
    for t in range(L):
        o, tt = O.decode_step(q[:, t], kc, vc, pos, W, math.sqrt(D))
        if t >= prefill:
            outs.append(o)
            taus.append(tt)
        kc, vc, pos = O.decode_append(kc, vc, pos, k[:, t], v[:, t], W)
    np.savez_compressed(os.path.join(HERE, name), **f32(q=q, k=k, v=v, W=np.int64(W),
                        prefill=np.int64(prefill), out=np.stack(outs, 1), tau=np.stack(taus, 1)))


def rope_case(name, B, T, H, D, off, seed):
    x = draw(seed, B, T, H, D)
    dy = draw(seed + 1, B, T, H, D)
    cos, sin = O.rope_tables(T + off, D)
    np.savez_compressed(os.path.join(HERE, name), **f32(
        x=x, dy=dy, cos=cos, sin=sin, off=np.int64(off),
        y=O.rope_apply(x, cos, sin, off), dx=O.rope_apply_adjoint(dy, cos, sin, off)))


CASES = {
    "window_f32_small.npz": lambda: window_case("window_f32_small.npz", 2, 32, 4, 16, 8, seed=1),
    "window_bf16_d64.npz": lambda: window_case("window_bf16_d64.npz", 1, 130, 2, 64, 64, seed=2,
                                               std=0.5, bf16=True),
    "global_bf16_d64.npz": lambda: global_case("global_bf16_d64.npz", 1, 80, 2, 64, 16, seed=3,
                                               bf16=True),
    "global_f32_small.npz": lambda: global_case("global_f32_small.npz", 1, 40, 2, 16, 8, seed=4),
    "decode_bf16_d64.npz": lambda: decode_case("decode_bf16_d64.npz", 2, 2, 64, 32, 40, 4, seed=5,
                                               bf16=True),
    "rope_small.npz": lambda: rope_case("rope_small.npz", 1, 20, 2, 16, 5, seed=6),
}


if __name__ == "__main__":
    for name, fn in CASES.items():
        fn()
        print("wrote", name, os.path.getsize(os.path.join(HERE, name)), "bytes")
