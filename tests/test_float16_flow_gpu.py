"""float16 Q / K / V on the split-operand MFMA kernels.

The reference's Triton kernel loads any dtype and computes in float32
(kernel.py:71-98).  Here a float16 value enters the bf16 MFMAs as two bf16
terms, which hold it exactly (11 significant bits, and bf16 spans
float16's exponent range), so every product of two float16 operands is
exact; the float32 P, P' and G go in as two terms as well.  Outputs are
float16, so the bound is float16's own rounding: relative L2 1e-3 on out,
dQ, dK, dV (float16 rounds at 2^-11 = 4.9e-4 relative) and an elementwise
absolute 4.9e-4 on tau (values <= 1), against the float64 oracle.
"""
import math

import pytest
import torch

from tests._util import f64, make_inputs, max_abs, rel_l2
from tests.test_window_gpu import hip_run, last_kernel, oracle_run
from tests.test_global_gpu import hip_run as global_hip_run, oracle_run as global_oracle_run

pytestmark = pytest.mark.gpu

REL = 1e-3
TAU_ABS = 2.0 ** -11


def check(hip, ref, tau_checked):
    out, tau, grads = hip
    for name, g, r in zip(("out", "dQ", "dK", "dV"), (out,) + tuple(grads), (ref[0],) + tuple(ref[2])):
        assert g.dtype == torch.float16, name
        err = rel_l2(f64(g), r)
        print(f"  {name}: rel L2 err {err:.3e}", flush=True)
        assert err <= REL, f"{name}: rel L2 err {err:.3e} > {REL:.0e}"
    if tau_checked:
        err = max_abs(f64(tau), ref[1])
        print(f"  tau: max abs err {err:.3e}", flush=True)
        assert tau.dtype == torch.float16 and err <= TAU_ABS, f"tau: {err:.3e}"


SHAPES = {"117m": (8, 1024, 12, 64, 64), "350m": (2, 1024, 16, 64, 256), "d32": (4, 256, 4, 32, 32),
          "ragged": (2, 300, 3, 64, 100)}


@pytest.mark.parametrize("normalize", [None, "mass", "count"])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_float16_flow_window(dev, shape, normalize):
    """out, tau and the three gradients (tau's gradient included)."""
    from bozo_amd import _lib as L
    B, T, H, D, W = SHAPES[shape]
    inp = make_inputs(B, T, H, D, seed=120 + W + D + T, std=0.5, dtype=torch.float16, W=W, dtau_std=0.1)
    print(f"[f16 flow] {shape} B{B} T{T} H{H} D{D} W{W} normalize={normalize}", flush=True)
    hip = hip_run(inp, W, math.sqrt(D), dev, normalize=normalize, return_tau=True, use_dtau=True)
    assert last_kernel() == L.KERNEL_SPLIT_F16
    check(hip, oracle_run(inp, W, math.sqrt(D), normalize=normalize, use_dtau=True), True)


@pytest.mark.parametrize("W,T", [(64, 1024), (7, 130)])
def test_float16_flow_bias(dev, W, T):
    """With the pre-sigmoid bias [B, T, W] (float32, broadcast over heads)."""
    from bozo_amd import _lib as L
    B, H, D = 2, 3, 64
    inp = make_inputs(B, T, H, D, seed=125 + W, std=0.5, dtype=torch.float16, W=W, dtau_std=0.1,
                      bias_std=0.5, bias_shape=(B, T, W))
    hip = hip_run(inp, W, 8.0, dev, normalize="mass", return_tau=True, use_bias=True, use_dtau=True)
    assert last_kernel() == L.KERNEL_SPLIT_F16
    check(hip, oracle_run(inp, W, 8.0, normalize="mass", use_bias=True, use_dtau=True), True)


@pytest.mark.parametrize("D,T,Wl", [(64, 130, 16), (32, 97, 16), (64, 200, 130)])
def test_float16_flow_global(dev, D, T, Wl):
    """The global block with a bias [B, T, T], tau_local (over one key
    block, or three) and its gradient."""
    from bozo_amd import _lib as L
    B, H = 2, 3
    inp = make_inputs(B, T, H, D, seed=127 + D + T, std=0.5, dtype=torch.float16, W=Wl, dtau_std=0.1,
                      bias_std=0.5, bias_shape=(B, T, T))
    scale = math.sqrt(D)
    hip = global_hip_run(inp, scale, dev, W_local=Wl, use_bias=True, use_dtl=True)
    assert int(L.lib().tension_last_kernel()) == L.KERNEL_SPLIT_F16
    check(hip, global_oracle_run(inp, scale, W_local=Wl, use_bias=True, use_dtl=True), True)
