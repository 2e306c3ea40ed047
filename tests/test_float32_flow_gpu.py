"""The reference's float32 flow on the split-operand MFMA kernels.

Without autocast the reference calls the op with float32 Q, K and V
(its Triton path takes "CUDA float32/bfloat16", triton_tension/ops.py:202,
and computes in float32, kernel.py:71-98).  Here every float32 operand --
V included -- enters the bf16 MFMAs as three bf16 terms, and every output
(out, tau, dQ, dK, dV) is float32: all of them are held to the fp32 bound,
max-abs 1e-5 absolute, against the float64 oracle.  Shapes: the reference's
117M layer (B8 H12 T1024 W64), its 350M preset's local layer (W256, 16
heads), its default model (head dim 32, W32), and the
global block; and the float32 calls that stay on the exact kernels (other
head dims, unaligned rows), at the same bound.
"""
import ctypes
import math

import pytest
import torch

from tests._util import f64, make_inputs, max_abs
from tests.test_window_gpu import check_fp32, compare, hip_run, last_kernel, oracle_run
from tests.test_global_gpu import hip_run as global_hip_run, oracle_run as global_oracle_run

pytestmark = pytest.mark.gpu

SHAPES = {"117m": (8, 1024, 12, 64, 64), "350m": (2, 1024, 16, 64, 256), "d32": (4, 256, 4, 32, 32)}


@pytest.mark.parametrize("normalize", [None, "mass", "count"])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_float32_flow_window(dev, shape, normalize):
    """out, tau and the three gradients (tau's gradient included) at the fp32
    bound, on the split kernels with V as three terms."""
    from bozo_amd import _lib as L
    B, T, H, D, W = SHAPES[shape]
    inp = make_inputs(B, T, H, D, seed=90 + W + D, std=0.5, W=W, dtau_std=0.1)
    print(f"[f32 flow] {shape} B{B} T{T} H{H} D{D} W{W} normalize={normalize}", flush=True)
    hip = hip_run(inp, W, math.sqrt(D), dev, normalize=normalize, return_tau=True, use_dtau=True)
    assert last_kernel() == L.KERNEL_SPLIT_F32V
    assert all(g.dtype == torch.float32 for g in hip[2])
    compare(hip, oracle_run(inp, W, math.sqrt(D), normalize=normalize, use_dtau=True), torch.float32, True)


@pytest.mark.parametrize("W,T", [(64, 1024), (100, 300), (7, 130)])
def test_float32_flow_bias(dev, W, T):
    """With the pre-sigmoid bias [B, T, W] (float32, broadcast over heads),
    tau-mass, tau and its gradient; ragged T and a window that is not a
    multiple of the tile."""
    from bozo_amd import _lib as L
    B, H, D = 2, 3, 64
    inp = make_inputs(B, T, H, D, seed=95 + W, std=0.5, W=W, dtau_std=0.1, bias_std=0.5, bias_shape=(B, T, W))
    hip = hip_run(inp, W, 8.0, dev, normalize="mass", return_tau=True, use_bias=True, use_dtau=True)
    assert last_kernel() == L.KERNEL_SPLIT_F32V
    compare(hip, oracle_run(inp, W, 8.0, normalize="mass", use_bias=True, use_dtau=True), torch.float32, True)


@pytest.mark.parametrize("W,D,tau", [(64, 64, True), (256, 64, False), (65, 32, True)])
def test_float32_flow_saved_rows_match_recompute(dev, W, D, tau):
    """tension_window_bwd_saved (coefficients from the forward's rows and tau
    mass, one pass) against tension_window_bwd (a first pass over the band
    forms them) through the C ABI, float32 V: equal to float32 rounding, and
    both at the fp32 bound against the float64 oracle."""
    from bozo_amd import _lib as L
    B, T, H = 2, 300, 3
    inp = make_inputs(B, T, H, D, seed=97 + W + D, std=0.5, W=W, dtau_std=0.1 if tau else None)
    q, k, v, dO = (inp[n].to(dev) for n in ("Q", "K", "V", "dO"))
    dtau = inp["dTau"].to(dev) if tau else None
    scale = math.sqrt(D)
    lib, st = L.lib(), L.stream_handle(dev)
    out = torch.empty_like(q)
    mass = torch.empty(B, T, H, device=dev)
    L.check(lib.tension_window_fwd(L.buf(q), L.buf(k), L.buf(v), L.buf(out), None, None, L.buf(mass),
                                   B, T, H, D, W, ctypes.c_double(scale), L.NORM_MASS, st), "fwd")
    assert int(lib.tension_last_kernel()) == L.KERNEL_SPLIT_F32V
    res = []
    for saved in (False, True):
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ws = torch.empty(lib.tension_window_bwd_workspace(B, T, H, L.F32, L.NORM_MASS), dtype=torch.uint8,
                         device=dev)
        common = (L.buf(q), L.buf(k), L.buf(v), L.buf(dO), L.buf(dtau), None)
        tail = (L.buf(dq), L.buf(dk), L.buf(dv), ctypes.c_void_p(ws.data_ptr()), B, T, H, D, W,
                ctypes.c_double(scale), L.NORM_MASS, st)
        if saved:
            L.check(lib.tension_window_bwd_saved(*common, L.buf(out), L.buf(mass), *tail), "saved")
        else:
            L.check(lib.tension_window_bwd(*common, *tail), "recompute")
        assert int(lib.tension_last_kernel()) == L.KERNEL_SPLIT_F32V
        res.append((dq, dk, dv))
    torch.cuda.synchronize()
    for name, a, b_ in zip(("dQ", "dK", "dV"), res[0], res[1]):
        err = float((a - b_).abs().max())
        print(f"  {name}: saved vs recompute max abs {err:.2e}", flush=True)
        assert err <= 1e-6, (name, err)
    _, _, grads = oracle_run(inp, W, scale, normalize="mass", use_dtau=tau)
    for r in res:
        for got, want, name in zip(r, grads, ("dQ", "dK", "dV")):
            check_fp32(got, want, name)


@pytest.mark.parametrize("D,T,Wl", [(64, 130, 16), (32, 97, 16), (64, 256, 16), (64, 256, 100)])
def test_float32_flow_global(dev, D, T, Wl):
    """The global block (model.py:217-238) with float32 Q / K / V, a bias
    [B, T, T], tau_local (over one key block, or two) and its gradient: out,
    dQ, dK, dV and tau_local at the fp32 bound."""
    from bozo_amd import _lib as L
    B, H = 2, 3
    inp = make_inputs(B, T, H, D, seed=99 + D + T, std=0.5, W=Wl, dtau_std=0.1, bias_std=0.5, bias_shape=(B, T, T))
    scale = math.sqrt(D)
    hip = global_hip_run(inp, scale, dev, W_local=Wl, use_bias=True, use_dtl=True)
    assert int(L.lib().tension_last_kernel()) == L.KERNEL_SPLIT_F32V
    ref = global_oracle_run(inp, scale, W_local=Wl, use_bias=True, use_dtl=True)
    got = (hip[0], hip[1], *hip[2])
    want = (ref[0], ref[1], *ref[2])
    for name, g, r in zip(("out", "tau_local", "dQ", "dK", "dV"), got, want):
        err = max_abs(f64(g), r)
        print(f"  {name}: max abs err {err:.3e}", flush=True)
        assert g.dtype == torch.float32 and err <= 1e-5, f"{name}: {err:.3e}"


@pytest.mark.parametrize("D,aligned", [(16, True), (128, True), (64, False)])
def test_float32_exact_kernels(dev, D, aligned):
    """float32 calls the split kernels do not take -- head dims other than
    32 / 64, rows that are not 16-byte aligned (here Q, K, V are views one
    element into a wider buffer) -- run on the exact kernels, at the same
    fp32 bound."""
    from bozo_amd import causal_tension, _lib as L
    B, T, H, W = 2, 150, 3, 40
    inp = make_inputs(B, T, H, D, seed=130 + D, std=0.5, W=W, dtau_std=0.1)
    if aligned:
        Q, K, V = (inp[n].to(dev).requires_grad_(True) for n in "QKV")
        leaves = (Q, K, V)
    else:
        base = [torch.zeros(B, T, H, D + 1, device=dev) for _ in range(3)]
        for b_, n in zip(base, "QKV"):
            b_[..., 1:].copy_(inp[n].to(dev))
        leaves = tuple(b_.requires_grad_(True) for b_ in base)
        Q, K, V = (b_[..., 1:] for b_ in leaves)
        assert Q.data_ptr() % 16 != 0
    out, tau = causal_tension(Q, K, V, W, math.sqrt(D), return_tau=True, normalize="mass")
    assert last_kernel() == L.KERNEL_EXACT
    loss = (out * inp["dO"].to(dev)).sum() + (tau * inp["dTau"].to(dev)).sum()
    grads = torch.autograd.grad(loss, leaves)
    if not aligned:
        grads = tuple(g[..., 1:] for g in grads)
    torch.cuda.synchronize()
    assert last_kernel() == L.KERNEL_EXACT
    compare((out, tau, grads), oracle_run(inp, W, math.sqrt(D), normalize="mass", use_dtau=True), torch.float32,
            True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_strided_kv_views(dev, dtype):
    """model.py:206-207 splits one fused wkv projection: K and V are views of
    one [B, T, H, 2 D] tensor (row stride 2 D).  The split kernels read them
    in place in the float32 and float16 flows too; forward and backward
    against the float64 oracle (float32 at its 1e-5 bound, float16 at 1e-3
    relative L2)."""
    from bozo_amd import causal_tension, _lib as L
    from tests._util import rel_l2
    B, T, H, D, W = 2, 200, 3, 64, 64
    inp = make_inputs(B, T, H, D, seed=140, std=0.5, dtype=dtype, W=W)
    kv = torch.cat([inp["K"], inp["V"]], dim=-1).to(dev).requires_grad_(True)
    q = inp["Q"].to(dev).requires_grad_(True)
    k, v = kv[..., :D], kv[..., D:]
    assert k.stride(2) == 2 * D
    out = causal_tension(q, k, v, W, 8.0, normalize="mass")
    assert last_kernel() == (L.KERNEL_SPLIT_F32V if dtype == torch.float32 else L.KERNEL_SPLIT_F16)
    dq, dkv = torch.autograd.grad((out.float() * inp["dO"].to(dev).float()).sum(), (q, kv))
    ref = oracle_run(inp, W, 8.0, normalize="mass")
    got = (out, dq, dkv[..., :D], dkv[..., D:])
    want = (ref[0],) + tuple(ref[2])
    for name, g, r in zip(("out", "dQ", "dK", "dV"), got, want):
        if dtype == torch.float32:
            check_fp32(g, r, name)
        else:
            err = rel_l2(f64(g), r)
            print(f"  {name}: rel L2 err {err:.3e}", flush=True)
            assert err <= 1e-3, (name, err)
