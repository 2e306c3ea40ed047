"""Parity of the global (full causal, diagonal included) block kernels
against the float64 oracle (restating model.py:217-238)."""
import math

import numpy as np
import pytest
import torch

from oracle import tension_oracle as O
from tests._util import f64, make_inputs, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def hip_run(inp, scale, dev, *, W_local=None, use_bias=False, use_dtl=False):
    from bozo_amd import global_tension
    Q, K, V = (inp[n].to(dev).requires_grad_(True) for n in "QKV")
    bias = inp["bias"].to(dev) if use_bias else None
    res = global_tension(Q, K, V, scale, bias=bias, W_local=W_local)
    out, tl = res if W_local else (res, None)
    loss = (out.float() * inp["dO"].to(dev).float()).sum()
    if use_dtl:
        loss = loss + (tl.float() * inp["dTau"].to(dev).float()).sum()
    loss.backward()
    torch.cuda.synchronize()
    return out, tl, (Q.grad, K.grad, V.grad)


def oracle_run(inp, scale, *, W_local=None, use_bias=False, use_dtl=False):
    Q, K, V, dO = f64(inp["Q"]), f64(inp["K"]), f64(inp["V"]), f64(inp["dO"])
    bias = f64(inp["bias"]) if use_bias else None
    dtl = f64(inp["dTau"]) if use_dtl else None
    out, mass, tl = O.global_forward(Q, K, V, scale, bias, W_local)
    grads = O.global_backward(Q, K, V, scale, dO, bias, dtl)
    return out, tl, grads


def check(hip, ref, dtype, tl_checked=False):
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    metric = max_abs if dtype == torch.float32 else rel_l2
    for name, g, r in zip(("out", "dQ", "dK", "dV"), (hip[0],) + tuple(hip[2]), (ref[0],) + tuple(ref[2])):
        err = metric(f64(g), r)
        assert err <= tol, f"{name}: err {err:.3e} > {tol:.1e}"
    if tl_checked:
        lim = 1e-5 if dtype == torch.float32 else 4e-3
        assert max_abs(f64(hip[1]), ref[1]) <= lim


@pytest.mark.parametrize("use_bias,use_tl", [(True, False), (False, True), (True, True)])
def test_global_bf16_bias_tau_local(dev, use_bias, use_tl):
    """The dedicated global kernels with each optional operand: bias [B,T,T]
    and the tau_local output / dtau_local input (W_local = 64)."""
    B, H, T, D = 2, 2, 200, 64
    inp = make_inputs(B, T, H, D, seed=7, std=0.5, dtype=torch.bfloat16, W=64, dtau_std=0.1,
                      bias_std=0.5, bias_shape=(B, T, T))
    wl = 64 if use_tl else None
    hip = hip_run(inp, 8.0, dev, W_local=wl, use_bias=use_bias, use_dtl=use_tl)
    ref = oracle_run(inp, 8.0, W_local=wl, use_bias=use_bias, use_dtl=use_tl)
    check(hip, ref, torch.bfloat16, use_tl)


@pytest.mark.parametrize("B,H,T,wl", [(2, 4, 200, None), (2, 4, 200, 16), (1, 8, 130, 64), (2, 4, 64, None),
                                      (1, 8, 64, 16), (3, 1, 129, None)])
def test_global_bf16_bias_xcd_groups(dev, B, H, T, wl):
    """A bias with B * H a multiple of 8 (the heads of a sequence grouped on
    XCDs, gl_slot) and not (3 x 1), ragged and whole tiles, one query tile
    (T = 64: the dQ kernel's single block), and with tau_local (the forward
    loading the next block's bias behind its score products)."""
    D = 64
    inp = make_inputs(B, T, H, D, seed=B * 1000 + T, std=0.5, dtype=torch.bfloat16, W=wl or 1,
                      dtau_std=0.1 if wl else None, bias_std=0.5, bias_shape=(B, T, T))
    print(f"[global bias] B{B} H{H} T{T} W_local={wl}", flush=True)
    hip = hip_run(inp, 8.0, dev, W_local=wl, use_bias=True, use_dtl=wl is not None)
    ref = oracle_run(inp, 8.0, W_local=wl, use_bias=True, use_dtl=wl is not None)
    check(hip, ref, torch.bfloat16, wl is not None)


@pytest.mark.parametrize("pad", [1, 4])
def test_global_bf16_bias_row_views(dev, pad):
    """The bias as a view into wider rows (row stride T + pad): with pad 4
    the rows stay 16-byte aligned and the kernels read a block's bias in
    16-byte pieces (the last, ragged block element by element); with pad 1
    every load is an element load."""
    B, H, T, D = 2, 3, 200, 64
    inp = make_inputs(B, T, H, D, seed=11 + pad, std=0.5, dtype=torch.bfloat16, W=64)
    wide = torch.randn(B, T, T + pad, generator=torch.Generator().manual_seed(pad)) * 0.5
    inp["bias"] = wide[:, :, :T]
    from bozo_amd import global_tension
    Q, K, V = (inp[n].to(dev).requires_grad_(True) for n in "QKV")
    bias = wide.to(dev)[:, :, :T]
    assert bias.stride(1) == T + pad
    out = global_tension(Q, K, V, 8.0, bias=bias)
    (out.float() * inp["dO"].to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    ref = oracle_run(inp, 8.0, use_bias=True)
    check((out, None, (Q.grad, K.grad, V.grad)), ref, torch.bfloat16)


def test_config3_bf16_full_size(dev):
    """B4 H12 T2048 d64 bf16, full causal, tau-mass."""
    B, H, T, D = 4, 12, 2048, 64
    inp = make_inputs(B, T, H, D, seed=2, std=0.5, dtype=torch.bfloat16, rope=False)
    check(hip_run(inp, 8.0, dev), oracle_run(inp, 8.0), torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [1, 33, 64, 130])
def test_global_small(dev, dtype, T):
    D = 64
    inp = make_inputs(2, T, 3, D, seed=T, std=0.5, dtype=dtype, W=min(16, T), dtau_std=0.1,
                      bias_std=0.5, bias_shape=(2, T, T))
    hip = hip_run(inp, 8.0, dev, W_local=16, use_bias=True, use_dtl=True)
    ref = oracle_run(inp, 8.0, W_local=16, use_bias=True, use_dtl=True)
    check(hip, ref, dtype, True)


def test_global_without_diagonal_equals_window(dev):
    """Global with the diagonal biased to -inf equals the local window of W=T
    (tau-mass normalised): the two kernels agree through the public ops."""
    from bozo_amd import causal_tension, global_tension
    B, T, H, D = 2, 96, 2, 32
    inp = make_inputs(B, T, H, D, seed=21, dtype=torch.float32)
    Q, K, V = (inp[n].to(dev) for n in "QKV")
    nodiag = torch.zeros(B, T, T, device=dev)
    nodiag[:, torch.arange(T), torch.arange(T)] = -1e30
    a = global_tension(Q, K, V, math.sqrt(D), bias=nodiag)
    b = causal_tension(Q, K, V, T, math.sqrt(D), normalize="mass")
    assert max_abs(f64(a), f64(b)) <= 1e-5


def test_gradcheck_float64(dev):
    from bozo_amd import global_tension
    torch.manual_seed(3)
    B, T, H, D = 1, 12, 2, 8
    Q, K, V = (torch.randn(B, T, H, D, device=dev, dtype=torch.float64, requires_grad=True)
               for _ in range(3))
    bias = torch.randn(B, T, T, device=dev, dtype=torch.float64) * 0.3

    def fn(q, k, v):
        return global_tension(q, k, v, math.sqrt(D), bias=bias, W_local=5)

    assert torch.autograd.gradcheck(fn, (Q, K, V), eps=1e-6, atol=1e-6, rtol=1e-5)


def test_backward_saved_rows_match_band_recompute(dev):
    """tension_global_bwd given the forward's out and mass rows (tau-mass
    coefficients from one pass over those rows) and without them (band
    recompute): both against the oracle and against each other (bf16, d64)."""
    from bozo_amd import _lib as L
    B, H, T, D = 2, 3, 200, 64
    inp = make_inputs(B, T, H, D, seed=5, std=0.5, dtype=torch.bfloat16, rope=False)
    Q, K, V, dO = (inp[n].to(dev).contiguous() for n in ("Q", "K", "V", "dO"))
    dO = dO.to(torch.bfloat16)
    out = torch.empty_like(Q)
    mass = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    lib = L.lib()
    L.check(lib.tension_global_fwd(L.buf(Q), L.buf(K), L.buf(V), L.buf(out), None, None, L.buf(mass),
                                   B, T, H, D, 0, 8.0, 0, L.stream_handle()), "fwd")
    ws = torch.empty(lib.tension_global_bwd_workspace(B, T, H, L.F32, 0), dtype=torch.uint8, device=dev)
    grads = {}
    for name, o, m in (("saved", out, mass), ("band", None, None)):
        g = [torch.empty_like(Q) for _ in range(3)]
        L.check(lib.tension_global_bwd(L.buf(Q), L.buf(K), L.buf(V), L.buf(dO), None, None, L.buf(o), L.buf(m),
                                       L.buf(g[0]), L.buf(g[1]), L.buf(g[2]), ws.data_ptr(), B, T, H, D, 0,
                                       8.0, 0, L.stream_handle()), name)
        torch.cuda.synchronize()
        grads[name] = g
    ref = O.global_backward(f64(inp["Q"]), f64(inp["K"]), f64(inp["V"]), 8.0, f64(dO.cpu()), None, None)
    for i, n in enumerate(("dQ", "dK", "dV")):
        for route in ("saved", "band"):
            err = rel_l2(f64(grads[route][i]), ref[i])
            assert err <= 2e-2, f"{route} {n}: {err:.3e}"
        assert rel_l2(f64(grads["saved"][i]), f64(grads["band"][i])) <= 1e-2, n
    mo, _, _ = O.global_forward(f64(inp["Q"]), f64(inp["K"]), f64(inp["V"]), 8.0, None, None)
    assert rel_l2(f64(out), mo) <= 2e-2


def test_global_row_stride_beyond_32bit_offsets(dev):
    """K / V rows 33,554,496 elements apart (64 rows span more than 2^32
    bytes): the dedicated forward keeps per-lane tile offsets in 32 bits, so
    the host sends such calls to the band kernel's 64-bit sources.  The views
    sit in 6.6 GB allocations of which only the rows are written."""
    B, H, T, D = 1, 1, 100, 64
    s1 = (1 << 25) + 64
    inp = make_inputs(B, T, H, D, seed=31, std=0.5, dtype=torch.bfloat16, rope=False)

    def spread(x):
        base = torch.empty((T - 1) * s1 + D, dtype=x.dtype, device=dev)
        view = base.as_strided((B, T, H, D), (T * s1, s1, D, 1))
        view.copy_(x.to(dev))
        return view

    from bozo_amd import global_tension
    Q = inp["Q"].to(dev).requires_grad_(True)
    K = spread(inp["K"]).requires_grad_(True)
    V = spread(inp["V"]).requires_grad_(True)
    print(f"[global stride] s1={s1} K stride {K.stride()}", flush=True)
    out = global_tension(Q, K, V, 8.0)
    (out.float() * inp["dO"].to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    ref = oracle_run(inp, 8.0)
    check((out, None, (Q.grad, K.grad, V.grad)), ref, torch.bfloat16)


@pytest.mark.parametrize("flow,D,T", [("bf16", 32, 200), ("bf16", 32, 64), ("f32qk", 64, 130), ("f32qk", 32, 97)])
def test_global_split_kernels(dev, flow, D, T):
    """The global block on the split-operand kernels: bf16 at head dim 32
    (the reference's default model under autocast, model.py:33-36,219) and
    float32 Q / K with a bf16 V (three bf16 terms per float32 value: the
    fp32 bound, max-abs 1e-5, on out, dQ, dK and tau_local), with bias,
    tau_local and its gradient."""
    from bozo_amd import _lib as L
    B, H, Wl = 2, 3, 16
    dt = torch.bfloat16 if flow == "bf16" else torch.float32
    inp = make_inputs(B, T, H, D, seed=40 + D + T, std=0.5, dtype=dt, W=Wl, dtau_std=0.1,
                      bias_std=0.5, bias_shape=(B, T, T))
    inp["V"] = inp["V"].to(torch.bfloat16)
    scale = math.sqrt(D)
    hip = hip_run(inp, scale, dev, W_local=Wl, use_bias=True, use_dtl=True)
    assert int(L.lib().tension_last_kernel()) == (L.KERNEL_SPLIT_BF16 if flow == "bf16" else L.KERNEL_SPLIT_F32)
    ref = oracle_run(inp, scale, W_local=Wl, use_bias=True, use_dtl=True)
    if flow == "bf16":
        check(hip, ref, torch.bfloat16, True)
        return
    for name, g, r in zip(("out", "dQ", "dK"), (hip[0], hip[2][0], hip[2][1]), (ref[0], ref[2][0], ref[2][1])):
        err = max_abs(f64(g), r)
        print(f"  {name}: max abs err {err:.3e}", flush=True)
        assert err <= 1e-5, f"{name}: {err:.3e}"
    assert rel_l2(f64(hip[2][2]), ref[2][2]) <= 2e-2
    assert max_abs(f64(hip[1]), ref[1]) <= 1e-5
