"""Parity of the local-window HIP kernels against the float64 oracle.

Mirrors the reference's kernel tests (triton_tension/test.py,
triton_tension/test_tau.py) with the oracle in place of the unfold
reference, plus the benchmark configs and the edge cases of the band.
Tolerances: float32 absolute max-abs 1e-5 on out, dQ, dK, dV and tau
(raw sums included); bfloat16 relative L2 <= 2e-2 for out/dQ/dK/dV and an
elementwise absolute bound of 4e-3 on tau (tau in [0,1], bf16 ulp at 1 is
2^-8, rounding error <= 2^-9).  Every check prints the error it measured.

Launch geometry: the bf16 W <= 64 kernels split each (b, h) sequence by the
grid size, so the same inputs exercise different code at different B*H
(``fused_geometry``).  The tests at the 117M training geometry (B8 H12 T1024)
run exactly the kernel variants the model step and the tau benchmark run.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tension_oracle as O
from tests._util import f64, fused_geometry, make_inputs, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def hip_run(inp, W, scale, dev, *, normalize=None, return_tau=False, use_bias=False,
            use_dtau=False, backward=True):
    from bozo_amd import causal_tension
    Q, K, V = (inp[n].to(dev).requires_grad_(backward) for n in "QKV")
    bias = inp["bias"].to(dev) if use_bias else None
    res = causal_tension(Q, K, V, W, scale, return_tau=return_tau, bias=bias, normalize=normalize)
    out, tau = res if return_tau else (res, None)
    grads = (None, None, None)
    if backward:
        loss = (out.float() * inp["dO"].to(dev).float()).sum()
        if use_dtau:
            loss = loss + (tau.float() * inp["dTau"].to(dev).float()).sum()
        loss.backward()
        grads = (Q.grad, K.grad, V.grad)
    torch.cuda.synchronize()
    return out, tau, grads


def oracle_run(inp, W, scale, *, normalize=None, use_bias=False, use_dtau=False):
    Q, K, V, dO = f64(inp["Q"]), f64(inp["K"]), f64(inp["V"]), f64(inp["dO"])
    bias = f64(inp["bias"]) if use_bias else None
    dTau = f64(inp["dTau"]) if use_dtau else None
    msg, tau = O.window_forward(Q, K, V, W, scale, bias)
    if normalize == "mass":
        out, _ = O.normalize_mass(msg, tau)
        grads = O.window_backward_normalized(Q, K, V, W, scale, dO, dTau, bias)
    elif normalize == "count":
        out = O.normalize_count(msg, W)
        cnt = O.valid_count(Q.shape[1], W)[None, :, None, None]
        grads = O.window_backward(Q, K, V, W, scale, dO / cnt, dTau, bias)
    else:
        out = msg
        grads = O.window_backward(Q, K, V, W, scale, dO, dTau, bias)
    return out, tau, grads


def check_fp32(got, want, what, tol=1e-5):
    err = max_abs(f64(got), want)
    print(f"  {what}: max abs err {err:.3e} (|ref| max {float(np.max(np.abs(want))) if want.size else 0:.3g})",
          flush=True)
    assert err <= tol, f"{what}: max abs err {err:.3e} > {tol:.1e}"


def check_bf16(got, want, what, tol=2e-2):
    err = rel_l2(f64(got), want)
    print(f"  {what}: rel L2 err {err:.3e}", flush=True)
    assert err <= tol, f"{what}: rel L2 err {err:.3e} > {tol:.1e}"


def compare(hip, ref, dtype, tau_checked):
    out, tau, grads = hip
    rout, rtau, rgrads = ref
    chk = check_fp32 if dtype in (torch.float32, torch.float64) else check_bf16
    chk(out, rout, "out")
    for n, g, r in zip(("dQ", "dK", "dV"), grads, rgrads):
        if g is not None:
            chk(g, r, n)
    if tau_checked:
        err = max_abs(f64(tau), rtau)
        lim = 1e-5 if dtype in (torch.float32, torch.float64) else 4e-3
        print(f"  tau: max abs err {err:.3e}", flush=True)
        assert err <= lim, f"tau: max abs err {err:.3e} > {lim:.1e}"


# ------------------------------------------------------------ benchmark configs

@pytest.mark.parametrize("with_tau", [False, True])
def test_config1_fp32_normalised(dev, with_tau):
    """B4 H4 T256 d32 W32 fp32, RoPE, out = sum tau v / sum tau."""
    B, H, T, D, W = 4, 4, 256, 32, 32
    inp = make_inputs(B, T, H, D, seed=0, W=W, dtau_std=0.1 if with_tau else None)
    hip = hip_run(inp, W, math.sqrt(D), dev, normalize="mass", return_tau=with_tau, use_dtau=with_tau)
    ref = oracle_run(inp, W, math.sqrt(D), normalize="mass", use_dtau=with_tau)
    compare(hip, ref, torch.float32, with_tau)


@pytest.mark.parametrize("normalize", [None, "mass", "count"])
def test_config2_bf16_full_size(dev, normalize):
    """BASELINE config 2 at full size: B8 H12 T1024 d64 W64 bf16 (MFMA path).
    "count" without tau is the model's cross-entropy-only step."""
    B, H, T, D, W = 8, 12, 1024, 64, 64
    print(f"[c2] geometry (fwd tiles/wg, bwd runs, longest run) = {fused_geometry(B, H, T)}", flush=True)
    inp = make_inputs(B, T, H, D, seed=1, std=0.5, dtype=torch.bfloat16)
    hip = hip_run(inp, W, 8.0, dev, normalize=normalize)
    ref = oracle_run(inp, W, 8.0, normalize=normalize)
    compare(hip, ref, torch.bfloat16, False)


def test_config2_bf16_with_tau_and_dtau(dev):
    """Config 2 with tau materialised [B,T,H,W] and a gradient through it."""
    B, H, T, D, W = 2, 12, 1024, 64, 64
    inp = make_inputs(B, T, H, D, seed=1, std=0.5, dtype=torch.bfloat16, W=W, dtau_std=0.1)
    hip = hip_run(inp, W, 8.0, dev, normalize="mass", return_tau=True, use_dtau=True)
    ref = oracle_run(inp, W, 8.0, normalize="mass", use_dtau=True)
    compare(hip, ref, torch.bfloat16, True)


@pytest.mark.parametrize("B,H,T,normalize,tau", [(8, 12, 1024, None, False), (8, 12, 1024, "count", False),
                                                  (8, 12, 1024, "mass", False), (8, 12, 1024, "mass", True),
                                                  (1, 2, 192, "mass", False), (1, 2, 192, None, True)])
def test_config2_geometry_bias(dev, B, H, T, normalize, tau):
    """A [B,T,W] bias at the config-2 launch geometry (B8 H12 T1024 W64
    bf16): the fast forward (two tiles per workgroup, the second tile's bias
    loaded while the first computes) and the fast backward (runs of 3-4
    tiles and a halo step, each step's bias issued ahead of the next step's
    loads); with tau the backward takes the bias with dTau on the generic
    path.  The small shape has one-tile workgroups and runs."""
    D, W = 64, 64
    chunk, runs, longest = fused_geometry(B, H, T)
    print(f"[c2 bias] normalize={normalize} tau={tau} fwd tiles/wg={min(chunk, 2)} bwd runs={runs} "
          f"longest={longest}", flush=True)
    inp = make_inputs(B, T, H, D, seed=5, std=0.5, dtype=torch.bfloat16, W=W, bias_std=0.5,
                      bias_shape=(B, T, W), dtau_std=0.1 if tau else None)
    hip = hip_run(inp, W, 8.0, dev, normalize=normalize, return_tau=tau, use_bias=True, use_dtau=tau)
    ref = oracle_run(inp, W, 8.0, normalize=normalize, use_bias=True, use_dtau=tau)
    compare(hip, ref, torch.bfloat16, tau)


@pytest.mark.parametrize("normalize", [None, "count", "mass"])
def test_117m_geometry_tau_and_dtau(dev, normalize):
    """The kernel variants of the model's aux-loss step and of the tau
    benchmark, at their own launch geometry (B8 H12 T1024 W64 bf16): the
    fast forward emitting tau with two tiles per workgroup, and the fast
    backward taking dTau in runs of 3-4 tiles (dTau rows handed from step to
    step through the exchange tiles) plus a halo step."""
    B, H, T, D, W = 8, 12, 1024, 64, 64
    chunk, runs, longest = fused_geometry(B, H, T)
    print(f"[117m tau] normalize={normalize} fwd tiles/wg={min(chunk, 2)} bwd runs={runs} "
          f"longest={longest}", flush=True)
    assert min(chunk, 2) == 2 and longest >= 3
    inp = make_inputs(B, T, H, D, seed=11, std=0.5, dtype=torch.bfloat16, W=W, dtau_std=0.1)
    hip = hip_run(inp, W, 8.0, dev, normalize=normalize, return_tau=True, use_dtau=True)
    ref = oracle_run(inp, W, 8.0, normalize=normalize, use_dtau=True)
    compare(hip, ref, torch.bfloat16, True)


@pytest.mark.parametrize("normalize", [None, "count", "mass"])
@pytest.mark.parametrize("B,H,T", [(1, 2, 64), (2, 3, 320), (1, 12, 1024), (8, 16, 512), (2, 90, 640)])
def test_fast_path_dtau_bf16(dev, normalize, B, H, T):
    """The W = 64, T % 64 == 0 bf16 backward with a gradient through tau
    (the model's aux-loss step): dTau rows staged per wave.  The first three
    shapes give one-tile runs (a halo step after every tile), B8 H16 T512
    runs of two tiles."""
    D, W = 64, 64
    print(f"[fast dtau] B={B} H={H} T={T} geometry={fused_geometry(B, H, T)}", flush=True)
    inp = make_inputs(B, T, H, D, seed=T + H, std=0.5, dtype=torch.bfloat16, W=W, dtau_std=0.1)
    hip = hip_run(inp, W, 8.0, dev, normalize=normalize, return_tau=True, use_dtau=True)
    ref = oracle_run(inp, W, 8.0, normalize=normalize, use_dtau=True)
    compare(hip, ref, torch.bfloat16, True)


# ------------------------------------------------------------ reference kernel tests

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_forward_reference_shape(dev, dtype):
    """triton_tension/test.py:59-73 (seed 0; B2 T32 H4 HD16 W8)."""
    inp = make_inputs(2, 32, 4, 16, seed=0, rope=False, dtype=dtype)
    hip = hip_run(inp, 8, 4.0, dev, backward=False)
    ref = oracle_run(inp, 8, 4.0)
    compare(hip, ref, dtype, False)


def test_manual_grad_reference_shape(dev):
    """triton_tension/test.py:95-128 (seed 2; B2 T24 H4 HD16 W8, fp32)."""
    inp = make_inputs(2, 24, 4, 16, seed=2, rope=False)
    compare(hip_run(inp, 8, 4.0, dev), oracle_run(inp, 8, 4.0), torch.float32, False)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bias_forward_backward(dev, dtype):
    """triton_tension/test.py:131-149,175-209 (bias [B,T,W] * 0.5)."""
    inp = make_inputs(2, 32, 4, 16, seed=10, rope=False, dtype=dtype, bias_std=0.5,
                      bias_shape=(2, 32, 8))
    compare(hip_run(inp, 8, 4.0, dev, use_bias=True), oracle_run(inp, 8, 4.0, use_bias=True),
            dtype, False)


def test_bias_mfma_path(dev):
    inp = make_inputs(2, 200, 3, 64, seed=12, std=0.5, dtype=torch.bfloat16, bias_std=0.5,
                      bias_shape=(2, 200, 64), W=64, dtau_std=0.1)
    hip = hip_run(inp, 64, 8.0, dev, normalize="mass", return_tau=True, use_bias=True, use_dtau=True)
    ref = oracle_run(inp, 64, 8.0, normalize="mass", use_bias=True, use_dtau=True)
    compare(hip, ref, torch.bfloat16, True)


def test_large_bf16_spot_check(dev):
    """triton_tension/test.py:212-227 (seed 3; B4 T512 H12 HD64 W64 bf16)."""
    inp = make_inputs(4, 512, 12, 64, seed=3, rope=False, dtype=torch.bfloat16)
    compare(hip_run(inp, 64, 8.0, dev), oracle_run(inp, 64, 8.0), torch.bfloat16, False)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_forward_tau(dev, dtype):
    """triton_tension/test_tau.py:28-44."""
    D = 16 if dtype == torch.float32 else 64
    inp = make_inputs(2, 32, 4, D, seed=0, rope=False, dtype=dtype)
    hip = hip_run(inp, 8, math.sqrt(D), dev, return_tau=True, backward=False)
    compare(hip, oracle_run(inp, 8, math.sqrt(D)), dtype, True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_output_identical_with_without_tau(dev, dtype):
    """triton_tension/test_tau.py:47-60: requesting tau does not change Out (exact)."""
    from bozo_amd import causal_tension
    D = 16 if dtype == torch.float32 else 64
    inp = make_inputs(2, 70, 2, D, seed=1, rope=False, dtype=dtype)
    Q, K, V = (inp[n].to(dev) for n in "QKV")
    a = causal_tension(Q, K, V, 6, math.sqrt(D))
    b, _ = causal_tension(Q, K, V, 6, math.sqrt(D), return_tau=True)
    assert torch.equal(a, b)


def test_backward_through_tau(dev):
    """triton_tension/test_tau.py:63-99 (dTau * 0.1, raw output)."""
    inp = make_inputs(2, 24, 4, 16, seed=2, rope=False, W=8, dtau_std=0.1)
    hip = hip_run(inp, 8, 4.0, dev, return_tau=True, use_dtau=True)
    compare(hip, oracle_run(inp, 8, 4.0, use_dtau=True), torch.float32, True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backward_tau_unused(dev, dtype):
    """triton_tension/test_tau.py:102-127: unused tau leaves the grads unchanged."""
    from bozo_amd import causal_tension
    D = 16 if dtype == torch.float32 else 64
    inp = make_inputs(2, 90, 4, D, seed=3, rope=False, dtype=dtype)
    grads = []
    for rt in (False, True):
        Q, K, V = (inp[n].to(dev).requires_grad_(True) for n in "QKV")
        r = causal_tension(Q, K, V, 8, math.sqrt(D), return_tau=rt)
        out = r[0] if rt else r
        (out.float() * inp["dO"].to(dev).float()).sum().backward()
        grads.append((Q.grad, K.grad, V.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_memory_vs_unfold(dev):
    """triton_tension/test_tau.py:130-159: peak < unfold footprint / 4."""
    from bozo_amd import causal_tension
    B, T, H, D, W = 4, 1024, 16, 64, 256
    g = torch.Generator(device=dev).manual_seed(4)
    Q, K, V = (torch.randn(B, T, H, D, device=dev, dtype=torch.bfloat16, generator=g) for _ in range(3))
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    before = torch.cuda.memory_allocated()
    out, tau = causal_tension(Q, K, V, W, 8.0, return_tau=True)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - before
    unfold_bytes = B * T * H * W * D * 2
    assert peak < unfold_bytes / 4
    assert tau.shape == (B, T, H, W) and tau.dtype == torch.bfloat16


# ------------------------------------------------------------ float64 gradcheck

@pytest.mark.parametrize("normalize", [None, "mass", "count"])
@pytest.mark.parametrize("use_bias", [False, True])
def test_gradcheck_float64_on_gpu(dev, normalize, use_bias):
    """Unlike the reference (whose float64 gradcheck falls back to PyTorch,
    ops.py:217), this exercises the HIP backward kernels."""
    from bozo_amd import causal_tension
    torch.manual_seed(1)
    B, T, H, D, W = 1, 16, 2, 16, 6
    Q, K, V = (torch.randn(B, T, H, D, device=dev, dtype=torch.float64, requires_grad=True)
               for _ in range(3))
    bias = torch.randn(B, T, W, device=dev, dtype=torch.float64) * 0.3 if use_bias else None

    def fn(q, k, v):
        return causal_tension(q, k, v, W, math.sqrt(D), return_tau=True, bias=bias, normalize=normalize)

    assert torch.autograd.gradcheck(fn, (Q, K, V), eps=1e-6, atol=1e-7, rtol=1e-6)


# ------------------------------------------------------------ band edge cases

@pytest.mark.parametrize("T,W", [(1, 4), (5, 8), (64, 64), (65, 64), (100, 64), (130, 1),
                                 (300, 256), (200, 32), (77, 100)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_band_edges(dev, T, W, dtype):
    D = 64
    inp = make_inputs(2, T, 3, D, seed=T * 7 + W, std=0.5, dtype=dtype, W=W, dtau_std=0.1)
    hip = hip_run(inp, W, 8.0, dev, normalize="mass", return_tau=True, use_dtau=True)
    ref = oracle_run(inp, W, 8.0, normalize="mass", use_dtau=True)
    compare(hip, ref, dtype, True)


@pytest.mark.parametrize("D", [8, 16, 32, 128])
def test_other_head_dims_exact_path(dev, D):
    inp = make_inputs(2, 50, 2, D, seed=D, dtype=torch.bfloat16, W=12, dtau_std=0.1)
    hip = hip_run(inp, 12, math.sqrt(D), dev, normalize="mass", return_tau=True, use_dtau=True)
    ref = oracle_run(inp, 12, math.sqrt(D), normalize="mass", use_dtau=True)
    compare(hip, ref, torch.bfloat16, True)


def test_float16(dev):
    inp = make_inputs(2, 70, 2, 64, seed=5, std=0.5, dtype=torch.float16)
    compare(hip_run(inp, 16, 8.0, dev, normalize="mass"), oracle_run(inp, 16, 8.0, normalize="mass"),
            torch.bfloat16, False)


def test_strided_views_like_wkv_split(dev):
    """model.py:206-207 splits a fused wkv projection: K and V are strided
    views (innermost stride 1); the kernels read them in place."""
    from bozo_amd import causal_tension
    B, T, H, D, W = 2, 130, 4, 64, 64
    g = torch.Generator().manual_seed(9)
    kv = (torch.randn(B, T, H, 2 * D, generator=g) * 0.5).to(torch.bfloat16)
    q = (torch.randn(B, T, H, D, generator=g) * 0.5).to(torch.bfloat16)
    k, v = kv.split(D, dim=-1)
    out = causal_tension(q.to(dev), kv.to(dev)[..., :D], kv.to(dev)[..., D:], W, 8.0, normalize="mass")
    msg, tau = O.window_forward(f64(q), f64(k), f64(v), W, 8.0)
    ref, _ = O.normalize_mass(msg, tau)
    check_bf16(out, ref, "out")


def check_mixed(hip, ref, tau_checked):
    """The split-operand kernels carry every float32 operand as three bf16
    terms (24 significant bits, like float32 itself): the float32 outputs
    (out -- raw sums included --, dQ, dK, tau) are held to the fp32 bound,
    max-abs 1e-5 absolute, and the bf16 dV to 2e-2 relative L2."""
    out, tau, grads = hip
    assert out.dtype == torch.float32 and grads[0].dtype == torch.float32
    assert grads[1].dtype == torch.float32 and grads[2].dtype == torch.bfloat16
    check_fp32(out, ref[0], "out")
    check_fp32(grads[0], ref[2][0], "dQ")
    check_fp32(grads[1], ref[2][1], "dK")
    check_bf16(grads[2], ref[2][2], "dV")
    if tau_checked:
        assert tau.dtype == torch.float32
        check_fp32(tau, ref[1], "tau")


def mixed_inputs(B, T, H, seed, W=None, dtau_std=None, bias_std=None, D=64):
    """The reference's autocast flow: fp32 RoPE'd Q / K (model.py:75-81), bf16 V."""
    inp = make_inputs(B, T, H, D, seed=seed, std=0.5, W=W, dtau_std=dtau_std, bias_std=bias_std,
                      bias_shape=(B, T, W) if bias_std else None)
    inp["V"] = inp["V"].to(torch.bfloat16)
    return inp


def last_kernel():
    from bozo_amd import _lib as L
    return int(L.lib().tension_last_kernel())


def test_mixed_dtypes_autocast_like(dev):
    """Under autocast the reference feeds fp32 (RoPE'd) Q/K with bf16 V: the
    split-operand MFMA kernels."""
    from bozo_amd import _lib as L
    inp = mixed_inputs(2, 96, 2, seed=6)
    check_mixed(hip_run(inp, 32, 8.0, dev, normalize="mass"), oracle_run(inp, 32, 8.0, normalize="mass"), False)
    assert last_kernel() == L.KERNEL_SPLIT_F32


@pytest.mark.parametrize("normalize", [None, "mass", "count"])
def test_mixed_dtypes_117m_geometry(dev, normalize):
    """The reference's autocast dtype flow at the 117M layer shape (B8 H12
    T1024 W64): fp32 Q / K, bf16 V, tau emitted (fp32) and a gradient
    through it."""
    inp = mixed_inputs(8, 1024, 12, seed=21, W=64, dtau_std=0.1)
    print(f"[mixed 117m] normalize={normalize}", flush=True)
    hip = hip_run(inp, 64, 8.0, dev, normalize=normalize, return_tau=True, use_dtau=True)
    ref = oracle_run(inp, 64, 8.0, normalize=normalize, use_dtau=True)
    check_mixed(hip, ref, True)


@pytest.mark.parametrize("normalize", [None, "mass", "count"])
def test_mixed_dtypes_350m_window(dev, normalize):
    """The reference's 350M preset (train.py:246-256: W = 256, 16 heads of
    64) in its autocast flow, fp32 Q / K with bf16 V, at B2 T1024: tau
    emitted and its gradient, every normalisation, on the split kernels
    (five key blocks per query tile; the tau-mass dQ takes two passes)."""
    from bozo_amd import _lib as L
    inp = mixed_inputs(2, 1024, 16, seed=22, W=256, dtau_std=0.1)
    print(f"[mixed 350m W256] normalize={normalize}", flush=True)
    hip = hip_run(inp, 256, 8.0, dev, normalize=normalize, return_tau=True, use_dtau=True)
    assert last_kernel() == L.KERNEL_SPLIT_F32
    ref = oracle_run(inp, 256, 8.0, normalize=normalize, use_dtau=True)
    check_mixed(hip, ref, True)


@pytest.mark.parametrize("normalize", [None, "mass", "count"])
def test_mixed_dtypes_head_dim_32(dev, normalize):
    """The reference's default model (dim 128, 4 heads: head dim 32,
    model.py:33-36) in its autocast flow at the config-1 shape (B4 H4 T256
    W32): fp32 Q / K, bf16 V on the split kernels."""
    from bozo_amd import _lib as L
    inp = mixed_inputs(4, 256, 4, seed=23, W=32, dtau_std=0.1, D=32)
    hip = hip_run(inp, 32, math.sqrt(32), dev, normalize=normalize, return_tau=True, use_dtau=True)
    assert last_kernel() == L.KERNEL_SPLIT_F32
    ref = oracle_run(inp, 32, math.sqrt(32), normalize=normalize, use_dtau=True)
    check_mixed(hip, ref, True)


@pytest.mark.parametrize("T,W", [(1, 4), (70, 64), (100, 17), (130, 64), (64, 1), (200, 65), (300, 129),
                                 (257, 256)])
def test_mixed_dtypes_band_edges_bias(dev, T, W):
    """Ragged T, windows around the block size, one-key windows and the bias
    on the split kernels."""
    inp = mixed_inputs(2, T, 3, seed=T + W, W=W, dtau_std=0.1, bias_std=0.5)
    hip = hip_run(inp, W, 8.0, dev, normalize="mass", return_tau=True, use_bias=True, use_dtau=True)
    ref = oracle_run(inp, W, 8.0, normalize="mass", use_bias=True, use_dtau=True)
    check_mixed(hip, ref, True)


@pytest.mark.parametrize("T,W,normalize", [(1, 4, "mass"), (70, 64, "count"), (100, 17, "mass"),
                                           (130, 64, None), (200, 33, "mass"), (400, 200, "mass"),
                                           (333, 300, None), (129, 128, "count")])
def test_mixed_dtypes_band_edges_plain(dev, T, W, normalize):
    """Ragged T without bias or dTau, windows up to 300."""
    inp = mixed_inputs(2, T, 3, seed=3 * T + W, W=W)
    hip = hip_run(inp, W, 8.0, dev, normalize=normalize)
    ref = oracle_run(inp, W, 8.0, normalize=normalize)
    check_mixed(hip, ref, False)


@pytest.mark.parametrize("T,W,normalize,bias,tau", [
    (256, 32, "mass", False, False),   # BASELINE config 1 shape in bf16
    (256, 32, None, True, True),
    (300, 100, "count", False, True),
    (129, 256, "mass", True, True),
    (64, 1, None, False, False),
])
def test_bf16_head_dim_32(dev, T, W, normalize, bias, tau):
    """bf16 at head dim 32 (the reference's default model, model.py:33-36)
    on the split kernels with one bf16 term per operand: the bf16 tolerance
    (2e-2 relative L2; tau elementwise 4e-3)."""
    from bozo_amd import _lib as L
    D = 32
    inp = make_inputs(4, T, 4, D, seed=T + W + 5, std=0.5, dtype=torch.bfloat16, W=W,
                      dtau_std=0.1 if tau else None, bias_std=0.5 if bias else None,
                      bias_shape=(4, T, W) if bias else None)
    hip = hip_run(inp, W, math.sqrt(D), dev, normalize=normalize, return_tau=tau, use_bias=bias, use_dtau=tau)
    assert last_kernel() == L.KERNEL_SPLIT_BF16
    ref = oracle_run(inp, W, math.sqrt(D), normalize=normalize, use_bias=bias, use_dtau=tau)
    compare(hip, ref, torch.bfloat16, tau)


@pytest.mark.parametrize("dtype,D,W,normalize,bias,dtau", [
    ("f32qk", 32, 17, "mass", False, False),   # dQ and dK / dV runs
    ("f32qk", 32, 64, "count", True, False),   # runs with a bias
    ("f32qk", 32, 64, None, False, True),      # dTau: dK / dV runs, dQ per tile
    ("f32qk", 64, 33, "mass", True, True),     # head dim 64: dK / dV runs
    ("bf16", 32, 48, "mass", True, True),      # one bf16 term: dK / dV runs
])
def test_backward_runs(dev, dtype, D, W, normalize, bias, dtau):
    """Local windows W <= 64 on shapes with more tiles than workgroups per
    (b, h): the split backward walks runs of consecutive tiles (dK / dV
    always, dQ for float32 Q / K at head dim 32 without dTau), with T ragged
    (the last tile partly past the sequence) so the runs end on a partial
    tile.  B * H = 128 on 16 tiles per sequence: 4 runs each on a 256-CU
    device."""
    from bozo_amd import _lib as L
    B, H, T = 32, 4, 1000
    seed = 100 + D + W
    if dtype == "f32qk":
        inp = mixed_inputs(B, T, H, seed=seed, W=W, dtau_std=0.1 if dtau else None,
                           bias_std=0.5 if bias else None, D=D)
    else:
        inp = make_inputs(B, T, H, D, seed=seed, std=0.5, dtype=torch.bfloat16, W=W,
                          dtau_std=0.1 if dtau else None, bias_std=0.5 if bias else None,
                          bias_shape=(B, T, W) if bias else None)
    print(f"[runs] {dtype} D={D} W={W} normalize={normalize} bias={bias} dtau={dtau}", flush=True)
    hip = hip_run(inp, W, math.sqrt(D), dev, normalize=normalize, return_tau=dtau, use_bias=bias, use_dtau=dtau)
    assert last_kernel() == (L.KERNEL_SPLIT_F32 if dtype == "f32qk" else L.KERNEL_SPLIT_BF16)
    ref = oracle_run(inp, W, math.sqrt(D), normalize=normalize, use_bias=bias, use_dtau=dtau)
    if dtype == "f32qk":
        check_mixed(hip, ref, dtau)
    else:
        compare(hip, ref, torch.bfloat16, dtau)


def test_strides_beyond_int32_take_exact_kernels(dev):
    """A batch stride above 2^31 elements: the MFMA and split kernels take
    32-bit strides, so the call runs on the exact kernels (strides read in
    place, 64-bit offsets), and matches the oracle.  Q, K, V are views with
    gaps into one 4.3 GB buffer."""
    from bozo_amd import _lib as L
    B, T, H, D, W = 2, 128, 2, 64, 16
    S = (1 << 31) + 64  # batch stride in elements
    n = T * H * D
    buf = torch.zeros(S + 3 * n, dtype=torch.bfloat16, device=dev)
    ref_in = make_inputs(B, T, H, D, seed=77, std=0.5, dtype=torch.bfloat16, W=W)
    views = {}
    for i, name in enumerate("QKV"):
        v = buf.as_strided((B, T, H, D), (S, H * D, D, 1), i * n)
        v.copy_(ref_in[name].to(dev))
        views[name] = v
    from bozo_amd import causal_tension
    Q, K, V = (views[c].detach().requires_grad_(True) for c in "QKV")
    assert Q.stride(0) == S
    out = causal_tension(Q, K, V, W, 8.0, normalize="mass")
    assert last_kernel() == L.KERNEL_EXACT
    (out.float() * ref_in["dO"].to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    assert last_kernel() == L.KERNEL_EXACT
    ref = oracle_run(ref_in, W, 8.0, normalize="mass")
    compare((out, None, (Q.grad, K.grad, V.grad)), ref, torch.bfloat16, False)
    del buf, views, Q, K, V, out


def test_empty_batch(dev):
    from bozo_amd import causal_tension
    Q = torch.zeros(0, 16, 2, 64, device=dev, dtype=torch.bfloat16)
    out = causal_tension(Q, Q, Q, 8, 8.0)
    assert out.shape == Q.shape


def test_deterministic(dev):
    """No atomics: two runs are bitwise identical."""
    inp = make_inputs(2, 300, 4, 64, seed=8, std=0.5, dtype=torch.bfloat16)
    a = hip_run(inp, 64, 8.0, dev, normalize="mass")
    b = hip_run(inp, 64, 8.0, dev, normalize="mass")
    assert torch.equal(a[0], b[0])
    for x, y in zip(a[2], b[2]):
        assert torch.equal(x, y)


def test_errors(dev):
    from bozo_amd import causal_tension
    Q = torch.zeros(1, 8, 1, 16, device=dev)
    with pytest.raises(RuntimeError):
        causal_tension(Q.cpu(), Q.cpu(), Q.cpu(), 4, 4.0)
    with pytest.raises(ValueError):
        causal_tension(Q, Q, Q, 4, 4.0, bias=torch.zeros(1, 8, 5, device=dev))
    with pytest.raises(ValueError):
        causal_tension(Q, Q, Q, 0, 4.0)


# ------------------------------------------------------------ fused backward runs

@pytest.mark.parametrize("B,H,T,W", [
    (1, 1, 1024, 64),   # 16 runs of one tile per (b,h): a halo step in every run
    (2, 48, 400, 64),   # 5 runs of 1-2 tiles, ragged last tile
    (64, 17, 65, 33),   # one run per (b,h) (no halo), W < 64
    (3, 2, 333, 17),
    (4, 64, 512, 64),   # 2 runs of 4 tiles: run 1 steps down from the sequence end (no halo)
    (2, 90, 640, 64),   # 3 runs of 3-4 tiles: boundaries met at the runs' ends and at their starts
])
@pytest.mark.parametrize("normalize", [None, "mass", "count"])
def test_fused_backward_runs_bf16(dev, B, H, T, W, normalize):
    """The bf16 backward for W <= 64 is one kernel that splits every (b,h)
    sequence into runs of tiles, odd runs stepping down, and recomputes the
    tile after each run (the halo); the grid size, and so the run length and
    count, depends on B*H."""
    inp = make_inputs(B, T, H, 64, seed=B * 1000 + T + W, std=0.5, dtype=torch.bfloat16,
                      bias_std=0.5, bias_shape=(B, T, W))
    use_bias = normalize == "mass"
    hip = hip_run(inp, W, 8.0, dev, normalize=normalize, use_bias=use_bias)
    ref = oracle_run(inp, W, 8.0, normalize=normalize, use_bias=use_bias)
    compare(hip, ref, torch.bfloat16, False)


@pytest.mark.parametrize("pad", [8, 4])
def test_tau_dtau_row_layouts_abi(dev, pad):
    """Through the C ABI, tau / dTau rows padded to 64 + pad slots: pad 8
    keeps 16-byte rows (the staged fast paths), pad 4 does not (the general
    kernels).  Either way the results equal the contiguous run's."""
    import ctypes
    from bozo_amd import _lib as L
    from bozo_amd import causal_tension
    B, T, H, D, W, scale = 2, 256, 3, 64, 64, 8.0
    g = torch.Generator(device=dev).manual_seed(pad)
    q, k, v, do = ((torch.randn(B, T, H, D, device=dev, generator=g) * 0.5).to(torch.bfloat16) for _ in range(4))
    dt = (torch.randn(B, T, H, W, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))
    out_ref, tau_ref = causal_tension(qq, kk, vv, W, scale, return_tau=True, normalize="mass")
    torch.autograd.backward([out_ref, tau_ref], [do, dt])

    lib = L.lib()
    st = L.stream_handle(dev)
    out = torch.empty_like(q)
    taup = torch.full((B, T, H, W + pad), float("nan"), device=dev, dtype=torch.bfloat16)
    tau = taup[..., :W]
    L.check(lib.tension_window_fwd(L.buf(q), L.buf(k), L.buf(v), L.buf(out), L.buf(tau), None, None,
                                   B, T, H, D, W, ctypes.c_double(scale), L.NORM_MASS, st), "fwd")
    dtp = torch.zeros((B, T, H, W + pad), device=dev, dtype=torch.bfloat16)
    dtp[..., :W] = dt
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    nws = lib.tension_window_bwd_workspace(B, T, H, L.F32, L.NORM_MASS)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
    L.check(lib.tension_window_bwd(L.buf(q), L.buf(k), L.buf(v), L.buf(do), L.buf(dtp[..., :W]), None,
                                   L.buf(dq), L.buf(dk), L.buf(dv), ctypes.c_void_p(ws.data_ptr() if nws else None),
                                   B, T, H, D, W, ctypes.c_double(scale), L.NORM_MASS, st), "bwd")
    torch.cuda.synchronize()
    if pad % 8 == 0:  # the same kernels as the contiguous run: the same bits
        assert torch.equal(out, out_ref.detach())
        assert torch.equal(tau, tau_ref.detach())
    else:  # other kernels: bf16 rounding of the same fp32 values
        assert (out.float() - out_ref.float()).abs().max().item() <= 2e-2 * out_ref.float().abs().max().item()
        assert (tau.float() - tau_ref.float()).abs().max().item() <= 4e-3
    assert torch.isnan(taup[..., W:]).all()  # the padding is not written
    for a, b in ((dq, qq.grad), (dk, kk.grad), (dv, vv.grad)):
        assert (a.float() - b.float()).abs().max().item() <= 2e-2 * b.float().abs().max().item()


@pytest.mark.parametrize("W,D,tau", [(256, 64, False), (256, 64, True), (65, 32, True), (100, 64, True)])
def test_window_bwd_saved_rows_match_recompute(dev, W, D, tau):
    """tension_window_bwd_saved (coefficients from the forward's float32 rows
    and tau mass, one pass) against tension_window_bwd (coefficients from a
    pass over the band) through the C ABI, autocast flow, tau-mass: equal to
    float32 rounding (max-abs 2e-7 on dQ, dK; dV bf16 to one rounding), and
    both against the float64 oracle at the fp32 bound."""
    import ctypes
    from bozo_amd import _lib as L
    B, T, H = 2, 300, 3
    inp = mixed_inputs(B, T, H, seed=70 + W + D, W=W, dtau_std=0.1 if tau else None, D=D)
    q, k, dO = (inp[n].to(dev) for n in ("Q", "K", "dO"))
    v = inp["V"].to(dev)
    dtau = inp["dTau"].to(dev) if tau else None
    scale = math.sqrt(D)
    lib, st = L.lib(), L.stream_handle(dev)
    out = torch.empty_like(q)
    mass = torch.empty(B, T, H, device=dev)
    L.check(lib.tension_window_fwd(L.buf(q), L.buf(k), L.buf(v), L.buf(out), None, None, L.buf(mass),
                                   B, T, H, D, W, ctypes.c_double(scale), L.NORM_MASS, st), "fwd")
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
        assert int(lib.tension_last_kernel()) == L.KERNEL_SPLIT_F32
        res.append((dq, dk, dv))
    torch.cuda.synchronize()
    for name, a, b_ in zip(("dQ", "dK"), res[0], res[1]):
        err = float((a - b_).abs().max())
        print(f"  {name}: saved vs recompute max abs {err:.2e}", flush=True)
        assert err <= 2e-7, (name, err)
    assert float((res[0][2].float() - res[1][2].float()).abs().max()) <= 2 ** -8 * float(res[0][2].float().abs().max())
    _, _, grads = oracle_run(inp, W, scale, normalize="mass", use_dtau=tau)
    for got, want, name in zip(res[1][:2], grads[:2], ("dQ", "dK")):
        check_fp32(got, want, name)
