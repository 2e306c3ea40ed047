"""Seeded sweeps of RoPE and of the fused tau regularisers.

RoPE: twenty configurations drawn once from a fixed generator -- batch,
length (1 to 129), heads, head dims 16 to 128 (the 16-byte kernel when D is
a multiple of 16 and the rows are 16-byte aligned, the generic one
otherwise), input dtypes bf16 / fp16 / fp32 / fp64, output dtype the input's,
float32 (the reference's promotion under autocast) or bf16, position offsets,
and strided inputs (a slice of a wider tensor, as the model's q / k views
of one projection are).  The forward is checked against the float64
restatement of model.py:75-81 (one rounding of the float32 result in a 16-bit
output: relative 2^-8 for bf16, 2^-10 for fp16; float32 max-abs 1e-5, float64
1e-12) and the backward against its adjoint.

Aux losses: twelve configurations of the fused diversity / consistency /
entropy losses (layers, batch, length, heads, W from 1 -- no consistency
terms -- to 64, float32 and bf16 taus, one or two window groups) against the
model's PyTorch restatements of model.py:498-611 (pinned by loops in the CPU
suite), values and dTau, with the tolerances of test_aux_loss_gpu.py.
"""
import numpy as np
import pytest
import torch

from bozo_amd import model as M
from oracle import tension_oracle as O
from tests._util import f64, max_abs, rel_l2
from tests.test_aux_loss_gpu import reference, taus_of

pytestmark = pytest.mark.gpu

_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32, "f64": torch.float64}


def _draw_rope(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        dt = str(rng.choice(["bf16", "bf16", "f16", "f32", "f32", "f64"]))
        out = str(rng.choice(["same", "f32", "bf16"])) if dt != "f64" else "same"
        cases.append((i, int(rng.choice([1, 2, 3])), int(rng.choice([1, 7, 50, 129])),
                      int(rng.choice([1, 3, 12])), int(rng.choice([16, 32, 40, 48, 64, 128])), dt, out,
                      int(rng.choice([0, 5, 100])), bool(rng.integers(2))))
    return cases


ROPE = _draw_rope(20, 2030)


@pytest.mark.parametrize("case", ROPE, ids=[f"{c[0]}-B{c[1]}T{c[2]}H{c[3]}D{c[4]}-{c[5]}-{c[6]}-p{c[7]}"
                                            f"{'-strided' if c[8] else ''}" for c in ROPE])
def test_rope_sweep(dev, case):
    from bozo_amd import rope
    i, B, T, H, D, dt, out, pos, strided = case
    dtype = _DT[dt]
    out_dtype = None if out == "same" else _DT[out]
    cos, sin = O.rope_tables(pos + T + 3, D)
    g = torch.Generator().manual_seed(1100 + i)
    base = torch.randn(B, T, H, 3 * D if strided else D, generator=g, dtype=torch.float64).to(dtype)
    x = base[..., D:2 * D] if strided else base            # a slice with a 3D row stride
    print(f"[rope sweep {case}]", flush=True)
    xd = base.to(dev)[..., D:2 * D] if strided else base.to(dev)
    xd = xd.detach().requires_grad_(True)
    y = rope(xd, torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev), pos_offset=pos, out_dtype=out_dtype)
    assert y.dtype == (out_dtype or dtype) and y.shape == x.shape
    want = O.rope_apply(f64(x), cos, sin, pos_offset=pos)
    if y.dtype in (torch.bfloat16, torch.float16):
        rel = 2 ** -8 if y.dtype == torch.bfloat16 else 2 ** -10
        err = float(np.max(np.abs(f64(y) - want) / np.maximum(np.abs(want), 1e-3)))
        assert err <= rel, f"forward: relative err {err:.3e} > {rel:.2e}"
    else:
        lim = 1e-12 if y.dtype == torch.float64 else 1e-5
        assert max_abs(f64(y), want) <= lim
    dy = torch.randn(B, T, H, D, generator=g, dtype=torch.float64).to(y.dtype)
    (y.double() * dy.to(dev).double()).sum().backward()
    dwant = O.rope_apply_adjoint(f64(dy), cos, sin, pos_offset=pos)
    if dtype in (torch.bfloat16, torch.float16):
        lim = 2e-2 if dtype == torch.bfloat16 else 2e-3
        assert rel_l2(f64(xd.grad), dwant) <= lim
    else:
        lim = 1e-12 if dtype == torch.float64 else 1e-5
        assert max_abs(f64(xd.grad), dwant) <= lim


def _draw_aux(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        cases.append((i, int(rng.choice([1, 2, 3, 6, 12])), int(rng.choice([1, 2, 3])),
                      int(rng.choice([3, 17, 64, 300, 1030])), int(rng.choice([1, 2, 4, 12])),
                      int(rng.choice([1, 2, 3, 8, 33, 64])), str(rng.choice(["f32", "bf16"])), bool(rng.integers(2))))
    return cases


AUX = _draw_aux(12, 2031)


@pytest.mark.parametrize("case", AUX, ids=[f"{c[0]}-L{c[1]}B{c[2]}T{c[3]}H{c[4]}W{c[5]}-{c[6]}"
                                           f"{'-grouped' if c[7] else ''}" for c in AUX])
def test_aux_losses_sweep(dev, case):
    i, L, B, T, H, W, dt, grouped = case
    dtype = _DT[dt]
    taus = taus_of(1200 + i, L, B, T, H, W, dtype, dev)
    groups = {W: list(range(0, L, 2)), 1024: list(range(1, L, 2))} if grouped and L > 1 else None
    print(f"[aux sweep {case}] workgroups/layer={-(-B * T * H // 1024)}", flush=True)
    a = [t.detach().float().requires_grad_(True) for t in taus]
    b = [t.detach().clone().requires_grad_(True) for t in taus]
    ra = reference(a, groups)
    fb = M.tension_aux_losses(b, groups)
    for x, y in zip(ra, fb):
        x, y = float(x.detach()), float(y.detach())
        assert abs(x - y) <= 1e-5 * max(1.0, abs(x)), (x, y)
    w = (0.7, 1.3, 2.1)
    sum(wi * x for wi, x in zip(w, ra)).backward()
    sum(wi * y for wi, y in zip(w, fb)).backward()
    for ga, gb in zip(a, b):
        assert gb.grad.dtype == dtype
        ref = ga.grad.double()
        err = (gb.grad.double() - ref).abs().max().item()
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        assert err <= tol * max(ref.abs().max().item(), 1e-12) + 1e-12, (err,)
