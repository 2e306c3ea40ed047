"""tension_global_bwd_noalloc: the global backward with its per-query
coefficients in the library's fixed device scratch instead of a caller
workspace.  Through the C ABI, two calls in a row (the second with a smaller
input, so stale scratch contents from the first would show) must give the
same dQ, dK, dV bits as tension_global_bwd with a caller workspace, on the
bf16 MFMA kernels, on the split kernels (float32 and float16 flows) and on
the exact kernels.  The refusal of
requests beyond the scratch happens before any HIP call and is checked on
the CPU (tests/test_abi.py)."""
import ctypes

import pytest
import torch

from bozo_amd import _lib as L

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, D, dtype, Wl, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    q, k, v, do = ((torch.randn(B, T, H, D, device=dev, generator=g) * 0.5).to(dtype) for _ in range(4))
    bias = torch.randn(B, T, T, device=dev, generator=g) * 0.5
    dtl = (torch.randn(B, T, H, Wl, device=dev, generator=g) * 0.1).to(dtype)
    return q, k, v, do, bias, dtl


def _forward(lib, q, k, v, bias, Wl, scale, st):
    B, T, H, D = q.shape
    out = torch.empty_like(q)
    tl = torch.empty(B, T, H, Wl, dtype=q.dtype, device=q.device)
    mass = torch.empty(B, T, H, dtype=torch.float32, device=q.device)
    L.check(lib.tension_global_fwd(L.buf(q), L.buf(k), L.buf(v), L.buf(out), L.buf(tl), L.buf(bias),
                                   L.buf(mass), B, T, H, D, Wl, ctypes.c_double(scale), 0, st), "fwd")
    return out, mass


def _backward(lib, noalloc, q, k, v, do, dtl, bias, out, mass, Wl, scale, st):
    B, T, H, D = q.shape
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    common = (L.buf(q), L.buf(k), L.buf(v), L.buf(do), L.buf(dtl), L.buf(bias), L.buf(out), L.buf(mass),
              L.buf(dq), L.buf(dk), L.buf(dv))
    if noalloc:
        r = lib.tension_global_bwd_noalloc(*common, B, T, H, D, Wl, ctypes.c_double(scale), 0, st)
    else:
        acc = L.F64 if q.dtype == torch.float64 else L.F32
        ws = torch.empty(lib.tension_global_bwd_workspace(B, T, H, acc, 0), dtype=torch.uint8, device=q.device)
        r = lib.tension_global_bwd(*common, ctypes.c_void_p(ws.data_ptr()), B, T, H, D, Wl,
                                   ctypes.c_double(scale), 0, st)
    L.check(r, "noalloc" if noalloc else "workspace")
    return dq, dk, dv


@pytest.mark.parametrize("dtype,D,shapes", [
    (torch.bfloat16, 64, [(2, 700, 12), (1, 300, 4)]),   # MFMA kernels
    (torch.float32, 32, [(2, 130, 3), (1, 70, 2)]),      # split kernels, float32 flow
    (torch.float16, 64, [(2, 300, 3), (1, 100, 2)]),     # split kernels, float16
    (torch.float32, 16, [(2, 130, 3), (1, 70, 2)]),      # exact kernels
])
def test_noalloc_matches_workspace_entry_point(dev, dtype, D, shapes):
    lib = L.lib()
    st = L.stream_handle(dev)
    Wl, scale = 16, D ** 0.5
    for i, (B, T, H) in enumerate(shapes):
        print(f"[noalloc] call {i}: B={B} T={T} H={H} D={D} {dtype}", flush=True)
        q, k, v, do, bias, dtl = _inputs(B, T, H, D, dtype, Wl, 100 + i, dev)
        out, mass = _forward(lib, q, k, v, bias, Wl, scale, st)
        a = _backward(lib, True, q, k, v, do, dtl, bias, out, mass, Wl, scale, st)
        b = _backward(lib, False, q, k, v, do, dtl, bias, out, mass, Wl, scale, st)
        torch.cuda.synchronize()
        for name, x, y in zip(("dQ", "dK", "dV"), a, b):
            assert torch.isfinite(x.float()).all(), name
            assert torch.equal(x, y), (name, (x.float() - y.float()).abs().max().item())

