"""Seeded sweep of the streaming decode step against the float64 oracle.

Thirty-two window-cache configurations drawn once from a fixed generator:
sequence and head counts, head dims 64 (the fast kernels) and 32 / 128 (the
exact kernel), windows from one slot to 512, a cache that is empty, partly
filled, exactly full or wrapped when the checked steps begin, every
normalisation (tau mass, valid count, raw), with and without the tau output,
and five dtype flows: bf16, float32 and float16 (the fast kernel at head
dim 64, float32 up to W = 512; the exact kernel otherwise), float64 (exact
kernel), and float32 q / K with a bf16 V cache (the reference's autocast
flow, float32-K fast kernel).  Each step must
equal the last row of the local window over the same sequence (the decode
contract; the oracle's window_forward / normalize_* are pinned by
test_oracle.py), computed in float64 from the rounded inputs.  Eight more
run the self-key step of a global layer's cache (every earlier token cached,
the new token a key too), which must equal the rows of global_forward.

Tolerances: float32 outputs and tau max-abs 1e-5 (raw sums: 1e-5 of their
largest magnitude), float64 1e-9, float16 relative L2 2e-3 (tau max-abs
1e-3), bf16 relative L2 2e-2 (tau max-abs 4e-3), as in test_decode_gpu.py.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tension_oracle as O
from tests._util import f64, max_abs, rel_l2

pytestmark = pytest.mark.gpu

_KINDS = {  # q / K dtype, V dtype
    "bf16": (torch.bfloat16, torch.bfloat16),
    "f32": (torch.float32, torch.float32),
    "f64": (torch.float64, torch.float64),
    "f16": (torch.float16, torch.float16),
    "f32k_bf16v": (torch.float32, torch.bfloat16),
}


def _draw(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        kind = str(rng.choice(["bf16", "bf16", "f32", "f64", "f16", "f32k_bf16v"]))
        D = 64 if kind == "f32k_bf16v" else int(rng.choice([64, 64, 32, 128]))
        W = int(rng.choice([1, 7, 33, 64, 65, 100, 256, 300, 512]))
        N = int(rng.choice([1, 2, 3]))
        H = int(rng.choice([1, 3, 4]))
        prefill = int(rng.choice([0, 1, W // 2, W, W + 3]))
        norm = str(rng.choice(["mass", "count", "raw"]))
        tau = bool(rng.integers(2))
        cases.append((i, kind, D, W, N, H, prefill, norm, tau))
    return cases


CASES = _draw(32, 2029)


def _inputs(N, L, H, D, seed, kind):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(N, L, H, D, generator=g, dtype=torch.float64) * 0.5 for _ in range(3))
    qk_dt, v_dt = _KINDS[kind]
    return q.to(qk_dt), k.to(qk_dt), v.to(v_dt)


def _check(what, got, want, kind, raw=False):
    g = f64(got)
    if kind in ("f32", "f32k_bf16v", "f64"):
        lim = 1e-9 if kind == "f64" else 1e-5
        if raw and want.size:
            lim *= max(1.0, float(np.max(np.abs(want))))
        err = max_abs(g, want)
    elif what == "tau":
        lim, err = (1e-3 if kind == "f16" else 4e-3), max_abs(g, want)
    else:
        lim, err = (2e-3 if kind == "f16" else 2e-2), rel_l2(g, want)
    assert err <= lim, f"{what}: err {err:.3e} > {lim:.1e}"
    return err


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}-D{c[2]}W{c[3]}N{c[4]}H{c[5]}p{c[6]}-{c[7]}"
                                             f"{'-tau' if c[8] else ''}" for c in CASES])
def test_decode_sweep(dev, case):
    from bozo_amd import TensionDecodeCache
    i, kind, D, W, N, H, prefill, norm, want_tau = case
    S = 4
    L = prefill + S
    q, k, v = _inputs(N, L, H, D, 700 + i, kind)
    qk_dt, v_dt = _KINDS[kind]
    print(f"[decode sweep {case}]", flush=True)
    cache = TensionDecodeCache(N, H, D, W, dtype=qk_dt, device=dev, v_dtype=v_dt)
    for t in range(prefill):
        cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), normalize=norm)
    msg, tau = O.window_forward(f64(q), f64(k), f64(v), W, math.sqrt(D))
    ref = {"mass": lambda: O.normalize_mass(msg, tau)[0], "count": lambda: O.normalize_count(msg, W),
           "raw": lambda: msg}[norm]()
    for t in range(prefill, L):
        r = cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), normalize=norm, return_tau=want_tau)
        out, tt = r if want_tau else (r, None)
        torch.cuda.synchronize()
        assert out.dtype == qk_dt
        e = _check("out", out, ref[:, t], kind, raw=norm == "raw")
        if want_tau:
            e2 = _check("tau", tt, tau[:, t], kind)
            print(f"  step {t}: out {e:.2e} tau {e2:.2e}", flush=True)
    # the ring holds the last min(L, W) keys, each in the slot its position maps to
    kc = cache.k.cpu()
    for t in range(max(0, L - W), L):
        assert torch.equal(kc[:, :, t % W], k[:, t]), t
    assert int(cache.pos[cache.cur][0]) == L


SELF = [(i, kind, W, prefill) for i, (kind, W, prefill) in enumerate([
    ("bf16", 64, 0), ("bf16", 96, 40), ("bf16", 300, 250), ("bf16", 1024, 700),
    ("f32", 40, 0), ("f32", 64, 30), ("f64", 50, 20), ("f16", 128, 100)])]


@pytest.mark.parametrize("case", SELF, ids=[f"{c[0]}-{c[1]}-W{c[2]}p{c[3]}" for c in SELF])
def test_decode_self_sweep(dev, case):
    """A global layer's cache (max_seq_len slots, never wrapped) with the new
    token as a key: the rows of the full causal block, diagonal included."""
    from bozo_amd import TensionDecodeCache
    i, kind, W, prefill = case
    N, H, D, S = 2, 3, 64, 4
    L = prefill + S
    assert L <= W
    q, k, v = _inputs(N, L, H, D, 900 + i, kind)
    qk_dt, v_dt = _KINDS[kind]
    print(f"[decode self sweep {case}]", flush=True)
    cache = TensionDecodeCache(N, H, D, W, dtype=qk_dt, device=dev, v_dtype=v_dt)
    for t in range(prefill):
        cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), include_self=True)
    ref = O.global_forward(f64(q), f64(k), f64(v), math.sqrt(D))[0]
    for t in range(prefill, L):
        out = cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), include_self=True)
        torch.cuda.synchronize()
        _check("out", out, ref[:, t], kind)
