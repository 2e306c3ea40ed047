"""Long sequences: the window op at up to T = 65573 and the global block at
T = 3000, forward and backward, against the float64 oracle.

The window op is local, which makes the check exact at any length: out and
dQ of rows [t0, t1) depend only on the inputs of rows [t0 - W, t1), and dK /
dV of those rows on the queries up to t1 + W - 1, whose own windows start at
or after t0 - W.  So each checked segment runs the oracle on rows
[t0 - W, t1 + W) (clipped to the sequence) and compares rows [t0, t1) of the
full-length HIP run.  Segments sit at the start, in the middle (not aligned
to the 64-row tiles, crossing the fused backward's run boundaries) and at
the end of the sequence.  The paths: the fused backward's fast path (W = 64,
T a multiple of 64), its general path (ragged T), the split backward
(W > 64) and the float32 exact kernels.  The global block has no such
locality; it is checked whole at T = 3000 (ragged, 47 tiles).

Tolerances as elsewhere: bf16 relative L2 2e-2 over the checked rows,
float32 max-abs 1e-5.
"""
import numpy as np
import pytest
import torch

from tests._util import f64, make_inputs, max_abs, rel_l2
from tests.test_global_gpu import hip_run as global_hip_run
from tests.test_global_gpu import oracle_run as global_oracle_run
from tests.test_window_gpu import hip_run, oracle_run

pytestmark = pytest.mark.gpu


def _segments(T, W):
    mid = T // 2 - 97
    return [(0, 200), (mid, mid + 256), (T - 200, T)]


@pytest.mark.parametrize("dtype,T,H,W,norm", [
    (torch.bfloat16, 65536, 3, 64, "mass"),      # fused backward, fast path
    (torch.bfloat16, 65573, 2, 64, "count"),     # fused backward, ragged T
    (torch.bfloat16, 40000, 2, 100, "mass"),     # split backward (W > 64)
    (torch.float32, 20000, 2, 64, "mass"),       # exact kernels
])
def test_window_long_sequence_segments(dev, dtype, T, H, W, norm):
    D = 64
    inp = make_inputs(1, T, H, D, seed=T + W, std=0.5, rope=False, dtype=dtype)
    print(f"[long window {dtype} T={T} H={H} W={W} {norm}]", flush=True)
    out, _, grads = hip_run(inp, W, 8.0, dev, normalize=norm)
    got = [f64(out)] + [f64(g) for g in grads]
    for t0, t1 in _segments(T, W):
        a, b = max(0, t0 - W), min(T, t1 + W)
        seg = {k: (v[:, a:b] if v is not None else None) for k, v in inp.items()}
        rout, _, rgrads = oracle_run(seg, W, 8.0, normalize=norm)
        for what, g, r in zip(("out", "dQ", "dK", "dV"), got, (rout,) + tuple(rgrads)):
            g, r = g[:, t0:t1], r[:, t0 - a:t1 - a]
            if dtype == torch.float32:
                err, lim = max_abs(g, r), 1e-5
            else:
                err, lim = rel_l2(g, r), 2e-2
            print(f"  rows [{t0}, {t1}) {what}: {err:.2e}", flush=True)
            assert err <= lim, f"rows [{t0}, {t1}) {what}: {err:.3e} > {lim:.0e}"


@pytest.mark.parametrize("dtype,T", [(torch.bfloat16, 3000), (torch.float32, 1500)])
def test_global_long_sequence(dev, dtype, T):
    B, H, D = 1, 1, 64
    inp = make_inputs(B, T, H, D, seed=T, std=0.5, rope=False, dtype=dtype)
    print(f"[long global {dtype} T={T}]", flush=True)
    out, _, grads = global_hip_run(inp, 8.0, dev)
    rout, _, rgrads = global_oracle_run(inp, 8.0)
    for what, g, r in zip(("out", "dQ", "dK", "dV"), (out,) + tuple(grads), (rout,) + tuple(rgrads)):
        if dtype == torch.float32:
            err, lim = max_abs(f64(g), r), 1e-5
        else:
            err, lim = rel_l2(f64(g), r), 2e-2
        print(f"  {what}: {err:.2e}", flush=True)
        assert err <= lim, f"{what}: {err:.3e} > {lim:.0e}"
