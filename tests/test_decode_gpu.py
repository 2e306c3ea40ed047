"""Streaming decode and RoPE kernels against the oracle.

Decode has no reference kernel; the contract (survey row A11) is that each
step equals the last row of the tau-mass-normalised local window over the
same sequence (causality, ts_bridge/streaming_parity.py:20-24), which the
oracle's own tests pin.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tension_oracle as O
from tests._util import f64, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def seq_inputs(N, L, H, D, seed, std=0.5):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(N, L, H, D, generator=g) * std for _ in range(3)]


@pytest.mark.parametrize("dtype,D,W,prefill", [
    (torch.bfloat16, 64, 64, 64),     # fast path, warm cache
    (torch.bfloat16, 64, 32, 5),      # fast path, filling cache
    (torch.bfloat16, 64, 1, 2),       # fast path, one slot (31 rows past W)
    (torch.bfloat16, 64, 33, 40),     # fast path, rows past W in the last pass
    (torch.bfloat16, 64, 100, 7),     # fast path, filling, W not a multiple of 32
    (torch.bfloat16, 64, 160, 170),   # fast path, 4 passes, 96 rows past W
    (torch.bfloat16, 64, 288, 7),     # fast path, 8 passes
    (torch.bfloat16, 64, 384, 390),   # fast path, 8 passes
    (torch.bfloat16, 64, 512, 515),   # fast path, largest window
    (torch.float32, 64, 64, 70),      # fast path, float32 throughout
    (torch.float32, 64, 512, 515),    # fast path, float32, largest window it takes
    (torch.float32, 64, 600, 610),    # exact path (float32 beyond W = 512)
    (torch.float32, 32, 64, 70),      # exact path (D != 64)
    (torch.float16, 64, 64, 70),      # fast path, float16 throughout
    (torch.float16, 64, 1024, 1030),  # fast path, float16, 16 passes
    (torch.bfloat16, 32, 16, 3),      # exact path (D != 64)
])
def test_decode_matches_window_rows(dev, dtype, D, W, prefill):
    from bozo_amd import TensionDecodeCache
    N, H, S = 3, 4, 12
    L = prefill + S
    q, k, v = (t.to(dtype) for t in seq_inputs(N, L, H, D, seed=W + prefill))
    cache = TensionDecodeCache(N, H, D, W, dtype=dtype, device=dev)
    for t in range(prefill):
        cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev))
    msg, tau = O.window_forward(f64(q), f64(k), f64(v), W, math.sqrt(D))
    ref, _ = O.normalize_mass(msg, tau)
    for t in range(prefill, L):
        out, tt = cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), return_tau=True)
        torch.cuda.synchronize()
        if dtype == torch.float32:
            assert max_abs(f64(out), ref[:, t]) <= 1e-5
            assert max_abs(f64(tt), tau[:, t]) <= 1e-5
        elif dtype == torch.float16:
            assert rel_l2(f64(out), ref[:, t]) <= 1e-3
            assert max_abs(f64(tt), tau[:, t]) <= 2.0 ** -11
        else:
            assert rel_l2(f64(out), ref[:, t]) <= 2e-2
            assert max_abs(f64(tt), tau[:, t]) <= 4e-3
    assert int(cache.pos[cache.cur][0]) == L


@pytest.mark.parametrize("dtype,W,prefill", [
    (torch.bfloat16, 64, 10),    # fast path, filling
    (torch.bfloat16, 64, 70),    # fast path, wrapped
    (torch.float32, 16, 20),     # exact path
])
def test_decode_count_matches_window_rows(dev, dtype, W, prefill):
    from bozo_amd import TensionDecodeCache
    N, H, D, S = 2, 3, 64, 8
    L = prefill + S
    q, k, v = (t.to(dtype) for t in seq_inputs(N, L, H, D, seed=7 + W))
    cache = TensionDecodeCache(N, H, D, W, dtype=dtype, device=dev)
    for t in range(prefill):
        cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), normalize="count")
    msg, _ = O.window_forward(f64(q), f64(k), f64(v), W, math.sqrt(D))
    ref = O.normalize_count(msg, W)
    for t in range(prefill, L):
        out = cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), normalize="count")
        torch.cuda.synchronize()
        if dtype == torch.float32:
            assert max_abs(f64(out), ref[:, t]) <= 1e-5
        else:
            assert rel_l2(f64(out), ref[:, t]) <= 2e-2


@pytest.mark.parametrize("W,prefill", [(64, 64), (64, 5), (256, 260), (100, 7), (1024, 1030), (32, 3)])
@pytest.mark.parametrize("normalize", ["mass", "count"])
def test_decode_fp32_qk_bf16_v(dev, W, prefill, normalize):
    """The reference's autocast flow in generation: float32 (RoPE-promoted)
    q / K cache with a bf16 V cache -- the float32-K fast kernel; out and tau
    float32, held to max-abs 1e-5."""
    from bozo_amd import TensionDecodeCache
    N, H, D, S = 3, 4, 64, 6
    L = prefill + S
    q, k, v = seq_inputs(N, L, H, D, seed=W + prefill + 5)
    v = v.to(torch.bfloat16)
    cache = TensionDecodeCache(N, H, D, W, dtype=torch.float32, device=dev, v_dtype=torch.bfloat16)
    for t in range(prefill):
        cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), normalize=normalize)
    msg, tau = O.window_forward(f64(q), f64(k), f64(v), W, math.sqrt(D))
    ref = O.normalize_mass(msg, tau)[0] if normalize == "mass" else O.normalize_count(msg, W)
    for t in range(prefill, L):
        out, tt = cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), normalize=normalize,
                             return_tau=True)
        torch.cuda.synchronize()
        assert out.dtype == torch.float32 and tt.dtype == torch.float32
        assert max_abs(f64(out), ref[:, t]) <= 1e-5, (t, max_abs(f64(out), ref[:, t]))
        assert max_abs(f64(tt), tau[:, t]) <= 1e-5
    kd = cache.k[:, :, (L - 1) % W].cpu()
    assert torch.equal(kd, k[:, L - 1])  # the append keeps float32 keys exactly


@pytest.mark.parametrize("dtype,W,prefill", [
    (torch.bfloat16, 1024, 1000),  # fast path, 16 passes, nearly full
    (torch.bfloat16, 1024, 0),     # fast path, empty cache: the first rows are self only
    (torch.bfloat16, 300, 150),    # fast path, 8 passes
    (torch.bfloat16, 64, 3),       # fast path, one pass
    (torch.float32, 40, 20),       # exact path
    (torch.float16, 1024, 700),    # fast path, float16, 16 passes
])
def test_decode_self_matches_global_rows(dev, dtype, W, prefill):
    """include_self over a cache that holds every earlier token is the global
    block (keys s <= t), row by row."""
    from bozo_amd import TensionDecodeCache
    N, H, D, S = 2, 2, 64, 8
    L = prefill + S
    assert L <= W
    q, k, v = (t.to(dtype) for t in seq_inputs(N, L, H, D, seed=11 + W))
    cache = TensionDecodeCache(N, H, D, W, dtype=dtype, device=dev)
    cache.k[:, :, :prefill] = k[:, :prefill].permute(0, 2, 1, 3).to(dev)
    cache.v[:, :, :prefill] = v[:, :prefill].permute(0, 2, 1, 3).to(dev)
    cache.pos[cache.cur].fill_(prefill)
    ref, _, _ = O.global_forward(f64(q), f64(k), f64(v), math.sqrt(D))
    for t in range(prefill, L):
        out = cache.step(q[:, t].to(dev), k[:, t].to(dev), v[:, t].to(dev), include_self=True)
        torch.cuda.synchronize()
        if dtype == torch.float32:
            assert max_abs(f64(out), ref[:, t]) <= 1e-5
        else:
            assert rel_l2(f64(out), ref[:, t]) <= 2e-2
    assert torch.equal(cache.k[:, :, prefill:L].cpu(), k[:, prefill:L].permute(0, 2, 1, 3))
    with pytest.raises(Exception, match="not supported"):
        cache.step(q[:, 0].to(dev), k[:, 0].to(dev), v[:, 0].to(dev), include_self=True,
                   return_tau=True)


def test_decode_config4_shape_steps(dev):
    """BASELINE config 4 shape (64 seqs, H16, d64, W256 bf16): cache
    pre-filled with W tokens, then steps checked against the oracle's
    decode_step on the same ring contents."""
    from bozo_amd import decode_step
    N, H, D, W, S = 64, 16, 64, 256, 4
    g = torch.Generator().manual_seed(3)
    kc = (torch.randn(N, H, W, D, generator=g) * 0.5).to(torch.bfloat16)
    vc = (torch.randn(N, H, W, D, generator=g) * 0.5).to(torch.bfloat16)
    kd, vd = kc.to(dev), vc.to(dev)
    pos = torch.full((N,), W, dtype=torch.int32)
    pin, pout = pos.to(dev), torch.empty(N, dtype=torch.int32, device=dev)
    for s in range(S):
        q, kn, vn = ((torch.randn(N, H, D, generator=g) * 0.5).to(torch.bfloat16) for _ in range(3))
        tau = torch.empty(N, H, W, dtype=torch.bfloat16, device=dev)
        out = decode_step(q.to(dev), kn.to(dev), vn.to(dev), kd, vd, pin, pout, 8.0, True, tau)
        ro, rt = O.decode_step(f64(q), f64(kc), f64(vc), pos.numpy(), W, 8.0)
        assert rel_l2(f64(out), ro) <= 2e-2
        assert max_abs(f64(tau), rt) <= 4e-3
        kc_np, vc_np, pos_np = O.decode_append(kc.float().numpy(), vc.float().numpy(), pos.numpy(),
                                               kn.float().numpy(), vn.float().numpy(), W)
        kc, vc = torch.from_numpy(kc_np).to(torch.bfloat16), torch.from_numpy(vc_np).to(torch.bfloat16)
        pos = torch.from_numpy(pos_np.astype(np.int32))
        assert torch.equal(kd.cpu(), kc) and torch.equal(vd.cpu(), vc)
        assert torch.equal(pout.cpu(), pos)
        pin, pout = pout, pin


def test_decode_strided_views(dev):
    """Caches and rows as views with padding (the kernel reads strides, not
    shapes): caches sliced from [N, H + 1, W, D + 8] storage, q / k_new /
    v_new rows from [N, H, D + 16]; the fast kernel's 32-bit strides and
    the ring append land on the views, checked against the oracle."""
    from bozo_amd import decode_step
    N, H, D, W, S = 8, 4, 64, 96, 3
    g = torch.Generator().manual_seed(21)
    kbig = (torch.randn(N, H + 1, W, D + 8, generator=g) * 0.5).to(torch.bfloat16)
    vbig = (torch.randn(N, H + 1, W, D + 8, generator=g) * 0.5).to(torch.bfloat16)
    kbd, vbd = kbig.to(dev), vbig.to(dev)
    kd, vd = kbd[:, 1:, :, :D], vbd[:, 1:, :, :D]
    assert kd.stride() == ((H + 1) * W * (D + 8), W * (D + 8), D + 8, 1)
    kc, vc = kbig[:, 1:, :, :D].contiguous(), vbig[:, 1:, :, :D].contiguous()
    pos = torch.tensor([0, 1, 50, 95, 96, 97, 200, 7], dtype=torch.int32)
    pin, pout = pos.to(dev), torch.empty(N, dtype=torch.int32, device=dev)
    for s in range(S):
        rows = [(torch.randn(N, H, D + 16, generator=g) * 0.5).to(torch.bfloat16) for _ in range(3)]
        q, kn, vn = (r[:, :, 8:8 + D] for r in rows)
        qd, knd, vnd = (r.to(dev)[:, :, 8:8 + D] for r in rows)
        assert qd.stride(1) == D + 16
        tau = torch.empty(N, H, W, dtype=torch.bfloat16, device=dev)
        out = decode_step(qd, knd, vnd, kd, vd, pin, pout, 8.0, True, tau)
        ro, rt = O.decode_step(f64(q), f64(kc), f64(vc), pos.numpy(), W, 8.0)
        assert rel_l2(f64(out), ro) <= 2e-2
        assert max_abs(f64(tau), rt) <= 4e-3
        kc_np, vc_np, pos_np = O.decode_append(kc.float().numpy(), vc.float().numpy(), pos.numpy(),
                                               kn.float().numpy(), vn.float().numpy(), W)
        kc, vc = torch.from_numpy(kc_np).to(torch.bfloat16), torch.from_numpy(vc_np).to(torch.bfloat16)
        pos = torch.from_numpy(pos_np.astype(np.int32))
        assert torch.equal(kd.cpu(), kc) and torch.equal(vd.cpu(), vc)
        assert torch.equal(pout.cpu(), pos)
        pin, pout = pout, pin
    # the padding around the views is untouched
    assert torch.equal(kbd[:, 0].cpu(), kbig[:, 0]) and torch.equal(kbd[..., D:].cpu(), kbig[..., D:])


@pytest.mark.parametrize("dtype,out_dtype", [(torch.float32, None), (torch.bfloat16, torch.float32),
                                             (torch.float64, None), (torch.bfloat16, None)])
def test_rope(dev, dtype, out_dtype):
    from bozo_amd import rope
    B, T, H, D = 2, 50, 3, 64
    cos, sin = O.rope_tables(128, D)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, T, H, D, generator=g).to(dtype)
    xd = x.to(dev).requires_grad_(True)
    y = rope(xd, torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev), pos_offset=7,
             out_dtype=out_dtype)
    dy = torch.randn(B, T, H, D, generator=g)
    (y.double() * dy.to(dev).double()).sum().backward()
    want = O.rope_apply(f64(x), cos, sin, pos_offset=7)
    dwant = O.rope_apply_adjoint(dy.double().numpy(), cos, sin, pos_offset=7)
    assert y.dtype == (out_dtype or dtype)
    if y.dtype == torch.bfloat16:  # the 16-byte kernel: one bf16 rounding of the fp32 result
        assert np.max(np.abs(f64(y) - want) / np.maximum(np.abs(want), 1e-3)) <= 2 ** -8
    else:
        assert max_abs(f64(y), want) <= 1e-5
    tol = 1e-5 if dtype != torch.bfloat16 else 2e-2
    metric = max_abs if dtype != torch.bfloat16 else rel_l2
    assert metric(f64(xd.grad), dwant) <= tol


@pytest.mark.parametrize("D,dtype,out_dtype", [(32, torch.bfloat16, torch.float32), (48, torch.float32, None),
                                               (40, torch.bfloat16, torch.float32), (16, torch.float32, torch.bfloat16)])
def test_rope_head_dims(dev, D, dtype, out_dtype):
    """RoPE on the 16-byte path (D a multiple of 16: 32, 48, 16) and the
    generic one (D = 40), each dtype pair, forward and adjoint against the
    float64 restatement of model.py:75-81."""
    from bozo_amd import rope
    B, T, H = 2, 37, 3
    cos, sin = O.rope_tables(64, D)
    g = torch.Generator().manual_seed(D)
    x = torch.randn(B, T, H, D, generator=g).to(dtype)
    xd = x.to(dev).requires_grad_(True)
    y = rope(xd, torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev), pos_offset=5, out_dtype=out_dtype)
    dy = torch.randn(B, T, H, D, generator=g).to(y.dtype)
    (y.double() * dy.to(dev).double()).sum().backward()
    want = O.rope_apply(f64(x), cos, sin, pos_offset=5)
    dwant = O.rope_apply_adjoint(f64(dy), cos, sin, pos_offset=5)
    assert y.dtype == (out_dtype or dtype)
    if y.dtype == torch.bfloat16:
        assert np.max(np.abs(f64(y) - want) / np.maximum(np.abs(want), 1e-3)) <= 2 ** -8
    else:
        assert max_abs(f64(y), want) <= 1e-5
    if dtype == torch.bfloat16:
        assert rel_l2(f64(xd.grad), dwant) <= 2e-2
    else:
        assert max_abs(f64(xd.grad), dwant) <= 1e-5


def test_decode_config4_graph_replay_wraps(dev):
    """Config 4 through the path bench.py times: ``TensionDecodeCache.step``
    (position counters double-buffered on the device) captured 320 times in
    one HIP graph over a cache pre-filled with W = 256 tokens, then replayed.
    The ring wraps past its 256 slots; eight sequences are checked at every
    step against the oracle's decode_step over its decode_append ring, and
    the whole cache and counters after the replay against the known appends.
    The graph is replayed a second time from a restored state: same bits."""
    from bozo_amd import TensionDecodeCache
    N, H, D, W, S = 64, 16, 64, 256, 320
    sel = [0, 9, 17, 30, 41, 50, 58, 63]
    g = torch.Generator().manual_seed(3)
    kc = (torch.randn(N, H, W, D, generator=g) * 0.5).to(torch.bfloat16)
    vc = (torch.randn(N, H, W, D, generator=g) * 0.5).to(torch.bfloat16)
    q, k, v = ((torch.randn(S, N, H, D, generator=g) * 0.5).to(torch.bfloat16) for _ in range(3))
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    cache = TensionDecodeCache(N, H, D, W, dtype=torch.bfloat16, device=dev)

    def reset():
        cache.k.copy_(kc.to(dev))
        cache.v.copy_(vc.to(dev))
        cache.pos[0].fill_(W)
        cache.pos[1].fill_(-1)
        cache.cur = 0

    # one eager step on a scratch cache loads the library before capture
    scratch = TensionDecodeCache(N, H, D, W, dtype=torch.bfloat16, device=dev)
    scratch.step(qd[0], kd[0], vd[0])
    reset()
    torch.cuda.synchronize()
    print(f"[decode graph] capturing {S} steps", flush=True)
    graph = torch.cuda.CUDAGraph()
    outs = []
    with torch.cuda.graph(graph):
        for i in range(S):
            outs.append(cache.step(qd[i], kd[i], vd[i]))
    assert cache.cur == 0  # an even number of steps: the counters end in pos[0]
    reset()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    first = [o.clone() for o in outs]

    kc_s, vc_s = kc[sel].float().numpy(), vc[sel].float().numpy()
    pos = np.full(len(sel), W, dtype=np.int64)
    worst = 0.0
    for i in range(S):
        ro, _ = O.decode_step(q[i, sel].float().numpy(), kc_s, vc_s, pos, W, 8.0)
        worst = max(worst, rel_l2(f64(first[i][sel]), ro))
        assert rel_l2(f64(first[i][sel]), ro) <= 2e-2, (i, rel_l2(f64(first[i][sel]), ro))
        kc_s, vc_s, pos = O.decode_append(kc_s, vc_s, pos, k[i, sel].float().numpy(),
                                          v[i, sel].float().numpy(), W)
    print(f"  worst per-step rel L2 over {S} steps: {worst:.3e}", flush=True)
    # the ring after S appends: slot (W + i) % W holds step i's row for the last W steps
    want_k, want_v = kc.clone(), vc.clone()
    for i in range(S):
        want_k[:, :, (W + i) % W] = k[i]
        want_v[:, :, (W + i) % W] = v[i]
    assert torch.equal(cache.k.cpu(), want_k) and torch.equal(cache.v.cpu(), want_v)
    assert torch.equal(cache.pos[0].cpu(), torch.full((N,), W + S, dtype=torch.int32))
    reset()
    graph.replay()
    torch.cuda.synchronize()
    for i in range(S):
        assert torch.equal(outs[i], first[i]), i
