"""Benchmark of the MI355X sigmoid-tension hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-traffic]

Workload (the 117M-model shape the metric is quoted
on): windowed tension fwd+bwd, B=8 H=12 T=1024 d=64 W=64, bf16 storage with
fp32 accumulation, Q/K/V ~ 0.5 N(0,1) with RoPE (base 10000) on Q/K, upstream
grad ~ N(0,1), tau-mass normalised output (the north star's
out = sum tau v / sum tau), tau not materialised.  One step = forward +
backward (dQ, dK, dV) of one batch.

Method: NSETS independent input sets (more than the 256 MB Infinity Cache
in total) are generated on the GPU and rotated, so every step reads its
inputs from HBM.  The steps (1 forward + 1 fused backward kernel each,
launched through the public autograd op) are captured in HIP graphs, NSETS steps per
graph; the timed region runs exactly K steps between two events after a
synchronize.  Each kernel is then timed alone the same way (graphs of its
launches over the rotated sets, on the same stream) for the roofline entry;
``rocprofv3 --kernel-trace --marker-trace --stats`` of this command, read
back with ``--summarize``, gives the per-kernel durations in profiles/.

HBM traffic (``roofline.traffic``) is measured in the same run: two
``rocprofv3 --pmc`` passes (FETCH_SIZE, then WRITE_SIZE) over this script's
``--profile-kernels`` driver run as child processes, each counter calibrated
by the driver's 256 MiB device copy (``--no-traffic`` skips them; the field
is then null).

The CPU baseline times the reference's CPU path (unfold gather + tau-mass +
autograd, restated in oracle/torch_ref.py) in float32 on the host cores, on
a bounded sample (one of the 8 sequences, repeated for ~10 s).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
NSETS = 8                      # 8 x 50 MB of inputs > 256 MB Infinity Cache
METRIC = "tension fwd+bwd tokens/s at 117M shape (T=1024,W=64); % MFMA/HBM roofline"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def pairs_window(B, H, T, W):
    """Valid (query, key) pairs of the local band."""
    full = max(0, T - W) * W
    ramp = sum(min(t, W) for t in range(min(T, W)))
    return B * H * (full + ramp)


def rope_tables(T, D, dev):
    half = D // 2
    theta = 1.0 / (10000 ** (torch.arange(0, half).float() / half))
    freqs = torch.outer(torch.arange(T).float(), theta)
    return freqs.cos().to(dev), freqs.sin().to(dev)


def make_window_sets(n, B, T, H, D, dev, seed):
    from bozo_amd import rope
    cos, sin = rope_tables(T, D, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    sets = []
    for _ in range(n):
        q = torch.randn(B, T, H, D, device=dev, generator=g) * 0.5
        k = torch.randn(B, T, H, D, device=dev, generator=g) * 0.5
        v = torch.randn(B, T, H, D, device=dev, generator=g) * 0.5
        do = torch.randn(B, T, H, D, device=dev, generator=g)
        s = dict(Q=rope(q, cos, sin, out_dtype=torch.bfloat16).detach().requires_grad_(True),
                 K=rope(k, cos, sin, out_dtype=torch.bfloat16).detach().requires_grad_(True),
                 V=v.to(torch.bfloat16).requires_grad_(True), dO=do.to(torch.bfloat16))
        sets.append(s)
    torch.cuda.synchronize()
    return sets


def capture(fns, warm=2):
    """One HIP graph that runs fns[0](), fns[1](), ... in order (eager warm-up
    on a side stream first, as graph capture requires)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warm):
            for fn in fns:
                fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in fns:
            fn()
    torch.cuda.synchronize()
    return g


class Runner:
    """Replays units of work (one step, or one kernel launch) over the
    rotated input sets.  `ring` runs one unit on each of the NSETS sets in a
    single graph, so the hipGraphLaunch cost is paid once per NSETS units;
    `singles[i]` runs the unit on set i alone (for counts that are not a
    multiple of NSETS)."""

    def __init__(self, fns, warm=2):
        self.ring = capture(fns, warm)
        self.singles = [capture([f], 0) for f in fns]
        self.n = len(fns)

    def run(self, units):
        for _ in range(units // self.n):
            self.ring.replay()
        for i in range(units % self.n):
            self.singles[i].replay()


def time_units(runner, units, warmup, phase):
    """ms per unit over exactly `units` units; the timed region runs inside a
    roctx range named `phase` (rocprofv3 --marker-trace attributes the kernel
    dispatches of the range to it)."""
    runner.run(warmup)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.nvtx.range_push(phase)
    e0.record()
    runner.run(units)
    e1.record()
    torch.cuda.synchronize()
    torch.cuda.nvtx.range_pop()
    return e0.elapsed_time(e1) / units


def window_step_fn(s, W, scale, normalize, return_tau=False):
    from bozo_amd import causal_tension

    def fn():
        if return_tau:
            out, tau = causal_tension(s["Q"], s["K"], s["V"], W, scale, return_tau=True,
                                      normalize=normalize)
            return torch.autograd.grad((out, tau), (s["Q"], s["K"], s["V"]), (s["dO"], s["dTau"]))
        out = causal_tension(s["Q"], s["K"], s["V"], W, scale, normalize=normalize)
        return torch.autograd.grad(out, (s["Q"], s["K"], s["V"]), s["dO"])
    return fn


def kernel_fns(s, W, scale, flags):
    """One launch of each band kernel on set s, through C ABI entry points
    that launch exactly one kernel each: the forward, the fused backward
    (tension_window_bwd for W <= 64), and the split backward's dQ and dK/dV
    kernels (used for wider windows and the global block)."""
    from bozo_amd import _lib as L
    B, T, H, D = s["Q"].shape
    Q, K, V, dO = (s[n].detach() for n in ("Q", "K", "V", "dO"))
    out = torch.empty_like(Q)
    dq, dk, dv = torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)
    ws = torch.empty(max(1, L.lib().tension_window_bwd_workspace(B, T, H, L.F32, flags)),
                     dtype=torch.uint8, device=Q.device)
    lib = L.lib()
    bq, bk, bv, bo, bdo = (L.buf(t) for t in (Q, K, V, out, dO))
    bdq, bdk, bdv = L.buf(dq), L.buf(dk), L.buf(dv)
    # the ctypes buffers hold raw pointers only: every closure references
    # `keep`, so the tensors live as long as any launcher does (graph
    # capture empties torch's cache, which would unmap freed outputs)
    keep = (Q, K, V, dO, out, dq, dk, dv, ws)

    def fwd():
        _ = keep  # holds the tensors behind the raw pointers
        L.check(lib.tension_window_fwd(bq, bk, bv, bo, None, None, None, B, T, H, D, W, scale, flags,
                                       L.stream_handle()), "fwd")

    def dqf():
        _ = keep  # holds the tensors behind the raw pointers
        L.check(lib.tension_window_bwd_dq(bq, bk, bv, bdo, None, None, bdq, ws.data_ptr(),
                                          B, T, H, D, W, scale, flags, L.stream_handle()), "dq")

    def dkvf():
        _ = keep  # holds the tensors behind the raw pointers
        L.check(lib.tension_window_bwd_dkv(bq, bk, bv, bdo, None, None, bdk, bdv, ws.data_ptr(),
                                           B, T, H, D, W, scale, flags, L.stream_handle()), "dkv")

    def bwdf():
        _ = keep  # holds the tensors behind the raw pointers
        L.check(lib.tension_window_bwd(bq, bk, bv, bdo, None, None, bdq, bdk, bdv, ws.data_ptr(),
                                       B, T, H, D, W, scale, flags, L.stream_handle()), "bwd")
    return {"fwd": fwd, "bwd": bwdf, "dq": dqf, "dkv": dkvf}, keep


def kernel_bytes(B, T, H, D, W, el=2):
    """Algorithmic (compulsory) HBM bytes per launch of each kernel of the
    tau-mass-normalised step: every tensor the kernel must touch, once."""
    act = B * T * H * D * el           # one [B,T,H,D] bf16 tensor
    vec = B * T * H * 4                # one [B,T,H] fp32 tensor
    return {
        "fwd": 3 * act + act,                    # Q,K,V -> out
        "bwd": 4 * act + 3 * act,                # Q,K,V,dO -> dQ,dK,dV (fused)
        "dq": 4 * act + act + 2 * vec,           # Q,K,V,dO -> dQ, ws(a,c)
        "dkv": 4 * act + 2 * vec + 2 * act,      # Q,K,V,dO,ws -> dK,dV
    }


def host_cpus():
    """The host's CPUs as this process sees them: os.cpu_count(), the CPUs
    it may run on (affinity), the cgroup CPU quota, the CPU model, and the
    thread count the CPU baselines use -- every CPU the process can use
    (os.cpu_count() when nothing restricts it, as the reference's timing
    recipe sets torch.set_num_threads(os.cpu_count())), no more than the
    quota and the OMP_NUM_THREADS share the GPU box assigns to one GPU."""
    total = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = total
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
            if q != "max":
                quota = float(q) / float(per)
    except (OSError, ValueError):
        pass
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    threads = affinity
    if quota is not None:
        threads = min(threads, max(1, int(quota)))
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit() and int(share) > 0:
        threads = min(threads, int(share))
    return {"cpu_count": total, "affinity": affinity, "cgroup_quota": quota, "model": model,
            "threads": max(1, threads)}


def cpu_baseline(B, T, H, D, W, seconds=10.0):
    """Reference CPU path (unfold + tau-mass + autograd, fp32) on the host."""
    from oracle import torch_ref as R
    hc = host_cpus()
    cores = hc["threads"]
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(1)
    b = 1  # bounded sample: one sequence of the batch
    q, k, v = (torch.randn(b, T, H, D, generator=g) * 0.5 for _ in range(3))
    do = torch.randn(b, T, H, D, generator=g)

    def once():
        qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))
        msg, tau = R.unfold_tension(qq, kk, vv, W, math.sqrt(D), return_tau=True)
        out = R.normalize_mass(msg, tau)
        torch.autograd.grad(out, (qq, kk, vv), do)

    once()
    n, t0 = 0, time.perf_counter()
    while True:
        once()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 200:
            break
    return {"value": round(b * T * n / el, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "host": {k: hc[k] for k in ("model", "cpu_count", "affinity", "cgroup_quota")},
            "sample": f"{n} fwd+bwd passes of 1 sequence (T={T}, H={H}, d={D}, W={W}) fp32, "
                      f"unfold+tau-mass+autograd (oracle/torch_ref.py), {el:.1f} s on {cores} threads "
                      f"of {hc['model']} (os.cpu_count()={hc['cpu_count']})"}


class _ReferenceCpuOps:
    """Swap the model's tension ops for the reference's CPU path (unfold +
    normalisation, einsum global block, torch RoPE; oracle/torch_ref.py) for
    the CPU baselines of the model rows."""

    def __enter__(self):
        from bozo_amd import model as M
        from oracle import torch_ref as R

        def ct(Q, K, V, window, scale, return_tau=False, bias=None, *, normalize=None):
            raw, tau = R.unfold_tension(Q, K, V, window, scale, return_tau=True, bias=bias)
            if normalize == "mass":
                raw = R.normalize_mass(raw, tau)
            elif normalize == "count":
                raw = R.normalize_count(raw, window)
            return (raw, tau) if return_tau else raw

        def gt(Q, K, V, scale, bias=None, W_local=None):
            out, tl = R.global_block(Q, K, V, scale, bias=bias, W_local=W_local)
            return (out, tl) if W_local is not None else out

        self.M, self.saved = M, (M.causal_tension, M.global_tension, M.rope)
        M.causal_tension, M.global_tension = ct, gt
        M.rope = lambda x, cos, sin, pos_offset=0, out_dtype=None: R.rope(x, cos, sin, pos_offset)
        return self

    def __exit__(self, *exc):
        self.M.causal_tension, self.M.global_tension, self.M.rope = self.saved


def cpu_model_baselines(seconds=10.0):
    """The reference's CPU path for the model rows, fp32 on the host cores:
    one 117M training step (CE + aux losses, AdamW) on one 1024-token
    sequence, and the reference's generation step (forward over a 512-token
    context for one new token)."""
    import torch.nn.functional as F
    from bozo_amd import model as M
    cores = host_cpus()["threads"]
    torch.set_num_threads(cores)
    cfg = M.config_117m(use_triton=False, dropout=0.0)
    torch.manual_seed(4)
    m = M.TensionLM(cfg)
    opt = M.configure_adamw(m)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (1, 1025), generator=g)
    res = {"cores": cores, "kind": "port"}
    with _ReferenceCpuOps():
        n, t0 = 0, time.perf_counter()
        while n < 1 or (time.perf_counter() - t0 < seconds / 2 and n < 5):
            lg, hid, taus = m(ids[:, :-1], return_all=True)
            loss = (F.cross_entropy(lg.reshape(-1, cfg.vocab_size), ids[0, 1:])
                    + 0.01 * M.manifold_closure_loss(hid) + 0.02 * M.tension_diversity_loss(taus, m.window_groups))
            loss.backward()
            torch.nn.utils.clip_grad_norm_(m.parameters(), 1.0)
            opt.step()
            opt.zero_grad(set_to_none=True)
            n += 1
        el = time.perf_counter() - t0
        res["train_tokens_per_s"] = round(1024 * n / el, 1)
        res["train_sample"] = f"{n} steps of 1 x 1024 tokens, {el:.1f} s"
        m.eval()
        n, t0 = 0, time.perf_counter()
        with torch.no_grad():
            while n < 1 or (time.perf_counter() - t0 < seconds / 2 and n < 20):
                m(ids[:, :512])[:, -1]
                n += 1
        el = time.perf_counter() - t0
        res["generate_ms_per_token"] = round(el * 1e3 / n, 1)
        res["generate_sample"] = f"{n} re-forwards of a 512-token context, {el:.1f} s"
    return res


def bench_window(args, dev):
    B, H, T, D, W = 8, 12, 1024, 64, 64
    scale = math.sqrt(D)
    tokens = B * T
    P = pairs_window(B, H, T, W)
    flops = (4 + 8) * D * P
    sets = make_window_sets(NSETS, B, T, H, D, dev, seed=1)

    log(f"[bench] capturing step graphs (B{B} H{H} T{T} d{D} W{W} bf16, tau-mass)")
    steps = Runner([window_step_fn(s, W, scale, "mass") for s in sets])
    ms = time_units(steps, args.steps, args.warmup, "step")
    log(f"[bench] fwd+bwd {ms * 1e3:.1f} us/step")

    # per-kernel durations (same stream, graph of one launch per set)
    from bozo_amd import _lib as L
    kfns, keep = [], []
    for s in sets:
        f, kp = kernel_fns(s, W, scale, L.NORM_MASS)
        kfns.append(f)
        keep.append(kp)
    kbytes = kernel_bytes(B, T, H, D, W)
    per_kernel = {}
    for name in ("fwd", "bwd", "dq", "dkv"):
        if name == "dkv":  # its workspace must hold what dq wrote
            for f in kfns:
                f["dq"]()
        kr = Runner([f[name] for f in kfns], warm=1)
        kms = time_units(kr, max(NSETS * 10, args.steps), NSETS, f"kernel:{name}")
        del kr
        per_kernel[name] = {"us": round(kms * 1e3, 2),
                            "alg_bytes": kbytes[name],
                            "GBps": round(kbytes[name] / (kms * 1e-3) / 1e9, 1)}
        log(f"[bench] kernel {name}: {kms * 1e3:.2f} us, {per_kernel[name]['GBps']} GB/s algorithmic")
    # the step runs fwd + fused bwd; dq/dkv are the split backward, reported
    # for comparison only
    dom = max(("fwd", "bwd"), key=lambda k: per_kernel[k]["us"])
    d = per_kernel[dom]
    kname = {"fwd": "mfma_fwd_ring", "bwd": "mfma_bwd_fused", "dq": "mfma_bwd_dq", "dkv": "mfma_bwd_dkv"}

    # compulsory HBM bytes of one fwd+bwd: read Q,K,V, write out; read Q,K,V,dO,
    # write dQ,dK,dV
    step_bytes = 11 * B * T * H * D * 2
    result = {
        "metric": METRIC,
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "windowed sigmoid-tension fwd+bwd, tau-mass normalised (config 2)",
                   "B": B, "H": H, "T": T, "head_dim": D, "window": W, "global_batch": B,
                   "seq_len": T, "parallelism": "none (1 GPU)", "input_sets_rotated": NSETS},
        "roofline": {"bound": "hbm", "kernel": kname[dom],
                     "achieved": d["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(d["GBps"] / HBM_PEAK_GBS, 4), "traffic": None},
        "step": {"alg_bytes": step_bytes,
                 "hbm_GBps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                 "hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                 "alg_flops": flops,
                 "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 2),
                 "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                 "kernels": per_kernel},
    }

    # secondary variants: raw contract, and tau materialised + dTau (export path)
    del steps
    raw = Runner([window_step_fn(s, W, scale, None) for s in sets])
    result["variants"] = {"raw_out_ms": round(time_units(raw, args.steps, args.warmup, "step:raw"), 5)}
    del raw
    g = torch.Generator(device=dev).manual_seed(7)
    for s in sets:
        s["dTau"] = (torch.randn(B, T, H, W, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    tau = Runner([window_step_fn(s, W, scale, "mass", return_tau=True) for s in sets])
    result["variants"]["tau_materialised_ms"] = round(
        time_units(tau, args.steps, args.warmup, "step:tau"), 5)
    del tau
    # the reference's autocast dtype flow: fp32 RoPE'd Q / K, bf16 V, fp32 out
    # and dOut (the split-operand kernels)
    mixed = []
    for s in sets:
        mixed.append(dict(Q=s["Q"].detach().float().requires_grad_(True),
                          K=s["K"].detach().float().requires_grad_(True),
                          V=s["V"], dO=s["dO"].float()))
    del sets
    mx = Runner([window_step_fn(s, W, scale, "mass") for s in mixed])
    result["variants"]["mixed_dtype_ms"] = round(time_units(mx, args.steps, args.warmup, "step:mixed"), 5)
    del mx, mixed
    return result


def bench_window_variants(dev, steps, warmup):
    """The local-window op at the reference's other shipped shapes, fwd+bwd
    per step over 4 rotated input sets, tau-mass normalised:
      * the 350M preset's local layer (train.py:246-256: B4, 16 heads of 64,
        T1024, W256) in the reference's autocast flow -- RoPE'd float32 Q / K,
        bf16 V, float32 out / dOut (the split kernels, three bf16 terms per
        float32 value) -- with and without tau + dTau (the aux-loss step),
        and in bf16 (the dedicated bf16 kernels, W > 64 split backward);
      * head dim 32 in bf16 (the reference's default model, model.py:33-36):
        BASELINE config 1's shape (B4 H4 T256 W32) and a 32-sequence batch
        at T1024;
      * the reference's float32 flow (no autocast: Q, K, V, out, dOut and
        every gradient float32; the split kernels with V as three terms
        too) at the 117M layer, the 350M local layer and head dim 32;
      * float16 throughout (two terms per value) at the 117M and 350M
        layers."""
    def sets_for(B, H, T, D, W, flow, n=4, seed=11):
        raw = make_window_sets(n, B, T, H, D, dev, seed=seed)
        g = torch.Generator(device=dev).manual_seed(seed + 1)
        out = []
        for s in raw:
            if flow in ("f32qk", "f32"):
                v = s["V"].detach().float().requires_grad_(True) if flow == "f32" else s["V"]
                s = dict(Q=s["Q"].detach().float().requires_grad_(True),
                         K=s["K"].detach().float().requires_grad_(True), V=v, dO=s["dO"].float())
            if flow == "f16":
                s = {k: s[k].detach().half().requires_grad_(k != "dO") for k in ("Q", "K", "V", "dO")}
            dt = {"bf16": torch.bfloat16, "f16": torch.float16}.get(flow, torch.float32)
            s["dTau"] = (torch.randn(B, T, H, W, device=dev, generator=g) * 0.1).to(dt)
            out.append(s)
        return out

    from bozo_amd import _lib as L
    rows = []
    for name, (B, H, T, D, W), flow, tau in (
            ("350m_local_autocast", (4, 16, 1024, 64, 256), "f32qk", False),
            ("350m_local_autocast_tau", (4, 16, 1024, 64, 256), "f32qk", True),
            ("350m_local_bf16", (4, 16, 1024, 64, 256), "bf16", False),
            ("117m_local_autocast", (8, 12, 1024, 64, 64), "f32qk", False),
            ("d32_bf16_config1", (4, 4, 256, 32, 32), "bf16", False),
            ("d32_bf16_b32_t1024", (32, 4, 1024, 32, 32), "bf16", False),
            ("d32_autocast_b32_t1024", (32, 4, 1024, 32, 32), "f32qk", False),
            ("117m_local_f32", (8, 12, 1024, 64, 64), "f32", False),
            ("350m_local_f32", (4, 16, 1024, 64, 256), "f32", False),
            ("d32_f32_b32_t1024", (32, 4, 1024, 32, 32), "f32", False),
            ("117m_local_f16", (8, 12, 1024, 64, 64), "f16", False),
            ("350m_local_f16", (4, 16, 1024, 64, 256), "f16", False)):
        sets = sets_for(B, H, T, D, W, flow)
        run = Runner([window_step_fn(s, W, math.sqrt(D), "mass", return_tau=tau) for s in sets])
        ms = time_units(run, max(steps, 40), warmup, f"variant:{name}")
        kernel = int(L.lib().tension_last_kernel())
        del run, sets
        el_qk = 2 if flow in ("bf16", "f16") else 4
        el_v = 4 if flow == "f32" else 2
        # compulsory bytes: fwd reads Q, K, V, writes out; bwd reads Q, K, V, dO,
        # writes dQ, dK, dV (out / dO / dQ / dK in Q's dtype, V / dV in V's)
        nel = B * T * H * D
        step_bytes = nel * (el_qk * 2 + el_v + el_qk) + nel * (el_qk * 2 + el_v + el_qk + el_qk * 2 + el_v)
        if tau:
            step_bytes += 2 * B * T * H * W * el_qk
        rows.append({"name": name, "B": B, "H": H, "T": T, "head_dim": D, "window": W,
                     "dtype_flow": {"f32qk": "fp32 Q/K/out/dOut, bf16 V/dV", "f32": "fp32 throughout",
                                    "bf16": "bf16", "f16": "fp16 throughout"}[flow],
                     "tau_and_dtau": tau, "ms_per_step": round(ms, 5),
                     "tokens_per_s": round(B * T / (ms * 1e-3), 1), "alg_bytes": step_bytes,
                     "hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "kernel_family": {0: "exact", 1: "mfma_bf16", 2: "split_bf16", 3: "split_f32",
                                       4: "split_f32v", 5: "split_f16"}.get(kernel)})
        log(f"[bench] variant {rows[-1]}")
    return {"config": "window op at the reference's other shipped shapes (350M preset W256, head dim 32) "
                      "and in its float32 flow (and float16)",
            "rows": rows}


def profile_kernels(n, dev):
    """Counter-collection driver (run under rocprofv3 --pmc): n eager launches
    of each band kernel on rotated config-2 sets (bf16, then fp32 Q / K with
    bf16 V, then fp32 throughout and fp16 throughout), of the split kernels
    at the 350M preset's W = 256 shape (bf16 and fp32 Q / K), n config-4
    decode steps
    over 4 rotated caches and n config-3 global forward + backward calls, then
    a plain device copy of
    known size (256 MiB read + 256 MiB written) whose FETCH_SIZE/WRITE_SIZE
    readings calibrate the counters into bytes."""
    from bozo_amd import _lib as L
    B, H, T, D, W = 8, 12, 1024, 64, 64
    sets = make_window_sets(NSETS, B, T, H, D, dev, seed=1)
    fns = [kernel_fns(s, W, math.sqrt(D), L.NORM_MASS) for s in sets]
    for name in ("fwd", "bwd", "dq", "dkv"):
        for i in range(n):
            fns[i % NSETS][0][name]()
        torch.cuda.synchronize()
    del fns
    # the reference's autocast dtype flow: fp32 (RoPE'd) Q / K, bf16 V, fp32
    # out / dOut (the split-operand kernels xb_fwd / xb_dq / xb_dkv)
    mixed = [dict(Q=s["Q"].detach().float(), K=s["K"].detach().float(), V=s["V"].detach(),
                  dO=s["dO"].float()) for s in sets[:2]]
    del sets
    fns = [kernel_fns(s, W, math.sqrt(D), L.NORM_MASS) for s in mixed]
    for name in ("fwd", "dq", "dkv"):
        for i in range(n):
            fns[i % 2][0][name]()
        torch.cuda.synchronize()
    del fns, mixed
    # config 2 in the float32 flow (fp32 Q / K / V, V as three terms too) and
    # in fp16 (two terms per value), valid-count normalised (one-pass dQ)
    base = make_window_sets(2, B, T, H, D, dev, seed=5)
    flows = [{k: s[k].detach().float() for k in ("Q", "K", "V", "dO")} for s in base]
    flows += [{k: s[k].detach().half() for k in ("Q", "K", "V", "dO")} for s in base]
    del base
    fns = [kernel_fns(s, W, math.sqrt(D), L.NORM_COUNT) for s in flows]
    for name in ("fwd", "dq", "dkv"):
        for i in range(n):
            fns[i % 2][0][name]()       # float32 throughout
            fns[2 + i % 2][0][name]()   # float16 throughout
        torch.cuda.synchronize()
    del fns, flows
    # the 350M preset's local layer (B4 H16 T1024 W256) on the split kernels,
    # bf16 and in the autocast flow, valid-count normalised (its CE-only step;
    # distinct kernel instances from the tau-mass config-2 ones above)
    wide = make_window_sets(2, 4, T, 16, D, dev, seed=11)
    wide += [dict(Q=s["Q"].detach().float(), K=s["K"].detach().float(), V=s["V"].detach(),
                  dO=s["dO"].float()) for s in wide]
    fns = [kernel_fns(s, 256, math.sqrt(D), L.NORM_COUNT) for s in wide]
    for name in ("fwd", "dq", "dkv"):
        for i in range(n):
            fns[i % 2][0][name]()       # bf16
            fns[2 + i % 2][0][name]()   # fp32 Q / K, bf16 V
        torch.cuda.synchronize()
    del fns, wide
    # config-4 decode steps over 4 rotated caches, fresh q / k / v per step
    from bozo_amd import TensionDecodeCache
    N, Hd, Wd, NC = 64, 16, 256, 4
    g = torch.Generator(device=dev).manual_seed(3)
    caches = []
    for _ in range(NC):
        c = TensionDecodeCache(N, Hd, D, Wd, dtype=torch.bfloat16, device=dev)
        c.k.normal_(0.0, 0.5, generator=g)  # in place: no device copies besides the calibration
        c.v.normal_(0.0, 0.5, generator=g)
        c.pos[c.cur].fill_(Wd)
        caches.append(c)
    qkv = [(torch.randn(n, N, Hd, D, device=dev, generator=g) * 0.5).to(torch.bfloat16) for _ in range(3)]
    torch.cuda.synchronize()
    for i in range(n):
        caches[i % NC].step(qkv[0][i], qkv[1][i], qkv[2][i])
    torch.cuda.synchronize()
    del caches, qkv
    # config-3 global block: n forward and n backward calls (the backward runs
    # gl_dq, which forms the tau-mass coefficients, and gl_dkv)
    Bg, Hg, Tg = 4, 12, 2048
    q, k, v, do = ((torch.randn(Bg, Tg, Hg, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
                   for _ in range(4))
    out, mass = torch.empty_like(q), torch.empty(Bg, Tg, Hg, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    lib = L.lib()
    ws = torch.empty(lib.tension_global_bwd_workspace(Bg, Tg, Hg, L.F32, 0), dtype=torch.uint8, device=dev)
    for _ in range(n):
        L.check(lib.tension_global_fwd(L.buf(q), L.buf(k), L.buf(v), L.buf(out), None, None, L.buf(mass),
                                       Bg, Tg, Hg, D, 0, 8.0, 0, L.stream_handle()), "global fwd")
        L.check(lib.tension_global_bwd(L.buf(q), L.buf(k), L.buf(v), L.buf(do), None, None, L.buf(out),
                                       L.buf(mass), L.buf(dq), L.buf(dk), L.buf(dv), ws.data_ptr(), Bg, Tg, Hg,
                                       D, 0, 8.0, 0, L.stream_handle()), "global bwd")
    torch.cuda.synchronize()
    del q, k, v, do, out, mass, dq, dk, dv, ws
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] profile-kernels: {n} launches each of fwd/bwd/dq/dkv, decode, global fwd/bwd; 4 copies of 256 MiB")


def _phase_regions(cur):
    """(name, start, end) of the roctx ranges bench.py pushes, from a rocpd db."""
    out = []
    try:
        rows = cur.execute("select e.extdata, r.start, r.end from rocpd_region r "
                           "join rocpd_event e on e.id = r.event_id").fetchall()
    except Exception:  # noqa: BLE001 - older/newer schema: fall back to one phase
        return out
    for ext, a, b in rows:
        try:
            msg = json.loads(ext or "{}").get("message", "")
        except ValueError:
            msg = ""
        if msg.startswith(("step", "kernel:", "variant:", "global", "decode", "model:")):
            out.append((msg, a, b))
    return out


def _collect(paths):
    """Kernel durations per phase and per-dispatch counter means from rocprofv3
    rocpd databases (the *_results.db of --kernel-trace [--marker-trace] or
    --pmc runs of this script)."""
    import glob
    import sqlite3
    import statistics
    dbs = []
    for path in paths:
        dbs += [path] if path.endswith(".db") else sorted(glob.glob(os.path.join(path, "**", "*.db"),
                                                                    recursive=True))
    durations = []  # (db, [(phase, {kernel: [us, ...]})])
    counters = {}   # counter -> kernel -> (mean value per dispatch, dispatches)
    for db in dbs:
        cur = sqlite3.connect(db).cursor()
        kern = cur.execute("select name, start, end from kernels").fetchall()
        pmc = cur.execute("select name, counter_name, avg(counter_value), count(*) from pmc_events "
                          "group by name, counter_name").fetchall()
        if pmc:
            for n, cn, v, cnt in pmc:
                counters.setdefault(cn, {})[n.split("(")[0]] = (v, cnt)
            # calibration copies: the largest copy dispatches (the 256 MiB copies;
            # smaller set-up copies would dilute the mean)
            for cn, in cur.execute("select distinct counter_name from pmc_events").fetchall():
                vals = [v for v, in cur.execute(
                    "select counter_value from pmc_events where counter_name = ? and name like ?",
                    (cn, "__amd_rocclr_copyBuffer%")).fetchall()]
                big = [v for v in vals if vals and v >= 0.5 * max(vals)]
                if big:
                    counters[cn]["__amd_rocclr_copyBuffer"] = (statistics.mean(big), len(big))
            continue
        if not kern:
            continue
        phases = _phase_regions(cur) or [("all", min(k[1] for k in kern), max(k[2] for k in kern))]
        per = []
        for pname, a, b in phases:
            by = {}
            for n, s0, s1 in kern:
                if s0 >= a and s1 <= b:
                    by.setdefault(n.split("(")[0], []).append((s1 - s0) / 1e3)
            per.append((pname, by))
        durations.append((db, per))
    return durations, counters


def hbm_traffic(counters):
    """Copy-calibrated HBM bytes per launch {kernel: (read, write)} from
    FETCH_SIZE / WRITE_SIZE (KiB per dispatch) readings, or {} without them."""
    copy = "__amd_rocclr_copyBuffer"
    fe, wr = counters.get("FETCH_SIZE", {}), counters.get("WRITE_SIZE", {})
    if copy not in fe or copy not in wr:
        return {}, None
    known_kib = 256 * 1024  # the profile driver copies 256 MiB
    sf, sw = known_kib / fe[copy][0], known_kib / wr[copy][0]
    out = {}
    for n in sorted(set(fe) & set(wr)):
        if n == copy or "tension::" not in n:
            continue
        out[n] = (fe[n][0] * sf * 1024, wr[n][0] * sw * 1024)
    return out, (sf, sw)


def summarize(paths):
    """Print per-phase kernel statistics, counters and calibrated HBM traffic."""
    import statistics
    durations, counters = _collect(paths)
    for db, per in durations:
        print(f"# kernel durations: {os.path.basename(os.path.dirname(db))}/{os.path.basename(db)}")
        print("| phase | kernel | dispatches | mean us | median us | min us | max us |")
        print("|---|---|---|---|---|---|---|")
        for pname, by in per:
            tot = sum(sum(x) for x in by.values())
            ten = sum(sum(x) for n, x in by.items() if "tension::" in n)
            print(f"| {pname} | (all kernels: {tot / 1e3:.2f} ms; tension kernels {ten / 1e3:.2f} ms = "
                  f"{ten / max(tot, 1e-9):.1%}) | {sum(len(x) for x in by.values())} | | | | |")
            for n, d in sorted(by.items(), key=lambda kv: -sum(kv[1])):
                if sum(d) < 0.01 * tot:
                    continue
                print(f"| {pname} | {n} | {len(d)} | {statistics.mean(d):.2f} | {statistics.median(d):.2f} "
                      f"| {min(d):.2f} | {max(d):.2f} |")
        print()
    if counters:
        print("# counters (KiB per dispatch for FETCH_SIZE / WRITE_SIZE)")
        print("| kernel | counter | mean per dispatch | dispatches |")
        print("|---|---|---|---|")
        for cn, by in counters.items():
            for n, (v, cnt) in by.items():
                print(f"| {n[:70]} | {cn} | {v:.1f} | {cnt} |")
        traffic, cal = hbm_traffic(counters)
        if cal:
            print(f"\ncopy-kernel calibration: FETCH_SIZE x{cal[0]:.3f}, WRITE_SIZE x{cal[1]:.3f}")
            print("\n| kernel | HBM read MB | HBM write MB | total MB per launch |")
            print("|---|---|---|---|")
            for n, (r, w) in traffic.items():
                print(f"| {n} | {r / 1e6:.2f} | {w / 1e6:.2f} | {(r + w) / 1e6:.2f} |")


def rocprof_passes(passes, n=16, timeout=240):
    """Run this script's --profile-kernels driver under rocprofv3 once per
    pass, as child processes on the same GPU: a pass is a tuple of counters
    (one --pmc run; each run stays within the per-block counter limits) or
    None (a --kernel-trace run).  Returns (durations, counters, error): the
    parsed results of _collect, or the reason nothing was measured."""
    import shutil
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(exe):
        return [], {}, "rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="bench_pmc_", dir="/tmp")
    env = dict(os.environ, TMPDIR="/tmp")
    for i, counters in enumerate(passes):
        what = "--pmc " + " ".join(counters) if counters else "--kernel-trace"
        cmd = [exe, *what.split(), "-d", os.path.join(tmp, f"pass{i}"), "-o", "run", "--",
               sys.executable, os.path.abspath(__file__), "--profile-kernels", str(n)]
        log(f"[bench] rocprofv3 {what} over --profile-kernels {n} ...")
        try:
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, env=env, cwd=ROOT)
        except subprocess.TimeoutExpired:
            shutil.rmtree(tmp, ignore_errors=True)
            return [], {}, f"rocprofv3 {what} timed out"
        # rocprofv3 itself may end with a segmentation fault after the program
        # finished and its results are whole; the results decide
        if r.returncode not in (0, -11, 139) or "profile-kernels:" not in (r.stdout + r.stderr):
            shutil.rmtree(tmp, ignore_errors=True)
            return [], {}, f"rocprofv3 {what} failed (rc {r.returncode})"
    try:
        durations, counters = _collect([tmp])
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return durations, counters, None


TRAFFIC_PASSES = (("FETCH_SIZE",), ("WRITE_SIZE",))
UTIL_PASS = ("MfmaUtil", "VALUBusy")  # SQ_VALU_MFMA_BUSY_CYCLES, SQ_ACTIVE_INST_VALU, GRBM_GUI_ACTIVE


def measure_traffic(n=16):
    """HBM bytes per launch and MFMA / VALU busy %, measured now: rocprofv3
    --pmc passes (FETCH_SIZE, WRITE_SIZE, MfmaUtil + VALUBusy) over the
    --profile-kernels driver, the byte counters calibrated by the driver's
    256 MiB device copy.  Returns ({kernel: bytes}, {kernel: (mfma %, valu %)},
    note)."""
    _, counters, err = rocprof_passes(TRAFFIC_PASSES + (UTIL_PASS,), n)
    if err:
        return {}, {}, err + ": traffic not measured"
    traffic, cal = hbm_traffic(counters)
    if not traffic:
        return {}, {}, "no calibrated FETCH_SIZE / WRITE_SIZE readings: traffic not measured"
    valu = counters.get("VALUBusy", {})
    util = {k: (round(v, 1), round(valu[k][0], 1) if k in valu else None)
            for k, (v, _) in counters.get("MfmaUtil", {}).items() if "tension::" in k}
    return ({k: int(r + w) for k, (r, w) in traffic.items()}, util,
            f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE / MfmaUtil+VALUBusy in this run, {n} launches per "
            f"kernel, bytes copy-calibrated x{cal[0]:.3f} / x{cal[1]:.3f}")


def kernel_counters(n=16):
    """Markdown table per tension kernel of the --profile-kernels driver:
    rocprofv3 kernel-trace mean duration, MFMA busy % (MfmaUtil: MFMA busy
    cycles over all SIMDs' active cycles), VALU busy %, copy-calibrated HBM
    traffic and GB/s over the 8 TB/s peak."""
    import statistics
    passes = (None,) + TRAFFIC_PASSES + (UTIL_PASS,)
    durations, counters, err = rocprof_passes(passes, n)
    if err:
        print(f"kernel counters not measured: {err}")
        return
    dur = {}
    for _, per in durations:
        for _, by in per:
            for k, d in by.items():
                dur.setdefault(k, []).extend(d)
    traffic, cal = hbm_traffic(counters)
    get = lambda cn, k: counters.get(cn, {}).get(k, (float("nan"), 0))[0]  # noqa: E731
    print(f"{n} launches per kernel; bytes calibrated x{cal[0]:.3f} (FETCH_SIZE) / x{cal[1]:.3f} "
          "(WRITE_SIZE) against the driver's 256 MiB copy\n")
    print("| kernel | launches | mean us | MFMA busy % | VALU busy % | HBM MB (read+write) | HBM GB/s "
          "| of 8 TB/s |")
    print("|---|---|---|---|---|---|---|---|")
    for k in sorted(dur, key=lambda k: -statistics.mean(dur[k])):
        if "tension::" not in k:
            continue
        us = statistics.mean(dur[k])
        rw = traffic.get(k)
        mb = (rw[0] + rw[1]) / 1e6 if rw else float("nan")
        gbs = mb * 1e6 / (us * 1e-6) / 1e9
        print(f"| {k} | {len(dur[k])} | {us:.2f} | {get('MfmaUtil', k):.1f} | {get('VALUBusy', k):.1f} "
              f"| {mb:.2f} | {gbs:.0f} | {gbs / HBM_PEAK_GBS:.1%} |")


def bench_global(dev, steps, warmup):
    """Config 3: global block B4 H12 T2048 d64 bf16, fwd+bwd (MFMA-bound),
    over 4 rotated input sets (4 x 50 MB of Q, K, V, dO plus their
    gradients and the forward's out: more than the 256 MB Infinity Cache)."""
    from bozo_amd import global_tension
    B, H, T, D = 4, 12, 2048, 64
    g = torch.Generator(device=dev).manual_seed(2)
    sets = []
    for _ in range(4):
        q, k, v = ((torch.randn(B, T, H, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
                   .requires_grad_(True) for _ in range(3))
        sets.append(dict(Q=q, K=k, V=v, dO=torch.randn(B, T, H, D, device=dev, generator=g)
                         .to(torch.bfloat16)))

    def step_fn(s):
        def fn():
            out = global_tension(s["Q"], s["K"], s["V"], math.sqrt(D))
            return torch.autograd.grad(out, (s["Q"], s["K"], s["V"]), s["dO"])
        return fn
    run = Runner([step_fn(s) for s in sets])
    ms = time_units(run, steps, warmup, "global")
    pairs = B * H * T * (T + 1) // 2
    flops = 12 * D * pairs
    return {"config": "global block B4 H12 T2048 d64 bf16 fwd+bwd, 4 rotated input sets (config 3)",
            "ms_per_step": round(ms, 4), "tokens_per_s": round(B * T / (ms * 1e-3), 1),
            "alg_flops": flops, "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 2),
            "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}


def bench_decode(dev, reps):
    """Config 4: streaming decode, 64 sequences x H16 x d64, W=256 bf16 ring
    caches pre-filled with W tokens.  Four independent caches (4 x 67 MB,
    more than the 256 MB Infinity Cache) are stepped in rotation so every
    step reads its cache from HBM; 512 steps are captured in one HIP graph."""
    from bozo_amd import TensionDecodeCache
    N, H, D, W, S, NC = 64, 16, 64, 256, 512, 4
    g = torch.Generator(device=dev).manual_seed(3)
    caches = []
    for _ in range(NC):
        cache = TensionDecodeCache(N, H, D, W, dtype=torch.bfloat16, device=dev)
        cache.k.copy_((torch.randn(N, H, W, D, device=dev, generator=g) * 0.5).to(torch.bfloat16))
        cache.v.copy_((torch.randn(N, H, W, D, device=dev, generator=g) * 0.5).to(torch.bfloat16))
        cache.pos[cache.cur].fill_(W)
        caches.append(cache)
    q, k, v = ((torch.randn(S, N, H, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
               for _ in range(3))
    run = Runner([lambda: [caches[i % NC].step(q[i], k[i], v[i]) for i in range(S)]], warm=1)
    ms = time_units(run, reps, 1, "decode") / S
    step_bytes = 2 * N * H * W * D * 2 + 4 * N * H * D * 2
    traffic = None  # filled in by main() from this run's counter passes
    return {"config": "decode 64 seqs H16 d64 W256 bf16, 4 rotated caches, 512 steps per graph (config 4)",
            "us_per_step": round(ms * 1e3, 3), "steps_per_s": round(1e3 / ms, 1),
            "alg_bytes_per_step": step_bytes,
            "GBps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": traffic}


def bench_model(dev, steps, warmup, aux, fast_rope=False, compiled=False):
    """Config 5: one TensionLM-117M training step (random init, bf16
    autocast, AdamW as train.py:894-902, clip 1.0) on B8 x T1024 token ids
    ~ U[0, 32768).  ``aux``: the reference default, return_all with tau
    emitted by every layer and the four aux losses computed (weights 0.01,
    0.02, 0, 0 as train.py:135-140 -- all four are evaluated there too; the
    three tau losses in the fused kernels); otherwise CE only (local layers
    on the valid-count path, no tau).  ``fast_rope``: rotated Q / K stay bf16
    (the bf16 kernels) instead of the reference's float32 promotion.
    ``compiled``: the model under torch.compile(dynamic=False,
    mode="default") as train.py:776-780 runs it (the tension kernels enter
    the graph as the bozo:: custom operators); compilation happens in the
    warmup steps."""
    import gc
    import torch.nn.functional as F
    from bozo_amd import model as M
    gc.collect()
    torch.cuda.empty_cache()  # blocks cached by the earlier benches would be split for this one
    cfg = M.config_117m(use_triton=True, fast_rope=fast_rope)
    torch.manual_seed(4)
    m = M.TensionLM(cfg).to(dev).train()
    opt = M.configure_adamw(m, lr=3e-4, weight_decay=0.1, fused=True)
    fwd = m
    if compiled:
        torch._dynamo.reset()
        fwd = torch.compile(m, dynamic=False, mode="default")
    t_c = time.perf_counter()
    B, T = 8, 1024
    g = torch.Generator(device=dev).manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (B, T + 1), device=dev, generator=g)
    inputs, targets = ids[:, :-1], ids[:, 1:]

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            if aux:
                logits, hidden, taus = fwd(inputs, return_all=True)
            else:
                logits = fwd(inputs)
            loss = F.cross_entropy(logits.reshape(-1, cfg.vocab_size), targets.reshape(-1))
            if aux:  # all four computed, as the reference does; the tau ones fused
                div, cons, ent = M.tension_aux_losses(taus, m.window_groups)
                loss = (loss + 0.01 * M.manifold_closure_loss(hidden) + 0.02 * div
                        + 0.0 * cons + 0.0 * ent)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(m.parameters(), 1.0)
        opt.step()
        opt.zero_grad(set_to_none=True)
        return loss

    for _ in range(warmup):
        loss = step()
    torch.cuda.synchronize()
    warm_s = time.perf_counter() - t_c
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    torch.cuda.nvtx.range_push("model:" + ("aux" if aux else "ce") + (":fast_rope" if fast_rope else "")
                               + (":compiled" if compiled else ""))
    e0.record()
    for _ in range(steps):
        loss = step()
    e1.record()
    torch.cuda.synchronize()
    torch.cuda.nvtx.range_pop()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ms = e0.elapsed_time(e1) / steps
    res = {"config": "TensionLM-117M training step B8 T1024 bf16 autocast AdamW (config 5), "
                     + ("aux losses + tau (reference default)" if aux else "CE only")
                     + (", bf16 Q/K (fast_rope)" if fast_rope else ", fp32 RoPE'd Q/K (reference dtype flow)")
                     + (", torch.compile (train.py:776-780)" if compiled else ", eager"),
           "ms_per_step": round(ms, 3), "wall_ms_per_step": round(wall, 3),
           "warmup_s": round(warm_s, 1),
           "tokens_per_s": round(B * T / (ms * 1e-3), 1), "params": m.num_params,
           "final_loss": round(float(loss.item()), 4)}
    del m, opt, fwd
    if compiled:
        torch._dynamo.reset()
    torch.cuda.empty_cache()
    return res


def bench_generation(dev, prompt=512, new=128):
    """TensionLM-117M generation, logits of one new token per sequence
    (sampling excluded), bf16 autocast, random init: the reference's method
    (re-running the forward over the context for every token, model.py:
    719-768) against the cached step on the decode kernel, eager and
    replayed from a HIP graph, for 1 and 64 sequences."""
    from bozo_amd import model as M
    from bozo_amd.generation import TensionKVCache
    cfg = M.config_117m(use_triton=True)
    torch.manual_seed(4)
    m = M.TensionLM(cfg).to(dev).eval()
    g = torch.Generator(device=dev).manual_seed(5)
    res = {"config": f"TensionLM-117M generation, prompt {prompt}, {new} new tokens, bf16 autocast, "
                     "logits only"}

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for i in range(n):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        ids = torch.randint(0, cfg.vocab_size, (64, prompt + new), device=dev, generator=g)
        m(ids[:1, :prompt])
        ms = timed(lambda i: m(ids[:1, :prompt + i + 1])[:, -1], 16)
        res["reforward_ms_per_token_n1"] = round(ms, 3)
        for N in (1, 64):
            for mode in ("eager", "graph"):
                cache = TensionKVCache(m, N)
                cache.prefill(ids[:N, :prompt])
                step = cache.step if mode == "eager" else cache.graph_step
                step(ids[:N, prompt])  # warm-up (and capture)
                ms = timed(lambda i: step(ids[:N, prompt + 1 + i]), new - 1)
                res[f"cached_{mode}_ms_per_step_n{N}"] = round(ms, 4)
                res[f"cached_{mode}_tokens_per_s_n{N}"] = round(N / (ms * 1e-3), 1)
                del cache
    del m
    torch.cuda.empty_cache()
    return res


def bench_export(dev, reps=20):
    """Tau export reductions at the 117M shape: 9 local layers of tau
    [1, 1024, 12, 64] bf16 (sigmoid of 2 N(0,1), a spread like a trained
    model's), per-head profile + head-masked aggregate + Gini + edge
    selection on the device, against the reference's host path (copy to the
    host, numpy reductions: oracle/export_ref.py) timed on this host."""
    from bozo_amd import export as E
    from oracle import export_ref as X
    Ln, B, T, H, W = 9, 1, 1024, 12, 64
    g = torch.Generator(device=dev).manual_seed(6)
    taus = [torch.sigmoid(torch.randn(B, T, H, W, device=dev, generator=g) * 2).to(torch.bfloat16)
            for _ in range(Ln)]
    mask = torch.zeros(Ln, H, dtype=torch.bool)
    mask[:, ::3] = True

    def device_path():
        st = E.head_stats(taus)
        agg = E.aggregate_tau(taus, mask)
        gini, mean = E.concentration(agg)
        emit = E._valid(T, W, dev) & (agg >= 0.6)
        return st, torch.nonzero(emit).cpu(), agg[emit].cpu()

    device_path()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        device_path()
    torch.cuda.synchronize()
    dev_ms = (time.perf_counter() - t0) * 1e3 / reps
    # the two kernels alone
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        E.head_stats(taus)
    e1.record()
    torch.cuda.synchronize()
    stats_us = e0.elapsed_time(e1) * 1e3 / reps
    e0.record()
    for _ in range(reps):
        E.aggregate_tau(taus, mask)
    e1.record()
    torch.cuda.synchronize()
    agg_us = e0.elapsed_time(e1) * 1e3 / reps

    t0 = time.perf_counter()
    n_cpu = 0
    while time.perf_counter() - t0 < 5.0 or n_cpu == 0:
        np_taus = [t.float().cpu().numpy() for t in taus]
        X.head_stats(np_taus)
        agg = X.aggregate(np_taus, mask.numpy())
        X.concentration(agg)
        X.edges(agg, 0.6)
        n_cpu += 1
    cpu_ms = (time.perf_counter() - t0) * 1e3 / n_cpu
    tau_bytes = Ln * B * T * H * W * 2
    return {"config": "tau export reductions, 9 layers x [1,1024,12,64] bf16 (117M shape)",
            "device_ms": round(dev_ms, 3), "head_stats_us": round(stats_us, 1),
            "aggregate_us": round(agg_us, 1),
            "aggregate_GBps": round(tau_bytes / (agg_us * 1e-6) / 1e9, 1),
            "cpu_reference_path_ms": round(cpu_ms, 1), "cpu_cores": 1}


def bench_bias(dev, n_edges=50000, T=1024, W=64):
    """Graph-bias builder: a 50k-edge content map, a 1024-token context,
    the [1, T, W] window bias and the [1, T, T] global bias built on the
    device (content ids on the host, one lookup kernel each), against the
    reference's Python loops (oracle/bias_ref.py) on this host."""
    import numpy as np
    from bozo_amd.bias import GraphBias
    from oracle import bias_ref as R

    class Tok:
        def id_to_token(self, i):
            return f"w{i}"

    r = np.random.default_rng(7)
    V = 4000
    src, dst = r.integers(0, V, n_edges), r.integers(0, V, n_edges)
    edge_map = {(f"w{a}", f"w{b}"): float(r.random()) for a, b in zip(src, dst)}
    ids = r.integers(0, V, T).tolist()
    gb = GraphBias(edge_map, alpha=0.5)
    tok = Tok()
    gb.local_bias(ids, tok, window=W, device=dev)  # table build + warm-up
    res = {"config": f"graph bias, {len(edge_map)} edges, T={T} W={W}"}
    for name, fn in (("local", lambda: gb.local_bias(ids, tok, window=W, device=dev)),
                     ("global", lambda: gb.global_bias(ids, tok, device=dev))):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        res[f"{name}_device_ms"] = round((time.perf_counter() - t0) * 1e2, 3)
    contents = [tok.id_to_token(i) for i in ids]
    t0 = time.perf_counter()
    R.local_bias(edge_map, 0.5, contents, W)
    res["local_cpu_reference_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
    t0 = time.perf_counter()
    R.global_bias(edge_map, 0.5, contents[:256])
    res["global_cpu_reference_ms_T256"] = round((time.perf_counter() - t0) * 1e3, 1)
    res["cpu_cores"] = 1
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc passes that measure HBM traffic")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--kernel-counters", type=int, default=0, metavar="N",
                    help="per-kernel table of duration, MFMA / VALU busy %%, counted MFMA TFLOP/s and HBM "
                         "traffic from rocprofv3 passes over --profile-kernels N")
    ap.add_argument("--profile-kernels", type=int, default=0, metavar="N",
                    help="only launch each band kernel N times (counter collection)")
    ap.add_argument("--summarize", metavar="PATH", nargs="+",
                    help="print per-phase kernel stats / calibrated traffic of rocprofv3 output "
                         "dirs or .db files and exit")
    ap.add_argument("--model-only", action="store_true",
                    help="only the TensionLM-117M training step (config 5), one JSON line per variant")
    ap.add_argument("--window-only", action="store_true",
                    help="only the config-2 step (with its variants) and the other window shapes")
    ap.add_argument("--generation-only", action="store_true",
                    help="only the cached-generation, tau-export and graph-bias timings")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every box has one GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.profile_kernels:
        profile_kernels(args.profile_kernels, dev)
        return
    if args.kernel_counters:
        kernel_counters(args.kernel_counters)
        return
    if args.generation_only:
        print(json.dumps(bench_generation(dev)), flush=True)
        print(json.dumps(bench_export(dev)), flush=True)
        print(json.dumps(bench_bias(dev)), flush=True)
        return
    if args.model_only:
        for compiled in (False, True):
            for fast in (False, True):
                for aux in (False, True):
                    log(f"[bench] config 5, aux={aux}, fast_rope={fast}, compiled={compiled} ...")
                    print(json.dumps(bench_model(dev, args.steps, args.warmup, aux, fast, compiled)),
                          flush=True)
        if not args.no_cpu:
            print(json.dumps({"cpu_model_baselines": cpu_model_baselines(args.cpu_seconds)}), flush=True)
        return
    result = bench_window(args, dev)
    log("[bench] window op at the other shipped shapes ...")
    variants = bench_window_variants(dev, 40, 5)
    if args.window_only:
        result["other_configs"] = [variants]
        print(json.dumps(result), flush=True)
        return
    log("[bench] global block (config 3) ...")
    others = [variants, bench_global(dev, 20, 3)]
    log(f"[bench] {others[-1]}")
    log("[bench] decode (config 4) ...")
    others.append(bench_decode(dev, 4))
    log(f"[bench] {others[-1]}")
    for fast, compiled in ((False, False), (True, False), (False, True)):
        for aux in (False, True):
            log(f"[bench] TensionLM-117M training step (config 5, aux={aux}, fast_rope={fast}, "
                f"compiled={compiled}) ...")
            others.append(bench_model(dev, 10, 5, aux, fast, compiled))
            log(f"[bench] {others[-1]}")
    log("[bench] tau export reductions ...")
    others.append(bench_export(dev))
    log(f"[bench] {others[-1]}")
    log("[bench] graph bias builder ...")
    others.append(bench_bias(dev))
    log(f"[bench] {others[-1]}")
    log("[bench] TensionLM-117M cached generation ...")
    others.append(bench_generation(dev))
    log(f"[bench] {others[-1]}")
    result["other_configs"] = others
    if not args.no_traffic:
        log("[bench] HBM traffic: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes ...")
        traffic, util, note = measure_traffic()
        pick = lambda key: next((v for k, v in traffic.items() if key in k), None)  # noqa: E731
        busy = lambda key: next((v for k, v in util.items() if key in k), None)  # noqa: E731
        result["roofline"]["traffic"] = pick({"mfma_bwd_fused": "mfma_bwd_fused<1, false, false, true>",
                                              "mfma_fwd_ring": "mfma_fwd_ring<1, false, false, true>"}
                                             [result["roofline"]["kernel"]])
        result["roofline"]["traffic_source"] = note
        for name, key in (("fwd", "mfma_fwd_ring<1, false, false, true>"),
                          ("bwd", "mfma_bwd_fused<1, false, false, true>")):
            result["step"]["kernels"][name]["traffic"] = pick(key)
            result["step"]["kernels"][name]["mfma_valu_busy_pct"] = busy(key)
        for o in others:
            if o["config"].startswith("decode"):
                o["traffic"] = pick("decode_bf16_d64")
            if o["config"].startswith("global block"):
                o["traffic"] = {k.split("::")[-1]: v for k, v in traffic.items()
                                if "gl_" in k or "coef_from_out" in k} or None
                o["mfma_valu_busy_pct"] = {k.split("::")[-1]: v for k, v in util.items() if "gl_" in k} or None
        log(f"[bench] traffic: {note}; {result['roofline']['traffic']} bytes per dominant launch")
    if not args.no_cpu:
        log("[bench] CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(1, 1024, 12, 64, 64, args.cpu_seconds)
        log("[bench] CPU baselines of the model rows ...")
        others.append({"config": "reference CPU path of the 117M model (fp32)",
                       **cpu_model_baselines(args.cpu_seconds)})
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
