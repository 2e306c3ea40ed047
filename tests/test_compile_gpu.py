"""The kernels as torch.library operators under torch.compile.

The reference compiles its model (train.py:776-780, dynamic=False, mode
"default").  Here the tension kernels enter a compiled graph as the bozo::
custom operators: torch.library.opcheck checks their schemas, fake
kernels and autograd registration against the real kernels; a full-graph
compile of causal_tension / global_tension / rope equals the eager call
bit for bit (the same kernels run, forward and backward); and the compiled
TensionLM (inductor, the reference's setting) gives the eager model's loss
and gradients within floating-point reassociation of the inductor-fused
elementwise work."""
import pytest
import torch
import torch.nn.functional as F

from bozo_amd import model as M
from bozo_amd.ops import causal_tension, global_tension, rope

pytestmark = pytest.mark.gpu


def qkv(B, T, H, D, dtype, dev, seed, requires_grad=False):
    g = torch.Generator(device="cpu").manual_seed(seed)
    ts = [(0.5 * torch.randn(B, T, H, D, generator=g)).to(dev, dtype) for _ in range(3)]
    return [t.requires_grad_(requires_grad) for t in ts]


@pytest.mark.parametrize("dtype,W,tau,flags,bias", [
    (torch.bfloat16, 64, True, 1, False),   # MFMA kernels, tau-mass
    (torch.bfloat16, 64, False, 2, False),  # MFMA, valid-count
    (torch.float32, 17, True, 0, True),     # split kernels (float32 flow), raw sum, bias
    (torch.float16, 100, True, 1, False),   # split kernels (float16), tau-mass, W > 64
    (torch.float64, 9, False, 1, False),    # exact kernels
])
def test_opcheck_window(dev, dtype, W, tau, flags, bias):
    B, T, H, D = 2, 200, 3, 64
    q, k, v = qkv(B, T, H, D, dtype, dev, 1, requires_grad=True)
    b = torch.randn(B, T, W, device=dev) if bias else None
    print(f"[opcheck window] {dtype} W={W} tau={tau} flags={flags} bias={bias}", flush=True)
    torch.library.opcheck(torch.ops.bozo.window_fwd.default, (q, k, v, W, 8.0, tau, b, flags))


@pytest.mark.parametrize("Wl", [0, 64])
def test_opcheck_global(dev, Wl):
    q, k, v = qkv(2, 150, 2, 64, torch.bfloat16, dev, 2, requires_grad=True)
    print(f"[opcheck global] Wl={Wl}", flush=True)
    torch.library.opcheck(torch.ops.bozo.global_fwd.default, (q, k, v, 8.0, None, Wl))


def test_opcheck_rope(dev):
    x = qkv(2, 50, 3, 64, torch.bfloat16, dev, 3, requires_grad=True)[0]
    m = M.RotaryEmbedding(64, 64).to(dev)
    print("[opcheck rope]", flush=True)
    torch.library.opcheck(torch.ops.bozo.rope.default, (x, m.cos, m.sin, 7, torch.float32, 0))


def run(fn, inputs, cot_seed=9):
    """Outputs and input gradients of fn under fixed random cotangents."""
    res = fn(*inputs)
    outs = res if isinstance(res, tuple) else (res,)
    g = torch.Generator(device="cpu").manual_seed(cot_seed)
    loss = sum((o.float() * torch.randn(o.shape, generator=g).to(o.device)).sum() for o in outs)
    grads = torch.autograd.grad(loss, inputs)
    return [o.detach() for o in outs], grads


def assert_same(a, b):
    for x, y in zip(a[0] + list(a[1]), b[0] + list(b[1])):
        assert torch.equal(x, y), (x - y).abs().max().item()


@pytest.mark.parametrize("dtype,normalize,tau", [(torch.bfloat16, "mass", True),
                                                 (torch.bfloat16, "count", False),
                                                 (torch.float32, None, True)])
def test_compiled_window_equals_eager(dev, dtype, normalize, tau):
    B, T, H, D, W = 2, 300, 4, 64, 64
    bias = torch.randn(B, T, W, device=dev)

    def fn(q, k, v):
        return causal_tension(q, k, v, W, 8.0, return_tau=tau, bias=bias, normalize=normalize)

    print(f"[compile window] {dtype} {normalize} tau={tau}", flush=True)
    torch._dynamo.reset()
    cfn = torch.compile(fn, backend="aot_eager", fullgraph=True, dynamic=False)
    eager = run(fn, qkv(B, T, H, D, dtype, dev, 4, True))
    comp = run(cfn, qkv(B, T, H, D, dtype, dev, 4, True))
    assert_same(eager, comp)


@pytest.mark.parametrize("W_local", [None, 64])
def test_compiled_global_equals_eager(dev, W_local):
    def fn(q, k, v):
        return global_tension(q, k, v, 8.0, W_local=W_local)

    print(f"[compile global] W_local={W_local}", flush=True)
    torch._dynamo.reset()
    cfn = torch.compile(fn, backend="aot_eager", fullgraph=True, dynamic=False)
    assert_same(run(fn, qkv(2, 260, 2, 64, torch.bfloat16, dev, 5, True)),
                run(cfn, qkv(2, 260, 2, 64, torch.bfloat16, dev, 5, True)))


def test_compiled_rope_equals_eager(dev):
    m = M.RotaryEmbedding(64, 128).to(dev)

    def fn(x):
        return rope(x, m.cos, m.sin, 3, out_dtype=torch.float32)

    torch._dynamo.reset()
    cfn = torch.compile(fn, backend="aot_eager", fullgraph=True, dynamic=False)
    assert_same(run(fn, qkv(2, 100, 3, 64, torch.bfloat16, dev, 6, True)[:1]),
                run(cfn, qkv(2, 100, 3, 64, torch.bfloat16, dev, 6, True)[:1]))


def test_dynamic_shapes_equal_eager(dev):
    """One dynamic-shape compile (symbolic T) serves several sequence lengths,
    ragged ones included; every call equals the eager op bit for bit."""
    W = 64

    def fn(q, k, v):
        out, tau = causal_tension(q, k, v, W, 8.0, return_tau=True, normalize="mass")
        return out, tau, global_tension(q, k, v, 8.0)

    torch._dynamo.reset()
    cfn = torch.compile(fn, backend="aot_eager", fullgraph=True, dynamic=True)
    for T in (130, 256, 333):
        print(f"[compile dynamic] T={T}", flush=True)
        assert_same(run(fn, qkv(2, T, 2, 64, torch.bfloat16, dev, T, True)),
                    run(cfn, qkv(2, T, 2, 64, torch.bfloat16, dev, T, True)))


@pytest.mark.timeout(600)
@pytest.mark.parametrize("autocast,aux", [(False, False), (True, False), (True, True)])
def test_compiled_model_step_matches_eager(dev, autocast, aux):
    """One training step of a small TensionLM compiled as train.py:776-780
    (inductor, dynamic=False, mode "default") against the eager model: the
    loss and every parameter gradient, fp32 to 1e-4 relative L2 (inductor
    reassociates the fused norm / SwiGLU arithmetic), bf16 autocast to
    2e-2."""
    cfg = M.TensionConfig(vocab_size=256, dim=128, num_layers=4, num_heads=2, window=64,
                          max_seq_len=256, dropout=0.0, global_every=2, use_rope=True,
                          use_triton=True)
    torch.manual_seed(7)
    m = M.TensionLM(cfg).to(dev).train()
    ids = torch.randint(0, cfg.vocab_size, (2, 201), generator=torch.Generator().manual_seed(8)).to(dev)
    x, y = ids[:, :-1], ids[:, 1:]

    def step(model):
        m.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            if aux:
                logits, hidden, taus = model(x, return_all=True)
            else:
                logits = model(x)
            loss = F.cross_entropy(logits.float().reshape(-1, cfg.vocab_size), y.reshape(-1))
            if aux:
                div, cons, ent = M.tension_aux_losses(taus, m.window_groups)
                loss = loss + 0.01 * M.manifold_closure_loss(hidden) + 0.02 * div + 0.1 * cons + 0.1 * ent
        loss.backward()
        return loss.item(), [p.grad.detach().clone() for p in m.parameters() if p.grad is not None]

    print(f"[compile model] autocast={autocast} aux={aux}", flush=True)
    le, ge = step(m)
    torch._dynamo.reset()
    cm = torch.compile(m, dynamic=False, mode="default", fullgraph=True)
    lc, gc = step(cm)
    lc2, gc2 = step(cm)  # a second call runs the cached graph
    tol = 2e-2 if autocast else 1e-4
    print(f"  loss eager {le:.6f} compiled {lc:.6f}", flush=True)
    assert abs(lc - le) <= tol * abs(le)
    assert abs(lc2 - lc) <= 1e-6 * abs(lc)
    for a, b, b2 in zip(ge, gc, gc2):
        for c in (b, b2):
            rel = ((a - c).norm() / a.norm().clamp_min(1e-30)).item()
            assert rel <= tol, rel
    torch._dynamo.reset()
