"""The torch.library registration of the kernels (bozo::window_fwd /
window_bwd, global_fwd / global_bwd, rope), CPU side: every operator is
registered with the schema the compiled path calls, and its fake-tensor
kernel gives the shapes and dtypes the real kernel writes (what torch.compile
traces the reference's compiled model with, train.py:776-780).  The GPU side
(opcheck and compiled-vs-eager equality) is in test_compile_gpu.py."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import bozo_amd  # noqa: F401  (registers the operators)


OPS = ("window_fwd", "window_bwd", "global_fwd", "global_bwd", "rope")


@pytest.mark.parametrize("name", OPS)
def test_registered(name):
    op = getattr(torch.ops.bozo, name).default
    assert not op._schema.is_mutable
    # every argument and return is a plain value or tensor, nothing aliased
    assert all(a.alias_info is None for a in op._schema.arguments)
    assert all(r.alias_info is None for r in op._schema.returns)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("return_tau", [False, True])
def test_window_fake_shapes(dtype, return_tau):
    with FakeTensorMode():
        q = torch.empty(2, 100, 3, 64, dtype=dtype, device="cuda")
        bias = torch.empty(2, 100, 17, device="cuda")
        out, tau = torch.ops.bozo.window_fwd(q, q, q, 17, 8.0, return_tau, bias, 1)
        assert out.shape == q.shape and out.dtype == dtype and out.device.type == "cuda"
        assert tau.shape == ((2, 100, 3, 17) if return_tau else (0,)) and tau.dtype == dtype
        dq, dk, dv = torch.ops.bozo.window_bwd(q, q, q, out, tau if return_tau else None, bias, 17, 8.0, 1)
        assert all(t.shape == q.shape and t.dtype == dtype for t in (dq, dk, dv))


@pytest.mark.parametrize("Wl", [0, 64])
def test_global_fake_shapes(Wl):
    with FakeTensorMode():
        q = torch.empty(2, 300, 4, 64, dtype=torch.bfloat16, device="cuda")
        out, tl, mass = torch.ops.bozo.global_fwd(q, q, q, 8.0, None, Wl)
        assert out.shape == q.shape and out.dtype == q.dtype
        assert tl.shape == ((2, 300, 4, Wl) if Wl else (0,))
        assert mass.shape == (2, 300, 4) and mass.dtype == torch.float32
        dq, dk, dv = torch.ops.bozo.global_bwd(q, q, q, out, tl if Wl else None, None, out, mass, Wl, 8.0)
        assert all(t.shape == q.shape for t in (dq, dk, dv))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_rope_fake_shapes(out_dtype):
    with FakeTensorMode():
        x = torch.empty(2, 50, 3, 64, dtype=torch.bfloat16, device="cuda")
        c = torch.empty(128, 32, device="cuda")
        y = torch.ops.bozo.rope(x, c, c, 5, out_dtype, 0)
        assert y.shape == x.shape and y.dtype == out_dtype


def test_autograd_registered():
    """The forward operators carry an autograd formula (the backward
    operators are what it calls)."""
    for name in ("window_fwd", "global_fwd", "rope"):
        op = getattr(torch.ops.bozo, name).default
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "Autograd")


def _trace(fn, *args, **kw):
    """Dynamo's full-graph trace of fn on fake CUDA tensors (no GPU
    needed): the names of the bozo operators in the captured graph."""
    seen = []

    def backend(gm, example_inputs):
        seen.extend(str(n.target) for n in gm.graph.nodes if "bozo" in str(n.target))
        return gm.forward

    torch._dynamo.reset()
    out = torch.compile(fn, backend=backend, fullgraph=True, dynamic=False)(*args, **kw)
    return out, seen


@pytest.mark.parametrize("return_tau,normalize", [(False, None), (True, "mass"), (False, "count")])
def test_causal_tension_traces_without_break(return_tau, normalize):
    from bozo_amd.ops import causal_tension
    with FakeTensorMode(allow_non_fake_inputs=True), torch.device("cuda"):
        q = torch.empty(2, 100, 3, 64, dtype=torch.bfloat16)
        bias = torch.empty(2, 100, 9)
        res, seen = _trace(causal_tension, q, q, q, 9, 8.0, return_tau=return_tau, bias=bias,
                           normalize=normalize)
        out = res[0] if return_tau else res
        assert out.shape == q.shape
        if return_tau:
            assert res[1].shape == (2, 100, 3, 9)
    assert seen == ["bozo.window_fwd"]


@pytest.mark.parametrize("autocast", [False, True])
@pytest.mark.parametrize("return_all", [False, True])
def test_model_traces_without_break(autocast, return_all):
    """The whole TensionLM forward is one graph: RoPE on q and k of each
    layer, the window op on the local layer, the global op on the global
    layer (train.py:776-780 compiles this module)."""
    from bozo_amd import model as M
    cfg = M.TensionConfig(vocab_size=80, dim=128, num_layers=2, num_heads=2, window=6, max_seq_len=64,
                          dropout=0.1, global_every=2, use_rope=True, use_triton=True)
    with FakeTensorMode(allow_non_fake_inputs=True), torch.device("cuda"):
        m = M.TensionLM(cfg)
        ids = torch.zeros(2, 40, dtype=torch.long)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            res, seen = _trace(m, ids, return_all=return_all)
        logits = res[0] if return_all else res
        assert logits.shape == (2, 40, 80)
        if return_all:
            assert [tuple(t.shape) for t in res[2]] == [(2, 40, 2, 6), (2, 40, 2, 6)]
    assert seen == ["bozo.rope"] * 2 + ["bozo.window_fwd"] \
        + ["bozo.rope"] * 2 + ["bozo.global_fwd"]
