"""The fused tau regularisers (tension_aux_loss_fwd / _bwd behind
model.tension_aux_losses) against the model's PyTorch restatements of the
reference losses (model.py:498-611), which the CPU suite pins with loops:
loss values and dTau."""
import math

import pytest
import torch

from bozo_amd import model as M

pytestmark = pytest.mark.gpu


def taus_of(seed, L, B, T, H, W, dtype, dev):
    g = torch.Generator().manual_seed(seed)
    out = []
    for l in range(L):
        x = torch.rand(B, T, H, W, generator=g)
        x = x ** (1 + 3 * (l % 3))          # spread rows: some peaky, some flat
        if l % 2:
            x = 0.02 + 0.05 * x             # low-mean rows (the 0.05 floor)
        if l == 0:
            x = 0.75 + 0.25 * x             # high-mean rows (the 0.8 ceiling)
        out.append(x.to(dtype).to(dev))
    return out


def reference(taus, groups):
    return (M.tension_diversity_loss(taus, groups), M.constraint_consistency_loss(taus),
            M.tension_entropy_loss(taus))


@pytest.mark.parametrize("L,B,T,H,W,dtype,grouped", [
    (4, 2, 37, 3, 64, torch.float32, True),
    (3, 1, 20, 2, 5, torch.float32, False),
    (2, 2, 9, 2, 3, torch.float32, False),     # n = 1
    (2, 1, 12, 2, 2, torch.float32, False),    # no consistency terms (W < 3)
    (2, 1, 5, 2, 8, torch.float32, False),     # T too short for the terms
    (12, 2, 64, 4, 64, torch.bfloat16, True),  # the model's shape class
    # more than one workgroup per layer (1024 rows each): blocks that start
    # mid-sequence and mid-row-group, neighbours across block edges, and the
    # host sum of the partials; T = 1000 is not a multiple of the block
    (12, 2, 1024, 12, 64, torch.bfloat16, True),
    (3, 2, 1000, 12, 64, torch.float32, True),
    # wider windows: two and four 8-slot chunks per lane (the 350M preset's
    # W = 256, train.py:246-256), ragged widths and float32 / bf16 rows
    (8, 2, 1024, 16, 256, torch.float32, True),
    (8, 1, 700, 16, 256, torch.bfloat16, True),
    (3, 2, 129, 3, 200, torch.float32, False),
    (3, 2, 65, 2, 128, torch.bfloat16, False),
    (2, 2, 100, 3, 100, torch.float32, False),
    (2, 1, 40, 2, 77, torch.bfloat16, False),   # element loads (W not a multiple of 8)
])
def test_fused_aux_losses_match_reference(dev, L, B, T, H, W, dtype, grouped):
    taus = taus_of(L * 100 + W, L, B, T, H, W, dtype, dev)
    groups = {W: list(range(0, L, 2)), 1024: list(range(1, L, 2))} if grouped else None
    print(f"[aux] L={L} B={B} T={T} H={H} W={W} {dtype} grouped={grouped} "
          f"workgroups/layer={-(-B * T * H // 1024)}", flush=True)
    a = [t.detach().float().requires_grad_(True) for t in taus]    # reference in fp32
    b = [t.detach().clone().requires_grad_(True) for t in taus]    # fused, tau's own dtype
    ra = reference(a, groups)
    fb = M.tension_aux_losses(b, groups)
    for x, y in zip(ra, fb):
        x, y = float(x.detach()), float(y.detach())
        assert abs(x - y) <= 1e-5 * max(1.0, abs(x)), (x, y)
    w = (0.7, 1.3, 2.1)   # distinct upstream weights per loss
    sum(wi * x for wi, x in zip(w, ra)).backward()
    sum(wi * y for wi, y in zip(w, fb)).backward()
    for ga, gb in zip(a, b):
        assert gb.grad.dtype == dtype
        ref = ga.grad.double()
        err = (gb.grad.double() - ref).abs().max().item()
        scale = ref.abs().max().item()
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        assert err <= tol * max(scale, 1e-12) + 1e-12, (err, scale)


def test_fused_aux_losses_mixed_layer_dtypes(dev):
    """fp32 taus of local layers beside bf16 tau_local of global layers (the
    reference dtype flow under autocast): one fused pass, each layer read in
    its own dtype, dTau returned in it."""
    L, B, T, H, W = 6, 2, 300, 4, 64
    taus = taus_of(99, L, B, T, H, W, torch.float32, dev)
    taus = [t.to(torch.bfloat16) if l % 3 == 2 else t for l, t in enumerate(taus)]
    groups = {W: [0, 1, 3, 4], 1024: [2, 5]}
    a = [t.detach().float().requires_grad_(True) for t in taus]
    b = [t.detach().clone().requires_grad_(True) for t in taus]
    ra = reference(a, groups)
    fb = M.tension_aux_losses(b, groups)
    for x, y in zip(ra, fb):
        assert abs(float(x) - float(y)) <= 1e-5 * max(1.0, abs(float(x))), (float(x), float(y))
    sum(wi * x for wi, x in zip((0.7, 1.3, 2.1), ra)).backward()
    sum(wi * y for wi, y in zip((0.7, 1.3, 2.1), fb)).backward()
    for ga, gb, t in zip(a, b, taus):
        assert gb.grad.dtype == t.dtype
        ref = ga.grad.double()
        tol = 1e-5 if t.dtype == torch.float32 else 1e-2
        assert (gb.grad.double() - ref).abs().max().item() <= tol * ref.abs().max().item() + 1e-12


def test_fused_aux_losses_in_the_model(dev):
    """return_all taus of a bf16 model: fused and reference losses give the
    same loss and the same parameter gradients (through the kernels' dTau)."""
    cfg = M.TensionConfig(vocab_size=128, dim=128, num_layers=4, num_heads=2, window=64, max_seq_len=256,
                          dropout=0.0, global_every=2, use_rope=True, use_triton=True)
    torch.manual_seed(0)
    m = M.TensionLM(cfg).to(dev).train()
    ids = torch.randint(0, 128, (2, 200), generator=torch.Generator().manual_seed(1)).to(dev)
    grads = []
    for fused in (False, True):
        m.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, hid, taus = m(ids, return_all=True)
            if fused:
                div, cons, ent = M.tension_aux_losses(taus, m.window_groups)
            else:
                f = [t.float() for t in taus]
                div, cons, ent = reference(f, m.window_groups)
            loss = 0.02 * div + 0.1 * cons + 0.05 * ent + 0.01 * M.manifold_closure_loss(hid)
        loss.backward()
        grads.append((loss.item(), {n: p.grad.detach().float().clone() for n, p in m.named_parameters()
                                    if p.grad is not None}))
    (la, ga), (lb, gb) = grads
    assert abs(la - lb) <= 1e-4 * abs(la)
    for n in ga:
        d = (ga[n] - gb[n]).norm().item()
        r = ga[n].norm().item()
        assert d <= 2e-2 * r + 1e-9, (n, d, r)
