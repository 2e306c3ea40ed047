"""CPU checks of the TensionLM integration (bozo_amd/model.py).

The kernel ops are swapped for the torch CPU restatement of the reference's
tension path (oracle/torch_ref.py) so the module wiring can run here; it is
compared with the functional restatement of the reference forward
(oracle/model_ref.py), a second formulation written from the reference's
model.py independently of the module code.  The aux losses are compared with
pure-Python loops written from their definitions (model.py:489-611).
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from bozo_amd import model as M
from oracle import model_ref, torch_ref


def _ct(Q, K, V, window, scale, return_tau=False, bias=None, *, normalize=None):
    raw, tau = torch_ref.unfold_tension(Q, K, V, window, scale, return_tau=True, bias=bias)
    if normalize == "mass":
        raw = torch_ref.normalize_mass(raw, tau)
    elif normalize == "count":
        raw = torch_ref.normalize_count(raw, window)
    return (raw, tau) if return_tau else raw


def _gt(Q, K, V, scale, bias=None, W_local=None):
    out, tl = torch_ref.global_block(Q, K, V, scale, bias=bias, W_local=W_local)
    return (out, tl) if W_local is not None else out


def _rope(x, cos, sin, pos_offset=0, out_dtype=None):
    return torch_ref.rope(x, cos, sin, pos_offset)


@pytest.fixture
def cpu_ops(monkeypatch):
    monkeypatch.setattr(M, "causal_tension", _ct)
    monkeypatch.setattr(M, "global_tension", _gt)
    monkeypatch.setattr(M, "rope", _rope)


def small_cfg(**kw):
    cfg = dict(vocab_size=50, dim=32, num_layers=4, num_heads=4, window=5, max_seq_len=24,
               dropout=0.0, global_every=2)
    cfg.update(kw)
    return M.TensionConfig(**cfg)


def perturbed_model(cfg, seed=0):
    torch.manual_seed(seed)
    m = M.TensionLM(cfg).double()
    with torch.no_grad():  # move every parameter off its init value (norm scales, phases)
        for p in m.parameters():
            p.add_(0.05 * torch.randn_like(p))
    return m


@pytest.mark.parametrize("use_rope", [True, False])
@pytest.mark.parametrize("use_triton", [True, False])
@pytest.mark.parametrize("return_all", [False, True])
def test_module_matches_functional_reference(cpu_ops, use_rope, use_triton, return_all):
    cfg = small_cfg(use_rope=use_rope, use_triton=use_triton)
    m = perturbed_model(cfg).eval()
    g = torch.Generator().manual_seed(1)
    B, T = 2, 19
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=g)
    bias = torch.randn(B, T, cfg.window, generator=g, dtype=torch.float64) * 0.5
    bias_g = torch.randn(B, T, T, generator=g, dtype=torch.float64) * 0.5
    sd = {k: v.detach() for k, v in m.state_dict().items()}
    with torch.no_grad():
        got = m(ids, return_all=return_all, tau_bias=bias, tau_bias_global=bias_g)
        ref = model_ref.forward(sd, cfg, ids, return_all, bias, bias_g)
    if return_all:
        (lg, hg, tg), (lr, hr, tr) = got, ref
        assert torch.allclose(hg, hr, atol=1e-12, rtol=1e-10)
        assert len(tg) == cfg.num_layers
        for a, b in zip(tg, tr):
            assert a.shape == b.shape
            assert torch.allclose(a, b, atol=1e-12)
    else:
        lg, lr = got, ref
    assert torch.allclose(lg, lr, atol=1e-10, rtol=1e-10)


def test_grad_checkpoint_uses_mass_path(cpu_ops):
    """With checkpointing in training mode every local layer runs with tau
    returned (tau-mass normalised), as model.py:367-376 does."""
    cfg = small_cfg(use_rope=True, use_triton=True, use_grad_checkpoint=True)
    m = perturbed_model(cfg).train()
    ids = torch.randint(0, cfg.vocab_size, (2, 16), generator=torch.Generator().manual_seed(2))
    sd = {k: v.detach() for k, v in m.state_dict().items()}
    got = m(ids)
    ref = model_ref.forward(sd, cfg, ids, True)[0]
    assert torch.allclose(got.detach(), ref, atol=1e-10)
    got.sum().backward()
    assert all(p.grad is not None for p in m.parameters())


def test_causality(cpu_ops):
    cfg = small_cfg(use_rope=True, use_triton=True)
    m = perturbed_model(cfg).eval()
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, cfg.vocab_size, (1, 20), generator=g)
    ids2 = ids.clone()
    ids2[0, 12:] = (ids2[0, 12:] + 7) % cfg.vocab_size
    with torch.no_grad():
        a, b = m(ids), m(ids2)
    assert torch.equal(a[:, :12], b[:, :12])
    assert not torch.allclose(a[:, 12:], b[:, 12:])


def test_parameter_layout_and_global_layers():
    cfg = small_cfg(use_rope=True)
    m = M.TensionLM(cfg)
    names = dict(m.named_parameters())
    expect = {"embedding.weight": (50, 32), "final_norm.scale": (32,)}
    for i in range(4):
        p = f"blocks.{i}."
        expect.update({p + "pre_norm.scale": (32,), p + "tension.wq.weight": (32, 32),
                       p + "tension.wk.weight": (32, 32), p + "tension.wv.weight": (32, 32),
                       p + "tension.wo.weight": (32, 32), p + "tension.norm.scale": (32,),
                       p + "oscillate.freqs": (32,), p + "oscillate.phases": (32,),
                       p + "oscillate.amp": (1,), p + "ffn.gate.weight": (96, 32),
                       p + "ffn.val.weight": (96, 32), p + "ffn.proj.weight": (32, 96),
                       p + "ffn.norm.scale": (32,)})
    assert {k: tuple(v.shape) for k, v in names.items()} == expect  # lm_head tied to embedding
    assert m.lm_head.weight is m.embedding.weight
    assert [b.global_layer for b in m.blocks] == [False, True, False, True]
    assert m.window_groups == {5: [0, 2], 24: [1, 3]}
    no_rope = M.TensionLM(small_cfg(use_rope=False))
    sd = no_rope.state_dict()
    assert "pos_embedding.weight" in sd and "blocks.0.tension.wkv.weight" in sd
    assert tuple(sd["blocks.0.tension.wkv.weight"].shape) == (64, 32)


def test_init_scales():
    cfg = small_cfg(num_layers=8, dim=128)
    torch.manual_seed(0)
    m = M.TensionLM(cfg)
    std = lambda t: t.detach().float().std().item()  # noqa: E731
    assert abs(std(m.embedding.weight) - 0.02) < 2e-3
    assert abs(std(m.blocks[0].tension.wq.weight) - 0.02 / math.sqrt(8)) < 1e-3
    assert abs(std(m.blocks[0].tension.wo.weight) - 0.02 / math.sqrt(16)) < 1e-3
    assert abs(std(m.blocks[0].ffn.proj.weight) - 0.02 / math.sqrt(16)) < 1e-3


def test_117m_parameter_count():
    with torch.device("meta"):
        m = M.TensionLM(M.config_117m())
    n = m.num_params
    assert 117_000_000 < n < 117_500_000, n
    assert [i for i, b in enumerate(m.blocks) if b.global_layer] == [3, 7, 11]


def test_rope_tables_match_functional_reference():
    rot = M.RotaryEmbedding(64, 1024)
    cos, sin = model_ref.rope_tables(64, 1024, dtype=torch.float32)
    assert torch.equal(rot.cos, cos) and torch.equal(rot.sin, sin)


# ------------------------------------------------------------------ aux losses

def _taus(seed, shapes):
    g = torch.Generator().manual_seed(seed)
    return [torch.rand(*s, generator=g, dtype=torch.float64) for s in shapes]


def loops_diversity(taus, groups):
    total = 0.0
    for W, idx in groups.items():
        ents = []
        for i in idx:
            t = taus[i].numpy()
            B, T, H, Wd = t.shape
            for b in range(B):
                for r in range(T):
                    for h in range(H):
                        s = sum(t[b, r, h]) + 1e-8
                        ents.append(-sum((x / s) * math.log(x / s + 1e-8) for x in t[b, r, h]))
        total += max(math.log(W) - sum(ents) / len(ents), 0.0)
    return total / max(len(groups), 1)


def loops_consistency(taus):
    total, count = 0.0, 0
    for t in taus:
        t = t.numpy()
        B, T, H, W = t.shape
        if W < 3 or T < 3:
            continue
        n = min(W - 2, 4)
        T_out = T - (n + 1)
        if T_out <= 0:
            continue
        vals = []
        for w1 in range(1, n + 1):
            for j in range(T_out):
                r = w1 + 1 + j
                for b in range(B):
                    for h in range(H):
                        vals.append(max(t[b, r, h, w1 - 1] * t[b, r - 1, h, 0] - t[b, r, h, w1], 0.0))
        total += sum(vals) / len(vals)
        count += 1
    return total / max(count, 1)


def loops_entropy(taus):
    total = 0.0
    for t in taus:
        t = t.numpy()
        m = t.mean(-1).ravel()
        total += sum(max(0.05 - x, 0) for x in m) / m.size + sum(max(x - 0.8, 0) for x in m) / m.size
    return total / len(taus)


def test_diversity_loss_vs_loops():
    taus = _taus(0, [(2, 5, 2, 4), (2, 5, 2, 3), (2, 5, 2, 4)])
    taus[0] = taus[0] ** 6  # peaky rows, so the relu is active
    groups = {4: [0, 2], 9: [1]}
    got = M.tension_diversity_loss(taus, groups).item()
    assert got > 0
    assert abs(got - loops_diversity(taus, groups)) < 1e-12
    got2 = M.tension_diversity_loss(taus).item()  # groups from the tau widths
    assert abs(got2 - loops_diversity(taus, {4: [0, 2], 3: [1]})) < 1e-12


def test_consistency_loss_vs_loops():
    taus = _taus(1, [(2, 9, 3, 6), (1, 7, 2, 3), (1, 4, 1, 8), (1, 9, 1, 2)])
    got = M.constraint_consistency_loss(taus).item()
    assert got > 0
    assert abs(got - loops_consistency(taus)) < 1e-12


def test_entropy_loss_vs_loops():
    taus = _taus(2, [(2, 6, 2, 5), (1, 6, 3, 4)])
    taus[0] = taus[0] * 0.08
    taus[1] = 0.7 + 0.3 * taus[1]
    got = M.tension_entropy_loss(taus).item()
    assert got > 0
    assert abs(got - loops_entropy(taus)) < 1e-12


def test_closure_loss_and_empty_lists():
    h = torch.randn(3, 7, 5, dtype=torch.float64, requires_grad=True)
    loss = M.manifold_closure_loss(h)
    assert abs(loss.item() - ((h[:, -1] - h[:, 0]) ** 2).mean().item()) < 1e-14
    loss.backward()
    assert torch.count_nonzero(h.grad[:, 0]) == 0  # the first position is detached
    for fn in (M.tension_diversity_loss, M.constraint_consistency_loss, M.tension_entropy_loss):
        assert fn([]).item() == 0.0


def test_aux_losses_catch_planted_mistakes():
    """A wrong slot in the consistency loss or a missing eps in the diversity
    loss changes the value (so the loop comparisons above are not vacuous)."""
    taus = _taus(4, [(1, 9, 2, 6)])
    ref = loops_consistency(taus)
    t = taus[0]
    wrong = F.relu(t[:, 2:6, :, 0] * t[:, 1:5, :, 1] - t[:, 2:6, :, 1]).mean().item()
    assert abs(wrong - ref) > 1e-6
    groups = {6: [0]}
    peaky = [taus[0] ** 8]
    p = peaky[0] / peaky[0].sum(-1, keepdim=True)
    no_eps = F.relu(math.log(6) + (p * torch.log(p)).sum(-1).mean()).item()
    assert abs(no_eps - loops_diversity(peaky, groups)) > 1e-12
    assert np.isfinite(M.tension_diversity_loss(peaky, groups).item())


def test_configure_adamw_groups():
    m = M.TensionLM(small_cfg())
    opt = M.configure_adamw(m, lr=3e-4, weight_decay=0.1)
    decay, nodecay = opt.param_groups
    assert decay["weight_decay"] == 0.1 and nodecay["weight_decay"] == 0.0
    assert all(p.dim() >= 2 for p in decay["params"]) and all(p.dim() < 2 for p in nodecay["params"])
    assert opt.defaults["betas"] == (0.9, 0.95) and opt.defaults["eps"] == 1e-8
    n = sum(p.numel() for g in opt.param_groups for p in g["params"])
    assert n == m.num_params


# ------------------------------------------------------------------ sampling

def reference_sample(logits, ids, temp, top_p, rep_penalty, generator):
    """The reference's sampling steps (model.py:634-650) written as its loop."""
    logits = logits.float().clone()
    for tok in set(ids[-32:]):
        if logits[tok] > 0:
            logits[tok] /= rep_penalty
        else:
            logits[tok] *= rep_penalty
    logits = logits / max(temp, 1e-5)
    probs = F.softmax(logits, dim=-1)
    sorted_p, sorted_i = torch.sort(probs, descending=True)
    cum_p = torch.cumsum(sorted_p, dim=-1)
    mask = (cum_p - sorted_p) < top_p
    sorted_p[~mask] = 0.0
    sorted_p /= sorted_p.sum()
    return sorted_i[torch.multinomial(sorted_p, 1, generator=generator).item()].item()


@pytest.mark.parametrize("seed", range(6))
def test_sample_next_matches_reference_loop(seed):
    from bozo_amd.generation import sample_next
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(300, generator=g) * 3
    hist = torch.randint(0, 300, (50,), generator=g).tolist()
    temp, top_p = [(0.8, 0.92), (1.5, 0.5), (1e-7, 0.92), (0.7, 1.0), (1.0, 0.1), (0.5, 0.99)][seed]
    a = sample_next(logits, hist, temp, top_p, 1.3, torch.Generator().manual_seed(100 + seed))
    b = reference_sample(logits, hist, temp, top_p, 1.3, torch.Generator().manual_seed(100 + seed))
    assert a == b
    # the penalty only touches the last 32 tokens, by sign
    assert sample_next(logits, [], 1e-7, 0.9) == int(torch.argmax(logits))


GOLDEN_MODEL = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_ref_cpu.npz")


@pytest.mark.parametrize("case", ["rope", "rope_osc_bias", "learned_pos", "learned_pos_bias"])
def test_model_ref_matches_reference_fixture(case):
    """oracle/model_ref.py against the reference TensionLM itself: vectors
    written by tests/golden/make_model_golden.py, which ran the reference's
    model.py on the CPU in float64 (its unfold and einsum paths,
    model.py:181-287,436-480).  Same seeded parameters (RoPE on / off,
    oscillation on / off, a global layer every 2nd block, graph biases on
    both layer kinds): logits, hidden state and every layer's tau to 1e-10;
    this build's four aux losses (bozo_amd/model.py) on model_ref's taus to
    1e-10; the gradient of sum(logits * g) + aux terms with respect to every
    parameter to 1e-5 relative (stored in float32)."""
    from tests.golden.make_model_golden import weights
    d = np.load(GOLDEN_MODEL)
    pre = case + "/"
    use_rope, use_osc, biases = (bool(x) for x in d[pre + "cfg"])
    cfg = M.TensionConfig(vocab_size=53, dim=16, num_layers=4, num_heads=2, window=3, ffn_mult=3,
                          max_seq_len=16, dropout=0.0, use_rope=use_rope, use_oscillation=use_osc,
                          use_triton=False, global_every=2)
    shapes = []
    for item in d[pre + "params"]:
        name, sh = str(item).rsplit(":", 1)
        shapes.append((name, tuple(int(x) for x in sh.split("x"))))
    sd = {k: torch.from_numpy(v).requires_grad_(True) for k, v in weights(shapes, int(d[pre + "seed"])).items()}
    ids = torch.from_numpy(d[pre + "ids"])
    bias = torch.from_numpy(d[pre + "bias"]) if biases else None
    bias_g = torch.from_numpy(d[pre + "bias_global"]) if biases else None
    logits, hidden, taus = model_ref.forward(sd, cfg, ids, True, bias, bias_g)
    close = lambda a, b, tol: float((a.detach() - torch.from_numpy(b)).abs().max()) <= tol  # noqa: E731
    assert close(logits, d[pre + "logits"], 1e-10)
    assert close(hidden, d[pre + "hidden"], 1e-10)
    for i, t in enumerate(taus):
        assert close(t, d[pre + f"tau/{i}"], 1e-10), i
    groups = M.TensionLM(cfg).window_groups
    div = M.tension_diversity_loss(taus, groups)
    cons = M.constraint_consistency_loss(taus)
    ent = M.tension_entropy_loss(taus)
    clo = M.manifold_closure_loss(hidden)
    got = torch.stack([div, cons, ent, clo]).detach().numpy()
    assert np.max(np.abs(got - d[pre + "aux"])) <= 1e-10, (got, d[pre + "aux"])
    upstream = torch.from_numpy(d[pre + "upstream"])
    loss = (logits * upstream).sum() + 0.3 * div + 0.2 * cons + 0.1 * ent + 0.05 * clo
    loss.backward()
    for name, _ in shapes:
        want = d[pre + "grad/" + name].astype(np.float64)
        err = float(np.max(np.abs(sd[name].grad.numpy() - want)) / max(np.max(np.abs(want)), 1e-30))
        assert err <= 1e-5, (name, err)
