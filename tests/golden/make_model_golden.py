"""Writes tests/golden/model_ref_cpu.npz: input / output vectors of the
reference TensionLM (model.py) run on the CPU in float64, for pinning the
functional restatement oracle/model_ref.py.

The reference's own model is the only thing that fixes its wiring (the order
of norms, residuals, oscillation, FFN, the local / global layer choice, the
RoPE promotion, weight tying); the other checks of oracle/model_ref.py compare
it with this build's module code, which could share a misreading.  So this
script imports the reference's model.py -- in the build container only, where
/root/reference exists; the GPU box never sees it -- and records, for four
small configurations (RoPE on / off, oscillation on / off, a global layer
every 2nd block, graph biases on the local and global layers):

* the token ids and the biases (the parameters are not stored: ``weights``
  below fills them from a seed, in the reference's parameter order, and the
  test rebuilds them the same way);
* logits, the final hidden state and every layer's tau (return_all=True,
  model.py:436-480; on the CPU the local layers take the unfold path,
  model.py:269-287, and the global ones the einsum path, 217-238);
* the four aux losses (model.py:489-611) on those taus;
* the gradient of loss = sum(logits * g) + aux terms with respect to every
  parameter (g a fixed seeded tensor), stored in float32.

Dropout is 0 (the gradients are those of train mode without dropout).

    python tests/golden/make_model_golden.py [/root/reference]
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = [
    # name, use_rope, use_oscillation, biases
    ("rope", True, False, False),
    ("rope_osc_bias", True, True, True),
    ("learned_pos", False, True, False),
    ("learned_pos_bias", False, False, True),
]


def weights(named_shapes, seed):
    """Parameter values for (name, shape) pairs in order: norm scales near 1,
    everything else N(0, 0.1^2), from numpy's PCG64 with `seed`."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in named_shapes:
        x = rng.standard_normal(shape) * 0.1
        if name.endswith("scale"):
            x = 1.0 + x
        out[name] = x
    return out


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import model as R  # the reference's model.py (torch only)

    torch.set_default_dtype(torch.float64)
    out = {}
    for ci, (name, use_rope, use_osc, biases) in enumerate(CASES):
        cfg = R.TensionConfig(vocab_size=53, dim=16, num_layers=4, num_heads=2, window=3, ffn_mult=3,
                              max_seq_len=16, dropout=0.0, use_rope=use_rope, use_oscillation=use_osc,
                              use_triton=False, global_every=2)
        m = R.TensionLM(cfg).double().train()
        shapes = [(k, tuple(p.shape)) for k, p in m.named_parameters()]
        vals = weights(shapes, 100 + ci)
        with torch.no_grad():
            for k, p in m.named_parameters():
                p.copy_(torch.from_numpy(vals[k]))
        g = torch.Generator().manual_seed(200 + ci)
        B, T = 2, 12
        ids = torch.randint(0, cfg.vocab_size, (B, T), generator=g)
        bias = torch.randn(B, T, cfg.window, generator=g) * 0.5 if biases else None
        bias_g = torch.randn(B, T, T, generator=g) * 0.5 if biases else None
        upstream = torch.randn(B, T, cfg.vocab_size, generator=g)
        logits, hidden, taus = m(ids, return_all=True, tau_bias=bias, tau_bias_global=bias_g)
        div = R.tension_diversity_loss(taus, m.window_groups)
        cons = R.constraint_consistency_loss(taus)
        ent = R.tension_entropy_loss(taus)
        clo = R.manifold_closure_loss(hidden)
        loss = (logits * upstream).sum() + 0.3 * div + 0.2 * cons + 0.1 * ent + 0.05 * clo
        loss.backward()
        pre = f"{name}/"
        out[pre + "cfg"] = np.array([int(use_rope), int(use_osc), int(biases)])
        out[pre + "seed"] = np.array(100 + ci)
        out[pre + "ids"] = ids.numpy()
        out[pre + "upstream"] = upstream.numpy()
        if biases:
            out[pre + "bias"] = bias.numpy()
            out[pre + "bias_global"] = bias_g.numpy()
        out[pre + "params"] = np.array([f"{k}:{'x'.join(map(str, sh))}" for k, sh in shapes])
        for k, p in m.named_parameters():
            out[pre + "grad/" + k] = p.grad.detach().numpy().astype(np.float32)
        out[pre + "logits"] = logits.detach().numpy()
        out[pre + "hidden"] = hidden.detach().numpy()
        for i, t in enumerate(taus):
            out[pre + f"tau/{i}"] = t.detach().numpy()
        out[pre + "aux"] = np.array([float(x.detach()) for x in (div, cons, ent, clo)])
    path = os.path.join(HERE, "model_ref_cpu.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(CASES)} configurations)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
