"""PyTorch-on-CPU restatement of the reference's CPU tension path.

TEST INFRASTRUCTURE ONLY (see ``oracle/tension_oracle.py``).  Used two ways:

* as an independent second formulation that pins the numpy oracle (tests),
* as the CPU baseline that ``bench.py`` times on the GPU box's host cores
  (``cpu_baseline.kind == "port"``): the reference's own CPU path is this
  unfold gather plus autograd, which cannot travel to the box, so it is
  restated here.

The formulation deliberately follows the reference's steps, because it is the
thing being timed and cross-checked:
* ``unfold_tension``  <- ``triton_tension/ops.py:29-63`` (pad W zeros in
  front of the time axis, ``unfold`` windows of W, w=0 oldest, validity mask
  t+w >= W, sigmoid(dots/scale + bias) * mask, sum tau*v).
* ``normalize_mass`` / ``normalize_count`` <- ``model.py:257-258,281-282`` and
  ``model.py:159-163,264``.
* ``global_block`` <- ``model.py:217-238`` (einsum scores, tril incl.
  diagonal, tau-mass, tau_local down-sample quirk).
* ``rope`` <- ``model.py:66-81``.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

MASS_EPS = 1e-6


def _window_views(z: torch.Tensor, W: int) -> torch.Tensor:
    """[B,T,H,C] -> [B,T,H,W,C] look-back windows, w=0 oldest, zero-padded."""
    B, T, H, C = z.shape
    zt = z.permute(0, 2, 3, 1)                   # B H C T
    zp = F.pad(zt, (W, 0), value=0.0)             # B H C (W+T)
    win = zp.unfold(-1, W, 1)[:, :, :, :T, :]     # B H C T W
    return win.permute(0, 3, 1, 4, 2)             # B T H W C


def unfold_tension(Q, K, V, W: int, scale: float, return_tau: bool = False,
                   bias=None):
    """Raw sum tau*v (and tau [B,T,H,W]) in the dtype of Q."""
    B, T, H, D = Q.shape
    win = _window_views(torch.cat([K, V], dim=-1), W)
    wk, wv = win[..., :D], win[..., D:]
    t = torch.arange(T).unsqueeze(1)
    w = torch.arange(W).unsqueeze(0)
    valid = (t + w >= W).to(Q.dtype)[None, :, None, :]        # 1 T 1 W
    x = (Q.unsqueeze(3) * wk).sum(-1) / scale                  # B T H W
    if bias is not None:
        x = x + bias.to(x.dtype).unsqueeze(2)
    tau = torch.sigmoid(x) * valid
    msg = (tau.unsqueeze(-1) * wv).sum(3)
    return (msg, tau) if return_tau else msg


def normalize_mass(msg, tau):
    return msg / tau.sum(-1).clamp(min=MASS_EPS).unsqueeze(-1)


def normalize_count(msg, W: int):
    T = msg.shape[1]
    t = torch.arange(T).unsqueeze(1)
    w = torch.arange(W).unsqueeze(0)
    cnt = (t + w >= W).to(msg.dtype).sum(-1).clamp(min=1)
    return msg / cnt[None, :, None, None]


def global_block(Q, K, V, scale: float, bias=None, W_local: int | None = None):
    """Returns (out, tau_local or None), out tau-mass normalised."""
    B, T, H, D = Q.shape
    x = torch.einsum("bthd,bshd->bths", Q, K) / scale
    tril = torch.tril(torch.ones(T, T, dtype=x.dtype))
    if bias is not None:
        x = x + bias.to(x.dtype).unsqueeze(2)
    tau = torch.sigmoid(x) * tril.unsqueeze(0).unsqueeze(2)
    mass = tau.sum(-1).clamp(min=MASS_EPS)
    out = torch.einsum("bths,bshd->bthd", tau, V) / mass.unsqueeze(-1)
    tau_local = None
    if W_local is not None:
        tau_local = tau[:, :, :, :T].flip(-1)[:, :, :, :min(W_local, T)]
    return out, tau_local


def rope(x, cos, sin, pos_offset: int = 0):
    T = x.shape[1]
    c = cos[pos_offset:pos_offset + T].to(x.dtype).unsqueeze(0).unsqueeze(2)
    s = sin[pos_offset:pos_offset + T].to(x.dtype).unsqueeze(0).unsqueeze(2)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)
