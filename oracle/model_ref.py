"""Functional CPU restatement of the reference TensionLM forward.

TEST INFRASTRUCTURE ONLY: imported by tests (never by the product path) to
check the wiring of ``bozo_amd/model.py`` -- the order of norms, residuals,
dropout-free paths, RoPE, the local/global layer choice and the weight tying
-- independently of its module code.  It reads a ``state_dict`` and runs the
reference forward as plain functions over torch CPU tensors (any float dtype,
float64 in the tests), with the tension op from ``oracle/torch_ref.py``.

Follows (reference ``model.py``):
* ``forward``         <- ``TensionLM.forward`` 436-480 (embedding, learned
  positions without RoPE, blocks, final norm, tied head);
* ``_block``          <- ``TensionBlock._impl`` 351-359 (pre_norm, tension,
  oscillation, FFN);
* ``_tension``        <- ``MultiHeadCausalTensionLayer.forward`` 181-287:
  global layers 217-238, local Triton path 247-267 (count normalisation when
  no tau is asked for), unfold path 269-287 (tau-mass);
* ``_oscillate``      <- ``OscillatoryModulation.forward`` 307-312;
* ``_ffn``            <- ``TensionFFN.forward`` 327-330;
* ``_rms``            <- ``RMSNorm.forward`` 94-99 (the fallback formula,
  which is what ``F.rms_norm`` computes);
* RoPE tables         <- ``RotaryEmbedding.__init__`` 66-73.
Dropout is the identity (eval mode / p = 0).
"""
from __future__ import annotations

import math

import torch

from . import torch_ref


def _rms(x, w, eps=1e-6):
    return x * (x.pow(2).mean(-1, keepdim=True) + eps).rsqrt() * w


def _lin(x, w):
    return x @ w.t()


def rope_tables(head_dim: int, max_seq_len: int, base: int = 10_000, dtype=torch.float64):
    half = head_dim // 2
    theta = 1.0 / (base ** (torch.arange(0, half).float() / half))
    freqs = torch.outer(torch.arange(max_seq_len).float(), theta)
    return freqs.cos().to(dtype), freqs.sin().to(dtype)


def _tension(sd, pre, x, cfg, is_global, return_tau, bias):
    B, T, D = x.shape
    H = cfg.num_heads
    HD = D // H
    scale = math.sqrt(HD)
    q = _lin(x, sd[pre + "wq.weight"]).view(B, T, H, HD)
    if cfg.use_rope:
        k = _lin(x, sd[pre + "wk.weight"]).view(B, T, H, HD)
        v = _lin(x, sd[pre + "wv.weight"]).view(B, T, H, HD)
        cos, sin = rope_tables(HD, cfg.max_seq_len, dtype=x.dtype)
        q = torch_ref.rope(q, cos, sin)
        k = torch_ref.rope(k, cos, sin)
    else:
        kv = _lin(x, sd[pre + "wkv.weight"]).view(B, T, H, 2 * HD)
        k, v = kv[..., :HD], kv[..., HD:]
    wo, nw = sd[pre + "wo.weight"], sd[pre + "norm.scale"]
    if is_global:
        msg, tau = torch_ref.global_block(q, k, v, scale, bias=bias,
                                          W_local=min(cfg.window, T))
        return _rms(x + _lin(msg.reshape(B, T, D), wo), nw), tau
    W = cfg.window
    raw, tau = torch_ref.unfold_tension(q, k, v, W, scale, return_tau=True, bias=bias)
    if cfg.use_triton and not return_tau:
        msg = torch_ref.normalize_count(raw, W)
    else:
        msg = torch_ref.normalize_mass(raw, tau)
    return _rms(x + _lin(msg.reshape(B, T, D), wo), nw), tau


def _oscillate(sd, pre, x):
    T = x.shape[1]
    pos = torch.arange(T, dtype=x.dtype)[:, None]
    mod = torch.sin(pos * sd[pre + "freqs"] + sd[pre + "phases"])
    return x * (1.0 + sd[pre + "amp"] * mod[None])


def _ffn(sd, pre, x):
    g = _lin(x, sd[pre + "gate.weight"])
    h = g * torch.sigmoid(g) * _lin(x, sd[pre + "val.weight"])
    return _rms(x + _lin(h, sd[pre + "proj.weight"]), sd[pre + "norm.scale"])


def _block(sd, i, x, cfg, return_tau, bias, bias_global):
    pre = f"blocks.{i}."
    is_global = cfg.global_every > 0 and (i + 1) % cfg.global_every == 0
    h = _rms(x, sd[pre + "pre_norm.scale"])
    h, tau = _tension(sd, pre + "tension.", h, cfg, is_global, return_tau,
                      bias_global if is_global else bias)
    if cfg.use_oscillation:
        h = _oscillate(sd, pre + "oscillate.", h)
    return _ffn(sd, pre + "ffn.", h), tau


def forward(sd: dict, cfg, input_ids, return_all: bool = False, tau_bias=None, tau_bias_global=None):
    """Reference TensionLM forward from a state_dict; returns logits, or
    (logits, hidden, taus) with ``return_all``."""
    B, T = input_ids.shape
    emb = sd["embedding.weight"]
    x = emb[input_ids]
    if not cfg.use_rope:
        x = x + sd["pos_embedding.weight"][:T][None]
    taus = []
    for i in range(cfg.num_layers):
        x, tau = _block(sd, i, x, cfg, return_all, tau_bias, tau_bias_global)
        taus.append(tau)
    hidden = _rms(x, sd["final_norm.scale"])
    logits = _lin(hidden, emb)
    return (logits, hidden, taus) if return_all else logits
