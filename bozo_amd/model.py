"""TensionLM on the MI355X kernels: the model around the tension op.

The reference model (``model.py``) with its tension layers running through
this package's HIP kernels instead of the Triton kernel / unfold / einsum
paths:

* local layers (``model.py:240-287``): ``causal_tension`` with the
  normalisation fused into the kernel -- valid-count when the layer does not
  return its tau (the reference's Triton path, ``model.py:259-264``),
  tau-mass when it does (``model.py:250-258``);
* global layers (``model.py:217-238``): ``global_tension`` (full causal,
  diagonal included, tau-mass normalised, the ``tau_local`` down-sample);
* RoPE (``model.py:54-81``): the ``rope`` kernel on the float32 tables.

Everything else is ordinary PyTorch (linear layers on hipBLASLt, RMSNorm,
SwiGLU, embeddings), with the reference's structure, parameter names and
initialisation, so a reference checkpoint's ``state_dict`` loads as is.
Class, function and argument names follow the reference (``TensionConfig``,
``TensionLM``, the four aux losses of ``model.py:489-611``).

Dtype flow: RoPE promotes like the reference's (``model.py:75-81``: a bf16
projection times the float32 tables gives float32 Q / K under autocast), so
the local layers see float32 Q / K with a bf16 V, which the op runs on its
split-operand MFMA kernels; global layers under autocast take bf16 Q / K /
V, as the reference's autocast einsum does (``model.py:219,230``).  With
``TensionConfig.fast_rope`` the rotated Q / K stay in the projection's dtype
instead (bf16 under autocast: the bf16 MFMA kernels, half the Q / K bytes).

Differences, by design:
* there is no CPU path (the kernels run on the GPU only);
* ``fast_rope`` (default off) is an addition;
* gradient checkpointing (``use_grad_checkpoint``) recomputes the block with
  ``torch.utils.checkpoint`` as the reference does.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor, nn
from torch.utils.checkpoint import checkpoint

from .ops import autocast_inputs, causal_tension, global_tension, rope


@dataclass
class TensionConfig:
    """Same fields and defaults as the reference config (``model.py:26-49``)."""
    vocab_size: int = 2048
    dim: int = 128
    num_layers: int = 4
    num_heads: int = 4
    window: int = 8
    ffn_mult: int = 3
    max_seq_len: int = 256
    dropout: float = 0.10
    use_grad_checkpoint: bool = False
    use_oscillation: bool = True
    use_rope: bool = False
    use_triton: bool = False  # selects the reference's Triton-path normalisation (see the layer)
    global_every: int = 0
    # not in the reference: keep rotated Q / K in the projection's dtype
    # instead of promoting them to the float32 tables' dtype (model.py:75-81)
    fast_rope: bool = False

    @property
    def head_dim(self) -> int:
        if self.dim % self.num_heads:
            raise ValueError("dim must be divisible by num_heads")
        return self.dim // self.num_heads


def config_117m(**overrides) -> TensionConfig:
    """The 117M model of the benchmark (12 layers, dim 768, 12 heads, vocab
    32768, W = 64, a global layer every 4th, RoPE, T = 1024)."""
    cfg = dict(vocab_size=32768, dim=768, num_layers=12, num_heads=12, window=64, ffn_mult=3,
               max_seq_len=1024, dropout=0.10, use_rope=True, global_every=4)
    cfg.update(overrides)
    return TensionConfig(**cfg)


class RotaryEmbedding(nn.Module):
    """Half-split rotary embedding; theta_i = base^(-i/half), float32 cos/sin
    tables of max_seq_len rows (``model.py:54-81``)."""

    def __init__(self, head_dim: int, max_seq_len: int, base: int = 10_000, promote: bool = True):
        super().__init__()
        self.promote = promote
        half = head_dim // 2
        # float32 throughout, as the reference builds its tables
        inv = 1.0 / (base ** (torch.arange(half, dtype=torch.float32) / half))
        ang = torch.arange(max_seq_len, dtype=torch.float32)[:, None] * inv[None, :]
        self.register_buffer("cos", ang.cos(), persistent=False)
        self.register_buffer("sin", ang.sin(), persistent=False)

    def forward(self, x: Tensor, T: int, pos_offset: int = 0) -> Tensor:
        # the reference's x * cos - ... promotes to the wider of x and the tables
        out = torch.promote_types(x.dtype, self.cos.dtype) if self.promote else None
        return rope(x, self.cos, self.sin, pos_offset, out_dtype=out)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.scale = nn.Parameter(torch.ones(dim))

    def forward(self, x: Tensor) -> Tensor:
        return F.rms_norm(x, x.shape[-1:], self.scale, self.eps)


class MultiHeadCausalTensionLayer(nn.Module):
    """One tension layer: projections, the tension op, output projection,
    residual and RMSNorm (``model.py:103-287``).  Parameter names match the
    reference (``wq``, ``wk``/``wv`` with RoPE, ``wkv`` without, ``wo``,
    ``norm``).

    Local layers follow the reference's two paths, both on the kernel here:
    with ``use_triton`` and no tau requested, valid-count normalisation and
    dropout before ``wo`` (``model.py:259-264``); otherwise tau-mass
    normalisation and dropout after ``wo`` (``model.py:250-258`` and the
    unfold path ``model.py:269-287``, which agree)."""

    def __init__(self, cfg: TensionConfig, global_layer: bool = False):
        super().__init__()
        self.global_layer = global_layer
        self.window = cfg.max_seq_len if global_layer else cfg.window
        self.local_window = cfg.window
        self.count_norm = cfg.use_triton and not global_layer
        self.num_heads = cfg.num_heads
        self.head_dim = cfg.head_dim
        self.scale = math.sqrt(self.head_dim)
        D = cfg.dim
        self.wq = nn.Linear(D, D, bias=False)
        self.rope_enabled = cfg.use_rope
        if cfg.use_rope:
            self.wk = nn.Linear(D, D, bias=False)
            self.wv = nn.Linear(D, D, bias=False)
            self.wkv = None
            self.rope = RotaryEmbedding(cfg.head_dim, cfg.max_seq_len, promote=not cfg.fast_rope)
        else:
            self.wkv = nn.Linear(D, 2 * D, bias=False)
            self.wk = self.wv = None
            self.rope = None
        self.wo = nn.Linear(D, D, bias=False)
        self.norm = RMSNorm(D)
        self.dropout = nn.Dropout(cfg.dropout)
        # called with the layer's (k, v) [B,T,H,HD] after RoPE when set (the
        # generation cache's prefill reads them here)
        self.kv_sink = None

    def _qkv(self, x: Tensor, pos_offset: int = 0):
        B, T, D = x.shape
        H, HD = self.num_heads, self.head_dim
        q = self.wq(x).view(B, T, H, HD)
        if self.rope_enabled:
            k = self.wk(x).view(B, T, H, HD)
            v = self.wv(x).view(B, T, H, HD)
            q, k = self.rope(q, T, pos_offset), self.rope(k, T, pos_offset)
        else:
            k, v = self.wkv(x).view(B, T, H, 2 * HD).split(HD, dim=-1)
        return q, k, v

    def forward(self, x: Tensor, return_tensions: bool = False, tau_bias: Optional[Tensor] = None):
        B, T, D = x.shape
        q, k, v = self._qkv(x)
        if self.global_layer:
            q, k, v = autocast_inputs(q, k, v)
        if self.kv_sink is not None:
            self.kv_sink(k, v)
        if self.global_layer:
            res = global_tension(q, k, v, self.scale, bias=tau_bias,
                                 W_local=self.local_window if return_tensions else None)
            msg, tau = res if return_tensions else (res, None)
            out = self.norm(x + self.dropout(self.wo(msg.reshape(B, T, D))))
            return (out, tau) if return_tensions else out
        if return_tensions or not self.count_norm:
            res = causal_tension(q, k, v, self.window, self.scale, return_tau=return_tensions,
                                 bias=tau_bias, normalize="mass")
            msg, tau = res if return_tensions else (res, None)
            out = self.norm(x + self.dropout(self.wo(msg.reshape(B, T, D))))
            return (out, tau) if return_tensions else out
        msg = causal_tension(q, k, v, self.window, self.scale, bias=tau_bias, normalize="count")
        return self.norm(x + self.wo(self.dropout(msg).reshape(B, T, D)))


class OscillatoryModulation(nn.Module):
    """x * (1 + amp * sin(pos * freq + phase)), per channel (``model.py:292-312``)."""

    def __init__(self, cfg: TensionConfig):
        super().__init__()
        self.freqs = nn.Parameter(torch.randn(cfg.dim) * 0.02)
        self.phases = nn.Parameter(torch.zeros(cfg.dim))
        self.amp = nn.Parameter(torch.full((1,), 0.1))
        self.register_buffer("pos_buf", torch.arange(cfg.max_seq_len, dtype=torch.float)[:, None],
                             persistent=False)

    def forward(self, x: Tensor) -> Tensor:
        T = x.shape[1]
        return x * (1.0 + self.amp * torch.sin(self.pos_buf[:T] * self.freqs + self.phases)[None])


class TensionFFN(nn.Module):
    """SwiGLU feed-forward with residual and RMSNorm (``model.py:317-330``)."""

    def __init__(self, cfg: TensionConfig):
        super().__init__()
        hidden = cfg.dim * cfg.ffn_mult
        self.gate = nn.Linear(cfg.dim, hidden, bias=False)
        self.val = nn.Linear(cfg.dim, hidden, bias=False)
        self.proj = nn.Linear(hidden, cfg.dim, bias=False)
        self.norm = RMSNorm(cfg.dim)
        self.dropout = nn.Dropout(cfg.dropout)

    def forward(self, x: Tensor) -> Tensor:
        return self.norm(x + self.dropout(self.proj(F.silu(self.gate(x)) * self.val(x))))


class TensionBlock(nn.Module):
    def __init__(self, cfg: TensionConfig, global_layer: bool = False):
        super().__init__()
        self.pre_norm = RMSNorm(cfg.dim)
        self.tension = MultiHeadCausalTensionLayer(cfg, global_layer=global_layer)
        self.oscillate = OscillatoryModulation(cfg) if cfg.use_oscillation else None
        self.ffn = TensionFFN(cfg)
        self.use_ckpt = cfg.use_grad_checkpoint
        self.global_layer = global_layer

    def _osc(self, x: Tensor) -> Tensor:
        return self.oscillate(x) if self.oscillate is not None else x

    def _body(self, x: Tensor, return_tensions: bool, tau_bias: Optional[Tensor]):
        h = self.pre_norm(x)
        if return_tensions:
            h, tau = self.tension(h, return_tensions=True, tau_bias=tau_bias)
            return self.ffn(self._osc(h)), tau
        return self.ffn(self._osc(self.tension(h, tau_bias=tau_bias)))

    def forward(self, x: Tensor, return_tensions: bool = False, tau_bias: Optional[Tensor] = None):
        if self.use_ckpt and self.training:
            out, tau = checkpoint(lambda y: self._body(y, True, tau_bias), x, use_reentrant=False)
            return (out, tau) if return_tensions else out
        return self._body(x, return_tensions, tau_bias)


class TensionLM(nn.Module):
    """Embedding, blocks (global every ``global_every``-th: layers i with
    (i + 1) % global_every == 0), final RMSNorm, tied LM head
    (``model.py:382-485``)."""

    def __init__(self, cfg: TensionConfig):
        super().__init__()
        self.cfg = cfg
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.dim)
        self.emb_drop = nn.Dropout(cfg.dropout)
        if cfg.use_rope:
            self.pos_embedding = None
        else:
            self.pos_embedding = nn.Embedding(cfg.max_seq_len, cfg.dim)
            self.register_buffer("pos_buf", torch.arange(cfg.max_seq_len)[None], persistent=False)
        self.blocks = nn.ModuleList(
            TensionBlock(cfg, global_layer=cfg.global_every > 0 and (i + 1) % cfg.global_every == 0)
            for i in range(cfg.num_layers))
        groups: dict = {}
        for i, blk in enumerate(self.blocks):
            groups.setdefault(blk.tension.window, []).append(i)
        self.window_groups = groups
        self.final_norm = RMSNorm(cfg.dim)
        self.lm_head = nn.Linear(cfg.dim, cfg.vocab_size, bias=False)
        self.lm_head.weight = self.embedding.weight
        self._init_weights()

    def _init_weights(self):
        std, depth = 0.02, self.cfg.num_layers
        nn.init.normal_(self.embedding.weight, std=std)
        if self.pos_embedding is not None:
            nn.init.normal_(self.pos_embedding.weight, std=std)
        for name, m in self.named_modules():
            if isinstance(m, nn.Linear) and m is not self.lm_head:
                out_proj = name.endswith(("wo", "proj"))
                nn.init.normal_(m.weight, std=std / math.sqrt((2 if out_proj else 1) * depth))

    def forward(self, input_ids: Tensor, return_all: bool = False, tau_bias: Optional[Tensor] = None,
                tau_bias_global: Optional[Tensor] = None):
        B, T = input_ids.shape
        if T > self.cfg.max_seq_len:
            raise ValueError(f"sequence length {T} exceeds max_seq_len {self.cfg.max_seq_len}")
        x = self.embedding(input_ids)
        if self.pos_embedding is not None:
            x = x + self.pos_embedding(self.pos_buf[:, :T])
        x = self.emb_drop(x)
        tensions = []
        for blk in self.blocks:
            bias = tau_bias_global if blk.global_layer else tau_bias
            if return_all:
                x, tau = blk(x, return_tensions=True, tau_bias=bias)
                tensions.append(tau)
            else:
                x = blk(x, tau_bias=bias)
        hidden = self.final_norm(x)
        logits = self.lm_head(hidden)
        return (logits, hidden, tensions) if return_all else logits

    @property
    def num_params(self) -> int:
        return sum(p.numel() for p in self.parameters())


def configure_adamw(model: nn.Module, lr: float = 3e-4, weight_decay: float = 0.1, **kw):
    """AdamW as the reference trains (``train.py:894-902``): weight decay on
    parameters with dim >= 2 only, betas (0.9, 0.95), eps 1e-8.  Extra
    keywords (e.g. ``fused=True``) go to ``torch.optim.AdamW``."""
    decay = [p for p in model.parameters() if p.requires_grad and p.dim() >= 2]
    nodecay = [p for p in model.parameters() if p.requires_grad and p.dim() < 2]
    return torch.optim.AdamW([{"params": decay, "weight_decay": weight_decay},
                              {"params": nodecay, "weight_decay": 0.0}],
                             lr=lr, betas=(0.9, 0.95), eps=1e-8, **kw)


# ------------------------------------------------------------------ aux losses
# Regularisers on the hidden states and the per-layer tau [B,T,H,W]
# (model.py:489-611); ordinary PyTorch, differentiable through the kernels'
# tau output (its gradient enters the backward as dTau).

def manifold_closure_loss(hidden: Tensor) -> Tensor:
    """MSE of the last position's hidden state to the (detached) first."""
    return F.mse_loss(hidden[:, -1], hidden[:, 0].detach())


def tension_diversity_loss(all_tensions: list, window_groups: Optional[dict] = None) -> Tensor:
    """Per window size W: relu(log W - mean entropy of tau normalised over the
    window), averaged over the window sizes present."""
    if not all_tensions:
        return torch.tensor(0.0)
    if window_groups is None:
        window_groups = {}
        for i, t in enumerate(all_tensions):
            window_groups.setdefault(t.shape[-1], []).append(i)
    total = torch.zeros((), device=all_tensions[0].device)
    for W, idx in window_groups.items():
        tau = torch.stack([all_tensions[i] for i in idx])
        p = tau / (tau.sum(-1, keepdim=True) + 1e-8)
        ent = -(p * torch.log(p + 1e-8)).sum(-1)
        total = total + F.relu(math.log(W) - ent.mean())
    return total / max(len(window_groups), 1)


def constraint_consistency_loss(all_tensions: list) -> Tensor:
    """Transitivity: for w1 = 1 .. min(W-2, 4), tau[t, w1-1] * tau[t-1, 0]
    should not exceed tau[t, w1] (slot index w = 0 oldest), over the rows t
    where every w1 is defined; mean of the violations per layer, averaged over
    the layers with W >= 3 and T large enough."""
    if not all_tensions:
        return torch.tensor(0.0)
    total = torch.zeros((), device=all_tensions[0].device)
    count = 0
    for tau in all_tensions:
        B, T, H, W = tau.shape
        if W < 3 or T < 3:
            continue
        n = min(W - 2, 4)
        T_out = T - (n + 1)
        if T_out <= 0:
            continue
        t0 = torch.arange(2, n + 2, device=tau.device)  # first row of each w1 = 1..n
        rows = t0[:, None] + torch.arange(T_out, device=tau.device)[None]  # n x T_out
        w1 = torch.arange(n, device=tau.device)[:, None]
        leg1 = tau[:, rows, :, w1.expand_as(rows)]          # B n T_out H
        leg2 = tau[:, rows - 1, :, torch.zeros_like(rows)]
        comb = tau[:, rows, :, (w1 + 1).expand_as(rows)]
        total = total + F.relu(leg1 * leg2 - comb).mean()
        count += 1
    return total / max(count, 1)


def tension_entropy_loss(all_tensions: list) -> Tensor:
    """Mean over layers of relu(0.05 - m).mean() + relu(m - 0.80).mean(), m
    the mean tau over the window of each (token, head)."""
    if not all_tensions:
        return torch.tensor(0.0)
    total = torch.zeros((), device=all_tensions[0].device)
    for tau in all_tensions:
        m = tau.mean(-1)
        total = total + F.relu(0.05 - m).mean() + F.relu(m - 0.80).mean()
    return total / len(all_tensions)


# ------------------------------------------------------------------ fused aux losses

def _cons_n(W: int, T: int) -> int:
    if W < 3 or T < 3:
        return 0
    n = min(W - 2, 4)
    return n if T - (n + 1) > 0 else 0


_GROUP_MATS: dict = {}


def _group_mats(groups, L: int, nrow: int, dev):
    key = (groups, L, nrow, str(dev))
    if key not in _GROUP_MATS:
        memb = torch.zeros(len(groups), L, dtype=torch.float64)
        for gi, (_, idx) in enumerate(groups):
            for i in idx:
                memb[gi, i] = 1.0 / (len(idx) * nrow)
        logw = torch.tensor([lw for lw, _ in groups], dtype=torch.float64)
        _GROUP_MATS[key] = (memb.to(dev), logw.to(dev))
    return _GROUP_MATS[key]


_AUX_DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float64)


class _AuxLossFn(torch.autograd.Function):
    """Diversity, consistency and entropy losses of every layer's tau in one
    HIP pass forward and one backward (tension_aux_loss_fwd / _bwd)."""

    @staticmethod
    def forward(ctx, groups, *taus):
        from . import _lib as Lb
        L = len(taus)
        B, T, H, W = taus[0].shape
        dev = taus[0].device
        rows = [t if t.stride(-1) == 1 else t.contiguous() for t in taus]
        arr = (Lb.TensionBuf * L)(*[Lb.buf(t).contents for t in rows])
        lib = Lb.lib()
        P = lib.tension_aux_loss_partials(B, T, H)
        part = torch.empty(L, P, 4, dtype=torch.float64, device=dev)
        with torch.cuda.device(dev):
            Lb.check(lib.tension_aux_loss_fwd(arr, L, B, T, H, W, part.data_ptr(),
                                              torch.cuda.current_stream(dev).cuda_stream), "tension_aux_loss_fwd")
        acc = part.sum(1)                                     # [L, 4]
        nrow = B * T * H
        # window groups as a [G, L] membership matrix scaled by 1 / (|group|
        # nrow), built once per (groups, L, device): indexing by Python lists
        # here would copy the index to the device and stall the host
        memb, logw = _group_mats(groups, L, nrow, dev)
        gap = logw - memb @ acc[:, 0]                         # [G]
        div = F.relu(gap).sum() / max(len(groups), 1)
        active = memb.t() @ (gap > 0).double()                # [L]: 1 / (|group| nrow) where active
        n = _cons_n(W, T)
        cons = torch.zeros((), dtype=torch.float64, device=dev)
        if n:
            cons = (acc[:, 1] / (n * B * (T - n - 1) * H)).sum() / L
        ent = ((acc[:, 2] + acc[:, 3]) / nrow).sum() / L
        ctx.save_for_backward(*rows)
        ctx.active, ctx.meta = active, (len(groups), n, L, B, T, H, W)
        return div.float(), cons.float(), ent.float()

    @staticmethod
    def backward(ctx, g_div, g_cons, g_ent):
        from . import _lib as Lb
        rows = ctx.saved_tensors
        G, n, L, B, T, H, W = ctx.meta
        dev = rows[0].device
        coef = torch.zeros(L, 3, dtype=torch.float32, device=dev)
        if g_div is not None:
            coef[:, 0] = (-g_div.double() / max(G, 1) * ctx.active).float()
        if g_cons is not None and n:
            coef[:, 1] = (g_cons.double() / (L * n * B * (T - n - 1) * H)).float()
        if g_ent is not None:
            coef[:, 2] = (g_ent.double() / (L * B * T * H)).float()
        dts = [torch.empty_like(t) for t in rows]
        arr = (Lb.TensionBuf * L)(*[Lb.buf(t).contents for t in rows])
        darr = (Lb.TensionBuf * L)(*[Lb.buf(t).contents for t in dts])
        with torch.cuda.device(dev):
            Lb.check(Lb.lib().tension_aux_loss_bwd(arr, darr, L, B, T, H, W, coef.data_ptr(),
                                                   torch.cuda.current_stream(dev).cuda_stream),
                     "tension_aux_loss_bwd")
        return (None, *dts)


def tension_aux_losses(all_tensions: list, window_groups: Optional[dict] = None):
    """(tension_diversity_loss, constraint_consistency_loss,
    tension_entropy_loss) of the same taus, in one fused pass on the GPU
    when every tau has one [B, T, H, W] shape with W <= 256 (the model's
    layers, e.g. the 350M preset's W = 256; each layer in its own float dtype, e.g. the float32 tau of the
    local layers beside the global layers' bf16 tau_local under autocast,
    all read into float32); otherwise the three functions above."""
    if not all_tensions:
        z = torch.tensor(0.0)
        return z, z, z
    shape = tuple(all_tensions[0].shape)
    fused = (all_tensions[0].is_cuda and len(all_tensions) <= 32 and shape[-1] <= 256
             and all(tuple(t.shape) == shape and t.device == all_tensions[0].device and t.dtype in _AUX_DTYPES
                     for t in all_tensions))
    if not fused:
        return (tension_diversity_loss(all_tensions, window_groups),
                constraint_consistency_loss(all_tensions), tension_entropy_loss(all_tensions))
    if window_groups is None:
        window_groups = {shape[-1]: list(range(len(all_tensions)))}
    groups = tuple((math.log(Wg), tuple(idx)) for Wg, idx in window_groups.items())
    return _AuxLossFn.apply(groups, *all_tensions)


from .generation import TensionKVCache, generate_cached, sample_next  # noqa: E402,F401
