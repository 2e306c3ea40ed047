"""KV-cached generation for TensionLM on the streaming decode kernel.

The reference generates by re-running the whole forward over the last
``max_seq_len`` tokens for every new token (``model.py:617-652`` and
``generate_cached`` ``model.py:719-768``, whose TODO at 736-739 asks for a
per-layer cache).  A tension layer only reads keys/values of earlier
positions, so one token can be advanced through all layers from caches:

* local layers keep a ring of the last W post-RoPE K/V rows per (sequence,
  head) and run ``tension_decode_step`` with the same normalisation as the
  full forward (valid count on the reference's Triton path without tau,
  tau mass otherwise);
* global layers keep every earlier row (a ring of ``max_seq_len`` slots that
  never wraps) and run the step with the new token as a key too (keys s <= t,
  tau-mass normalised);
* RoPE and the oscillatory modulation take the token's absolute position.

Each step therefore reads O(W) cached rows per local layer instead of
re-running O(T W) work.  The result equals the full forward's last row as
long as the sequence fits ``max_seq_len``; beyond that the reference slides
its context window (every position shifts, so no cache can serve it) and
``generate_cached`` re-runs the forward over the window, as the reference
does.

Sampling (``sample_next``) restates the reference's: repetition penalty over
the last 32 tokens, temperature, top-p nucleus, one multinomial draw
(``model.py:634-650``).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from .ops import TensionDecodeCache, autocast_inputs, decode_step, rope


class TensionKVCache:
    """Per-layer K/V caches of N sequences advancing in lock step.

    ``prefill(ids)`` runs the model's forward over the prompt [N, T] and
    keeps each layer's last W (local) / all (global) post-RoPE K/V rows;
    ``step(next_ids)`` advances one token per sequence and returns its
    logits [N, vocab].  The model must be in eval mode (dropout off)."""

    def __init__(self, model, N: int, return_all: bool = False):
        """``return_all``: every step computes what ``model(ctx,
        return_all=True)`` gives for the new token -- the forward the
        reference's streaming exporter runs per step (ts_bridge/streaming.py
        :26-33): local layers tau-mass normalised (model.py:250-258) and,
        with ``return_tau``, the global layers' down-sampled ``tau_local``
        row (model.py:231-237) beside the local layers' tau rows."""
        self.model = model
        self.N = N
        self.return_all = bool(return_all)
        self.t = 0  # tokens cached per sequence
        cfg = model.cfg
        self.windows = [cfg.max_seq_len if b.global_layer else cfg.window for b in model.blocks]
        self.layers: list[Optional[TensionDecodeCache]] = [None] * len(model.blocks)

    def _fill(self, i: int, k: Tensor, v: Tensor):
        N, T, H, HD = k.shape
        layer = self.model.blocks[i].tension
        c = self.layers[i]
        if c is None or c.k.dtype != k.dtype or c.v.dtype != v.dtype:
            c = TensionDecodeCache(N, H, HD, self.windows[i], dtype=k.dtype, device=k.device,
                                   scale=layer.scale, v_dtype=v.dtype)
            self.layers[i] = c
        W = c.W
        s = max(0, T - W)
        slots = torch.arange(s, T, device=k.device) % W
        c.k[:, :, slots] = k[:, s:].transpose(1, 2)
        c.v[:, :, slots] = v[:, s:].transpose(1, 2)
        c.pos[c.cur].fill_(T)

    @torch.no_grad()
    def prefill(self, ids: Tensor):
        """Forward over the prompt ids [N, T] (T <= max_seq_len) filling the
        caches; returns the logits [N, T, vocab], or with ``return_all``
        (logits, taus) of ``model(ids, return_all=True)``."""
        model = self.model
        N, T = ids.shape
        if N != self.N:
            raise ValueError(f"prefill: {N} sequences, cache built for {self.N}")
        if not 1 <= T <= model.cfg.max_seq_len:
            raise ValueError(f"prefill: prompt length {T} outside [1, {model.cfg.max_seq_len}]")
        if model.training:
            raise RuntimeError("generation needs model.eval() (dropout off)")
        layers = [b.tension for b in model.blocks]
        for i, layer in enumerate(layers):
            layer.kv_sink = (lambda k, v, i=i: self._fill(i, k, v))
        try:
            res = model(ids, return_all=True) if self.return_all else model(ids)
        finally:
            for layer in layers:
                layer.kv_sink = None
        self.t = T
        return (res[0], res[2]) if self.return_all else res

    def _check_step(self):
        cfg = self.model.cfg
        if self.t == 0:
            raise RuntimeError("step before prefill")
        if self.t >= cfg.max_seq_len:
            raise ValueError(f"position {self.t} is past max_seq_len {cfg.max_seq_len}")
        if self.model.training:
            raise RuntimeError("generation needs model.eval() (dropout off)")

    def _advance(self):
        for c in self.layers:
            c.cur = 1 - c.cur
        self.t += 1

    @torch.no_grad()
    def step(self, next_ids: Tensor, return_tau: bool = False):
        """Advance every sequence by one token (ids [N]) at position ``t``;
        returns logits [N, vocab] and, with ``return_tau``, the new token's
        tau row [N, H, W] of every local layer -- the last row of the full
        forward's tau -- and, in ``return_all`` mode, the global layers'
        ``tau_local`` row [N, H, min(W, t + 1)] (slot j = key t - j, the
        last row of model.py:231-237); None for global layers otherwise."""
        self._check_step()
        taus = [] if return_tau else None
        logits = self._step_device(next_ids, [c.cur for c in self.layers], taus, self.t)
        self._advance()
        return (logits, taus) if return_tau else logits

    @torch.no_grad()
    def graph_step(self, next_ids: Tensor) -> Tensor:
        """``step`` replayed from a HIP graph (captured on the first call, one
        graph per parity of the position counters).  Returns a view of the
        graph's static logits buffer [N, vocab], overwritten by the next
        call.  The result is the eager step's."""
        self._check_step()
        if self._graphs is None:
            self._capture()
        par = self.layers[0].cur
        self._ids.copy_(next_ids)
        self._graphs[par].replay()
        self._advance()
        return self._logits[par]

    _graphs = None

    def _capture(self):
        dev = self.layers[0].k.device
        self._ids = torch.zeros(self.N, dtype=torch.long, device=dev)
        saved = [(c.k.clone(), c.v.clone(), c.pos[0].clone(), c.pos[1].clone()) for c in self.layers]
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):  # warm-up launches (library set-up) outside the capture
            for par in (0, 1):
                self._step_device(self._ids, [par] * len(self.layers), None, None)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        for c, (k, v, p0, p1) in zip(self.layers, saved):
            c.k.copy_(k)
            c.v.copy_(v)
            c.pos[0].copy_(p0)
            c.pos[1].copy_(p1)
        graphs, logits = [], []
        pool = None
        for par in (0, 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                logits.append(self._step_device(self._ids, [par] * len(self.layers), None, None))
            pool = g.pool()
            graphs.append(g)
        torch.cuda.synchronize(dev)
        self._graphs, self._logits = graphs, logits

    def _step_device(self, next_ids: Tensor, parities, taus, t):
        """One token through the model with its position read from the layer
        caches' device counters (no host value of t), so the same launches
        can be captured once and replayed at every position.  ``t`` (host
        position) is only needed for the global layers' tau rows."""
        model = self.model
        N = next_ids.shape[0]
        c0 = self.layers[0]
        pos = c0.pos[parities[0]][:1].long()  # [1]: position of the new token
        x = model.embedding(next_ids.view(N, 1))
        if model.pos_embedding is not None:
            x = x + model.pos_embedding(pos.view(1, 1))
        # per-position tables, gathered once for every layer
        rot = None
        first = model.blocks[0].tension
        if first.rope_enabled:
            rot = (first.rope.cos.index_select(0, pos), first.rope.sin.index_select(0, pos))
        fpos = None
        for blk, c, par in zip(model.blocks, self.layers, parities):
            h = blk.pre_norm(x)
            h = _layer_step(blk.tension, h, c, par, rot, taus, self.return_all, t)
            if blk.oscillate is not None:
                osc = blk.oscillate
                if fpos is None:
                    fpos = osc.pos_buf.index_select(0, pos)
                h = h * (1.0 + osc.amp * torch.sin(fpos * osc.freqs + osc.phases)[None])
            ffn = blk.ffn
            y = ffn.proj(torch.nn.functional.silu(ffn.gate(h)) * ffn.val(h))
            # the residual in the stream's dtype (same values as x + y)
            x = ffn.norm(h + y.to(h.dtype))
        return model.lm_head(model.final_norm(x))[:, 0]


def _layer_step(layer, x: Tensor, cache: TensionDecodeCache, par: int, rot, taus,
                return_all: bool = False, t: Optional[int] = None):
    """One token through a tension layer: x [N, 1, D]; ``rot`` the RoPE
    (cos, sin) rows [1, HD/2] of its position; cache counters pos[par] ->
    pos[1 - par].  ``return_all``: the normalisation of the return_all
    forward (tau mass in every local layer) and, when taus are collected,
    the global layer's tau_local row for position ``t``."""
    N, _, D = x.shape
    H, HD = layer.num_heads, layer.head_dim
    q = layer.wq(x).view(N, 1, H, HD)
    if layer.rope_enabled:
        k = layer.wk(x).view(N, 1, H, HD)
        v = layer.wv(x).view(N, 1, H, HD)
        # promoted like the full forward's RoPE (model.py:75-81) unless fast_rope
        out = torch.promote_types(q.dtype, rot[0].dtype) if layer.rope.promote else None
        q, k = rope(q, *rot, out_dtype=out), rope(k, *rot, out_dtype=out)
    else:
        k, v = layer.wkv(x).view(N, 1, H, 2 * HD).split(HD, dim=-1)
    q, k, v = q[:, 0], k[:, 0], v[:, 0]
    if layer.global_layer:  # the full forward's autocast inputs of the global block
        q, k, v = autocast_inputs(q, k, v)
    pin, pout = cache.pos[par], cache.pos[1 - par]
    if layer.global_layer:
        out = decode_step(q, k, v, cache.k, cache.v, pin, pout, cache.scale, "mass", None, True)
        if taus is not None:
            taus.append(_global_tau_row(layer, q, cache, t) if return_all else None)
    else:
        tau = None
        if taus is not None:
            tau = torch.empty(N, H, cache.W, dtype=q.dtype, device=q.device)
            taus.append(tau)
        norm = "count" if layer.count_norm and not return_all else "mass"
        out = decode_step(q, k, v, cache.k, cache.v, pin, pout, cache.scale, norm, tau)
    return layer.norm(x + layer.wo(out.reshape(N, 1, D)).to(x.dtype))


def _global_tau_row(layer, q: Tensor, cache: TensionDecodeCache, t: int) -> Tensor:
    """Last row of a global layer's ``tau_local`` at position t (the cache
    already holds keys 0..t, slot = position): slot j = sigmoid(q . k_{t-j}
    / scale) for j < min(W_local, t + 1), the flipped, cut-down score row of
    model.py:231-237.  A side output of the streaming export (float32
    scores, rounded to q's dtype), computed from the cached keys."""
    Wl = min(layer.local_window, t + 1)
    keys = cache.k[:, :, t + 1 - Wl:t + 1].flip(2).float()            # [N, H, Wl, D]
    s = torch.matmul(keys, q.float()[..., None])[..., 0] / cache.scale  # [N, H, Wl]
    return torch.sigmoid(s).to(q.dtype)


def sample_next(logits: Tensor, history: list, temp: float = 0.8, top_p: float = 0.92,
                rep_penalty: float = 1.3, generator: Optional[torch.Generator] = None) -> int:
    """Next token from one logits row [vocab] (model.py:634-650)."""
    logits = logits.float().clone()
    recent = sorted(set(history[-32:]))
    if recent:
        idx = torch.tensor(recent, device=logits.device)
        sel = logits[idx]
        logits[idx] = torch.where(sel > 0, sel / rep_penalty, sel * rep_penalty)
    logits = logits / max(temp, 1e-5)
    probs = torch.softmax(logits, dim=-1)
    sorted_p, sorted_i = torch.sort(probs, descending=True)
    cum_p = torch.cumsum(sorted_p, dim=-1)
    keep = (cum_p - sorted_p) < top_p
    sorted_p[~keep] = 0.0
    sorted_p /= sorted_p.sum()
    return int(sorted_i[torch.multinomial(sorted_p, 1, generator=generator).item()].item())


@torch.no_grad()
def generate_cached(model, input_ids: list, max_new: int = 200, temp: float = 0.8,
                    top_p: float = 0.92, rep_penalty: float = 1.3,
                    generator: Optional[torch.Generator] = None, use_graph: bool = True) -> list:
    """Autoregressive generation with per-layer K/V caches (same arguments
    and result as the reference's ``generate_cached``, model.py:719-768).
    ``use_graph``: replay each cached step from a HIP graph."""
    model.eval()
    device = next(model.parameters()).device
    max_ctx = model.cfg.max_seq_len
    ids = list(input_ids)
    if not ids or max_new <= 0:
        return ids
    cache = TensionKVCache(model, 1)
    logits = cache.prefill(torch.tensor([ids[-max_ctx:]], dtype=torch.long, device=device))[0, -1]
    for i in range(max_new):
        nxt = sample_next(logits, ids, temp, top_p, rep_penalty, generator)
        ids.append(nxt)
        if i == max_new - 1:
            break
        if len(ids) <= max_ctx:
            nid = torch.tensor([nxt], dtype=torch.long, device=device)
            logits = (cache.graph_step(nid) if use_graph else cache.step(nid))[0]
        else:  # the reference's context slides past max_seq_len: re-run the window
            ctx = torch.tensor([ids[-max_ctx:]], dtype=torch.long, device=device)
            logits = model(ctx)[0, -1]
    return ids
