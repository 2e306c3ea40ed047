"""CPU oracle for the sigmoid-tension hot path (float64 numpy).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``bozo_amd``) imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may use it, and only as the checker.

It restates, in vectorised float64 numpy, what the reference computes on the
hot path (all citations are relative to the reference repository root):

* local window forward: ``triton_tension/ops.py:29-63`` (``_ref_forward``)
  and ``triton_tension/kernel.py:41-125`` -- tau[t,w] = sigmoid(q_t.k_s/scale
  + bias[b,t,w]) for s = t-(W-w), zero where s < 0; msg_t = sum_w tau.v_s.
* normalisations: tau-mass ``model.py:257-258,281-282`` and valid-count
  ``model.py:159-163,264``.
* local window backward: ``triton_tension/kernel.py:145-152`` (dQ) and
  ``kernel.py:247-255,308-329`` (dK/dV, dTau index w = W-delta).
* global (full causal, diagonal included) block: ``model.py:217-238``,
  including the ``tau_local`` down-sample quirk at ``model.py:231-237``.
* RoPE: ``model.py:54-81`` (half-split rotation).
* streaming decode: the last row of the tau-mass-normalised local window
  (``ts_bridge/streaming.py:100-127`` reads tau[:, -1]; causality argument in
  ``ts_bridge/streaming_parity.py:20-24``).

How each function is pinned (checked against something other than itself) is
listed in ``PINS`` at the bottom and exercised by ``tests/test_oracle.py``:
brute-force pure-Python loops written directly from the index definitions,
an independent torch ``unfold`` restatement with autograd
(``oracle/torch_ref.py``), finite differences, and closed-form invariants.
"""
from __future__ import annotations

import numpy as np

MASS_EPS = 1e-6  # model.py:227,257,281  clamp(min=1e-6)


# --------------------------------------------------------------------------
# elementwise helpers
# --------------------------------------------------------------------------

def sigmoid(x: np.ndarray) -> np.ndarray:
    """Numerically stable logistic function in float64."""
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    pos = x >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-x[pos]))
    ex = np.exp(x[~pos])
    out[~pos] = ex / (1.0 + ex)
    return out


def _f64(a):
    return None if a is None else np.asarray(a, dtype=np.float64)


# --------------------------------------------------------------------------
# RoPE  (model.py:54-81)
# --------------------------------------------------------------------------

def rope_tables(max_len: int, head_dim: int, base: float = 10000.0):
    """cos/sin tables [max_len, head_dim//2] in float32, as the model's
    non-persistent buffers (model.py:66-73): theta_i = base^(-i/half),
    freqs = outer(pos, theta)."""
    half = head_dim // 2
    theta = (1.0 / (np.float32(base) ** (np.arange(half, dtype=np.float32)
                                         / np.float32(half)))).astype(np.float32)
    pos = np.arange(max_len, dtype=np.float32)
    freqs = np.outer(pos, theta).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def rope_apply(x, cos, sin, pos_offset: int = 0):
    """x [B,T,H,D] -> rotated x (model.py:75-81): half-split, not interleaved.
    Rows t use table row pos_offset + t."""
    x = _f64(x)
    T, half = x.shape[1], x.shape[-1] // 2
    c = _f64(cos)[pos_offset:pos_offset + T][None, :, None, :]
    s = _f64(sin)[pos_offset:pos_offset + T][None, :, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def rope_apply_adjoint(dy, cos, sin, pos_offset: int = 0):
    """Gradient of rope_apply w.r.t. its input (the transposed rotation)."""
    dy = _f64(dy)
    T, half = dy.shape[1], dy.shape[-1] // 2
    c = _f64(cos)[pos_offset:pos_offset + T][None, :, None, :]
    s = _f64(sin)[pos_offset:pos_offset + T][None, :, None, :]
    d1, d2 = dy[..., :half], dy[..., half:]
    return np.concatenate([d1 * c + d2 * s, -d1 * s + d2 * c], axis=-1)


# --------------------------------------------------------------------------
# local window  (triton_tension/ops.py:29-63, kernel.py:41-341)
# --------------------------------------------------------------------------

def window_forward(Q, K, V, W: int, scale: float, bias=None):
    """Raw windowed tension.

    Q, K, V : [B,T,H,D];  bias : [B,T,W] or None (broadcast over heads).
    Returns (msg [B,T,H,D], tau [B,T,H,W]).  Slot w looks at key
    s = t - (W - w); slots with s < 0 hold tau = 0 and contribute nothing
    (ops.py:50-58, kernel.py:82-86,109).
    """
    Q, K, V, bias = _f64(Q), _f64(K), _f64(V), _f64(bias)
    B, T, H, D = Q.shape
    msg = np.zeros((B, T, H, D))
    tau = np.zeros((B, T, H, W))
    for w in range(W):
        back = W - w                     # t - s
        if back >= T:
            continue                     # no query has this key in range
        x = np.einsum("bthd,bthd->bth", Q[:, back:], K[:, :T - back]) / scale
        if bias is not None:
            x = x + bias[:, back:, w][:, :, None]
        p = sigmoid(x)
        tau[:, back:, :, w] = p
        msg[:, back:] += p[..., None] * V[:, :T - back]
    return msg, tau


def valid_count(T: int, W: int) -> np.ndarray:
    """model.py:159-163: number of slots with t + w >= W, clamped to >= 1."""
    t = np.arange(T)
    return np.maximum(np.minimum(t, W), 1).astype(np.float64)


def normalize_mass(msg, tau):
    """Tau-mass normalisation (model.py:257-258,281-282).
    Returns (out, mass) with mass = sum_w tau (unclamped)."""
    mass = tau.sum(-1)
    return msg / np.maximum(mass, MASS_EPS)[..., None], mass


def normalize_count(msg, W: int):
    """Valid-count normalisation (model.py:264)."""
    T = msg.shape[1]
    return msg / valid_count(T, W)[None, :, None, None]


def window_backward(Q, K, V, W: int, scale: float, dmsg, dtau=None, bias=None):
    """Gradients of a loss L(msg, tau) w.r.t. Q, K, V, given dL/dmsg and
    (optionally) dL/dtau, for the raw op.

    Per valid pair (t, s=t-(W-w)):
        g     = dmsg_t . v_s + dtau[t,w]              (kernel.py:211-217)
        ddot  = g * tau * (1 - tau)                   (kernel.py:219)
        dQ_t += ddot * k_s / scale;  dK_s += ddot * q_t / scale   (221, 330)
        dV_s += tau * dmsg_t                          (kernel.py:317)
    Bias receives no gradient (ops.py:184-187).
    """
    Q, K, V, dmsg = _f64(Q), _f64(K), _f64(V), _f64(dmsg)
    dtau, bias = _f64(dtau), _f64(bias)
    B, T, H, D = Q.shape
    dQ, dK, dV = np.zeros_like(Q), np.zeros_like(K), np.zeros_like(V)
    for w in range(W):
        back = W - w
        if back >= T:
            continue
        q, k, v, do = Q[:, back:], K[:, :T - back], V[:, :T - back], dmsg[:, back:]
        x = np.einsum("bthd,bthd->bth", q, k) / scale
        if bias is not None:
            x = x + bias[:, back:, w][:, :, None]
        p = sigmoid(x)
        g = np.einsum("bthd,bthd->bth", do, v)
        if dtau is not None:
            g = g + dtau[:, back:, :, w]
        dd = g * p * (1.0 - p)
        dQ[:, back:] += dd[..., None] * k / scale
        dK[:, :T - back] += dd[..., None] * q / scale
        dV[:, :T - back] += p[..., None] * do
    return dQ, dK, dV


def window_backward_normalized(Q, K, V, W: int, scale: float, dout, dtau=None,
                               bias=None):
    """Gradients through out = msg / max(mass, 1e-6) (and optionally tau),
    derived by the chain rule on top of ``window_backward``:
        dmsg_t  = dout_t / m_t
        dmass_t = -(dout_t . msg_t) / m_t^2   if mass_t >= 1e-6 else 0
    and, because mass_t = sum_w tau[t,w], dmass_t is added to dtau on every
    valid slot."""
    msg, tau = window_forward(Q, K, V, W, scale, bias)
    mass = tau.sum(-1)
    m = np.maximum(mass, MASS_EPS)
    dout = _f64(dout)
    dmsg = dout / m[..., None]
    dmass = -np.einsum("bthd,bthd->bth", dout, msg) / (m * m)
    dmass = np.where(mass >= MASS_EPS, dmass, 0.0)
    dt = np.broadcast_to(dmass[..., None], tau.shape).copy()
    if dtau is not None:
        dt = dt + _f64(dtau)
    return window_backward(Q, K, V, W, scale, dmsg, dt, bias)


# --------------------------------------------------------------------------
# global full-causal block  (model.py:217-238)
# --------------------------------------------------------------------------

def global_forward(Q, K, V, scale: float, bias=None, W_local: int | None = None):
    """Full causal sigmoid tension, diagonal INCLUDED (tril, model.py:221).

    bias: [B,T,T] indexed [b, t, s] (model.py:224-225).
    Returns (out, mass, tau_local) where out = (tau @ v) / max(mass, 1e-6)
    and tau_local = tau[..., :T].flip(-1)[..., :min(W_local, T)]
    (model.py:235-236): slot j holds key s = T-1-j for every query row
    (an absolute, not query-relative, key index).  tau_local is None when
    W_local is None.
    """
    Q, K, V, bias = _f64(Q), _f64(K), _f64(V), _f64(bias)
    B, T, H, D = Q.shape
    tril = np.tril(np.ones((T, T)))
    out = np.zeros_like(Q)
    mass = np.zeros((B, T, H))
    Wl = None if W_local is None else min(W_local, T)
    tau_local = None if W_local is None else np.zeros((B, T, H, Wl))
    for b in range(B):
        for h in range(H):
            x = Q[b, :, h] @ K[b, :, h].T / scale
            if bias is not None:
                x = x + bias[b]
            p = sigmoid(x) * tril
            mass[b, :, h] = p.sum(-1)
            out[b, :, h] = (p @ V[b, :, h]) / np.maximum(mass[b, :, h], MASS_EPS)[:, None]
            if tau_local is not None:
                tau_local[b, :, h, :] = p[:, ::-1][:, :Wl]
    return out, mass, tau_local


def global_backward(Q, K, V, scale: float, dout, bias=None, dtau_local=None):
    """Gradients of L(out, tau_local) for ``global_forward`` (chain rule):
    dtau[t,s] = (dout_t.v_s - dout_t.out_t)/m_t (mass term only where
    mass_t >= 1e-6) + dtau_local[t, T-1-s] for s >= T-W_local;
    ddot = dtau*tau*(1-tau) on s <= t; dQ = ddot K/scale, dK = ddot^T Q/scale,
    dV = (tau/m)^T dout."""
    Q, K, V, dout = _f64(Q), _f64(K), _f64(V), _f64(dout)
    bias, dtau_local = _f64(bias), _f64(dtau_local)
    B, T, H, D = Q.shape
    tril = np.tril(np.ones((T, T)))
    dQ, dK, dV = np.zeros_like(Q), np.zeros_like(K), np.zeros_like(V)
    for b in range(B):
        for h in range(H):
            q, k, v, do = Q[b, :, h], K[b, :, h], V[b, :, h], dout[b, :, h]
            x = q @ k.T / scale
            if bias is not None:
                x = x + bias[b]
            p = sigmoid(x) * tril
            mass = p.sum(-1)
            m = np.maximum(mass, MASS_EPS)
            msg = p @ v
            out = msg / m[:, None]
            dmsg = do / m[:, None]
            dmass = np.where(mass >= MASS_EPS, -(do * out).sum(-1) / m, 0.0)
            dp = dmsg @ v.T + dmass[:, None]
            if dtau_local is not None:
                Wl = dtau_local.shape[-1]
                # slot j <-> key T-1-j
                dp[:, T - Wl:] += dtau_local[b, :, h, ::-1]
            dd = dp * p * (1.0 - p) * tril
            dQ[b, :, h] = dd @ k / scale
            dK[b, :, h] = dd.T @ q / scale
            dV[b, :, h] = p.T @ dmsg
    return dQ, dK, dV


# --------------------------------------------------------------------------
# streaming decode
# --------------------------------------------------------------------------

def decode_step(q, k_cache, v_cache, pos, W: int, scale: float,
                normalize=True, self_kv=None):
    """One decode step over a ring cache.

    q [N,H,D]; k_cache/v_cache [N,H,W,D]; pos [N] = number of tokens already
    appended for each sequence.  Slot i holds the most recent position p with
    p % W == i.  The query attends to positions max(0,pos-W)..pos-1 (strictly
    past, like the local window) and, with ``self_kv`` = (k_new, v_new)
    [N,H,D], to the new token itself (the global block's diagonal).
    ``normalize``: True / "mass" (tau mass), "count" (number of keys,
    max(min(pos, W) + self, 1)) or False (raw).  Returns (out [N,H,D], tau
    [N,H,W]) with tau in window order (w=0 oldest: key position pos-W+w),
    zero on empty slots (the self key's tau is not part of it).
    """
    q, kc, vc = _f64(q), _f64(k_cache), _f64(v_cache)
    N, H, D = q.shape
    out = np.zeros((N, H, D))
    tau = np.zeros((N, H, W))
    for n in range(N):
        P = int(pos[n])
        mass = np.zeros(H)
        for w in range(W):
            p = P - W + w
            if p < 0:
                continue
            slot = p % W
            x = (q[n] * kc[n, :, slot]).sum(-1) / scale
            tau[n, :, w] = sigmoid(x)
            out[n] += tau[n, :, w][:, None] * vc[n, :, slot]
        mass += tau[n].sum(-1)
        keys = min(P, W)
        if self_kv is not None:
            kn, vn = _f64(self_kv[0])[n], _f64(self_kv[1])[n]
            ts = sigmoid((q[n] * kn).sum(-1) / scale)
            out[n] += ts[:, None] * vn
            mass += ts
            keys += 1
        if normalize is True or normalize == "mass":
            out[n] /= np.maximum(mass, MASS_EPS)[:, None]
        elif normalize == "count":
            out[n] /= max(keys, 1)
    return out, tau


def decode_append(k_cache, v_cache, pos, k_new, v_new, W: int):
    """Write the new token's k/v into slot pos % W (in place on copies) and
    return (k_cache, v_cache, pos + 1)."""
    kc, vc = np.array(k_cache, copy=True), np.array(v_cache, copy=True)
    for n in range(kc.shape[0]):
        slot = int(pos[n]) % W
        kc[n, :, slot] = k_new[n]
        vc[n, :, slot] = v_new[n]
    return kc, vc, np.asarray(pos) + 1


# --------------------------------------------------------------------------
# brute-force loop restatements (tiny inputs only; written from the index
# definitions, used to pin the vectorised versions above)
# --------------------------------------------------------------------------

def _sig1(x: float) -> float:
    import math
    return 1.0 / (1.0 + math.exp(-x)) if x >= 0 else math.exp(x) / (1.0 + math.exp(x))


def window_forward_loops(Q, K, V, W, scale, bias=None):
    Q, K, V = np.asarray(Q, np.float64), np.asarray(K, np.float64), np.asarray(V, np.float64)
    B, T, H, D = Q.shape
    msg = np.zeros((B, T, H, D))
    tau = np.zeros((B, T, H, W))
    for b in range(B):
        for t in range(T):
            for h in range(H):
                for w in range(W):
                    s = t - (W - w)
                    if s < 0:
                        continue
                    dot = 0.0
                    for d in range(D):
                        dot += float(Q[b, t, h, d]) * float(K[b, s, h, d])
                    x = dot / scale
                    if bias is not None:
                        x += float(bias[b, t, w])
                    p = _sig1(x)
                    tau[b, t, h, w] = p
                    for d in range(D):
                        msg[b, t, h, d] += p * float(V[b, s, h, d])
    return msg, tau


def global_forward_loops(Q, K, V, scale, bias=None, W_local=None):
    """Loops over (b, t, h, s) from the definitions of model.py:217-238.
    With W_local, also returns tau_local from its index definition
    (model.py:235-236: tau[..., :T].flip(-1)[..., :min(W_local, T)]): slot j
    of every query row holds the weight of key s = T-1-j, zero where that key
    lies after the query (s > t)."""
    Q, K, V = np.asarray(Q, np.float64), np.asarray(K, np.float64), np.asarray(V, np.float64)
    B, T, H, D = Q.shape
    out = np.zeros((B, T, H, D))
    Wl = None if W_local is None else min(W_local, T)
    tl = None if Wl is None else np.zeros((B, T, H, Wl))
    for b in range(B):
        for h in range(H):
            for t in range(T):
                acc = np.zeros(D)
                mass = 0.0
                for s in range(t + 1):
                    x = float(Q[b, t, h] @ K[b, s, h]) / scale
                    if bias is not None:
                        x += float(bias[b, t, s])
                    p = _sig1(x)
                    mass += p
                    acc += p * V[b, s, h]
                out[b, t, h] = acc / max(mass, MASS_EPS)
                if tl is not None:
                    for j in range(Wl):
                        s = T - 1 - j
                        if s <= t:
                            x = float(Q[b, t, h] @ K[b, s, h]) / scale
                            if bias is not None:
                                x += float(bias[b, t, s])
                            tl[b, t, h, j] = _sig1(x)
    return out if tl is None else (out, tl)


# Which check pins each function (all in tests/test_oracle.py).
PINS = {
    "window_forward": "brute-force loops; torch unfold restatement; K=0 -> tau=1/2; "
                      "bias +-inf -> tau 1/0; zero on s<0; prefix invariance",
    "window_backward": "torch autograd through the unfold restatement (fp64); "
                       "central finite differences; V-linearity of dV",
    "window_backward_normalized": "torch autograd through unfold + tau-mass; finite differences",
    "normalize_mass/normalize_count": "K=0 closed form (window mean of V); valid_count formula",
    "global_forward": "brute-force loops (tau_local from its index definition); diag-masked global == "
                      "window W=T; torch einsum restatement",
    "global_backward": "torch autograd through the einsum restatement; finite differences",
    "decode_step": "equals last rows of window_forward + tau-mass / valid-count normalisation over "
                   "a sequence; with self_kv, the rows of global_forward",
    "rope_apply": "norm preservation; relative-position identity; adjoint = inverse rotation",
}
