"""Pins for the CPU oracle (runs on CPU, no GPU).

Every oracle function is checked against something other than itself:
brute-force loops written from the index definitions, the torch ``unfold``
restatement of the reference CPU path with autograd, central finite
differences, library routines and closed forms.  The last test plants
plausible mistakes in copies of the oracle and shows that these pins fail.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tension_oracle as O
from oracle import torch_ref as R


def rnd(seed, *shape, scale=1.0):
    g = np.random.default_rng(seed)
    return g.standard_normal(shape) * scale


def close(a, b, tol=1e-10):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    err = np.max(np.abs(a - b)) if a.size else 0.0
    assert err <= tol, f"max abs err {err:.3e} > {tol:.1e}"


def t64(a, grad=False):
    return torch.tensor(np.asarray(a), dtype=torch.float64, requires_grad=grad)


# ---------------------------------------------------------------- forward

@pytest.mark.parametrize("B,T,H,D,W", [(2, 9, 2, 4, 3), (1, 5, 1, 3, 7), (1, 6, 2, 2, 1)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_window_forward_matches_loops(B, T, H, D, W, with_bias):
    Q, K, V = rnd(1, B, T, H, D), rnd(2, B, T, H, D), rnd(3, B, T, H, D)
    bias = rnd(4, B, T, W) if with_bias else None
    msg, tau = O.window_forward(Q, K, V, W, math.sqrt(D), bias)
    msg2, tau2 = O.window_forward_loops(Q, K, V, W, math.sqrt(D), bias)
    close(msg, msg2)
    close(tau, tau2)


@pytest.mark.parametrize("with_bias", [False, True])
def test_window_forward_matches_torch_unfold(with_bias):
    B, T, H, D, W = 2, 32, 4, 16, 8
    Q, K, V = rnd(5, B, T, H, D), rnd(6, B, T, H, D), rnd(7, B, T, H, D)
    bias = rnd(8, B, T, W) * 0.5 if with_bias else None
    msg, tau = O.window_forward(Q, K, V, W, 4.0, bias)
    m2, t2 = R.unfold_tension(t64(Q), t64(K), t64(V), W, 4.0, True,
                              None if bias is None else t64(bias))
    close(msg, m2.numpy())
    close(tau, t2.numpy())


def test_sigmoid_matches_library():
    from scipy.special import expit
    x = np.concatenate([rnd(9, 1000) * 30, [0.0, -800.0, 800.0, 1e-12]])
    close(O.sigmoid(x), expit(x), 1e-15)


def test_window_invariants():
    B, T, H, D, W = 2, 20, 3, 8, 6
    V = rnd(10, B, T, H, D)
    Q = rnd(11, B, T, H, D)
    K0 = np.zeros((B, T, H, D))
    msg, tau = O.window_forward(Q, K0, V, W, 2.0)
    t = np.arange(T)[:, None]
    w = np.arange(W)[None, :]
    valid = (t + w >= W)
    # K = 0 => tau = 1/2 exactly on valid slots, 0 elsewhere
    close(tau, np.broadcast_to(0.5 * valid[None, :, None, :], tau.shape), 0.0)
    # tau-mass output = plain mean of V over the strictly-past window
    out, mass = O.normalize_mass(msg, tau)
    want = np.zeros_like(V)
    for tt in range(1, T):
        lo = max(0, tt - W)
        want[:, tt] = V[:, lo:tt].mean(axis=1)
    close(out, want, 1e-12)
    close(mass, 0.5 * valid.sum(-1)[None, :, None] * np.ones((B, 1, H)))
    # valid-count normalisation: raw / max(min(t,W),1), here = mean/2
    close(O.normalize_count(msg, W), want * 0.5 * np.minimum(t[:, 0], W).clip(1)[None, :, None, None]
          / np.maximum(np.minimum(t[:, 0], W), 1)[None, :, None, None], 1e-12)
    # bias +-inf saturates tau to 1/0 on valid slots
    K = rnd(12, B, T, H, D)
    _, tau_hi = O.window_forward(Q, K, V, W, 2.0, np.full((B, T, W), 1e4))
    _, tau_lo = O.window_forward(Q, K, V, W, 2.0, np.full((B, T, W), -1e4))
    close(tau_hi, np.broadcast_to(valid[None, :, None, :], tau_hi.shape).astype(float), 0.0)
    close(tau_lo, np.zeros_like(tau_lo), 0.0)
    # bias = 0 is the unbiased path, exactly
    m_a, t_a = O.window_forward(Q, K, V, W, 2.0)
    m_b, t_b = O.window_forward(Q, K, V, W, 2.0, np.zeros((B, T, W)))
    close(m_a, m_b, 0.0)
    close(t_a, t_b, 0.0)
    # causality / prefix invariance
    m_p, t_p = O.window_forward(Q[:, :11], K[:, :11], V[:, :11], W, 2.0)
    close(m_a[:, :11], m_p, 0.0)
    close(t_a[:, :11], t_p, 0.0)


def test_valid_count_formula():
    # model.py:159-163 counts slots with t + w >= W and clamps at 1
    for T, W in [(10, 4), (3, 8), (64, 64)]:
        t = np.arange(T)[:, None]
        w = np.arange(W)[None, :]
        direct = np.maximum((t + w >= W).sum(-1), 1)
        close(O.valid_count(T, W), direct, 0.0)


# ---------------------------------------------------------------- backward

@pytest.mark.parametrize("with_bias,with_dtau", [(False, False), (True, False),
                                                 (False, True), (True, True)])
def test_window_backward_matches_autograd(with_bias, with_dtau):
    B, T, H, D, W = 2, 24, 4, 16, 8
    Q, K, V = rnd(20, B, T, H, D), rnd(21, B, T, H, D), rnd(22, B, T, H, D)
    dmsg = rnd(23, B, T, H, D)
    dtau = rnd(24, B, T, H, W) * 0.1 if with_dtau else None
    bias = rnd(25, B, T, W) * 0.5 if with_bias else None
    got = O.window_backward(Q, K, V, W, 4.0, dmsg, dtau, bias)
    q, k, v = t64(Q, True), t64(K, True), t64(V, True)
    msg, tau = R.unfold_tension(q, k, v, W, 4.0, True, None if bias is None else t64(bias))
    loss = (msg * t64(dmsg)).sum()
    if dtau is not None:
        loss = loss + (tau * t64(dtau)).sum()
    loss.backward()
    for g, x in zip(got, (q, k, v)):
        close(g, x.grad.numpy(), 1e-10)


@pytest.mark.parametrize("with_dtau", [False, True])
def test_window_backward_normalized_matches_autograd(with_dtau):
    B, T, H, D, W = 2, 20, 2, 8, 6
    Q, K, V = rnd(30, B, T, H, D), rnd(31, B, T, H, D), rnd(32, B, T, H, D)
    dout = rnd(33, B, T, H, D)
    dtau = rnd(34, B, T, H, W) * 0.1 if with_dtau else None
    bias = rnd(35, B, T, W) * 0.3
    got = O.window_backward_normalized(Q, K, V, W, 3.0, dout, dtau, bias)
    q, k, v = t64(Q, True), t64(K, True), t64(V, True)
    msg, tau = R.unfold_tension(q, k, v, W, 3.0, True, t64(bias))
    out = R.normalize_mass(msg, tau)
    loss = (out * t64(dout)).sum()
    if dtau is not None:
        loss = loss + (tau * t64(dtau)).sum()
    loss.backward()
    for g, x in zip(got, (q, k, v)):
        close(g, x.grad.numpy(), 1e-10)


def _fd_check(f, arrays, grads, eps=1e-6, tol=1e-6, n=12, seed=0):
    """Central differences of scalar f at n random coordinates of each array."""
    g = np.random.default_rng(seed)
    for a, ga in zip(arrays, grads):
        for _ in range(n):
            idx = tuple(g.integers(0, s) for s in a.shape)
            old = a[idx]
            a[idx] = old + eps
            fp = f()
            a[idx] = old - eps
            fm = f()
            a[idx] = old
            fd = (fp - fm) / (2 * eps)
            assert abs(fd - ga[idx]) <= tol * max(1.0, abs(fd)), (idx, fd, ga[idx])


def test_window_backward_finite_differences():
    B, T, H, D, W = 1, 10, 2, 4, 4
    Q, K, V = rnd(40, B, T, H, D), rnd(41, B, T, H, D), rnd(42, B, T, H, D)
    dout, dtau, bias = rnd(43, B, T, H, D), rnd(44, B, T, H, W), rnd(45, B, T, W)

    def loss():
        msg, tau = O.window_forward(Q, K, V, W, 2.0, bias)
        out, _ = O.normalize_mass(msg, tau)
        return float((out * dout).sum() + (tau * dtau).sum())

    grads = O.window_backward_normalized(Q, K, V, W, 2.0, dout, dtau, bias)
    _fd_check(loss, (Q, K, V), grads)


def test_dv_is_linear_in_dout():
    B, T, H, D, W = 1, 12, 2, 4, 5
    Q, K, V = rnd(46, B, T, H, D), rnd(47, B, T, H, D), rnd(48, B, T, H, D)
    d1, d2 = rnd(49, B, T, H, D), rnd(50, B, T, H, D)
    a = O.window_backward(Q, K, V, W, 2.0, d1)
    b = O.window_backward(Q, K, V, W, 2.0, d2)
    c = O.window_backward(Q, K, V, W, 2.0, 2 * d1 - 3 * d2)
    for x, y, z in zip(a, b, c):
        close(z, 2 * x - 3 * y, 1e-12)


# ---------------------------------------------------------------- global

@pytest.mark.parametrize("with_bias", [False, True])
def test_global_forward_matches_loops_and_torch(with_bias):
    B, T, H, D = 2, 12, 2, 4
    Q, K, V = rnd(60, B, T, H, D), rnd(61, B, T, H, D), rnd(62, B, T, H, D)
    bias = rnd(63, B, T, T) if with_bias else None
    out, mass, tl = O.global_forward(Q, K, V, 2.0, bias, W_local=5)
    close(out, O.global_forward_loops(Q, K, V, 2.0, bias), 1e-12)
    o2, tl2 = R.global_block(t64(Q), t64(K), t64(V), 2.0,
                             None if bias is None else t64(bias), W_local=5)
    close(out, o2.numpy(), 1e-12)
    close(tl, tl2.numpy(), 1e-12)


@pytest.mark.parametrize("T,Wl", [(12, 5), (9, 9), (7, 20)])
def test_tau_local_matches_index_loops(T, Wl):
    """tau_local (model.py:235-236) from a loop over its index definition,
    slot j = key T-1-j for every query row: not the flip / slice expression
    the oracle uses.  A query-relative reading (slot j = key t-j) differs."""
    B, H, D = 2, 2, 4
    Q, K, V = rnd(160 + T, B, T, H, D), rnd(161 + T, B, T, H, D), rnd(162 + T, B, T, H, D)
    bias = rnd(163 + T, B, T, T) * 0.5
    _, _, tl = O.global_forward(Q, K, V, 2.0, bias, W_local=Wl)
    out_l, tl_l = O.global_forward_loops(Q, K, V, 2.0, bias, W_local=Wl)
    assert tl.shape == (B, T, H, min(Wl, T))
    close(tl, tl_l, 1e-12)
    # the last query sees every key: its row is the full tau row reversed
    x = np.einsum("bhd,bshd->bhs", Q[:, -1], K) / 2.0 + bias[:, -1][:, None, :]
    close(tl[:, -1], (1 / (1 + np.exp(-x)))[..., ::-1][..., :min(Wl, T)], 1e-12)
    # query-relative slots (key t-j) are a different quantity
    rel = np.zeros_like(tl)
    for t in range(T):
        for j in range(min(Wl, T)):
            if t - j >= 0:
                xx = np.einsum("bhd,bhd->bh", Q[:, t], K[:, t - j]) / 2.0 + bias[:, t, t - j][:, None]
                rel[:, t, :, j] = 1 / (1 + np.exp(-xx))
    assert np.max(np.abs(rel - tl)) > 1e-3


def test_global_without_diagonal_equals_full_window():
    B, T, H, D = 2, 16, 2, 8
    Q, K, V = rnd(64, B, T, H, D), rnd(65, B, T, H, D), rnd(66, B, T, H, D)
    nodiag = np.zeros((B, T, T))
    nodiag[:, np.arange(T), np.arange(T)] = -1e30
    out, mass, _ = O.global_forward(Q, K, V, 2.5, nodiag)
    msg, tau = O.window_forward(Q, K, V, T, 2.5)
    out_w, mass_w = O.normalize_mass(msg, tau)
    close(out, out_w, 1e-12)
    close(mass, mass_w, 1e-12)


@pytest.mark.parametrize("with_bias,with_dtau", [(False, False), (True, True)])
def test_global_backward_matches_autograd(with_bias, with_dtau):
    B, T, H, D, Wl = 2, 14, 2, 4, 5
    Q, K, V = rnd(70, B, T, H, D), rnd(71, B, T, H, D), rnd(72, B, T, H, D)
    dout = rnd(73, B, T, H, D)
    bias = rnd(74, B, T, T) * 0.5 if with_bias else None
    dtl = rnd(75, B, T, H, Wl) * 0.1 if with_dtau else None
    got = O.global_backward(Q, K, V, 2.0, dout, bias, dtl)
    q, k, v = t64(Q, True), t64(K, True), t64(V, True)
    out, tl = R.global_block(q, k, v, 2.0, None if bias is None else t64(bias), W_local=Wl)
    loss = (out * t64(dout)).sum()
    if dtl is not None:
        loss = loss + (tl * t64(dtl)).sum()
    loss.backward()
    for g, x in zip(got, (q, k, v)):
        close(g, x.grad.numpy(), 1e-10)


def test_global_backward_finite_differences():
    B, T, H, D, Wl = 1, 8, 1, 4, 3
    Q, K, V = rnd(76, B, T, H, D), rnd(77, B, T, H, D), rnd(78, B, T, H, D)
    dout, dtl, bias = rnd(79, B, T, H, D), rnd(80, B, T, H, Wl), rnd(81, B, T, T)

    def loss():
        out, _, tl = O.global_forward(Q, K, V, 2.0, bias, Wl)
        return float((out * dout).sum() + (tl * dtl).sum())

    grads = O.global_backward(Q, K, V, 2.0, dout, bias, dtl)
    _fd_check(loss, (Q, K, V), grads)


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("prefill", [0, 3, 8])
def test_decode_equals_last_row_of_window(prefill):
    N, H, D, W, S = 3, 2, 4, 8, 13
    L = prefill + S
    q, k, v = rnd(90, N, L, H, D), rnd(91, N, L, H, D), rnd(92, N, L, H, D)
    kc = np.zeros((N, H, W, D))
    vc = np.zeros((N, H, W, D))
    pos = np.zeros(N, dtype=np.int64)
    for t in range(prefill):
        kc, vc, pos = O.decode_append(kc, vc, pos, k[:, t], v[:, t], W)
    msg, tau = O.window_forward(q, k, v, W, 2.0)
    out_w, _ = O.normalize_mass(msg, tau)
    for t in range(prefill, L):
        o, tt = O.decode_step(q[:, t], kc, vc, pos, W, 2.0)
        close(o, out_w[:, t], 1e-12)
        close(tt, tau[:, t], 1e-12)
        kc, vc, pos = O.decode_append(kc, vc, pos, k[:, t], v[:, t], W)


@pytest.mark.parametrize("prefill", [0, 5])
def test_decode_count_equals_window_count_rows(prefill):
    N, H, D, W, S = 2, 2, 4, 6, 9
    L = prefill + S
    q, k, v = rnd(93, N, L, H, D), rnd(94, N, L, H, D), rnd(95, N, L, H, D)
    kc, vc = np.zeros((N, H, W, D)), np.zeros((N, H, W, D))
    pos = np.zeros(N, dtype=np.int64)
    for t in range(prefill):
        kc, vc, pos = O.decode_append(kc, vc, pos, k[:, t], v[:, t], W)
    msg, _ = O.window_forward(q, k, v, W, 2.0)
    ref = O.normalize_count(msg, W)
    raw_o = None
    for t in range(prefill, L):
        o, _ = O.decode_step(q[:, t], kc, vc, pos, W, 2.0, normalize="count")
        close(o, ref[:, t], 1e-12)
        raw_o, _ = O.decode_step(q[:, t], kc, vc, pos, W, 2.0, normalize=False)
        close(raw_o, msg[:, t], 1e-12)
        kc, vc, pos = O.decode_append(kc, vc, pos, k[:, t], v[:, t], W)


def test_decode_self_equals_global_rows():
    """A cache that holds every earlier token plus the new token as a key is
    the global block (keys s <= t), row by row."""
    N, H, D, L = 2, 3, 4, 11
    W = L  # never wraps
    q, k, v = rnd(96, N, L, H, D), rnd(97, N, L, H, D), rnd(98, N, L, H, D)
    ref, _, _ = O.global_forward(q, k, v, 2.0)
    kc, vc = np.zeros((N, H, W, D)), np.zeros((N, H, W, D))
    pos = np.zeros(N, dtype=np.int64)
    for t in range(L):
        o, _ = O.decode_step(q[:, t], kc, vc, pos, W, 2.0, normalize=True, self_kv=(k[:, t], v[:, t]))
        close(o, ref[:, t], 1e-12)
        kc, vc, pos = O.decode_append(kc, vc, pos, k[:, t], v[:, t], W)


# ---------------------------------------------------------------- rope

def test_rope_properties():
    B, T, H, D = 1, 40, 2, 16
    cos, sin = O.rope_tables(64, D)
    x = rnd(100, B, T, H, D)
    y = O.rope_apply(x, cos, sin)
    close(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), 1e-5)
    # adjoint undoes the rotation (orthogonal map) up to the fp32 table error
    close(O.rope_apply_adjoint(y, cos, sin), x, 1e-5)
    # relative-position identity: <R_t q, R_s k> depends on t-s only
    q1 = np.broadcast_to(rnd(101, 1, 1, 1, D), (1, T, 1, D))
    k1 = np.broadcast_to(rnd(102, 1, 1, 1, D), (1, T, 1, D))
    rq, rk = O.rope_apply(q1, cos, sin), O.rope_apply(k1, cos, sin)
    d_a = (rq[0, 10, 0] * rk[0, 7, 0]).sum()
    d_b = (rq[0, 30, 0] * rk[0, 27, 0]).sum()
    assert abs(d_a - d_b) < 1e-4
    # pos 0 is the identity
    close(rq[0, 0, 0], q1[0, 0, 0], 0.0)
    # torch restatement agrees
    yt = R.rope(t64(x), torch.tensor(cos), torch.tensor(sin))
    close(y, yt.numpy(), 1e-12)


def test_rope_tables_match_torch_buffers():
    # model.py:68-73 computes the tables in float32 with torch; numpy's
    # float32 pow may differ by an ulp of theta, i.e. ~ S*ulp in the angle
    D, S = 64, 128
    half = D // 2
    theta = 1.0 / (10000 ** (torch.arange(0, half).float() / half))
    freqs = torch.outer(torch.arange(S).float(), theta)
    cos, sin = O.rope_tables(S, D)
    close(cos, freqs.cos().numpy(), 2e-5)
    close(sin, freqs.sin().numpy(), 2e-5)


# ---------------------------------------------------------------- the pins bite

def test_pins_catch_planted_mistakes():
    """Mutated copies of the oracle must FAIL the checks used above."""
    B, T, H, D, W = 1, 9, 2, 4, 3
    Q, K, V = rnd(110, B, T, H, D), rnd(111, B, T, H, D), rnd(112, B, T, H, D)
    ref_msg, ref_tau = O.window_forward_loops(Q, K, V, W, 2.0)

    # (a) window order reversed (w=0 newest, as in tension_lm.py:126)
    msg, tau = O.window_forward(Q, K, V, W, 2.0)
    with pytest.raises(AssertionError):
        close(tau[..., ::-1], ref_tau)
    # (b) self included in the local window (off-by-one: s = t - W + w + 1)
    Kshift = np.concatenate([K[:, 1:], np.zeros_like(K[:, :1])], axis=1)
    Vshift = np.concatenate([V[:, 1:], np.zeros_like(V[:, :1])], axis=1)
    bad_msg, _ = O.window_forward(Q, Kshift, Vshift, W, 2.0)
    with pytest.raises(AssertionError):
        close(bad_msg, ref_msg)
    # (c) dropped dtau term / wrong sign in dK against autograd
    dmsg, dtau = rnd(113, B, T, H, D), rnd(114, B, T, H, W)
    q, k, v = t64(Q, True), t64(K, True), t64(V, True)
    m, t = R.unfold_tension(q, k, v, W, 2.0, True)
    ((m * t64(dmsg)).sum() + (t * t64(dtau)).sum()).backward()
    dQ_nodtau, _, _ = O.window_backward(Q, K, V, W, 2.0, dmsg, None)
    with pytest.raises(AssertionError):
        close(dQ_nodtau, q.grad.numpy(), 1e-10)
    _, dK, _ = O.window_backward(Q, K, V, W, 2.0, dmsg, dtau)
    with pytest.raises(AssertionError):
        close(-dK, k.grad.numpy(), 1e-10)
    # (d) transposed global scores (k.q^T instead of q.k^T)
    out, _, _ = O.global_forward(Q, K, V, 2.0)
    bad, _, _ = O.global_forward(K, Q, V, 2.0)
    with pytest.raises(AssertionError):
        close(bad, out, 1e-12)
