"""Host side of the MI355X sigmoid-tension op: autograd Functions over the
C ABI of libtension_hip.so.

Drop-in for ``triton_tension.ops`` of the reference:

    from bozo_amd import causal_tension
    out          = causal_tension(Q, K, V, window=64, scale=8.0)
    out, tau     = causal_tension(Q, K, V, window=64, scale=8.0, return_tau=True)

Same name, arguments, defaults, return types and dtypes as
``triton_tension/ops.py:192-224``; ``_CausalTensionFn`` keeps the reference
Function's arity and gradient semantics (``ops.py:73-187``).  Differences,
all additive or stricter:

* ``normalize=`` (keyword only, default ``None`` = the reference's raw
  ``sum tau*v``): ``"mass"`` fuses the tau-mass normalisation of
  ``model.py:257-258,281-282`` into the kernel (forward and backward),
  ``"count"`` the valid-count one of ``model.py:264``.
* There is no CPU fallback.  The reference routes CPU and float64 inputs to a
  PyTorch unfold path (``ops.py:217-219``); here CPU tensors raise, and
  float64 runs on the GPU through the exact kernels, so ``gradcheck`` in
  float64 exercises the HIP backward itself.
* Inputs may be strided (unit innermost stride) and of mixed float dtypes;
  each is read in its own dtype (no upcast copies).  Outputs are returned in
  ``Q.dtype`` (``ops.py:122-124``); gradients in each input's dtype
  (``ops.py:186-187``).
"""
from __future__ import annotations

import math
from typing import Optional

import torch
from torch import Tensor

from . import _lib as L

_NORMS = {None: 0, "raw": 0, "mass": L.NORM_MASS, "count": L.NORM_COUNT}


def _on_gpu(*ts: Optional[Tensor]) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "bozo_amd tension ops run on the ROCm GPU only (got a CPU tensor); "
                "the CPU reference lives in oracle/ and is test infrastructure")


def _same_device(ref: Tensor, *ts: Optional[Tensor]) -> None:
    """The kernels read every operand on the device of the first one."""
    for t in ts:
        if t is not None and t.device != ref.device:
            raise ValueError(f"all tensors must be on {ref.device}, got one on {t.device}")


def _rows(t: Optional[Tensor]) -> Optional[Tensor]:
    """Unit innermost stride is all the kernels need."""
    if t is None:
        return None
    if t.dim() == 0 or t.stride(-1) != 1 or t.numel() == 0:
        return t.contiguous()
    return t


def _acc_code(*ts: Tensor) -> int:
    return L.F64 if any(t.dtype == torch.float64 for t in ts) else L.F32


def _side(t: Optional[Tensor], like: Tensor) -> Optional[Tensor]:
    """Side inputs (bias) are kept in float32, as the reference does
    (ops.py:93), or float64 for float64 calls."""
    if t is None:
        return None
    return _rows(t.to(torch.float64 if like.dtype == torch.float64 else torch.float32))


def _stream(t: Tensor):
    return L.stream_handle(t.device)


def _ws(nbytes: int, dev) -> Optional[Tensor]:
    return torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes > 0 else None


def _ptr(t: Optional[Tensor]):
    return None if t is None else t.data_ptr()


def _grads_like(*ts: Tensor):
    """Fresh contiguous gradient buffers (the layout the fake kernels of the
    registered operators report, whatever the inputs' strides)."""
    return tuple(torch.empty(t.shape, dtype=t.dtype, device=t.device) for t in ts)


# ----------------------------------------------------------------- local window

_EXACT_WARNED = set()


def _note_exact_path(what: str, Q: Tensor, K: Tensor, V: Tensor, pairs: int) -> None:
    """Warn once per dtype / head-dim combination when a large call ran on the
    exact kernels (one thread per row, no MFMA): mixes other than float32
    Q / K with a bf16 or float32 V, head dims other than 32 / 64 or
    unaligned rows.  float64 is exact on purpose."""
    if pairs < (1 << 20) or Q.dtype == torch.float64:
        return
    if int(L.lib().tension_last_kernel()) != L.KERNEL_EXACT:
        return
    key = (what, Q.dtype, K.dtype, V.dtype, Q.shape[-1])
    if key in _EXACT_WARNED:
        return
    _EXACT_WARNED.add(key)
    import warnings
    warnings.warn(f"{what}: Q/K/V {Q.dtype}/{K.dtype}/{V.dtype} with head dim {Q.shape[-1]} ran on the exact "
                  "(non-MFMA) kernels, one thread per row; the MFMA kernels take bf16, float16, or float32 "
                  "Q/K with a bf16 or float32 V, at head dim 32 or 64 with 16-byte aligned rows", RuntimeWarning,
                  stacklevel=3)


def _window_fwd(Q, K, V, W, scale, tau, bias, flags, mass):
    B, T, H, D = Q.shape
    out = torch.empty(B, T, H, D, dtype=Q.dtype, device=Q.device)
    with torch.cuda.device(Q.device):
        L.check(L.lib().tension_window_fwd(
            L.buf(Q), L.buf(K), L.buf(V), L.buf(out), L.buf(tau), L.buf(bias), L.buf(mass),
            B, T, H, D, W, float(scale), flags, _stream(Q)), "tension_window_fwd")
    _note_exact_path("causal_tension", Q, K, V, B * T * H * min(int(W), T))
    return out


class _CausalTensionFn(torch.autograd.Function):
    """Counterpart of the reference's ``_CausalTensionFn`` (ops.py:73-187)."""

    @staticmethod
    def forward(ctx, Q, K, V, W: int, scale: float, return_tau: bool, bias, normalize=None):
        B, T, H, D = Q.shape
        flags = _NORMS[normalize]
        Bias = _side(bias, Q)
        if Bias is not None and tuple(Bias.shape) != (B, T, W):
            raise ValueError(f"bias must be [B, T, W]=[{B}, {T}, {W}], got {tuple(Bias.shape)}")
        tau = torch.empty(B, T, H, W, dtype=Q.dtype, device=Q.device) if return_tau else None
        # the backward recomputes tau from the inputs; with float32 Q / K
        # under tau-mass it takes the per-query coefficients from the
        # forward's float32 rows and tau mass where that is the faster dQ
        # (tension_window_bwd_saved: one pass over the band instead of two)
        rows = _saved_rows_flow(Q, K, V, W, flags)
        mass = torch.empty(B, T, H, dtype=torch.float32, device=Q.device) if rows else None
        out = _window_fwd(Q, K, V, W, scale, tau, Bias, flags, mass)
        if rows:
            ctx.save_for_backward(Q, K, V, Bias, out, mass)
        else:
            ctx.save_for_backward(Q, K, V, Bias)
        ctx.rows = rows
        ctx.W, ctx.scale, ctx.flags = W, scale, flags
        ctx.return_tau = return_tau
        if return_tau:
            return out, tau
        return out

    @staticmethod
    def backward(ctx, *grads):
        if ctx.rows:
            Q, K, V, Bias, out, mass = ctx.saved_tensors
        else:
            (Q, K, V, Bias), out, mass = ctx.saved_tensors, None, None
        dTau = grads[1] if ctx.return_tau else None
        dQ, dK, dV = _window_bwd(Q, K, V, grads[0], dTau, Bias, ctx.W, ctx.scale, ctx.flags, out, mass)
        return dQ, dK, dV, None, None, None, None, None


def _saved_rows_flow(Q: Tensor, K: Tensor, V: Tensor, W: int, flags: int) -> bool:
    """Tau-mass with float32 Q / K at head dim 32 / 64, where the backward
    takes its coefficients from the forward's rows: with a bf16 V (the
    reference's autocast flow) for windows wider than 64 (narrower bands
    form them in registers, which is faster), with a float32 V at every
    window (its dQ kernel keeps no band in registers)."""
    if not (flags & L.NORM_MASS) or Q.dtype != torch.float32 or K.dtype != torch.float32 \
            or Q.shape[-1] not in (32, 64):
        return False
    if V.dtype == torch.bfloat16:
        return W > 64
    return V.dtype == torch.float32


def _window_bwd(Q, K, V, dOut, dTau, Bias, W, scale, flags, out=None, mass=None):
    B, T, H, D = Q.shape
    dOut = _rows(dOut) if dOut is not None else torch.zeros_like(Q)
    dTau = _rows(dTau)
    dQ, dK, dV = _grads_like(Q, K, V)
    lib = L.lib()
    ws = _ws(lib.tension_window_bwd_workspace(B, T, H, _acc_code(Q, K, V), flags), Q.device)
    with torch.cuda.device(Q.device):
        if out is not None:
            L.check(lib.tension_window_bwd_saved(
                L.buf(Q), L.buf(K), L.buf(V), L.buf(dOut), L.buf(dTau), L.buf(Bias), L.buf(out),
                L.buf(mass), L.buf(dQ), L.buf(dK), L.buf(dV), _ptr(ws), B, T, H, D, W,
                float(scale), flags, _stream(Q)), "tension_window_bwd_saved")
        else:
            L.check(lib.tension_window_bwd(
                L.buf(Q), L.buf(K), L.buf(V), L.buf(dOut), L.buf(dTau), L.buf(Bias),
                L.buf(dQ), L.buf(dK), L.buf(dV), _ptr(ws), B, T, H, D, W,
                float(scale), flags, _stream(Q)), "tension_window_bwd")
    return dQ, dK, dV


def causal_tension(Q: Tensor, K: Tensor, V: Tensor, window: int, scale: float,
                   return_tau: bool = False, bias: Optional[Tensor] = None, *,
                   normalize: Optional[str] = None):
    """Fused causal sigmoid tension on the MI355X.

    Args:
        Q, K, V    : [B, T, H, HD] on the GPU (float32 / bfloat16 / float16 /
                     float64; bf16 with HD=64 takes the MFMA kernels).
        window     : causal look-back W (keys t-W .. t-1).
        scale      : dot-product divisor (typically sqrt(HD)).
        return_tau : also emit tau [B, T, H, W] (w=0 oldest).
        bias       : optional [B, T, W] pre-sigmoid bias, broadcast over H.
        normalize  : None (raw sum tau*v, the reference contract), "mass"
                     or "count" (fused normalisations).
    Returns:
        out [B, T, H, HD] in Q.dtype, and tau [B, T, H, W] when return_tau.
    """
    _on_gpu(Q, K, V, bias)
    if Q.dim() != 4 or K.shape != Q.shape or V.shape != Q.shape:
        raise ValueError(f"Q, K, V must share one [B, T, H, HD] shape, got "
                         f"{tuple(Q.shape)}, {tuple(K.shape)}, {tuple(V.shape)}")
    _same_device(Q, K, V, bias)
    if normalize not in _NORMS:
        raise ValueError(f"normalize must be one of {list(_NORMS)}")
    if int(window) < 1:
        raise ValueError("window must be >= 1")
    if torch.compiler.is_compiling():  # the registered op, which torch.compile traces through
        Bias = _side(bias, Q)
        out, tau = torch.ops.bozo.window_fwd(Q, K, V, int(window), float(scale), bool(return_tau), Bias,
                                             _NORMS[normalize])
        return (out, tau) if return_tau else out
    return _CausalTensionFn.apply(_rows(Q), _rows(K), _rows(V), int(window), float(scale),
                                  bool(return_tau), bias, normalize)


# ----------------------------------------------------------------- global block

class _GlobalTensionFn(torch.autograd.Function):
    """Full-causal (diagonal included), tau-mass-normalised block; replaces
    the einsum path of model.py:217-238."""

    @staticmethod
    def forward(ctx, Q, K, V, scale: float, bias, W_local):
        B, T, H, D = Q.shape
        Bias = _side(bias, Q)
        if Bias is not None and tuple(Bias.shape) != (B, T, T):
            raise ValueError(f"global bias must be [B, T, T]=[{B}, {T}, {T}], got {tuple(Bias.shape)}")
        Wl = 0 if W_local is None else min(int(W_local), T)
        out, tl, mass = _global_fwd(Q, K, V, scale, Bias, Wl)
        ctx.save_for_backward(Q, K, V, Bias, out, mass)
        ctx.scale, ctx.Wl = scale, Wl
        if tl is not None:
            return out, tl
        return out

    @staticmethod
    def backward(ctx, *grads):
        Q, K, V, Bias, out, mass = ctx.saved_tensors
        dTl = grads[1] if ctx.Wl > 0 else None
        dQ, dK, dV = _global_bwd(Q, K, V, grads[0], dTl, Bias, out, mass, ctx.Wl, ctx.scale)
        return dQ, dK, dV, None, None, None


def _global_fwd(Q, K, V, scale, Bias, Wl):
    """out, tau_local (None when Wl is 0) and the tau mass of the global block."""
    B, T, H, D = Q.shape
    tl = torch.empty(B, T, H, Wl, dtype=Q.dtype, device=Q.device) if Wl > 0 else None
    out = torch.empty_like(Q)
    # the tau mass per query, kept with the output so the backward gets
    # its per-query coefficients from these rows (no band recompute)
    mass = torch.empty(B, T, H, dtype=torch.float32, device=Q.device)
    with torch.cuda.device(Q.device):
        L.check(L.lib().tension_global_fwd(
            L.buf(Q), L.buf(K), L.buf(V), L.buf(out), L.buf(tl), L.buf(Bias), L.buf(mass),
            B, T, H, D, Wl, float(scale), 0, _stream(Q)), "tension_global_fwd")
    _note_exact_path("global_tension", Q, K, V, B * H * T * (T + 1) // 2)
    return out, tl, mass


def _global_bwd(Q, K, V, dOut, dTl, Bias, out, mass, Wl, scale):
    B, T, H, D = Q.shape
    dOut = _rows(dOut) if dOut is not None else torch.zeros_like(Q)
    dTl = _rows(dTl) if Wl > 0 else None
    dQ, dK, dV = _grads_like(Q, K, V)
    lib = L.lib()
    ws = _ws(lib.tension_global_bwd_workspace(B, T, H, _acc_code(Q, K, V), 0), Q.device)
    with torch.cuda.device(Q.device):
        L.check(lib.tension_global_bwd(
            L.buf(Q), L.buf(K), L.buf(V), L.buf(dOut), L.buf(dTl), L.buf(Bias), L.buf(out),
            L.buf(mass), L.buf(dQ), L.buf(dK), L.buf(dV), _ptr(ws), B, T, H, D, Wl,
            float(scale), 0, _stream(Q)), "tension_global_bwd")
    return dQ, dK, dV


def global_tension(Q: Tensor, K: Tensor, V: Tensor, scale: float,
                   bias: Optional[Tensor] = None, W_local: Optional[int] = None):
    """Global layer of the reference (model.py:217-238) as one fused op.

    out = sum_{s<=t} tau*v / max(sum_{s<=t} tau, 1e-6),
    tau = sigmoid(q.k/scale + bias[b,t,s]).  With ``W_local`` also returns
    the reference's down-sampled ``tau_local`` [B,T,H,min(W_local,T)] whose
    slot j is key T-1-j (model.py:231-237)."""
    _on_gpu(Q, K, V, bias)
    if Q.dim() != 4 or K.shape != Q.shape or V.shape != Q.shape:
        raise ValueError("Q, K, V must share one [B, T, H, HD] shape")
    _same_device(Q, K, V, bias)
    if torch.compiler.is_compiling():  # the registered op, which torch.compile traces through
        B, T = Q.shape[:2]
        Bias = _side(bias, Q)
        if Bias is not None and tuple(Bias.shape) != (B, T, T):
            raise ValueError(f"global bias must be [B, T, T]=[{B}, {T}, {T}], got {tuple(Bias.shape)}")
        Wl = 0 if W_local is None else min(int(W_local), T)
        out, tl, _ = torch.ops.bozo.global_fwd(Q, K, V, float(scale), Bias, Wl)
        return (out, tl) if Wl > 0 else out
    return _GlobalTensionFn.apply(_rows(Q), _rows(K), _rows(V), float(scale), bias, W_local)


# ----------------------------------------------------------------- decode

_DECODE_NORMS = {True: L.NORM_MASS, "mass": L.NORM_MASS, "count": L.NORM_COUNT,
                 False: 0, None: 0, "raw": 0}


def _check_decode_operands(q, k_new, v_new, k_cache, v_cache, pos_in, pos_out, tau) -> None:
    """Shapes, devices and counter dtypes of one decode step.  The library
    sees strides only, so a cache, row or counter array smaller than q's
    [N, H, D] implies would be read past its end on the device."""
    if q.dim() != 3:
        raise ValueError(f"q must be [N, H, D], got {tuple(q.shape)}")
    N, H, D = q.shape
    if k_new.shape != q.shape or v_new.shape != q.shape:
        raise ValueError(f"k_new, v_new must be {tuple(q.shape)} like q, got "
                         f"{tuple(k_new.shape)}, {tuple(v_new.shape)}")
    if k_cache.dim() != 4 or (k_cache.shape[0], k_cache.shape[1], k_cache.shape[3]) != (N, H, D) \
            or v_cache.shape != k_cache.shape:
        raise ValueError(f"k_cache, v_cache must be [N, H, W, D] = [{N}, {H}, W, {D}] alike, got "
                         f"{tuple(k_cache.shape)}, {tuple(v_cache.shape)}")
    if pos_in.dtype != torch.int32 or (pos_out is not None and pos_out.dtype != torch.int32):
        raise TypeError("pos tensors must be int32")
    for name, t in (("pos_in", pos_in), ("pos_out", pos_out)):
        if t is not None and (tuple(t.shape) != (N,) or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous [N] = [{N}] tensor, got {tuple(t.shape)}")
    if tau is not None and tuple(tau.shape) != (N, H, k_cache.shape[2]):
        raise ValueError(f"tau must be [N, H, W] = [{N}, {H}, {k_cache.shape[2]}], got {tuple(tau.shape)}")
    _same_device(q, k_new, v_new, k_cache, v_cache, pos_in, pos_out, tau)


def decode_step(q: Tensor, k_new: Tensor, v_new: Tensor, k_cache: Tensor, v_cache: Tensor,
                pos_in: Tensor, pos_out: Optional[Tensor], scale: float,
                normalize=True, tau: Optional[Tensor] = None, include_self: bool = False) -> Tensor:
    """One streaming step (no autograd): attends q [N,H,D] to the cached
    window, then appends k_new/v_new at slot pos % W of the ring caches
    [N,H,W,D] (in place).  pos_in: int32 [N] on the GPU; pos_out receives
    pos_in + 1 when given.  ``normalize``: True / "mass" (tau mass), "count"
    (number of keys) or False / None (raw sum).  ``include_self``: the new
    token is a key too (a global layer's step; no tau then).  Returns out
    [N,H,D] in q.dtype."""
    _on_gpu(q, k_new, v_new, k_cache, v_cache, pos_in, pos_out, tau)
    _check_decode_operands(q, k_new, v_new, k_cache, v_cache, pos_in, pos_out, tau)
    N, H, D = q.shape
    W = k_cache.shape[2]
    if normalize not in _DECODE_NORMS:
        raise ValueError(f"normalize must be one of {list(_DECODE_NORMS)}")
    flags = _DECODE_NORMS[normalize] | (L.DECODE_SELF if include_self else 0)
    out = torch.empty_like(q)
    with torch.cuda.device(q.device):
        L.check(L.lib().tension_decode_step(
            L.buf(_rows(q)), L.buf(_rows(k_new)), L.buf(_rows(v_new)), L.buf(k_cache), L.buf(v_cache),
            L.buf(out), L.buf(tau), pos_in.data_ptr(), _ptr(pos_out), N, H, D, W, float(scale),
            flags, _stream(q)), "tension_decode_step")
    return out


class TensionDecodeCache:
    """Ring K/V cache of the last W tokens per (sequence, head) for streaming
    generation, with the position counters kept on the device (two buffers
    swapped each step, so a captured HIP graph can replay steps)."""

    def __init__(self, N: int, H: int, D: int, W: int, dtype=torch.bfloat16,
                 device="cuda", scale: Optional[float] = None, v_dtype=None):
        self.k = torch.zeros(N, H, W, D, dtype=dtype, device=device)
        self.v = torch.zeros(N, H, W, D, dtype=v_dtype or dtype, device=device)
        self.pos = [torch.zeros(N, dtype=torch.int32, device=device),
                    torch.zeros(N, dtype=torch.int32, device=device)]
        self.cur = 0
        self.W = W
        self.scale = float(scale) if scale is not None else math.sqrt(D)

    def step(self, q: Tensor, k_new: Tensor, v_new: Tensor, normalize=True,
             return_tau: bool = False, include_self: bool = False):
        tau = (torch.empty(q.shape[0], q.shape[1], self.W, dtype=q.dtype, device=q.device)
               if return_tau else None)
        pin, pout = self.pos[self.cur], self.pos[1 - self.cur]
        out = decode_step(q, k_new, v_new, self.k, self.v, pin, pout, self.scale, normalize, tau,
                          include_self)
        self.cur = 1 - self.cur
        return (out, tau) if return_tau else out


def autocast_inputs(*ts: Tensor):
    """Under CUDA autocast, the tensors in the autocast dtype: the dtype the
    reference's global block computes its einsums in (model.py:219,230);
    unchanged otherwise."""
    if ts[0].is_cuda and torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        return tuple(t.to(dt) for t in ts)
    return ts


# ----------------------------------------------------------------- RoPE

def _rope_call(x: Tensor, y: Tensor, cos: Tensor, sin: Tensor, pos_offset: int, inverse: int):
    B, T, H, D = x.shape
    with torch.cuda.device(x.device):
        L.check(L.lib().tension_rope(L.buf(x), L.buf(y), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
                                     B, T, H, D, pos_offset, inverse, _stream(x)), "tension_rope")


class _RopeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cos, sin, pos_offset, out_dtype):
        y = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
        _rope_call(x, y, cos, sin, pos_offset, 0)
        ctx.save_for_backward(cos, sin)
        ctx.pos_offset, ctx.in_dtype = pos_offset, x.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        cos, sin = ctx.saved_tensors
        dy = _rows(dy)
        dx = torch.empty(dy.shape, dtype=ctx.in_dtype, device=dy.device)
        _rope_call(dy, dx, cos, sin, ctx.pos_offset, 1)
        return dx, None, None, None, None


def rope(x: Tensor, cos: Tensor, sin: Tensor, pos_offset: int = 0,
         out_dtype: Optional[torch.dtype] = None) -> Tensor:
    """Half-split rotary embedding of x [B,T,H,D] with the model's float32
    cos/sin tables [S, D/2] (model.py:54-81).  ``out_dtype`` defaults to
    x.dtype (the reference promotes to float32 under autocast; pass
    torch.float32 to reproduce that)."""
    _on_gpu(x, cos, sin)
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise TypeError("cos/sin tables must be float32")
    if x.dim() != 4:
        raise ValueError(f"x must be [B, T, H, D], got {tuple(x.shape)}")
    _same_device(x, cos, sin)
    T, half = x.shape[1], x.shape[-1] // 2
    if cos.dim() != 2 or cos.shape[-1] != half or cos.shape[0] < pos_offset + T or sin.shape != cos.shape:
        raise ValueError("cos/sin tables do not cover the requested positions")
    if torch.compiler.is_compiling():  # the registered op, which torch.compile traces through
        return torch.ops.bozo.rope(x, cos.contiguous(), sin.contiguous(), int(pos_offset),
                                   out_dtype or x.dtype, 0)
    return _RopeFn.apply(_rows(x), cos.contiguous(), sin.contiguous(), int(pos_offset), out_dtype)


# ----------------------------------------------------------------- torch.library registration
#
# The same kernels as custom operators (bozo::window_fwd / window_bwd,
# global_fwd / global_bwd, rope) with fake-tensor shape functions and
# autograd formulas, so torch.compile traces a model through them without a
# graph break (the reference compiles its model, train.py:776-780).  The
# public functions call them while torch.compile traces and the autograd
# Functions above in eager mode.

@torch.library.custom_op("bozo::window_fwd", mutates_args=(), device_types="cuda")
def _op_window_fwd(Q: Tensor, K: Tensor, V: Tensor, window: int, scale: float, return_tau: bool,
                   bias: Optional[Tensor], flags: int) -> tuple[Tensor, Tensor]:
    B, T, H, _ = Q.shape
    if bias is not None and tuple(bias.shape) != (B, T, window):
        raise ValueError(f"bias must be [B, T, W]=[{B}, {T}, {window}], got {tuple(bias.shape)}")
    Q, K, V = _rows(Q), _rows(K), _rows(V)
    tau = torch.empty(B, T, H, window, dtype=Q.dtype, device=Q.device) if return_tau else Q.new_empty(0)
    out = _window_fwd(Q, K, V, window, scale, tau if return_tau else None, bias, flags, None)
    return out, tau


@_op_window_fwd.register_fake
def _(Q, K, V, window, scale, return_tau, bias, flags):
    B, T, H, D = Q.shape
    tau = Q.new_empty((B, T, H, window)) if return_tau else Q.new_empty(0)
    return Q.new_empty((B, T, H, D)), tau


@torch.library.custom_op("bozo::window_bwd", mutates_args=(), device_types="cuda")
def _op_window_bwd(Q: Tensor, K: Tensor, V: Tensor, dOut: Tensor, dTau: Optional[Tensor],
                   bias: Optional[Tensor], window: int, scale: float, flags: int) -> tuple[Tensor, Tensor, Tensor]:
    return _window_bwd(_rows(Q), _rows(K), _rows(V), dOut, dTau, bias, window, scale, flags)


@_op_window_bwd.register_fake
def _(Q, K, V, dOut, dTau, bias, window, scale, flags):
    return _grads_like(Q, K, V)


def _window_setup(ctx, inputs, output):
    Q, K, V, window, scale, return_tau, bias, flags = inputs
    ctx.save_for_backward(Q, K, V, bias)
    ctx.window, ctx.scale, ctx.return_tau, ctx.flags = window, scale, return_tau, flags


def _window_grad(ctx, d_out, d_tau):
    Q, K, V, bias = ctx.saved_tensors
    d_out = d_out if d_out is not None else torch.zeros_like(Q)
    dQ, dK, dV = torch.ops.bozo.window_bwd(Q, K, V, d_out, d_tau if ctx.return_tau else None, bias,
                                           ctx.window, ctx.scale, ctx.flags)
    return dQ, dK, dV, None, None, None, None, None


_op_window_fwd.register_autograd(_window_grad, setup_context=_window_setup)


@torch.library.custom_op("bozo::global_fwd", mutates_args=(), device_types="cuda")
def _op_global_fwd(Q: Tensor, K: Tensor, V: Tensor, scale: float, bias: Optional[Tensor],
                   Wl: int) -> tuple[Tensor, Tensor, Tensor]:
    out, tl, mass = _global_fwd(_rows(Q), _rows(K), _rows(V), scale, bias, Wl)
    return out, (tl if tl is not None else Q.new_empty(0)), mass


@_op_global_fwd.register_fake
def _(Q, K, V, scale, bias, Wl):
    B, T, H, D = Q.shape
    tl = Q.new_empty((B, T, H, Wl)) if Wl > 0 else Q.new_empty(0)
    return Q.new_empty((B, T, H, D)), tl, Q.new_empty((B, T, H), dtype=torch.float32)


@torch.library.custom_op("bozo::global_bwd", mutates_args=(), device_types="cuda")
def _op_global_bwd(Q: Tensor, K: Tensor, V: Tensor, dOut: Tensor, dTl: Optional[Tensor],
                   bias: Optional[Tensor], out: Tensor, mass: Tensor, Wl: int,
                   scale: float) -> tuple[Tensor, Tensor, Tensor]:
    return _global_bwd(_rows(Q), _rows(K), _rows(V), dOut, dTl, bias, out, mass, Wl, scale)


@_op_global_bwd.register_fake
def _(Q, K, V, dOut, dTl, bias, out, mass, Wl, scale):
    return _grads_like(Q, K, V)


def _global_setup(ctx, inputs, output):
    Q, K, V, scale, bias, Wl = inputs
    ctx.save_for_backward(Q, K, V, bias, output[0], output[2])
    ctx.scale, ctx.Wl = scale, Wl


def _global_grad(ctx, d_out, d_tl, d_mass):
    Q, K, V, bias, out, mass = ctx.saved_tensors
    d_out = d_out if d_out is not None else torch.zeros_like(Q)
    dQ, dK, dV = torch.ops.bozo.global_bwd(Q, K, V, d_out, d_tl if ctx.Wl > 0 else None, bias, out, mass,
                                           ctx.Wl, ctx.scale)
    return dQ, dK, dV, None, None, None


_op_global_fwd.register_autograd(_global_grad, setup_context=_global_setup)


@torch.library.custom_op("bozo::rope", mutates_args=(), device_types="cuda")
def _op_rope(x: Tensor, cos: Tensor, sin: Tensor, pos_offset: int, out_dtype: torch.dtype,
             inverse: int) -> Tensor:
    x = _rows(x)
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    _rope_call(x, y, cos, sin, pos_offset, inverse)
    return y


@_op_rope.register_fake
def _(x, cos, sin, pos_offset, out_dtype, inverse):
    return torch.empty(x.shape, dtype=out_dtype, device=x.device)


def _rope_setup(ctx, inputs, output):
    x, cos, sin, pos_offset, out_dtype, inverse = inputs
    ctx.save_for_backward(cos, sin)
    ctx.pos_offset, ctx.in_dtype, ctx.inverse = pos_offset, x.dtype, inverse


def _rope_grad(ctx, dy):
    cos, sin = ctx.saved_tensors
    return (torch.ops.bozo.rope(dy, cos, sin, ctx.pos_offset, ctx.in_dtype, 1 - ctx.inverse),
            None, None, None, None, None)


_op_rope.register_autograd(_rope_grad, setup_context=_rope_setup)
