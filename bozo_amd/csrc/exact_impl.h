// Exact (non-MFMA) band kernels (templates; instantiated by exact_*.hip): any input dtype (f32 / bf16 / f16 / f64),
// accumulation in A = float or double.  One thread owns one query row
// (forward, dQ) or one key row (dK/dV) and walks its band sequentially, so
// the result follows the reference's per-pair arithmetic in full precision:
// the dot is divided by scale (kernel.py:100), sigmoid is libm-accurate and
// every product is accumulated in A.  These kernels serve fp32 / fp64 /
// mixed-dtype calls (gradcheck runs through them in float64) and every shape
// the MFMA kernels do not take.
#pragma once

#include "kernels.h"

namespace tension {

template <typename A, int D>
__global__ __launch_bounds__(128) void exact_fwd(BandParams p) {
  touch_args(p);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.H * p.T;
  if (idx >= total) return;
  const int t = (int)(idx % p.T);
  const int64_t bh = idx / p.T;
  const int h = (int)(bh % p.H);
  const int b = (int)(bh / p.H);

  const int64_t qo = b * p.q.s0 + (int64_t)t * p.q.s1 + h * p.q.s2;
  A q[D], acc[D];
#pragma unroll
  for (int d = 0; d < D; d += 8) ld8<A>(p.q, qo + d, q + d);
#pragma unroll
  for (int d = 0; d < D; ++d) acc[d] = A(0);
  A mass = A(0);
  const A scale = (A)p.scale;

  const int s_lo = t - p.win > 0 ? t - p.win : 0;
  const int s_hi = t - 1 + p.diag;
  for (int s = s_lo; s <= s_hi; ++s) {
    const int64_t ko = b * p.k.s0 + (int64_t)s * p.k.s1 + h * p.k.s2;
    const int64_t vo = b * p.v.s0 + (int64_t)s * p.v.s1 + h * p.v.s2;
    A dot = A(0);
#pragma unroll
    for (int d = 0; d < D; d += 8) {
      A r[8];
      ld8<A>(p.k, ko + d, r);
#pragma unroll
      for (int i = 0; i < 8; ++i) dot += q[d + i] * r[i];
    }
    A x = dot / scale;
    if (p.bias.p) x += ld<A>(p.bias, bias_off(p, b, t, s));
    const A tau = sigmoid_exact(x);
    mass += tau;
#pragma unroll
    for (int d = 0; d < D; d += 8) {
      A r[8];
      ld8<A>(p.v, vo + d, r);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[d + i] += tau * r[i];
    }
    if (p.tau.p) {
      const int c = tau_col(p, t, s);
      if (c >= 0) st<A>(p.tau, tau_off(p.tau, b, t, h, c), tau);
    }
  }
  if (p.tau.p) {
    const int e = tau_empty_bound(p, t);
    for (int c = 0; c < e; ++c) st<A>(p.tau, tau_off(p.tau, b, t, h, c), A(0));
  }
  A inv = A(1);
  if (p.flags & TENSION_NORM_MASS) inv = A(1) / (mass > A(kMassEps) ? mass : A(kMassEps));
  if (p.flags & TENSION_NORM_COUNT) {
    const int cnt = t < p.W ? t : p.W;
    inv = A(1) / A(cnt > 1 ? cnt : 1);
  }
  const int64_t oo = b * p.out.s0 + (int64_t)t * p.out.s1 + h * p.out.s2;
#pragma unroll
  for (int d = 0; d < D; ++d) acc[d] *= inv;
#pragma unroll
  for (int d = 0; d < D; d += 8) st8<A>(p.out, oo + d, acc + d);
  if (p.mass.p) st<A>(p.mass, b * p.mass.s0 + (int64_t)t * p.mass.s1 + h * p.mass.s2, mass);
}

// Per-query coefficients of the backward:  dtau = a_t * (dO_t . v_s) - c_t
// (+ dTau).  raw: a = 1, c = 0; count: a = 1/max(min(t,W),1), c = 0.
// tau-mass (out = msg/m, m = max(sum tau, eps)): a = 1/m and
// c = (dO_t . msg_t)/m^2 = sum_s tau_s (dO_t . v_s) / m^2 while the mass is
// >= eps (the clamp passes no gradient below eps).  c is formed from the
// recomputed fp32/f64 band sums, never from the stored (possibly bf16) out:
// dO.v_s - dO.out cancels when a query has one dominant key.
template <typename A, int D>
__global__ __launch_bounds__(128) void exact_bwd_dq(BandParams p) {
  touch_args(p);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.H * p.T;
  if (idx >= total) return;
  const int t = (int)(idx % p.T);
  const int64_t bh = idx / p.T;
  const int h = (int)(bh % p.H);
  const int b = (int)(bh / p.H);

  const int64_t qo = b * p.q.s0 + (int64_t)t * p.q.s1 + h * p.q.s2;
  const int64_t go = b * p.dout.s0 + (int64_t)t * p.dout.s1 + h * p.dout.s2;
  A q[D], g[D], dq[D];
#pragma unroll
  for (int d = 0; d < D; d += 8) {
    ld8<A>(p.q, qo + d, q + d);
    ld8<A>(p.dout, go + d, g + d);
  }
#pragma unroll
  for (int d = 0; d < D; ++d) dq[d] = A(0);
  const A scale = (A)p.scale;
  const int s_lo = t - p.win > 0 ? t - p.win : 0;
  const int s_hi = t - 1 + p.diag;

  A ca = A(1), cc = A(0);
  if (p.flags & TENSION_NORM_MASS) {
    A mass = A(0), dsum = A(0);
    for (int s = s_lo; s <= s_hi; ++s) {
      const int64_t ko = b * p.k.s0 + (int64_t)s * p.k.s1 + h * p.k.s2;
      const int64_t vo = b * p.v.s0 + (int64_t)s * p.v.s1 + h * p.v.s2;
      A dot = A(0), gv = A(0);
#pragma unroll
      for (int d = 0; d < D; d += 8) {
        A rk[8], rv[8];
        ld8<A>(p.k, ko + d, rk);
        ld8<A>(p.v, vo + d, rv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dot += q[d + i] * rk[i];
          gv += g[d + i] * rv[i];
        }
      }
      A x = dot / scale;
      if (p.bias.p) x += ld<A>(p.bias, bias_off(p, b, t, s));
      const A tau = sigmoid_exact(x);
      mass += tau;
      dsum += tau * gv;
    }
    const A m = mass > A(kMassEps) ? mass : A(kMassEps);
    ca = A(1) / m;
    cc = mass >= A(kMassEps) ? dsum / (m * m) : A(0);
  } else if (p.flags & TENSION_NORM_COUNT) {
    const int cnt = t < p.W ? t : p.W;
    ca = A(1) / A(cnt > 1 ? cnt : 1);
  }
  if (p.ws && (p.flags & TENSION_NORM_MASS)) {
    const int64_t n = (int64_t)p.B * p.T * p.H;
    const int64_t wi = ((int64_t)b * p.T + t) * p.H + h;
    ((A*)p.ws)[wi] = ca;
    ((A*)p.ws)[n + wi] = cc;
  }
  for (int s = s_lo; s <= s_hi; ++s) {
    const int64_t ko = b * p.k.s0 + (int64_t)s * p.k.s1 + h * p.k.s2;
    const int64_t vo = b * p.v.s0 + (int64_t)s * p.v.s1 + h * p.v.s2;
    A dot = A(0), gv = A(0);
#pragma unroll
    for (int d = 0; d < D; d += 8) {
      A rk[8], rv[8];
      ld8<A>(p.k, ko + d, rk);
      ld8<A>(p.v, vo + d, rv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dot += q[d + i] * rk[i];
        gv += g[d + i] * rv[i];
      }
    }
    A x = dot / scale;
    if (p.bias.p) x += ld<A>(p.bias, bias_off(p, b, t, s));
    const A tau = sigmoid_exact(x);
    A dtau = gv * ca - cc;
    if (p.dtau.p) {
      const int c = tau_col(p, t, s);
      if (c >= 0) dtau += ld<A>(p.dtau, tau_off(p.dtau, b, t, h, c));
    }
    const A dd = dtau * tau * (A(1) - tau);
#pragma unroll
    for (int d = 0; d < D; d += 8) {
      A rk[8];
      ld8<A>(p.k, ko + d, rk);
#pragma unroll
      for (int i = 0; i < 8; ++i) dq[d + i] += dd * rk[i];
    }
  }
  const int64_t dqo = b * p.dq.s0 + (int64_t)t * p.dq.s1 + h * p.dq.s2;
#pragma unroll
  for (int d = 0; d < D; ++d) dq[d] /= scale;
#pragma unroll
  for (int d = 0; d < D; d += 8) st8<A>(p.dq, dqo + d, dq + d);
}

template <typename A, int D>
__global__ __launch_bounds__(128) void exact_bwd_dkv(BandParams p) {
  touch_args(p);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.H * p.T;
  if (idx >= total) return;
  const int s = (int)(idx % p.T);
  const int64_t bh = idx / p.T;
  const int h = (int)(bh % p.H);
  const int b = (int)(bh / p.H);

  const int64_t ko = b * p.k.s0 + (int64_t)s * p.k.s1 + h * p.k.s2;
  const int64_t vo = b * p.v.s0 + (int64_t)s * p.v.s1 + h * p.v.s2;
  A k[D], v[D], dk[D], dv[D];
#pragma unroll
  for (int d = 0; d < D; d += 8) {
    ld8<A>(p.k, ko + d, k + d);
    ld8<A>(p.v, vo + d, v + d);
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    dk[d] = A(0);
    dv[d] = A(0);
  }
  const A scale = (A)p.scale;
  const int64_t n = (int64_t)p.B * p.T * p.H;
  // queries that see key s: s + 1 - diag <= t <= s + win
  const int t_lo = s + 1 - p.diag;
  const int t_hi = (int64_t)s + p.win < p.T - 1 ? s + p.win : p.T - 1;
  for (int t = t_lo; t <= t_hi; ++t) {
    const int64_t qo = b * p.q.s0 + (int64_t)t * p.q.s1 + h * p.q.s2;
    const int64_t go = b * p.dout.s0 + (int64_t)t * p.dout.s1 + h * p.dout.s2;
    A dot = A(0), gv = A(0);
#pragma unroll
    for (int d = 0; d < D; d += 8) {
      A rq[8], rg[8];
      ld8<A>(p.q, qo + d, rq);
      ld8<A>(p.dout, go + d, rg);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dot += rq[i] * k[d + i];
        gv += rg[i] * v[d + i];
      }
    }
    A ca = A(1), cc = A(0);
    if (p.flags & TENSION_NORM_MASS) {
      const int64_t wi = ((int64_t)b * p.T + t) * p.H + h;
      ca = ((const A*)p.ws)[wi];
      cc = ((const A*)p.ws)[n + wi];
    } else if (p.flags & TENSION_NORM_COUNT) {
      const int cnt = t < p.W ? t : p.W;
      ca = A(1) / A(cnt > 1 ? cnt : 1);
    }
    A x = dot / scale;
    if (p.bias.p) x += ld<A>(p.bias, bias_off(p, b, t, s));
    const A tau = sigmoid_exact(x);
    A dtau = gv * ca - cc;
    if (p.dtau.p) {
      const int c = tau_col(p, t, s);
      if (c >= 0) dtau += ld<A>(p.dtau, tau_off(p.dtau, b, t, h, c));
    }
    const A dd = dtau * tau * (A(1) - tau);
    const A tv = tau * ca;
#pragma unroll
    for (int d = 0; d < D; d += 8) {
      A rq[8], rg[8];
      ld8<A>(p.q, qo + d, rq);
      ld8<A>(p.dout, go + d, rg);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dk[d + i] += dd * rq[i];
        dv[d + i] += tv * rg[i];
      }
    }
  }
  const int64_t dko = b * p.dk.s0 + (int64_t)s * p.dk.s1 + h * p.dk.s2;
  const int64_t dvo = b * p.dv.s0 + (int64_t)s * p.dv.s1 + h * p.dv.s2;
#pragma unroll
  for (int d = 0; d < D; ++d) dk[d] /= scale;
#pragma unroll
  for (int d = 0; d < D; d += 8) {
    st8<A>(p.dk, dko + d, dk + d);
    st8<A>(p.dv, dvo + d, dv + d);
  }
}

// Host launch of the exact kernel of PHASE (0 fwd, 1 dQ, 2 dK / dV) with
// accumulator A: one thread per (b, h, row), 128 per workgroup, head dims
// 8 .. 128.  Each (phase, accumulator) pair is instantiated in a unit of its
// own (exact_<phase>_<acc>.hip), so the six compile in parallel.
template <typename A, int PHASE, int D>
void exact_launch_d(const BandParams& p, hipStream_t st, unsigned grid) {
  if constexpr (PHASE == 0) hipLaunchKernelGGL((exact_fwd<A, D>), dim3(grid), dim3(128), 0, st, p);
  else if constexpr (PHASE == 1) hipLaunchKernelGGL((exact_bwd_dq<A, D>), dim3(grid), dim3(128), 0, st, p);
  else hipLaunchKernelGGL((exact_bwd_dkv<A, D>), dim3(grid), dim3(128), 0, st, p);
}

template <typename A, int PHASE>
int exact_launch(const BandParams& p, hipStream_t st, hipError_t* err) {
  const int64_t total = (int64_t)p.B * p.H * p.T;
  if ((total + 127) / 128 > 0x7fffffff) return kGridTooLarge;
  const unsigned grid = (unsigned)((total + 127) / 128);
  switch (p.D) {
    case 8: exact_launch_d<A, PHASE, 8>(p, st, grid); break;
    case 16: exact_launch_d<A, PHASE, 16>(p, st, grid); break;
    case 32: exact_launch_d<A, PHASE, 32>(p, st, grid); break;
    case 64: exact_launch_d<A, PHASE, 64>(p, st, grid); break;
    case 128: exact_launch_d<A, PHASE, 128>(p, st, grid); break;
    default: return -1;
  }
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
