// The "band" shared by the local-window and global kernels.
//
// A query t looks at keys s with
//     max(0, t - win) <= s <= t - 1 + diag
// local window (triton_tension/kernel.py:82-86): win = W, diag = 0
//     (strictly past, self excluded);
// global block (model.py:219-226): win = T + 1, diag = 1 (causal triangle,
//     self included).
// Column maps into the [.., W]-wide side tensors:
//   bias  local  [B,T,W]: w = s - t + W          (kernel.py:102-107)
//         global [B,T,T]: s                      (model.py:224-225)
//   tau   local  [B,T,H,W]: w = s - t + W
//         global tau_local [B,T,H,Wl]: j = T-1-s if j < Wl   (model.py:231-237)
#pragma once

#include "common.h"

namespace tension {

// Launcher result for a grid beyond 2^31 - 1 workgroups (0: launched, -1: no
// kernel for the request).
constexpr int kGridTooLarge = -2;

struct BandParams {
  Buf q, k, v;
  Buf out, tau, bias, mass;
  Buf dout, dtau, dq, dk, dv;
  void* ws;       // backward workspace: acc-typed a[B*T*H], c[B*T*H]
  int coef_pre;   // tau-mass backward: a, c computed from the saved out / mass
                  // rows (p.out, p.mass) instead of a pass over the band
  int B, T, H, D;
  int win, diag, glob;
  int W;          // local window (count normalisation)
  int Wtau;       // width of tau / dtau (local W, global Wl)
  double scale;
  int flags;
  int ntiles;     // 64-row tiles per (b,h) (MFMA kernels)
  int chunk;      // consecutive tiles per workgroup (MFMA ring kernels)
};

// BandParams in kernel-argument form: the same fields with 32-bit element
// strides (104 dwords against 162).  A band kernel reads its arguments with
// scalar loads, as many as its registers hold at a time; with the int64
// form the fused backward took five dependent rounds of them before its
// first tensor load, every workgroup at once.  band_args() refuses a
// stride outside int32 (such calls take the exact kernels); band_params()
// widens the fields back at kernel entry.
struct BufArg {
  const void* p;
  int dt;
  int s0, s1, s2, s3;
};

struct BandArgs {
  BufArg q, k, v;
  BufArg out, tau, bias, mass;
  BufArg dout, dtau, dq, dk, dv;
  void* ws;
  double scale;
  int coef_pre, B, T, H, D, win, diag, glob, W, Wtau, flags, ntiles, chunk;
};

inline bool buf_arg(const Buf& b, BufArg* a) {
  const int64_t lo = -0x7fffffffLL - 1, hi = 0x7fffffffLL;
  for (int64_t x : {b.s0, b.s1, b.s2, b.s3})
    if (x < lo || x > hi) return false;
  a->p = b.p;
  a->dt = b.dt;
  a->s0 = (int)b.s0;
  a->s1 = (int)b.s1;
  a->s2 = (int)b.s2;
  a->s3 = (int)b.s3;
  return true;
}

inline bool band_args(const BandParams& p, BandArgs* a) {
  const Buf* src[] = {&p.q, &p.k, &p.v, &p.out, &p.tau, &p.bias, &p.mass, &p.dout, &p.dtau, &p.dq, &p.dk, &p.dv};
  BufArg* dst[] = {&a->q, &a->k, &a->v, &a->out, &a->tau, &a->bias, &a->mass, &a->dout, &a->dtau, &a->dq, &a->dk, &a->dv};
  for (int i = 0; i < 12; ++i)
    if (!buf_arg(*src[i], dst[i])) return false;
  a->ws = p.ws;
  a->scale = p.scale;
  a->coef_pre = p.coef_pre;
  a->B = p.B; a->T = p.T; a->H = p.H; a->D = p.D;
  a->win = p.win; a->diag = p.diag; a->glob = p.glob; a->W = p.W; a->Wtau = p.Wtau;
  a->flags = p.flags; a->ntiles = p.ntiles; a->chunk = p.chunk;
  return true;
}

// The kernel-argument form of p for launchers behind launch_mfma /
// launch_split, which refuse a p whose strides band_args() rejects.
inline BandArgs to_args(const BandParams& p) {
  BandArgs a;
  band_args(p, &a);
  return a;
}

__device__ __forceinline__ Buf buf_of(const BufArg& a) {
  Buf b;
  b.p = a.p;
  b.dt = a.dt;
  b.s0 = a.s0;
  b.s1 = a.s1;
  b.s2 = a.s2;
  b.s3 = a.s3;
  return b;
}

__device__ __forceinline__ BandParams band_params(const BandArgs& a) {
  BandParams p;
  p.q = buf_of(a.q); p.k = buf_of(a.k); p.v = buf_of(a.v);
  p.out = buf_of(a.out); p.tau = buf_of(a.tau); p.bias = buf_of(a.bias); p.mass = buf_of(a.mass);
  p.dout = buf_of(a.dout); p.dtau = buf_of(a.dtau); p.dq = buf_of(a.dq); p.dk = buf_of(a.dk); p.dv = buf_of(a.dv);
  p.ws = a.ws;
  p.coef_pre = a.coef_pre;
  p.B = a.B; p.T = a.T; p.H = a.H; p.D = a.D;
  p.win = a.win; p.diag = a.diag; p.glob = a.glob; p.W = a.W; p.Wtau = a.Wtau;
  p.scale = a.scale;
  p.flags = a.flags; p.ntiles = a.ntiles; p.chunk = a.chunk;
  return p;
}

// Read one dword of every 64-byte line of a kernel's arguments at entry, in
// one batch of scalar loads: the argument reads the compiler places later,
// next to their uses, then hit the scalar cache instead of each waiting on
// memory in turn while every workgroup of the launch waits the same way.
template <typename A>
__device__ __forceinline__ void touch_args(const A& a) {
  const int* w = (const int*)&a;
  int x = 0;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(A) / 4); i += 16) x ^= w[i];
  asm volatile("" ::"s"(x));
}

__device__ __forceinline__ bool band_valid(const BandParams& p, int t, int s) {
  return s >= 0 && s >= t - p.win && s <= t - 1 + p.diag;
}

__device__ __forceinline__ int64_t bias_off(const BandParams& p, int b, int t, int s) {
  const int col = p.glob ? s : s - t + p.W;
  return (int64_t)b * p.bias.s0 + (int64_t)t * p.bias.s1 + (int64_t)col * p.bias.s2;
}

// Column of (t, s) in the bias (local [B,T,W]: s - t + W; global [B,T,T]: s).
__device__ __forceinline__ int bias_col(const BandParams& p, int t, int s) {
  return p.glob ? s : s - t + p.W;
}

// Column of (t, s) in tau / dtau, or -1 if the pair has no slot there.
__device__ __forceinline__ int tau_col(const BandParams& p, int t, int s) {
  if (p.glob) {
    const int j = p.T - 1 - s;
    return j < p.Wtau ? j : -1;
  }
  return s - t + p.W;
}

__device__ __forceinline__ int64_t tau_off(const Buf& b, int bb, int t, int h, int col) {
  return (int64_t)bb * b.s0 + (int64_t)t * b.s1 + (int64_t)h * b.s2 + col;
}

// Slots of tau row t that no valid key fills (and must read as 0):
// local: w < W - t (keys before the sequence start); global: j < T-1-t
// (keys after the query).  Returns the exclusive upper bound; slots are
// [0, bound).
__device__ __forceinline__ int tau_empty_bound(const BandParams& p, int t) {
  const int e = p.glob ? (p.T - 1 - t) : (p.W - t);
  return e < 0 ? 0 : (e > p.Wtau ? p.Wtau : e);
}

}  // namespace tension
