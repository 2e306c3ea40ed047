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
