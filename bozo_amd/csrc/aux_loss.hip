// The model's tau regularisers (model.py:498-611) in two passes over the
// materialised tau of every layer: the forward accumulates per-layer sums,
// the backward writes dTau from per-layer coefficients.
//
// Per row (b, t, h) of a layer, tau[0..W) (w = 0 oldest), all in fp32, each
// workgroup writing its four sums to its slot of the partials buffer:
//   diversity : S = sum tau, p = tau / (S + 1e-8),
//               ent = -sum p log(p + 1e-8)             (acc 0: sum of ent)
//   consistency (rows r with terms; n = min(W - 2, 4), T_out = T - n - 1):
//               for w1 = 1..n with w1 + 1 <= r <= w1 + T_out:
//               relu(tau[r, w1-1] * tau[r-1, 0] - tau[r, w1])  (acc 1)
//   entropy   : m = mean tau, relu(0.05 - m) (acc 2), relu(m - 0.8) (acc 3)
// Eight lanes share a row (16 bytes of bf16 each, W <= 64), so a wave load
// instruction reads eight whole 128-byte rows; row sums fold through DPP.
//
// Backward, with per-layer coefficients k = (k_div, k_cons, k_ent):
//   dTau[w]  = k_div (e_w - sum_v e_v p_v) / (S + 1e-8),  e = -(log(p + 1e-8) + p / (p + 1e-8))
//            + k_ent ([m > 0.8] - [m < 0.05]) / W
//            + k_cons (terms of row t: b for slot w1-1, -1 for slot w1, where
//              the term is active; terms of row t+1: its slot w1-1 value
//              for slot 0)
// so every row's gradient is written by the eight lanes that own it (no
// atomics).
#include "kernels.h"

namespace tension {

namespace {

constexpr float kDivEps = 1e-8f;  // model.py:527-528

// the eight values of lane chunk ch of a row (0 past W): one 16-byte load
// for a whole aligned bf16 chunk, element loads otherwise
__device__ __forceinline__ void row8(const Buf& b, int64_t off, int ch, int W, float* v) {
  const int64_t o = off + 8 * ch;
  if (b.dt == TENSION_BF16 && 8 * ch + 8 <= W && (o & 7) == 0) {
    const bf16x8 x = __builtin_bit_cast(bf16x8, *(const u16x8*)((const bf16*)b.p + o));
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)x[e];
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int w = 8 * ch + e;
    v[e] = w < W ? ld<float>(b, off + w) : 0.f;
  }
}

// store counterpart of row8
__device__ __forceinline__ void row8_store(const Buf& b, int64_t off, int ch, int W, const float* v) {
  const int64_t o = off + 8 * ch;
  if (b.dt == TENSION_BF16 && 8 * ch + 8 <= W && (o & 7) == 0) {
    bf16x8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (bf16)v[e];
    *(u16x8*)((bf16*)b.p + o) = __builtin_bit_cast(u16x8, x);
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (8 * ch + e < W) st<float>(b, off + 8 * ch + e, v[e]);
}

__device__ __forceinline__ float at(const Buf& b, int64_t off) { return ld<float>(b, off); }

// number of consistency terms n and the row range of term w1
__device__ __forceinline__ int cons_n(int W, int T) {
  if (W < 3 || T < 3) return 0;
  const int n = W - 2 < 4 ? W - 2 : 4;
  return T - (n + 1) > 0 ? n : 0;
}

}  // namespace

__global__ __launch_bounds__(256) void aux_loss_fwd_kernel(AuxLossParams p) {
  const int l = blockIdx.y;
  const Buf tb = p.tau[l];
  const int lane = threadIdx.x & 63, ch = lane & 7;
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
  const int64_t nrow = (int64_t)p.B * p.T * p.H;
  const bool live = row < nrow;
  const int64_t rr = live ? row : 0;
  const int h = (int)(rr % p.H), t = (int)((rr / p.H) % p.T), b = (int)(rr / ((int64_t)p.H * p.T));
  const int64_t off = b * tb.s0 + (int64_t)t * tb.s1 + h * tb.s2;
  float v[8];
  row8(tb, off, ch, p.W, v);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += v[e];
  s = row_sum8(s);
  const float inv = 1.f / (s + kDivEps);
  float ent = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (8 * ch + e < p.W) {
      const float pe = v[e] * inv;
      ent -= pe * __logf(pe + kDivEps);
    }
  }
  ent = row_sum8(ent);
  const float m = s / (float)p.W;
  float cons = 0.f;
  const int n = cons_n(p.W, p.T);
  if (ch == 0 && n > 0 && t >= 1) {
    const float prev0 = at(tb, off - tb.s1);  // tau[t-1, 0]
    const int T_out = p.T - (n + 1);
    for (int w1 = 1; w1 <= n; ++w1) {
      if (t < w1 + 1 || t > w1 + T_out) continue;
      const float x = at(tb, off + w1 - 1) * prev0 - at(tb, off + w1);
      cons += x > 0.f ? x : 0.f;
    }
  }
  // one lane per row contributes; the block's sums go to its own slot of
  // the partials buffer (summed by the caller: deterministic, no atomics)
  __shared__ double red[4][256 / 8];
  const int slot = threadIdx.x >> 3;
  if (ch == 0) {
    red[0][slot] = live ? (double)ent : 0.0;
    red[1][slot] = live ? (double)cons : 0.0;
    red[2][slot] = live && m < 0.05f ? (double)(0.05f - m) : 0.0;
    red[3][slot] = live && m > 0.8f ? (double)(m - 0.8f) : 0.0;
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    double a = 0.0;
    for (int i = 0; i < 256 / 8; ++i) a += red[threadIdx.x][i];
    p.acc[((int64_t)l * gridDim.x + blockIdx.x) * 4 + threadIdx.x] = a;
  }
}

__global__ __launch_bounds__(256) void aux_loss_bwd_kernel(AuxLossParams p) {
  const int l = blockIdx.y;
  const Buf tb = p.tau[l], db = p.dtau[l];
  const int lane = threadIdx.x & 63, ch = lane & 7;
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
  const int64_t nrow = (int64_t)p.B * p.T * p.H;
  if (row >= nrow) return;  // whole 8-lane groups leave together
  const int h = (int)(row % p.H), t = (int)((row / p.H) % p.T), b = (int)(row / ((int64_t)p.H * p.T));
  const int64_t off = b * tb.s0 + (int64_t)t * tb.s1 + h * tb.s2;
  const int64_t doff = b * db.s0 + (int64_t)t * db.s1 + h * db.s2;
  const float kdiv = p.coef[3 * l], kcons = p.coef[3 * l + 1], kent = p.coef[3 * l + 2];
  float v[8];
  row8(tb, off, ch, p.W, v);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += v[e];
  s = row_sum8(s);
  const float inv = 1.f / (s + kDivEps);
  float pe[8], ee[8], dot = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pe[e] = v[e] * inv;
    ee[e] = -(__logf(pe[e] + kDivEps) + pe[e] / (pe[e] + kDivEps));
    dot += 8 * ch + e < p.W ? ee[e] * pe[e] : 0.f;
  }
  dot = row_sum8(dot);
  const float m = s / (float)p.W;
  const float gent = kent * ((m > 0.8f ? 1.f : 0.f) - (m < 0.05f ? 1.f : 0.f)) / (float)p.W;
  float g[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) g[e] = kdiv * (ee[e] - dot) * inv + gent;
  // consistency: slots 0..n live in lane chunk 0 (n <= 4 < 8)
  const int n = cons_n(p.W, p.T);
  if (ch == 0 && n > 0 && kcons != 0.f) {
    const int T_out = p.T - (n + 1);
    if (t >= 1) {  // terms of row t: a = tau[t, w1-1], b = tau[t-1, 0], c = tau[t, w1]
      const float bprev = at(tb, off - tb.s1);
#pragma unroll
      for (int w1 = 1; w1 <= 4; ++w1) {
        if (w1 > n || t < w1 + 1 || t > w1 + T_out) continue;
        if (v[w1 - 1] * bprev - v[w1] > 0.f) {
          g[w1 - 1] += kcons * bprev;
          g[w1] -= kcons;
        }
      }
    }
    if (t + 1 < p.T) {  // terms of row t+1 use tau[t, 0] as b
      const int64_t on = off + tb.s1;
#pragma unroll
      for (int w1 = 1; w1 <= 4; ++w1) {
        if (w1 > n || t + 1 < w1 + 1 || t + 1 > w1 + T_out) continue;
        const float a = at(tb, on + w1 - 1);
        if (a * v[0] - at(tb, on + w1) > 0.f) g[0] += kcons * a;
      }
    }
  }
  row8_store(db, doff, ch, p.W, g);
}

int launch_aux_loss(bool bwd, const AuxLossParams& p, hipStream_t st, hipError_t* err) {
  const int64_t nrow = (int64_t)p.B * p.T * p.H;
  const dim3 grid((unsigned)((nrow * 8 + 255) / 256), (unsigned)p.L);
  if (bwd)
    hipLaunchKernelGGL(aux_loss_bwd_kernel, grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(aux_loss_fwd_kernel, grid, dim3(256), 0, st, p);
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
