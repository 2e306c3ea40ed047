// bf16 MFMA band backward, dQ half (local window and global block), head
// dim 64.  Query-centric like the forward: the four waves split the 64
// queries of the tile.  Per 64-key block:
//   S^T  = K Q^T,  dP^T = V dO^T          (A = K / V rows from LDS)
//   G    = (a_t dP - c_t + dTau) * P (1 - P) on the band          (fp32)
//   dQ^T += K^T G^T                        (A = K^T from a transposed tile)
// a_t, c_t are the per-query coefficients of the output normalisation
// (raw: 1, 0; valid-count: 1/n_t, 0; tau-mass: 1/m_t and
// sum_s P dP / m_t^2, the latter needing the whole band before any G).
// They are written to the workspace for the dK/dV kernel.
//
// HOLD: the band of every query spans at most two key blocks (local
// windows W <= 64): P and dP of both blocks stay in registers and K^T of
// both blocks in LDS, so one pass computes the coefficients and then G.
// Otherwise the tau-mass coefficients come from a first pass over the band,
// or (coef_pre) from the saved forward rows by coef_from_out.
#include "mfma_common.h"

namespace tension {

// Tau-mass coefficients from the forward's saved rows: out_t = msg_t / m'_t
// with m'_t = max(m_t, eps), so a_t = 1 / m'_t and
//   c_t = sum_s P dP / m'_t^2 = (dO_t . msg_t) / m'_t^2 = (dO_t . out_t) * a_t
// (0 when m_t < eps, as in the band pass).  Eight lanes per (b, t, h) row, 16
// bytes of out and dO each; the grid covers whole 8-lane groups, so a group
// is either fully inside [0, B*T*H) or fully outside.
__global__ __launch_bounds__(256) void coef_from_out(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  const int64_t n = (int64_t)p.B * p.T * p.H;
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;  // (b*T + t)*H + h
  const int ch = threadIdx.x & 7;
  if (row >= n) return;
  const int h = (int)(row % p.H);
  const int64_t bt = row / p.H;
  const int t = (int)(bt % p.T), b = (int)(bt / p.T);
  const bf16x8 o = load8((const bf16*)p.out.p + b * p.out.s0 + (int64_t)t * p.out.s1 + h * p.out.s2 + 8 * ch);
  const bf16x8 d = load8((const bf16*)p.dout.p + b * p.dout.s0 + (int64_t)t * p.dout.s1 + h * p.dout.s2 + 8 * ch);
  float dot = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) dot += (float)o[e] * (float)d[e];
  dot = row_sum8(dot);
  if (ch == 0) {
    const float m = ld<float>(p.mass, b * p.mass.s0 + (int64_t)t * p.mass.s1 + h * p.mass.s2);
    const float a = 1.f / (m > kMassEps ? m : kMassEps);
    ((float*)p.ws)[row] = a;
    ((float*)p.ws)[n + row] = m >= kMassEps ? dot * a : 0.f;
  }
}

__device__ __forceinline__ void scores_block(const bf16* Ks, const bf16* Vs, const bf16x8* qf,
                                             const bf16x8* gf, int g, int c, f32x4* s, f32x4* dp) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f32x4 a = {}, d = {};
    a = mfma(lds8(Ks + (16 * j + c) * kPitch + 8 * g), qf[0], a);
    a = mfma(lds8(Ks + (16 * j + c) * kPitch + 32 + 8 * g), qf[1], a);
    d = mfma(lds8(Vs + (16 * j + c) * kPitch + 8 * g), gf[0], d);
    d = mfma(lds8(Vs + (16 * j + c) * kPitch + 32 + 8 * g), gf[1], d);
    s[j] = a;
    dp[j] = d;
  }
}

template <int NORM, bool BIAS, bool DTAU, bool HOLD>
__global__ __launch_bounds__(kThreads) void mfma_bwd_dq(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  constexpr int NKT = HOLD ? 2 : 1;
  __shared__ __attribute__((aligned(16))) bf16 Ks[kTileElems];
  __shared__ __attribute__((aligned(16))) bf16 Vs[kTileElems];
  __shared__ __attribute__((aligned(16))) bf16 Kt[NKT][kTElems];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, p.glob != 0);
  const int b = id.b, h = id.h, T = p.T;
  const int t0 = id.tile * kTile;
  const int tq = t0 + wave * 16 + c;
  const bool qok = tq < T;
  const int tr = qok ? tq : T - 1;
  const int lo = tq - p.win > 0 ? tq - p.win : 0;
  const int hi = qok ? tq - 1 + p.diag : -1;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const bf16* gb_ = (const bf16*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;

  int s_lo = t0 - p.win;
  if (s_lo < 0) s_lo = 0;
  int s_hi = t0 + kTile - 2 + p.diag;
  if (s_hi > T - 1) s_hi = T - 1;
  const int kb_first = s_lo & ~(kTile - 1);

  TileRegs kr = tile_load(kb_, p.k.s1, kb_first, T, tid);
  TileRegs vr = tile_load(vb_, p.v.s1, kb_first, T, tid);
  TileRegs kr1, vr1;  // second block of a HOLD band, requested up front
  if (HOLD && kb_first + kTile <= s_hi) {
    kr1 = tile_load(kb_, p.k.s1, kb_first + kTile, T, tid);
    vr1 = tile_load(vb_, p.v.s1, kb_first + kTile, T, tid);
  }
  bf16x8 qf[2], gf[2];
  qf[0] = load8(qb_ + (int64_t)tr * p.q.s1 + 8 * g);
  qf[1] = load8(qb_ + (int64_t)tr * p.q.s1 + 32 + 8 * g);
  gf[0] = load8(gb_ + (int64_t)tr * p.dout.s1 + 8 * g);
  gf[1] = load8(gb_ + (int64_t)tr * p.dout.s1 + 32 + 8 * g);
  if (!qok) { qf[0] = bf16x8{}; qf[1] = bf16x8{}; gf[0] = bf16x8{}; gf[1] = bf16x8{}; }

  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;
  float ca = 1.f, cc = 0.f;
  if (NORM == NORM_COUNT_) {
    const int cnt = tq < p.W ? tq : p.W;
    ca = 1.f / (float)(cnt > 1 ? cnt : 1);
  }
  f32x4 acc[4] = {};

  auto finish_coeffs = [&](float msum, float dsum) {
    msum = wave_sum_g(msum);
    dsum = wave_sum_g(dsum);
    const float m = msum > kMassEps ? msum : kMassEps;
    ca = 1.f / m;
    cc = msum >= kMassEps ? dsum * ca * ca : 0.f;
    if (p.ws && qok && g == 0) {
      const int64_t n = (int64_t)p.B * p.T * p.H;
      const int64_t wi = ((int64_t)b * p.T + tq) * p.H + h;
      ((float*)p.ws)[wi] = ca;
      ((float*)p.ws)[n + wi] = cc;
    }
  };

  // G of one block from P (pv) and dP, then dQ^T += K^T G^T
  auto grad_block = [&](int kb0, const float (*pv)[4], const f32x4* dp, const bf16* kt) {
    float gd[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = key >= lo && key <= hi;
        float dt = dp[j][r] * ca - cc;
        if (DTAU && ok) {
          const int col = tau_col(p, tq, key);
          if (col >= 0) dt += ld<float>(p.dtau, tau_off(p.dtau, b, tq, h, col));
        }
        const float x = pv[j][r];
        gd[j][r] = ok ? dt * x * (1.f - x) : 0.f;
      }
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const bf16x8 pb = pack_b(gd[2 * kk], gd[2 * kk + 1]);
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m] = mfma(lds_tr8(kt, 16 * m + c, 32 * kk, g), pb, acc[m]);
    }
  };

  auto probs = [&](int kb0, const f32x4* s, float (*pv)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = (key >= lo) & (key <= hi);
        float b2 = 0.f;
        if (BIAS && ok) b2 = -kLog2e * ld<float>(p.bias, bias_off(p, b, tq, key));
        const float sg = sigmoid_scaled(s[j][r], k2, b2);  // select, not branch
        pv[j][r] = ok ? sg : 0.f;
      }
    }
  };

  if (HOLD) {
    // at most two key blocks; P and dP of both kept in registers
    const int nblk = s_hi < kb_first ? 0 : (s_hi - kb_first) / kTile + 1;
    float pv[2][4][4];
    f32x4 dpv[2][4];
    float msum = 0.f, dsum = 0.f;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      if (blk < nblk) {
        const int kb0 = kb_first + blk * kTile;
        __syncthreads();
        tile_store_rows(blk ? kr1 : kr, Ks, tid);
        tile_store_trans(blk ? kr1 : kr, Kt[blk & (NKT - 1)], tid);
        tile_store_rows(blk ? vr1 : vr, Vs, tid);
        __syncthreads();
        f32x4 s[4];
        scores_block(Ks, Vs, qf, gf, g, c, s, dpv[blk]);
        probs(kb0, s, pv[blk]);
        if (NORM == NORM_MASS_) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              msum += pv[blk][j][r];
              dsum += pv[blk][j][r] * dpv[blk][j][r];
            }
        }
      }
    }
    if (NORM == NORM_MASS_) finish_coeffs(msum, dsum);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
      if (blk < nblk) grad_block(kb_first + blk * kTile, pv[blk], dpv[blk], Kt[blk & (NKT - 1)]);
  } else {
    if (NORM == NORM_MASS_ && p.coef_pre) {
      if (qok) {
        const int64_t wi = ((int64_t)b * p.T + tq) * p.H + h;
        ca = ((const float*)p.ws)[wi];
        cc = ((const float*)p.ws)[(int64_t)p.B * p.T * p.H + wi];
      }
    } else if (NORM == NORM_MASS_) {
      float msum = 0.f, dsum = 0.f;
      for (int kb0 = kb_first; kb0 <= s_hi; kb0 += kTile) {
        __syncthreads();
        tile_store_rows(kr, Ks, tid);
        tile_store_rows(vr, Vs, tid);
        // the second pass starts again at the first block
        const int nxt = kb0 + kTile <= s_hi ? kb0 + kTile : kb_first;
        kr = tile_load(kb_, p.k.s1, nxt, T, tid);
        vr = tile_load(vb_, p.v.s1, nxt, T, tid);
        __syncthreads();
        f32x4 s[4], dp[4];
        float pv[4][4];
        scores_block(Ks, Vs, qf, gf, g, c, s, dp);
        probs(kb0, s, pv);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            msum += pv[j][r];
            dsum += pv[j][r] * dp[j][r];
          }
      }
      finish_coeffs(msum, dsum);
    }
    for (int kb0 = kb_first; kb0 <= s_hi; kb0 += kTile) {
      __syncthreads();
      tile_store_rows(kr, Ks, tid);
      tile_store_trans(kr, Kt[0], tid);
      tile_store_rows(vr, Vs, tid);
      if (kb0 + kTile <= s_hi) {
        kr = tile_load(kb_, p.k.s1, kb0 + kTile, T, tid);
        vr = tile_load(vb_, p.v.s1, kb0 + kTile, T, tid);
      }
      __syncthreads();
      f32x4 s[4], dp[4];
      float pv[4][4];
      scores_block(Ks, Vs, qf, gf, g, c, s, dp);
      probs(kb0, s, pv);
      grad_block(kb0, pv, dp, Kt[0]);
    }
  }
  if (!qok) return;
  bf16* drow = (bf16*)p.dq.p + b * p.dq.s0 + (int64_t)tq * p.dq.s1 + h * p.dq.s2;
  store_row4x4(drow, acc, inv_scale, g);
}

template <int NORM, bool BIAS, bool DTAU, bool HOLD>
static void go(const BandParams& p, hipStream_t st, unsigned nwg) {
  hipLaunchKernelGGL((mfma_bwd_dq<NORM, BIAS, DTAU, HOLD>), dim3(nwg), dim3(kThreads), 0, st, to_args(p));
}

template <int NORM, bool HOLD>
static void go_h(const BandParams& p, hipStream_t st, unsigned nwg, bool bias, bool dtau) {
  if (bias) {
    if (dtau) go<NORM, true, true, HOLD>(p, st, nwg); else go<NORM, true, false, HOLD>(p, st, nwg);
  } else {
    if (dtau) go<NORM, false, true, HOLD>(p, st, nwg); else go<NORM, false, false, HOLD>(p, st, nwg);
  }
}

template <int NORM>
static void go_n(const BandParams& p, hipStream_t st, unsigned nwg, bool bias, bool dtau, bool hold) {
  if (hold) go_h<NORM, true>(p, st, nwg, bias, dtau); else go_h<NORM, false>(p, st, nwg, bias, dtau);
}

void launch_gl_dq(const BandParams& p, hipStream_t st);

void launch_mfma_dq(const BandParams& p, hipStream_t st, unsigned nwg, int norm) {
  const bool bias = p.bias.p != nullptr, dtau = p.dtau.p != nullptr;
  // every query tile's band spans <= 2 key blocks iff the window is <= 64
  const bool hold = !p.glob && p.win <= kTile;
  if (norm == NORM_MASS_ && !hold && p.coef_pre) {
#ifndef TENSION_NO_GL_BWD
    if (p.glob) {  // bias and dtau_local included; the coefficients formed in-kernel
      launch_gl_dq(p, st);
      return;
    }
#endif
    const int64_t threads = (int64_t)p.B * p.T * p.H * 8;
    hipLaunchKernelGGL(coef_from_out, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, to_args(p));
  }
  switch (norm) {
    case NORM_MASS_: go_n<NORM_MASS_>(p, st, nwg, bias, dtau, hold); break;
    case NORM_COUNT_: go_n<NORM_COUNT_>(p, st, nwg, bias, dtau, false); break;
    default: go_n<NORM_RAW>(p, st, nwg, bias, dtau, false); break;
  }
}

}  // namespace tension
