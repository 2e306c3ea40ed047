// bf16 MFMA band backward, dK/dV half (local window and global block), head
// dim 64.  Key-centric: one workgroup owns a 64-key tile and the four waves
// split its keys (16 each), so every dK/dV row is produced by exactly one
// wave -- no atomics, deterministic.  For every 64-query block that sees
// the tile:
//   S  = Q K^T,  dP = dO V^T       (A = Q / dO rows from LDS, B = this
//                                    wave's K / V fragments)
//   P  = sigma(S/scale + bias),  G = (a_t dP - c_t + dTau) P (1 - P)
//   dV^T += dO^T (a P),  dK^T += Q^T G   (A = transposed Q / dO tiles)
// a_t, c_t come from the workspace written by the dQ kernel (tau-mass) or
// are closed-form (raw, valid-count).  The next query block's Q/dO rows are
// loaded from HBM while the current block is computed.
#include "mfma_common.h"

namespace tension {

template <int NORM, bool BIAS, bool DTAU>
__global__ __launch_bounds__(kThreads) void mfma_bwd_dkv(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  __shared__ __attribute__((aligned(16))) bf16 Qs[kTileElems];
  __shared__ __attribute__((aligned(16))) bf16 Gs[kTileElems];
  __shared__ __attribute__((aligned(16))) bf16 Qt[kTElems];
  __shared__ __attribute__((aligned(16))) bf16 Gt[kTElems];
  __shared__ float sa[kTile], sc[kTile];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  // key tile 0 sees the most queries in the global band: natural order is
  // already heaviest first
  const TileId id = tile_id(p, false);
  const int b = id.b, h = id.h, T = p.T;
  const int k0 = id.tile * kTile;
  const int tk = k0 + wave * 16 + c;
  const bool kok = tk < T;
  const int kr_ = kok ? tk : T - 1;
  // queries that see this lane's key: [qlo, qhi]
  const int qlo = tk + 1 - p.diag;
  const int64_t qhi64 = (int64_t)tk + p.win;
  const int qhi = !kok ? -1 : (qhi64 > T - 1 ? T - 1 : (int)qhi64);

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const bf16* gb_ = (const bf16*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;

  // query blocks that see keys [k0, k0+64): t in [k0 + 1 - diag, k0 + 63 + win]
  const int t_lo = k0 + 1 - p.diag;
  const int64_t t_hi64 = (int64_t)k0 + kTile - 1 + p.win;
  const int t_hi = t_hi64 > T - 1 ? T - 1 : (int)t_hi64;
  const int qb_first = t_lo & ~(kTile - 1);

  // two-deep register ring of Q/dO tiles (for W <= 64 both query blocks of
  // the band are requested up front)
  TileRegs qr[2], gr[2];
  qr[0] = tile_load(qb_, p.q.s1, qb_first, T, tid);
  gr[0] = tile_load(gb_, p.dout.s1, qb_first, T, tid);
  if (qb_first + kTile <= t_hi) {
    qr[1] = tile_load(qb_, p.q.s1, qb_first + kTile, T, tid);
    gr[1] = tile_load(gb_, p.dout.s1, qb_first + kTile, T, tid);
  }
  bf16x8 kf[2], vf[2];
  kf[0] = load8(kb_ + (int64_t)kr_ * p.k.s1 + 8 * g);
  kf[1] = load8(kb_ + (int64_t)kr_ * p.k.s1 + 32 + 8 * g);
  vf[0] = load8(vb_ + (int64_t)kr_ * p.v.s1 + 8 * g);
  vf[1] = load8(vb_ + (int64_t)kr_ * p.v.s1 + 32 + 8 * g);
  if (!kok) { kf[0] = bf16x8{}; kf[1] = bf16x8{}; vf[0] = bf16x8{}; vf[1] = bf16x8{}; }

  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;
  const int64_t nws = (int64_t)p.B * p.T * p.H;
  f32x4 dk[4] = {}, dv[4] = {};
  int slot = 0;
  for (int q0 = qb_first; q0 <= t_hi; q0 += kTile, slot ^= 1) {
    __syncthreads();
    {
      const TileRegs& qx = slot ? qr[1] : qr[0];
      const TileRegs& gx = slot ? gr[1] : gr[0];
      tile_store_rows(qx, Qs, tid);
      tile_store_trans(qx, Qt, tid);
      tile_store_rows(gx, Gs, tid);
      tile_store_trans(gx, Gt, tid);
    }
    if (tid < kTile) {
      const int t = q0 + tid;
      float a = 1.f, cc = 0.f;
      if (t < T) {
        if (NORM == NORM_MASS_) {
          const int64_t wi = ((int64_t)b * p.T + t) * p.H + h;
          a = ((const float*)p.ws)[wi];
          cc = ((const float*)p.ws)[nws + wi];
        } else if (NORM == NORM_COUNT_) {
          const int cnt = t < p.W ? t : p.W;
          a = 1.f / (float)(cnt > 1 ? cnt : 1);
        }
      }
      sa[tid] = a;
      sc[tid] = cc;
    }
    if (q0 + 2 * kTile <= t_hi) {
      if (slot) {
        qr[1] = tile_load(qb_, p.q.s1, q0 + 2 * kTile, T, tid);
        gr[1] = tile_load(gb_, p.dout.s1, q0 + 2 * kTile, T, tid);
      } else {
        qr[0] = tile_load(qb_, p.q.s1, q0 + 2 * kTile, T, tid);
        gr[0] = tile_load(gb_, p.dout.s1, q0 + 2 * kTile, T, tid);
      }
    }
    __syncthreads();
    float P[4][4], G[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 s = {}, dp = {};
      s = mfma(lds8(Qs + (16 * j + c) * kPitch + 8 * g), kf[0], s);
      s = mfma(lds8(Qs + (16 * j + c) * kPitch + 32 + 8 * g), kf[1], s);
      dp = mfma(lds8(Gs + (16 * j + c) * kPitch + 8 * g), vf[0], dp);
      dp = mfma(lds8(Gs + (16 * j + c) * kPitch + 32 + 8 * g), vf[1], dp);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ql = 16 * j + 4 * g + r;
        const int t = q0 + ql;
        const bool ok = t >= qlo && t <= qhi;
        float b2 = 0.f;
        if (BIAS && ok) b2 = -kLog2e * ld<float>(p.bias, bias_off(p, b, t, tk));
        const float pv = sigmoid_scaled(s[r], k2, b2);
        const float a = sa[ql];
        float dt = dp[r] * a - sc[ql];
        if (DTAU && ok) {
          const int col = tau_col(p, t, tk);
          if (col >= 0) dt += ld<float>(p.dtau, tau_off(p.dtau, b, t, h, col));
        }
        P[j][r] = ok ? pv * a : 0.f;
        G[j][r] = ok ? dt * pv * (1.f - pv) : 0.f;
      }
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const bf16x8 pb = pack_b(P[2 * kk], P[2 * kk + 1]);
      const bf16x8 gbb = pack_b(G[2 * kk], G[2 * kk + 1]);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        dv[m] = mfma(lds_tr8(Gt, 16 * m + c, 32 * kk, g), pb, dv[m]);
        dk[m] = mfma(lds_tr8(Qt, 16 * m + c, 32 * kk, g), gbb, dk[m]);
      }
    }
  }
  if (!kok) return;
  bf16* dkrow = (bf16*)p.dk.p + b * p.dk.s0 + (int64_t)tk * p.dk.s1 + h * p.dk.s2;
  bf16* dvrow = (bf16*)p.dv.p + b * p.dv.s0 + (int64_t)tk * p.dv.s1 + h * p.dv.s2;
  store_row4x4(dkrow, dk, inv_scale, g);
  store_row4x4(dvrow, dv, 1.f, g);
}

template <int NORM, bool BIAS, bool DTAU>
static void go(const BandParams& p, hipStream_t st, unsigned nwg) {
  hipLaunchKernelGGL((mfma_bwd_dkv<NORM, BIAS, DTAU>), dim3(nwg), dim3(kThreads), 0, st, to_args(p));
}

template <int NORM>
static void go_n(const BandParams& p, hipStream_t st, unsigned nwg, bool bias, bool dtau) {
  if (bias) {
    if (dtau) go<NORM, true, true>(p, st, nwg); else go<NORM, true, false>(p, st, nwg);
  } else {
    if (dtau) go<NORM, false, true>(p, st, nwg); else go<NORM, false, false>(p, st, nwg);
  }
}

void launch_gl_dkv(const BandParams& p, hipStream_t st);

void launch_mfma_dkv(const BandParams& p, hipStream_t st, unsigned nwg, int norm) {
  const bool bias = p.bias.p != nullptr, dtau = p.dtau.p != nullptr;
#ifndef TENSION_NO_GL_BWD
  // global block: the coefficients are in the workspace whichever way the dQ
  // phase produced them
  if (p.glob && norm == NORM_MASS_) {  // bias and dtau_local included
    launch_gl_dkv(p, st);
    return;
  }
#endif
  switch (norm) {
    case NORM_MASS_: go_n<NORM_MASS_>(p, st, nwg, bias, dtau); break;
    case NORM_COUNT_: go_n<NORM_COUNT_>(p, st, nwg, bias, dtau); break;
    default: go_n<NORM_RAW>(p, st, nwg, bias, dtau); break;
  }
}

}  // namespace tension
