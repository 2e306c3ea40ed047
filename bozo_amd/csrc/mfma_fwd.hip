// bf16 MFMA band forward (local window and global block), head dim 64.
//
// One workgroup per 64-query tile; the four waves split the queries (16
// each).  For every 64-key block of the tile's band:
//   S^T = K Q^T   (A = K rows read from LDS, B = this wave's Q fragment)
//   P   = sigma(S/scale + bias) on the band, 0 elsewhere      (fp32)
//   O^T += V^T P^T (A = V^T read transposed from the row-major V tile,
//                   B = P^T packed straight from the C layout of S^T)
// S^T leaves lane (g, c) holding keys 16j+4g+r of query c, which is already
// the B-operand layout of the P.V product once two 16-key groups are packed,
// so no shuffle of P is needed.
//
// K/V blocks stream HBM -> LDS with global_load_lds into a two-deep ring of
// tiles: the blocks n and n+1 are in flight while block n-1 is computed,
// and no register or LDS-store instruction touches the stream.
#include "mfma_common.h"

namespace tension {

template <int NORM, bool BIAS, bool TAU>
__global__ __launch_bounds__(kThreads) void mfma_fwd(BandParams p) {
  __shared__ __attribute__((aligned(16))) bf16 Kb[2][kDTile];
  __shared__ __attribute__((aligned(16))) bf16 Vb[2][kDTile];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, p.glob != 0);
  const int b = id.b, h = id.h, T = p.T;
  const int t0 = id.tile * kTile;
  const int tq = t0 + wave * 16 + c;
  const bool qok = tq < T;
  // keys of this lane's query: [lo, hi] (empty for rows past T)
  const int lo = tq - p.win > 0 ? tq - p.win : 0;
  const int hi = qok ? tq - 1 + p.diag : -1;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;

  int s_lo = t0 - p.win;
  if (s_lo < 0) s_lo = 0;
  int s_hi = t0 + kTile - 2 + p.diag;
  if (s_hi > T - 1) s_hi = T - 1;
  const int kb_first = s_lo & ~(kTile - 1);
  const int nblk = s_hi < kb_first ? 0 : (s_hi - kb_first) / kTile + 1;

  bf16x8 qf[2];
  {
    const int tr = qok ? tq : T - 1;
    qf[0] = load8(qb_ + (int64_t)tr * p.q.s1 + 8 * g);
    qf[1] = load8(qb_ + (int64_t)tr * p.q.s1 + 32 + 8 * g);
  }
  // each block is 4 load instructions per wave (2 for K, 2 for V)
  tile_async(kb_, p.k.s1, kb_first, T, Kb[0], wave, lane);
  tile_async(vb_, p.v.s1, kb_first, T, Vb[0], wave, lane);
  if (nblk > 1) {
    tile_async(kb_, p.k.s1, kb_first + kTile, T, Kb[1], wave, lane);
    tile_async(vb_, p.v.s1, kb_first + kTile, T, Vb[1], wave, lane);
  }
  if (!qok) { qf[0] = bf16x8{}; qf[1] = bf16x8{}; }

  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;
  f32x4 acc[4] = {};
  float msum = 0.f;

  for (int blk = 0; blk < nblk; ++blk) {
    const int kb0 = kb_first + blk * kTile;
    const bf16* Ks = Kb[blk & 1];
    const bf16* Vs = Vb[blk & 1];
    if (blk + 1 < nblk) wait_vm<4>(); else wait_vm<0>();
    __syncthreads();
    float pr[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 s = {};
      s = mfma(dt_row8(Ks, 16 * j + c, g), qf[0], s);
      s = mfma(dt_row8(Ks, 16 * j + c, 4 + g), qf[1], s);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = key >= lo && key <= hi;
        float b2 = 0.f;
        if (BIAS && ok) b2 = -kLog2e * ld<float>(p.bias, bias_off(p, b, tq, key));
        const float pv = ok ? sigmoid_scaled(s[r], k2, b2) : 0.f;
        if (TAU && ok) {
          const int col = tau_col(p, tq, key);
          if (col >= 0) st<float>(p.tau, tau_off(p.tau, b, tq, h, col), pv);
        }
        msum += pv;
        pr[j][r] = pv;
      }
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const bf16x8 pb = pack_b(pr[2 * kk], pr[2 * kk + 1]);
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m] = mfma(dt_tr8(Vs, m, 32 * kk, g, c), pb, acc[m]);
    }
    if (blk + 2 < nblk) {
      __syncthreads();  // every wave is done with this ring slot
      tile_async(kb_, p.k.s1, kb0 + 2 * kTile, T, Kb[blk & 1], wave, lane);
      tile_async(vb_, p.v.s1, kb0 + 2 * kTile, T, Vb[blk & 1], wave, lane);
    }
  }
  msum = wave_sum_g(msum);
  if (!qok) return;
  bf16* orow = (bf16*)p.out.p + b * p.out.s0 + (int64_t)tq * p.out.s1 + h * p.out.s2;
  store_row4x4(orow, acc, out_factor<NORM>(msum, tq, p.W), g);
  if (p.mass.p && g == 0)
    st<float>(p.mass, b * p.mass.s0 + (int64_t)tq * p.mass.s1 + h * p.mass.s2, msum);
  if (TAU) {
    const int e = tau_empty_bound(p, tq);
    for (int col = g; col < e; col += 4) st<float>(p.tau, tau_off(p.tau, b, tq, h, col), 0.f);
  }
}

template <int NORM, bool BIAS, bool TAU>
static void go(const BandParams& p, hipStream_t st, unsigned nwg) {
  hipLaunchKernelGGL((mfma_fwd<NORM, BIAS, TAU>), dim3(nwg), dim3(kThreads), 0, st, p);
}

template <int NORM>
static void go_n(const BandParams& p, hipStream_t st, unsigned nwg, bool bias, bool tau) {
  if (bias) {
    if (tau) go<NORM, true, true>(p, st, nwg); else go<NORM, true, false>(p, st, nwg);
  } else {
    if (tau) go<NORM, false, true>(p, st, nwg); else go<NORM, false, false>(p, st, nwg);
  }
}

void launch_mfma_fwd(const BandParams& p, hipStream_t st, unsigned nwg, int norm) {
  const bool bias = p.bias.p != nullptr, tau = p.tau.p != nullptr;
  switch (norm) {
    case NORM_MASS_: go_n<NORM_MASS_>(p, st, nwg, bias, tau); break;
    case NORM_COUNT_: go_n<NORM_COUNT_>(p, st, nwg, bias, tau); break;
    default: go_n<NORM_RAW>(p, st, nwg, bias, tau); break;
  }
}

}  // namespace tension
