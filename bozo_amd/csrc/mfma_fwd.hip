// bf16 MFMA band forward (local window and global block), head dim 64.
//
// The four waves of a workgroup split a 64-query tile (16 queries each).
// For every 64-key block of the tile's band:
//   S^T = K Q^T   (A = K rows read from LDS, B = this wave's Q fragment)
//   P   = sigma(S/scale + bias) on the band, 0 elsewhere      (fp32)
//   O^T += V^T P^T (A = V^T read transposed from the row-major V tile,
//                   B = P^T packed straight from the C layout of S^T)
// S^T leaves lane (g, c) holding keys 16j+4g+r of query c, which is already
// the B-operand layout of the P.V product once two 16-key groups are packed,
// so no shuffle of P is needed.  16-key sub-blocks outside the wave's band
// are skipped (see WaveBand).
//
// Two kernels share that block routine:
//   mfma_fwd_ring (local windows W <= 64): a workgroup owns `chunk`
//     consecutive query tiles of one (b,h).  Tile t needs key blocks t-1
//     and t; a three-slot ring of LDS tiles holds them while block t+1
//     streams in (global_load_lds), so each K/V block is fetched once per
//     chunk and its HBM latency overlaps the previous tile's arithmetic.
//     The slots are tiles of one LDS array selected at compile time; the
//     ring is synchronised with fence-free barriers after explicit copy
//     waits, so reads of one slot do not wait on the DMA into another.
//   mfma_fwd (any band, including the global block): one tile per workgroup,
//     key blocks streamed through a two-deep ring.
#include "mfma_common.h"

namespace tension {

// The raw bias (float32) of one key block's pairs for this lane's query tq:
// keys kb0 + 16 j + 4 g + r.  Rows past T read row T-1.  A group inside the
// band of every valid row of the wave (a wave-uniform test; row T-1's band
// holds it too) is one 16-byte load per lane; other pairs read their column
// clamped into the row, so pairs off the band read some element of the row.
// Such pairs are masked where the bias is used, and the -log2(e) factor is
// applied there: nothing waits for these loads before the products that
// follow them, and no lane-divergent branch surrounds them.
__device__ __forceinline__ void fwd_bias_load(const BandParams& p, int kb0, const WaveBand& wb, int b, int tq, int g,
                                              float (*x)[4]) {
  const int tr = tq < p.T ? tq : p.T - 1;
  const float* row = (const float*)p.bias.p + (int64_t)b * p.bias.s0 + (int64_t)tr * p.bias.s1;
  const int cmax = (p.glob ? p.T : p.W) - 1;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c0 = bias_col(p, tr, kb0 + 16 * j + 4 * g);
    if (p.bias.s2 == 1 && sub_kind(wb, kb0 + 16 * j) == 2) {
      __builtin_memcpy(x[j], row + c0, 16);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int cc = c0 + r < 0 ? 0 : (c0 + r > cmax ? cmax : c0 + r);
        x[j][r] = row[(int64_t)cc * p.bias.s2];
      }
    }
  }
}

// One key block of a query tile: S^T, P, O^T += V^T P^T (and the mass).
// braw: the block's raw bias (fwd_bias_load) when BIAS.
// MMA_MASS: the tau mass comes from the P.V product itself -- one more MFMA
// per 32 keys with an all-ones A operand sums the bf16-rounded P that the
// output is built from, so out = msg / mass holds exactly for the weights
// used (the tau-mass backward takes its coefficients from out and mass).
// The per-lane sum (msum, reduced over the lane groups afterwards) is used
// otherwise.
template <bool BIAS, bool TAU, bool MMA_MASS = false>
__device__ __forceinline__ void fwd_block(const BandParams& p, const bf16* Ks, const bf16* Vs, int kb0,
                                          const WaveBand& wb, int lo, int hi, int b, int h, int tq,
                                          int g, int c, const bf16x8* qf, float k2, f32x4* acc,
                                          float& msum, f32x4* macc, const float (*braw)[4]) {
  float pr[4][4];
  int kind[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kind[j] = sub_kind(wb, kb0 + 16 * j);
    if (kind[j] == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) pr[j][r] = 0.f;
      continue;
    }
    f32x4 s = {};
    s = mfma(dt_row8(Ks, 16 * j + c, g), qf[0], s);
    s = mfma(dt_row8(Ks, 16 * j + c, 4 + g), qf[1], s);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kb0 + 16 * j + 4 * g + r;
      // kind 2 covers every valid row of the wave; rows past T (hi < lo)
      // stay masked so no tau store leaves the tensors
      const bool ok = kind[j] == 2 ? hi >= lo : ((key >= lo) & (key <= hi));
      const float b2 = BIAS ? -kLog2e * braw[j][r] : 0.f;
      // computed on every lane (finite inputs) and selected: a conditional
      // sigmoid becomes a branch per element
      const float sg = sigmoid_scaled(s[r], k2, b2);
      const float pv = ok ? sg : 0.f;
      if (TAU && ok) {
        const int col = tau_col(p, tq, key);
        if (col >= 0) st<float>(p.tau, tau_off(p.tau, b, tq, h, col), pv);
      }
      if (!MMA_MASS) msum += pv;
      pr[j][r] = pv;
    }
  }
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    if (kind[2 * kk] == 0 && kind[2 * kk + 1] == 0) continue;
    const bf16x8 pb = pack_b(pr[2 * kk], pr[2 * kk + 1]);
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = mfma(dt_tr8(Vs, m, 32 * kk, g, c), pb, acc[m]);
    if (MMA_MASS) *macc = mfma(ones_bf16x8(), pb, *macc);
  }
}

// msum: this lane's partial tau mass (reduced over the lane groups here), or
// with `summed` the full mass already.
template <int NORM, bool TAU>
__device__ __forceinline__ void fwd_epilogue(const BandParams& p, int b, int h, int tq, int g,
                                             const f32x4* acc, float msum, bool summed = false) {
  if (!summed) msum = wave_sum_g(msum);
  if (tq >= p.T) return;
  bf16* orow = (bf16*)p.out.p + b * p.out.s0 + (int64_t)tq * p.out.s1 + h * p.out.s2;
  store_row4x4(orow, acc, out_factor<NORM>(msum, tq, p.W), g);
  if (p.mass.p && g == 0)
    st<float>(p.mass, b * p.mass.s0 + (int64_t)tq * p.mass.s1 + h * p.mass.s2, msum);
  if (TAU) {
    const int e = tau_empty_bound(p, tq);
    for (int col = g; col < e; col += 4) st<float>(p.tau, tau_off(p.tau, b, tq, h, col), 0.f);
  }
}

// A finished output row (bf16) held back until the next tile's wait: on
// gfx9 stores count in vmcnt, so a store issued before the wait for the
// next key block would make that wait cover the store's completion too.
struct OutRow {
  u16x4 v[4];
  int tq;
  float msum;
};

template <int NORM, bool TAU>
__device__ __forceinline__ OutRow fwd_finish(const BandParams& p, int b, int h, int tq, int g, const f32x4* acc,
                                             float msum, bool summed = false) {
  OutRow o;
  o.msum = summed ? msum : wave_sum_g(msum);
  o.tq = tq;
  const float f = out_factor<NORM>(o.msum, tq, p.W);
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) o.v[m][r] = bf16_bits((bf16)(acc[m][r] * f));
  if (TAU && tq < p.T) {
    const int e = tau_empty_bound(p, tq);
    for (int col = g; col < e; col += 4) st<float>(p.tau, tau_off(p.tau, b, tq, h, col), 0.f);
  }
  return o;
}

__device__ __forceinline__ void fwd_store(const BandParams& p, int b, int h, int g, const OutRow& o) {
  if (o.tq >= p.T) return;
  bf16* orow = (bf16*)p.out.p + b * p.out.s0 + (int64_t)o.tq * p.out.s1 + h * p.out.s2;
#pragma unroll
  for (int m = 0; m < 4; ++m) *(u16x4*)(orow + 16 * m + 4 * g) = o.v[m];
  if (p.mass.p && g == 0) st<float>(p.mass, b * p.mass.s0 + (int64_t)o.tq * p.mass.s1 + h * p.mass.s2, o.msum);
}

// FAST-path output: the wave's 16 x 64 bf16 rows pass through its own 2 KB
// of a free LDS slot (16-byte chunk k of row r at position k ^ (r & 7)) and
// leave as whole 128-byte rows, 16 bytes per lane, instead of four 32-byte
// pieces per row (partial-line writes), with non-temporal stores: the rows
// are not read again by this kernel, and streaming them out (rather than
// leaving dirty lines in L2 for the end-of-kernel write-back) measured
// 16.2 -> 14.0 us at config 2.  LDS operations of one wave execute in order,
// so the read-back needs no barrier.
__device__ __forceinline__ void fwd_store_staged(const BandParams& p, int b, int h, int g, int c, int lane, int w,
                                                 const OutRow& o, bf16* slot) {
  bf16* sb = slot + w * (16 * kTile);
#pragma unroll
  for (int m = 0; m < 4; ++m)  // d = 16m + 4g .. +3: chunk 2m + g/2, half g & 1
    *(u16x4*)(sb + c * kTile + 8 * ((2 * m + (g >> 1)) ^ (c & 7)) + 4 * (g & 1)) = o.v[m];
  const int row0 = o.tq - c;  // first query row of the wave
  bf16* obase = (bf16*)p.out.p + b * p.out.s0 + h * p.out.s2;
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const int rr = (lane >> 3) + 8 * n, cc = lane & 7;
    const u16x8 v = *(const u16x8*)(sb + rr * kTile + 8 * (cc ^ (rr & 7)));
    __builtin_nontemporal_store(v, (u16x8*)(obase + (int64_t)(row0 + rr) * p.out.s1 + 8 * cc));
  }
  if (p.mass.p && g == 0) st<float>(p.mass, b * p.mass.s0 + (int64_t)o.tq * p.mass.s1 + h * p.mass.s2, o.msum);
}

// FAST-path tau rows (W = 64, bf16, 16-byte rows): lane (g, c) holds the tau
// of query c at slots 16 s5 + 4 g + r - c (s5 = 0..4, r = 0..3), of which
// the ones inside [0, 64) -- each slot exactly once per query -- go to the
// wave's 16 x 64 staging rows (swizzled as the output rows); the rows then
// leave as 16-byte pieces.
__device__ __forceinline__ void fwd_store_tau_staged(const BandParams& p, int b, int h, int g, int c, int lane,
                                                     int w, int t0, const u16x4* tv, bf16* slot) {
  unsigned short* sb = (unsigned short*)(slot + w * (16 * kTile));
#pragma unroll
  for (int s5 = 0; s5 < 5; ++s5)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = 16 * s5 + 4 * g + r - c;
      if (col >= 0 && col < kTile) sb[c * kTile + 8 * ((col >> 3) ^ (c & 7)) + (col & 7)] = tv[s5][r];
    }
  bf16* tbase = (bf16*)p.tau.p + b * p.tau.s0 + h * p.tau.s2;
  const int row0 = t0 + 16 * w;
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const int rr = (lane >> 3) + 8 * n, cc = lane & 7;
    const u16x8 v = *(const u16x8*)(sb + rr * kTile + 8 * (cc ^ (rr & 7)));
    __builtin_nontemporal_store(v, (u16x8*)(tbase + (int64_t)(row0 + rr) * p.tau.s1 + 8 * cc));
  }
}

// ------------------------------------------------------------------ ring kernel (W <= 64)

// One query tile at W = 64 with T % 64 == 0 (bias: BIAS, bx): the band of
// wave w (queries t0 + 16w + c) is 16-key sub-blocks s = w .. w+4 of the
// 128 keys of blocks t-1 (s < 4) and t (s >= 4).  Sub-block w keeps key
// index kk = 4g + r >= c, sub-block w+4 keeps kk < c, the three between are
// whole, so the masks are two lane constants (mlo, mhi).  The P.V products
// run over the sub-block pairs (2 pr, 2 pr + 1), pr = w/2 .. w/2 + 2, with a
// zero half where the pair sticks out of the band; the tau mass comes from
// an all-ones A operand (the bf16 P the output is built from).  Sub-blocks
// of block t-1 are absent on tile 0.  The wave index is a template argument
// so that every band decision is static.  TV: the tau of the lane's pairs,
// sub-block s5 = 0..4 of the band, as bf16 bits in tv[s5] (zero where masked
// or absent).
template <int w, bool TV = false, bool BIAS = false>
__device__ __forceinline__ void fwd_tile_fast(const bf16* Ka, const bf16* Va, const bf16* Kb, const bf16* Vb,
                                              bool has_prev, int g, int c, const bf16x8* qf, float k2,
                                              const bool* mlo, const bool* mhi, f32x4* acc, f32x4& macc,
                                              u16x4* tv = nullptr, const float (*bx)[4] = nullptr,
                                              float bsc = 0.f) {
  const bf16x8 ones = ones_bf16x8();
#pragma unroll
  for (int pi = 0; pi < 3; ++pi) {
    const int pr = (w >> 1) + pi;  // 0..3
    if (pr < 2 && !has_prev) {
      if constexpr (TV) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int s5 = 2 * pr + h2 - w;
          if (s5 >= 0 && s5 <= 4) tv[s5] = u16x4{0, 0, 0, 0};
        }
      }
      continue;
    }
    const bf16* Kt = pr < 2 ? Ka : Kb;
    const bf16* Vt = pr < 2 ? Va : Vb;
    // V^T of the pair, read as counted asm (see dt_tr8_issue)
    TrRead vr[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) vr[m] = dt_tr8_issue(Vt, m, 32 * (pr & 1), g, c);
    float pv[2][4];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int s5 = 2 * pr + h2 - w;  // position in the band, 0..4
      if (s5 < 0 || s5 > 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pv[h2][r] = 0.f;
        continue;
      }
      const int row = 16 * ((2 * pr + h2) & 3) + c;
      // BIAS: the slot's bias (band_tile_bias with jrot = w: bx[s5 & 3]) times
      // the scale starts the accumulator, sigma(S / scale + bias) =
      // sigma((S + scale bias) / scale)
      f32x4 z = {};
      if constexpr (BIAS) {
#pragma unroll
        for (int r = 0; r < 4; ++r) z[r] = bx[s5 & 3][r] * bsc;
      }
      z = mfma(dt_row8(Kt, row, g), qf[0], z);
      z = mfma(dt_row8(Kt, row, 4 + g), qf[1], z);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(z[r] * k2));
        pv[h2][r] = s5 == 0 ? (mlo[r] ? x : 0.f) : (s5 == 4 ? (mhi[r] ? x : 0.f) : x);
      }
      if constexpr (TV) {
#pragma unroll
        for (int r = 0; r < 4; ++r) tv[s5][r] = bf16_bits((bf16)pv[h2][r]);
      }
    }
    const bf16x8 pb = pack_b(pv[0], pv[1]);
    tr_wait4(vr);
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = mfma(tr_join(vr[m]), pb, acc[m]);
    macc = mfma(ones, pb, macc);
  }
}

template <int NORM, bool BIAS, bool TAU, bool FAST>
__global__ __launch_bounds__(kThreads) void mfma_fwd_ring(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  // the six ring tiles form one LDS object (separate objects make the
  // compiler wait for every copy in flight before each ring read); the
  // slots are still chosen at compile time
  __shared__ __attribute__((aligned(16))) bf16 ring[6 * kDTile];
  bf16* const K0 = ring;
  bf16* const K1 = ring + kDTile;
  bf16* const K2 = ring + 2 * kDTile;
  bf16* const V0 = ring + 3 * kDTile;
  bf16* const V1 = ring + 4 * kDTile;
  bf16* const V2 = ring + 5 * kDTile;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar branches on it
  const int g = lane >> 4, c = lane & 15;
  const int nch = (p.ntiles + p.chunk - 1) / p.chunk;
  const int id = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);
  const int bh = id / nch;
  const int b = bh / p.H, h = bh % p.H, T = p.T;
  const int t_first = (id % nch) * p.chunk;
  const int t_end = t_first + p.chunk < p.ntiles ? t_first + p.chunk : p.ntiles;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const float k2 = -kLog2e * (float)(1.0 / p.scale);

  // key block gb (rows 64 gb ..) into a slot pair
  const TileSrc ksrc = tile_src(kb_, p.k.s1, T, wave, lane), vsrc = tile_src(vb_, p.v.s1, T, wave, lane);
  auto fetch = [&](int gb, bf16* Kd, bf16* Vd) {
    if (gb >= 0 && gb < p.ntiles) {
      tile_async_src(ksrc, gb * kTile, Kd, wave);
      tile_async_src(vsrc, gb * kTile, Vd, wave);
    }
  };
  bool mlo[4], mhi[4];  // FAST band masks of the first / last sub-block
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mlo[r] = 4 * g + r >= c;
    mhi[r] = 4 * g + r < c;
  }

  // Everything the first two tiles need is requested up front (the third
  // ring slot is free until tile t_first + 1): Q of both tiles and key
  // blocks t_first - 1 .. t_first + 1, so a two-tile workgroup makes one
  // round trip to HBM instead of two.
  bf16x8 qf[2], qn[2];
  const bool pre = t_first + 1 < t_end;
  if constexpr (FAST) {
    // At most two tiles, as straight-line code with every copy
    // unconditional inside its branch (block -1 reads as block 0, which the
    // first tile does not use), so that the compiler can count the copies in
    // flight: tile t_first reads slots 0 and 1 while block t_first + 1 and
    // the next Q fragment are still arriving.
    auto fetch_any = [&](int gb, bf16* Kd, bf16* Vd) {
      tile_async_src(ksrc, (gb > 0 ? gb : 0) * kTile, Kd, wave);
      tile_async_src(vsrc, (gb > 0 ? gb : 0) * kTile, Vd, wave);
    };
    // TAU: the tile's tau leaves through tv and fwd_store_tau_staged, every
    // slot included (no separate zero fill)
    u16x4 tv[5];
    // BIAS: each tile's bias (band_tile_bias, jrot = wave): tile t_first's
    // goes out before the next block's copies, tile t_first + 1's behind the
    // first wait, so that the products of tile t_first run under it
    float bias0[BIAS ? 4 : 1][4], bias1[BIAS ? 4 : 1][4];
    const float bsc = (float)p.scale;
    auto fast_tile = [&](int t, const bf16* Ka, const bf16* Va, const bf16* Kb, const bf16* Vb,
                         const float (*bx)[4]) -> OutRow {
      const int tq = t * kTile + wave * 16 + c;
      f32x4 acc[4] = {}, macc = {};
      // wave priority raised over the tile's arithmetic: a workgroup that is
      // staging and storing rows issues in its gaps (0.05-0.1 us at config 2)
      __builtin_amdgcn_s_setprio(1);
      switch (wave) {
        case 0: fwd_tile_fast<0, TAU, BIAS>(Ka, Va, Kb, Vb, t >= 1, g, c, qf, k2, mlo, mhi, acc, macc, tv, bx, bsc); break;
        case 1: fwd_tile_fast<1, TAU, BIAS>(Ka, Va, Kb, Vb, t >= 1, g, c, qf, k2, mlo, mhi, acc, macc, tv, bx, bsc); break;
        case 2: fwd_tile_fast<2, TAU, BIAS>(Ka, Va, Kb, Vb, t >= 1, g, c, qf, k2, mlo, mhi, acc, macc, tv, bx, bsc); break;
        default: fwd_tile_fast<3, TAU, BIAS>(Ka, Va, Kb, Vb, t >= 1, g, c, qf, k2, mlo, mhi, acc, macc, tv, bx, bsc); break;
      }
      __builtin_amdgcn_s_setprio(0);
      return fwd_finish<NORM, false>(p, b, h, tq, g, acc, macc[0], true);
    };
    if (pre) {
      load_qfrag(qb_, p.q.s1, t_first * kTile + wave * 16 + c, T, g, qf);
      fetch_any(t_first - 1, K0, V0);
      fetch_any(t_first, K1, V1);
      if constexpr (BIAS) band_tile_bias(p, b, t_first * kTile, wave, g, c, wave, bias0);
      fetch_any(t_first + 1, K2, V2);
      load_qfrag(qb_, p.q.s1, (t_first + 1) * kTile + wave * 16 + c, T, g, qn);
      wait_vm<6>();  // block t_first + 1 (4 copies) and qn (2 loads) may be in flight
      lds_barrier();
      if constexpr (BIAS) band_tile_bias(p, b, (t_first + 1) * kTile, wave, g, c, wave, bias1);
      const OutRow o0 = fast_tile(t_first, K0, V0, K1, V1, bias0);
      wait_vm<0>();
      lds_barrier();  // slots K0 / V0 (block t_first - 1) are free: they stage the rows
      fwd_store_staged(p, b, h, g, c, lane, wave, o0, K0);
      if constexpr (TAU) fwd_store_tau_staged(p, b, h, g, c, lane, wave, t_first * kTile, tv, V0);
      qf[0] = qn[0];
      qf[1] = qn[1];
      const OutRow o1 = fast_tile(t_first + 1, K1, V1, K2, V2, bias1);
      fwd_store_staged(p, b, h, g, c, lane, wave, o1, K0);
      if constexpr (TAU) fwd_store_tau_staged(p, b, h, g, c, lane, wave, (t_first + 1) * kTile, tv, V0);
    } else {
      load_qfrag(qb_, p.q.s1, t_first * kTile + wave * 16 + c, T, g, qf);
      fetch_any(t_first - 1, K0, V0);
      fetch_any(t_first, K1, V1);
      if constexpr (BIAS) band_tile_bias(p, b, t_first * kTile, wave, g, c, wave, bias0);
      wait_vm<0>();
      lds_barrier();
      const OutRow o0 = fast_tile(t_first, K0, V0, K1, V1, bias0);
      fwd_store_staged(p, b, h, g, c, lane, wave, o0, K2);  // slot 2 holds no block
      if constexpr (TAU) fwd_store_tau_staged(p, b, h, g, c, lane, wave, t_first * kTile, tv, V2);
    }
    return;
  }
  // the bias of tile t_first (the generic path; band_tile_bias), then one
  // tile ahead in each step
  float bcur[BIAS ? 4 : 1][4], bnext[BIAS ? 4 : 1][4];
  if constexpr (BIAS && !FAST) band_tile_bias(p, b, t_first * kTile, wave, g, c, 0, bcur);
  load_qfrag(qb_, p.q.s1, t_first * kTile + wave * 16 + c, T, g, qf);
  fetch(t_first - 1, K0, V0);
  fetch(t_first, K1, V1);
  if (pre) {
    fetch(t_first + 1, K2, V2);
    load_qfrag(qb_, p.q.s1, (t_first + 1) * kTile + wave * 16 + c, T, g, qn);
  }
  OutRow pend;             // the previous tile's output, stored after the next wait
  bool has_pend = false;
  bf16* stage = K2;        // FAST: the slot no block uses in the latest step

  // tile t = t_first + lt uses key blocks t-1 (slot lt % 3) and t (slot
  // (lt+1) % 3); block t+1 goes to slot (lt+2) % 3, freed by tile t-1
  // (for lt = 0 it was requested before the loop).
  auto tile_step = [&](int lt, const bf16* Ka, const bf16* Va, const bf16* Kb, const bf16* Vb,
                       bf16* Kn, bf16* Vn) -> bool {
    const int t = t_first + lt;
    if (t >= t_end) return false;
    // lt = 0 with the prefetch: the 4 DMA instructions of block t+1 and the
    // 2 loads of its Q fragment were issued after block t's, so <= 6 may
    // still be in flight
    if (lt == 0 && pre) wait_vm<6>(); else wait_vm<0>();
    lds_barrier();  // no fence: it would wait for the prefetch too
    const bool more = t + 1 < t_end;
    // FAST (at most two tiles per workgroup): slot Kn receives no block in
    // this step, and the tile that last read it finished before the barrier
    if (has_pend) {
      if (FAST) fwd_store_staged(p, b, h, g, c, lane, wave, pend, Kn); else fwd_store(p, b, h, g, pend);
    }
    stage = Kn;
    const int t0 = t * kTile;
    const int tq = t0 + wave * 16 + c;
    // the next tile's bias (after the last tile, this tile's again) goes out
    // ahead of the next tile's copies: the wait for those at the next step
    // covers it, and this tile's (bcur, loaded one step earlier) has nothing
    // outstanding when its products need it
    if constexpr (BIAS && !FAST) {
      band_tile_bias(p, b, (more ? t + 1 : t) * kTile, wave, g, c, 0, bnext);
      asm volatile("" ::: "memory");
    }
    if (more && lt > 0) {
      load_qfrag(qb_, p.q.s1, (t + 1) * kTile + wave * 16 + c, T, g, qn);
      fetch(t + 1, Kn, Vn);
    }
    f32x4 acc[4] = {};
    if (FAST) {
      f32x4 macc = {};
      switch (wave) {
        case 0: fwd_tile_fast<0>(Ka, Va, Kb, Vb, t >= 1, g, c, qf, k2, mlo, mhi, acc, macc); break;
        case 1: fwd_tile_fast<1>(Ka, Va, Kb, Vb, t >= 1, g, c, qf, k2, mlo, mhi, acc, macc); break;
        case 2: fwd_tile_fast<2>(Ka, Va, Kb, Vb, t >= 1, g, c, qf, k2, mlo, mhi, acc, macc); break;
        default: fwd_tile_fast<3>(Ka, Va, Kb, Vb, t >= 1, g, c, qf, k2, mlo, mhi, acc, macc); break;
      }
      pend = fwd_finish<NORM, TAU>(p, b, h, tq, g, acc, macc[0], true);
    } else {
      const int lo = tq - p.win > 0 ? tq - p.win : 0;
      const int hi = tq < T ? tq - 1 + p.diag : -1;  // hi < lo: no key for this row
      const WaveBand wb = wave_band(p, t0 + wave * 16);
      // rows past T hold row T-1 (finite) and are masked out entirely
      float msum = 0.f;
      // bcur serves both blocks (band_tile_bias)
      if (t >= 1) fwd_block<BIAS, TAU>(p, Ka, Va, t0 - kTile, wb, lo, hi, b, h, tq, g, c, qf, k2, acc, msum, nullptr, bcur);
      fwd_block<BIAS, TAU>(p, Kb, Vb, t0, wb, lo, hi, b, h, tq, g, c, qf, k2, acc, msum, nullptr, bcur);
      pend = fwd_finish<NORM, TAU>(p, b, h, tq, g, acc, msum);
    }
    has_pend = true;
    if (more) { qf[0] = qn[0]; qf[1] = qn[1]; }
    if constexpr (BIAS && !FAST) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) bcur[j][r] = bnext[j][r];
    }
    return true;
  };

  for (int lt = 0;; lt += 3) {
    if (!tile_step(lt, K0, V0, K1, V1, K2, V2)) break;
    if (!tile_step(lt + 1, K1, V1, K2, V2, K0, V0)) break;
    if (!tile_step(lt + 2, K2, V2, K0, V0, K1, V1)) break;
  }
  if (has_pend) {
    if (FAST) fwd_store_staged(p, b, h, g, c, lane, wave, pend, stage); else fwd_store(p, b, h, g, pend);
  }
}

// ------------------------------------------------------------------ streaming kernel

template <int NORM, bool BIAS, bool TAU>
__global__ __launch_bounds__(kThreads) void mfma_fwd(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  __shared__ __attribute__((aligned(16))) bf16 Kb[2][kDTile];
  __shared__ __attribute__((aligned(16))) bf16 Vb[2][kDTile];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, p.glob != 0);
  const int b = id.b, h = id.h, T = p.T;
  const int t0 = id.tile * kTile;
  const int tq = t0 + wave * 16 + c;
  const int lo = tq - p.win > 0 ? tq - p.win : 0;
  const int hi = tq < T ? tq - 1 + p.diag : -1;
  const WaveBand wb = wave_band(p, t0 + wave * 16);

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
  load_qfrag(qb_, p.q.s1, tq, T, g, qf);
  tile_async(kb_, p.k.s1, kb_first, T, Kb[0], wave, lane);
  tile_async(vb_, p.v.s1, kb_first, T, Vb[0], wave, lane);
  if (nblk > 1) {
    tile_async(kb_, p.k.s1, kb_first + kTile, T, Kb[1], wave, lane);
    tile_async(vb_, p.v.s1, kb_first + kTile, T, Vb[1], wave, lane);
  }
  if (tq >= T) { qf[0] = bf16x8{}; qf[1] = bf16x8{}; }
  const float k2 = -kLog2e * (float)(1.0 / p.scale);
  f32x4 acc[4] = {};
  f32x4 macc = {};
  float msum = 0.f;
  for (int blk = 0; blk < nblk; ++blk) {
    const int kb0 = kb_first + blk * kTile;
    if (blk + 1 < nblk) wait_vm<4>(); else wait_vm<0>();
    __syncthreads();
    float braw[BIAS ? 4 : 1][4];
    if constexpr (BIAS) fwd_bias_load(p, kb0, wb, b, tq, g, braw);
    fwd_block<BIAS, TAU, true>(p, Kb[blk & 1], Vb[blk & 1], kb0, wb, lo, hi, b, h, tq, g, c, qf, k2, acc, msum,
                               &macc, braw);
    if (blk + 2 < nblk) {
      __syncthreads();  // every wave is done with this ring slot
      tile_async(kb_, p.k.s1, kb0 + 2 * kTile, T, Kb[blk & 1], wave, lane);
      tile_async(vb_, p.v.s1, kb0 + 2 * kTile, T, Vb[blk & 1], wave, lane);
    }
  }
  fwd_epilogue<NORM, TAU>(p, b, h, tq, g, acc, macc[0], true);
}

// ------------------------------------------------------------------ launch

template <int NORM, bool BIAS, bool TAU>
static void go(const BandParams& p, hipStream_t st, unsigned nwg, bool ring) {
  if (ring) {
    const unsigned n = (unsigned)((int64_t)p.B * p.H * ((p.ntiles + p.chunk - 1) / p.chunk));
#ifndef TENSION_NO_FAST_FWD
    // the staged output stores need a free ring slot: at most two tiles per
    // workgroup
    // with tau: bf16 rows of 64 slots, 16-byte aligned (staged stores)
    const Buf& tb = p.tau;
    const bool tau_rows = !TAU || (tb.dt == TENSION_BF16 && ((tb.s0 | tb.s1 | tb.s2) & 7) == 0 &&
                                   ((uintptr_t)tb.p & 15) == 0);
    BandArgs a;
    if (!band_args(p, &a)) return;  // the host takes the ring kernel only with 32-bit strides
    if (tau_rows && p.win == kTile && p.T % kTile == 0) {
      if (a.chunk > 2) a.chunk = 2;
      const unsigned nq = (unsigned)((int64_t)a.B * a.H * ((a.ntiles + a.chunk - 1) / a.chunk));
      hipLaunchKernelGGL((mfma_fwd_ring<NORM, BIAS, TAU, true>), dim3(nq), dim3(kThreads), 0, st, a);
      return;
    }
#else
    BandArgs a;
    if (!band_args(p, &a)) return;
#endif
    hipLaunchKernelGGL((mfma_fwd_ring<NORM, BIAS, TAU, false>), dim3(n), dim3(kThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL((mfma_fwd<NORM, BIAS, TAU>), dim3(nwg), dim3(kThreads), 0, st, to_args(p));
  }
}

template <int NORM>
static void go_n(const BandParams& p, hipStream_t st, unsigned nwg, bool bias, bool tau, bool ring) {
  if (bias) {
    if (tau) go<NORM, true, true>(p, st, nwg, ring); else go<NORM, true, false>(p, st, nwg, ring);
  } else {
    if (tau) go<NORM, false, true>(p, st, nwg, ring); else go<NORM, false, false>(p, st, nwg, ring);
  }
}

void launch_gl_fwd(const BandParams& p, hipStream_t st);

void launch_mfma_fwd(const BandParams& p, hipStream_t st, unsigned nwg, int norm) {
  const bool bias = p.bias.p != nullptr, tau = p.tau.p != nullptr;
#ifndef TENSION_NO_GL_FWD
  // gl_fwd keeps each lane's offset within a 64-row K / V tile in 32 bits
  // (tile_lane); larger row strides take the band kernel's 64-bit sources
  if (p.glob && norm == NORM_MASS_ && rows_fit_view(kTile, p.k.s1) && rows_fit_view(kTile, p.v.s1)) {
    launch_gl_fwd(p, st);
    return;
  }
#endif
  const bool ring = !p.glob && p.win <= kTile && p.chunk > 0;
  switch (norm) {
    case NORM_MASS_: go_n<NORM_MASS_>(p, st, nwg, bias, tau, ring); break;
    case NORM_COUNT_: go_n<NORM_COUNT_>(p, st, nwg, bias, tau, ring); break;
    default: go_n<NORM_RAW>(p, st, nwg, bias, tau, ring); break;
  }
}

}  // namespace tension
