// bf16 MFMA band backward in one kernel (local windows W <= 64, head dim 64):
// dQ, dK and dV from a single pass over Q, K, V and dO, without atomics.
//
// A workgroup owns a run [tA, tB) of consecutive 64-row tiles of one (b, h):
// it writes dQ of query tiles tA..tB-1 and dK/dV of key blocks tA..tB-1.
// With W <= 64, query tile t sees key blocks t-1 and t, and key block k is
// seen by query tiles k and k+1, so step t (t = tA .. tB-1) completes dQ of
// tile t and dK/dV of block t-1; one extra "halo" step over query tile tB
// completes block tB-1 (the halo's dQ belongs to the next run and is not
// written).
//
// Step t, with K/V blocks t-1, t and the Q/dO tile t in LDS:
//   phase 1 (query-centric; wave w owns queries 16w..16w+15 of the tile):
//     S^T = K Q^T, dP^T = V dO^T over the 80-key band of its 16 queries
//     (five 16-key groups), P = sigma(S/scale + bias), the normalisation
//     coefficients a_t, c_t of those queries (in-wave: no workspace),
//     G = (a dP - c + dTau) P (1 - P),  dQ^T += K^T G^T  (registers),
//     and P' = a P, G into the exchange tiles X (bf16).
//   phase 2 (key-centric; wave w owns keys 16w..16w+15 of block t-1 and of
//     block t):  dV^T += dO^T P',  dK^T += Q^T G, with P' and G read back
//     transposed (ds_read_b64_tr_b16) from X and dO^T, Q^T from the tiles.
//     Block t-1 is complete after this phase and is written out.
// The next step's K/V block, Q/dO tile and Q/dO fragments are loaded into
// registers at the start of a step and stored to LDS behind the barriers.
//
// Exchange layout: for query group j and band slot sl (key group j + sl of
// the 128 keys of blocks t-1, t), a [16 query][16 key] bf16 sub-tile with a
// 32-byte row.  Phase-1 stores (lane (g,c): query c, keys 4g..4g+3) and
// phase-2 transposed reads (16 lanes: 4 rows x 16 keys) each touch 512
// contiguous bytes per wave instruction.
#include <type_traits>

#include "mfma_xchg.h"

namespace tension {

// Two waves per SIMD (two workgroups per CU): registers capped at 256.
#ifndef TENSION_BWD_WAVES_PER_EU
#define TENSION_BWD_WAVES_PER_EU 2
#endif

// FAST (W = 64, T a multiple of 64, no bias / dTau): the band of every
// 16-query group is the same five key groups -- slot 0 the old block's
// diagonal group (key >= query - 64, i.e. 4g + r >= c within the group),
// slots 1..3 entirely valid, slot 4 the new block's diagonal group (key <=
// query - 1, i.e. 4g + r < c) -- so the masks are two per-lane constants and
// no per-element index arithmetic is needed.
template <int NORM, bool BIAS, bool DTAU, bool FAST>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(TENSION_BWD_WAVES_PER_EU, TENSION_BWD_WAVES_PER_EU)))
void mfma_bwd_fused(BandParams p) {
  static_assert(!FAST || (!BIAS && !DTAU), "the fast path has no bias / dTau");
  __shared__ __attribute__((aligned(16))) bf16 Kt[2][kDTile];  // key block k in slot k & 1
  __shared__ __attribute__((aligned(16))) bf16 Vt[2][kDTile];
  __shared__ __attribute__((aligned(16))) bf16 Qt[kDTile];     // query tile of the step
  __shared__ __attribute__((aligned(16))) bf16 Ot[kDTile];     // dO tile of the step
  __shared__ __attribute__((aligned(16))) bf16 XP[kXElems];    // P' = a P
  __shared__ __attribute__((aligned(16))) bf16 XG[kXElems];    // G
#ifndef TENSION_BWD_DIRECT_STORES
  __shared__ __attribute__((aligned(16))) bf16 Stg[4 * 16 * kTile];  // per-wave output staging
#endif
  const int tid = threadIdx.x, lane = tid & 63;
  // the wave index is uniform across the wave; readfirstlane lets the
  // compiler see that, so every branch on it is a scalar branch
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  // output rows (dQ, dK, dV): row index `row` of lane c's row
#ifndef TENSION_BWD_DIRECT_STORES
  bf16* const stg = Stg + w * (16 * kTile);
#define STORE_ROWS(view, row, acc_, f_) seq_store_rows_staged(view, row, acc_, f_, g, c, lane, stg)
#else
#define STORE_ROWS(view, row, acc_, f_) seq_store_row4x4(view, (row) * (view).rs2, acc_, f_, g)
#endif
  const int nch = p.chunk;  // runs per (b, h)
  const int id = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);
  const int bh = id / nch, run = id % nch;
  const int b = bh / p.H, h = bh % p.H, T = p.T;
  const int tA = (int)((int64_t)run * p.ntiles / nch);
  const int tB = (int)((int64_t)(run + 1) * p.ntiles / nch);
  const int tE = tB < p.ntiles ? tB : tB - 1;  // last step (the halo when tB < ntiles)

  // per-sequence buffer views: rows >= T load as zeros, stores past T drop
  const SeqBuf sq = seq_view(p.q, b, h, T), sk = seq_view(p.k, b, h, T);
  const SeqBuf sv = seq_view(p.v, b, h, T), so = seq_view(p.dout, b, h, T);
  const SeqBuf sdq = seq_view(p.dq, b, h, T), sdk = seq_view(p.dk, b, h, T);
  const SeqBuf sdv = seq_view(p.dv, b, h, T);
  // thread tid moves 16 bytes of two staged tile rows (staged_row)
  const uint32_t lq = seq_lane_off(sq, tid), lk = seq_lane_off(sk, tid);
  const uint32_t lv = seq_lane_off(sv, tid), lo_ = seq_lane_off(so, tid);
  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;

  // ---- prologue: blocks tA-1 (if any) and tA, tile tA
  {
    const uint32_t r0 = (uint32_t)(tA * kTile);
    TileRegs k0 = seq_tile_load(sk, r0 * sk.rs2, lk);
    TileRegs v0 = seq_tile_load(sv, r0 * sv.rs2, lv);
    TileRegs q0 = seq_tile_load(sq, r0 * sq.rs2, lq);
    TileRegs o0 = seq_tile_load(so, r0 * so.rs2, lo_);
    if (tA >= 1) {
      const uint32_t rm = r0 - kTile;
      TileRegs km = seq_tile_load(sk, rm * sk.rs2, lk);
      TileRegs vm = seq_tile_load(sv, rm * sv.rs2, lv);
      tile_store_direct(km, Kt[(tA - 1) & 1], tid);
      tile_store_direct(vm, Vt[(tA - 1) & 1], tid);
    }
    tile_store_direct(k0, Kt[tA & 1], tid);
    tile_store_direct(v0, Vt[tA & 1], tid);
    tile_store_direct(q0, Qt, tid);
    tile_store_direct(o0, Ot, tid);
  }
  __syncthreads();
  // this wave's Q/dO fragments (query 16w + c, features 8g.., 32+8g..)
  bf16x8 qf[2], gf[2];
  qf[0] = dt_row8(Qt, 16 * w + c, g);
  qf[1] = dt_row8(Qt, 16 * w + c, 4 + g);
  gf[0] = dt_row8(Ot, 16 * w + c, g);
  gf[1] = dt_row8(Ot, 16 * w + c, 4 + g);

  // dK/dV of block t-1 (key group w), carried from step t-1 to step t
  f32x4 dk_old[4] = {}, dv_old[4] = {};
  // FAST: diagonal-group masks (1 valid, 0 not) for keys 4g + r of query c
  float mo[4], mn[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mo[r] = 4 * g + r >= c ? 1.f : 0.f;
    mn[r] = 1.f - mo[r];
  }

  // FAST phase 1 with all five slots live (steps t >= 1; the halo only with
  // tau-mass normalisation): slot sl is key group w + sl of blocks t-1, t;
  // slot 0 is the old block's diagonal group, slot 4 the new block's
  auto phase1_live = [&](int t, auto dq_tag) {
    constexpr bool DQ = decltype(dq_tag)::value;
    const bf16* Kold = Kt[(t + 1) & 1];
    const bf16* Vold = Vt[(t + 1) & 1];
    const bf16* Knew = Kt[t & 1];
    const bf16* Vnew = Vt[t & 1];
    f32x4 sv[kXSlots], dv[kXSlots];
#pragma unroll
    for (int sl = 0; sl < kXSlots; ++sl) {
      const int gg = w + sl;
      const bf16* Ks = (gg >> 2) ? Knew : Kold;
      const bf16* Vs = (gg >> 2) ? Vnew : Vold;
      const int row = 16 * (gg & 3) + c;
      f32x4 a = {}, d = {};
      a = mfma(dt_row8(Ks, row, g), qf[0], a);
      a = mfma(dt_row8(Ks, row, 4 + g), qf[1], a);
      d = mfma(dt_row8(Vs, row, g), gf[0], d);
      d = mfma(dt_row8(Vs, row, 4 + g), gf[1], d);
      sv[sl] = a;
      dv[sl] = d;
    }
    float pv[kXSlots][4];
    float ms[kXSlots], ds[kXSlots];
#pragma unroll
    for (int sl = 0; sl < kXSlots; ++sl) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = sigmoid_scaled(sv[sl][r], k2, 0.f);
        if (sl == 0) x *= mo[r];
        if (sl == kXSlots - 1) x *= mn[r];
        pv[sl][r] = x;
      }
      // short sums instead of one 20-long dependent chain
      ms[sl] = (pv[sl][0] + pv[sl][1]) + (pv[sl][2] + pv[sl][3]);
      ds[sl] = fmaf(pv[sl][0], dv[sl][0], pv[sl][1] * dv[sl][1]) + fmaf(pv[sl][2], dv[sl][2], pv[sl][3] * dv[sl][3]);
    }
    const int tq = t * kTile + 16 * w + c;
    float ca = 1.f, cc = 0.f;
    if (NORM == NORM_MASS_) {
      float msum = ((ms[0] + ms[1]) + (ms[2] + ms[3])) + ms[4];
      float dsum = ((ds[0] + ds[1]) + (ds[2] + ds[3])) + ds[4];
      msum = wave_sum_g(msum);
      dsum = wave_sum_g(dsum);
      ca = __builtin_amdgcn_rcpf(msum > kMassEps ? msum : kMassEps);
      cc = msum >= kMassEps ? dsum * ca * ca : 0.f;
    } else if (NORM == NORM_COUNT_) {
      const int cnt = tq < p.W ? tq : p.W;
      ca = __builtin_amdgcn_rcpf((float)(cnt > 1 ? cnt : 1));
    }
    u16x4 gb[kXSlots];
#pragma unroll
    for (int sl = 0; sl < kXSlots; ++sl) {
      float gq[4], pq[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = pv[sl][r];
        gq[r] = fmaf(dv[sl][r], ca, -cc) * fmaf(-x, x, x);
        pq[r] = x * ca;
      }
      gb[sl] = bf16x4_bits(gq[0], gq[1], gq[2], gq[3]);
      x_put_bits(XP, w, sl, g, c, bf16x4_bits(pq[0], pq[1], pq[2], pq[3]));
      x_put_bits(XG, w, sl, g, c, gb[sl]);
    }
    if constexpr (DQ) {
      f32x4 acc[4] = {};
      auto dq_pair = [&](int i, u16x4 lo4, u16x4 hi4) {
        const bf16* Ks = (i >> 1) ? Knew : Kold;
        const bf16x8 pb = join_bits(lo4, hi4);
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[m] = mfma(dt_tr8(Ks, m, 32 * (i & 1), g, c), pb, acc[m]);
      };
      const u16x4 z = {0, 0, 0, 0};
      if ((w & 1) == 0) {
        dq_pair(w >> 1, gb[0], gb[1]);
        dq_pair((w >> 1) + 1, gb[2], gb[3]);
        dq_pair((w >> 1) + 2, gb[4], z);
      } else {
        dq_pair(w >> 1, z, gb[0]);
        dq_pair((w >> 1) + 1, gb[1], gb[2]);
        dq_pair((w >> 1) + 2, gb[3], gb[4]);
      }
      STORE_ROWS(sdq, (uint32_t)tq, acc, inv_scale);
    }
  };

  for (int t = tA; t <= tE; ++t) {
    const bool halo = t >= tB;
    const bool more = t < tE;
    // ---- prefetch of step t+1 into registers
    TileRegs kn, vn, qn, on;
    if (more) {
      const uint32_t r0 = (uint32_t)((t + 1) * kTile);
      kn = seq_tile_load(sk, r0 * sk.rs2, lk);
      vn = seq_tile_load(sv, r0 * sv.rs2, lv);
      qn = seq_tile_load(sq, r0 * sq.rs2, lq);
      on = seq_tile_load(so, r0 * so.rs2, lo_);
    }

    // ---- phase 1: queries 16w..16w+15 of tile t
    if (FAST && t >= 1 && (!halo || NORM == NORM_MASS_)) {
      // every slot live: one branch-free block, so the LDS reads, MFMAs and
      // sigmoids of different slots overlap
      if (!halo)
        phase1_live(t, std::true_type{});
      else
        phase1_live(t, std::false_type{});
    } else {
    const bf16* Kold = Kt[(t + 1) & 1];  // block t-1
    const bf16* Vold = Vt[(t + 1) & 1];
    const bf16* Knew = Kt[t & 1];        // block t
    const bf16* Vnew = Vt[t & 1];
    const int tq = t * kTile + 16 * w + c;
    const int lo = tq - p.win > 0 ? tq - p.win : 0;
    const int hi = tq < T ? tq - 1 : -1;
    const bool rowok = hi >= lo;  // the query has at least one key
    const WaveBand wb = wave_band(p, t * kTile + 16 * w);
    float pv[kXSlots][4];
    f32x4 dpv[kXSlots];
    int kind[kXSlots];
    float msum = 0.f, dsum = 0.f;
#pragma unroll
    for (int sl = 0; sl < kXSlots; ++sl) {
      const int gg = w + sl;  // key group among the 8 of blocks t-1, t
      const int blk = gg >> 2, j = gg & 3;
      const int kb0 = (t - 1 + blk) * kTile + 16 * j;
      if (FAST) {
        const bool live = blk == 1 || t >= 1;
        kind[sl] = live ? (sl == 0 || sl == kXSlots - 1 ? 1 : 2) : 0;
      } else {
        kind[sl] = sub_kind(wb, kb0);
      }
      // the halo's new-block keys only feed its (unwritten) dQ; with tau-mass
      // normalisation they still enter the coefficients
      if (halo && blk == 1 && NORM != NORM_MASS_) kind[sl] = 0;
      if (kind[sl] == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pv[sl][r] = 0.f;
        dpv[sl] = f32x4{0.f, 0.f, 0.f, 0.f};
        continue;
      }
      const bf16* Ks = blk ? Knew : Kold;
      const bf16* Vs = blk ? Vnew : Vold;
      f32x4 s = {}, d = {};
      s = mfma(dt_row8(Ks, 16 * j + c, g), qf[0], s);
      s = mfma(dt_row8(Ks, 16 * j + c, 4 + g), qf[1], s);
      d = mfma(dt_row8(Vs, 16 * j + c, g), gf[0], d);
      d = mfma(dt_row8(Vs, 16 * j + c, 4 + g), gf[1], d);
      if (FAST) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = sigmoid_scaled(s[r], k2, 0.f);
          if (sl == 0) x *= mo[r];
          if (sl == kXSlots - 1) x *= mn[r];
          pv[sl][r] = x;
          if (NORM == NORM_MASS_) {
            msum += x;
            dsum = fmaf(x, d[r], dsum);
          }
        }
        dpv[sl] = d;
        continue;
      }
      const bool full = kind[sl] == 2;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 4 * g + r;
        const bool ok = full ? rowok : ((key >= lo) & (key <= hi));
        float b2 = 0.f;
        if (BIAS && ok) b2 = -kLog2e * ld<float>(p.bias, bias_off(p, b, tq, key));
        // computed on every lane (finite inputs) and selected: a conditional
        // sigmoid becomes a branch per element
        const float sg = sigmoid_scaled(s[r], k2, b2);
        const float x = ok ? sg : 0.f;
        pv[sl][r] = x;
        if (NORM == NORM_MASS_) {
          msum += x;
          dsum += x * d[r];
        }
      }
      dpv[sl] = d;
    }
    float ca = 1.f, cc = 0.f;
    if (NORM == NORM_MASS_) {
      msum = wave_sum_g(msum);
      dsum = wave_sum_g(dsum);
      const float m = msum > kMassEps ? msum : kMassEps;
      ca = 1.f / m;
      cc = msum >= kMassEps ? dsum * ca * ca : 0.f;
    } else if (NORM == NORM_COUNT_) {
      const int cnt = tq < p.W ? tq : p.W;
      ca = 1.f / (float)(cnt > 1 ? cnt : 1);
    }
    if (FAST) {
      // G = (a dP - c) P (1 - P): zero wherever P is masked to zero
      u16x4 gb[kXSlots];
#pragma unroll
      for (int sl = 0; sl < kXSlots; ++sl) {
        float gq[4], pq[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = pv[sl][r];
          gq[r] = fmaf(dpv[sl][r], ca, -cc) * fmaf(-x, x, x);
          pq[r] = x * ca;
        }
        gb[sl] = bf16x4_bits(gq[0], gq[1], gq[2], gq[3]);
        x_put_bits(XP, w, sl, g, c, bf16x4_bits(pq[0], pq[1], pq[2], pq[3]));
        x_put_bits(XG, w, sl, g, c, gb[sl]);
      }
      if (!halo) {
        f32x4 acc[4] = {};
        auto dq_pair = [&](int i, u16x4 lo4, u16x4 hi4) {
          const bf16* Ks = (i >> 1) ? Knew : Kold;
          const bf16x8 pb = join_bits(lo4, hi4);
#pragma unroll
          for (int m = 0; m < 4; ++m) acc[m] = mfma(dt_tr8(Ks, m, 32 * (i & 1), g, c), pb, acc[m]);
        };
        const u16x4 z = {0, 0, 0, 0};
        if ((w & 1) == 0) {
          if (kind[0] | kind[1]) dq_pair(w >> 1, gb[0], gb[1]);
          if (kind[2] | kind[3]) dq_pair((w >> 1) + 1, gb[2], gb[3]);
          if (kind[4]) dq_pair((w >> 1) + 2, gb[4], z);
        } else {
          if (kind[0]) dq_pair(w >> 1, z, gb[0]);
          if (kind[1] | kind[2]) dq_pair((w >> 1) + 1, gb[1], gb[2]);
          if (kind[3] | kind[4]) dq_pair((w >> 1) + 2, gb[3], gb[4]);
        }
        STORE_ROWS(sdq, (uint32_t)tq, acc, inv_scale);
      }
    } else {
    // G overwrites dP in place (dpv), P' = a P overwrites P (pv)
#pragma unroll
    for (int sl = 0; sl < kXSlots; ++sl) {
      const int gg = w + sl;
      const int kb0 = (t - 1 + (gg >> 2)) * kTile + 16 * (gg & 3);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 4 * g + r;
        const bool ok = kind[sl] != 0 && (kind[sl] == 2 ? rowok : ((key >= lo) & (key <= hi)));
        float dt = dpv[sl][r] * ca - cc;
        if (DTAU && ok) dt += ld<float>(p.dtau, tau_off(p.dtau, b, tq, h, key - tq + p.W));
        const float x = pv[sl][r];
        dpv[sl][r] = ok ? dt * x * (1.f - x) : 0.f;
        pv[sl][r] = x * ca;
      }
      const float gd4[4] = {dpv[sl][0], dpv[sl][1], dpv[sl][2], dpv[sl][3]};
      x_put(XP, w, sl, g, c, pv[sl]);
      x_put(XG, w, sl, g, c, gd4);
    }
    if (!halo) {
      // dQ^T += K^T G^T over 32-key pairs (key groups 2i, 2i+1); slot sl is
      // key group w + sl, so the pairing depends on the parity of w
      f32x4 acc[4] = {};
      auto dq_pair = [&](int i, const f32x4& lo4, const f32x4& hi4) {
        const bf16* Ks = (i >> 1) ? Knew : Kold;
        const float l[4] = {lo4[0], lo4[1], lo4[2], lo4[3]};
        const float u[4] = {hi4[0], hi4[1], hi4[2], hi4[3]};
        const bf16x8 pb = pack_b(l, u);
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[m] = mfma(dt_tr8(Ks, m, 32 * (i & 1), g, c), pb, acc[m]);
      };
      const f32x4 zz = {0.f, 0.f, 0.f, 0.f};
      if ((w & 1) == 0) {
        if (kind[0] | kind[1]) dq_pair(w >> 1, dpv[0], dpv[1]);
        if (kind[2] | kind[3]) dq_pair((w >> 1) + 1, dpv[2], dpv[3]);
        if (kind[4]) dq_pair((w >> 1) + 2, dpv[4], zz);
      } else {
        if (kind[0]) dq_pair(w >> 1, zz, dpv[0]);
        if (kind[1] | kind[2]) dq_pair((w >> 1) + 1, dpv[1], dpv[2]);
        if (kind[3] | kind[4]) dq_pair((w >> 1) + 2, dpv[3], dpv[4]);
      }
      STORE_ROWS(sdq, (uint32_t)tq, acc, inv_scale);
    }
    }  // !FAST
    }  // not all live
    __syncthreads();  // X written; every wave is done with block t-1

    if (more) {  // block t+1 replaces block t-1
      tile_store_direct(kn, Kt[(t + 1) & 1], tid);
      tile_store_direct(vn, Vt[(t + 1) & 1], tid);
    }

    // ---- phase 2: keys 16w..16w+15 of block t-1 (key group w) and of
    // block t (key group 4+w).  Query group j covers key groups j..j+4.
    const bool own_old = t >= 1 && t - 1 >= tA;
    const bool own_new = !halo;
    f32x4 dk_new[4] = {}, dv_new[4] = {};
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int j0 = 2 * kk;
      const bool need_old = own_old && j0 <= w;
      const bool need_new = own_new && j0 + 1 >= w;
      if (!need_old && !need_new) continue;
      bf16x8 aq[4], ao[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        aq[m] = dt_tr8(Qt, m, 32 * kk, g, c);
        ao[m] = dt_tr8(Ot, m, 32 * kk, g, c);
      }
      if (need_old) {
        const bf16x8 bp = x_pair(XP, j0, w - j0, true, w - j0 - 1, w >= j0 + 1, g, c);
        const bf16x8 bg = x_pair(XG, j0, w - j0, true, w - j0 - 1, w >= j0 + 1, g, c);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          dv_old[m] = mfma(ao[m], bp, dv_old[m]);
          dk_old[m] = mfma(aq[m], bg, dk_old[m]);
        }
      }
      if (need_new) {
        const bf16x8 bp = x_pair(XP, j0, 4 + w - j0, j0 >= w, 3 + w - j0, true, g, c);
        const bf16x8 bg = x_pair(XG, j0, 4 + w - j0, j0 >= w, 3 + w - j0, true, g, c);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          dv_new[m] = mfma(ao[m], bp, dv_new[m]);
          dk_new[m] = mfma(aq[m], bg, dk_new[m]);
        }
      }
    }
    if (own_old) {
      const uint32_t tk = (uint32_t)((t - 1) * kTile + 16 * w + c);
      STORE_ROWS(sdk, tk, dk_old, inv_scale);
      STORE_ROWS(sdv, tk, dv_old, 1.f);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      dk_old[m] = dk_new[m];
      dv_old[m] = dv_new[m];
    }
    __syncthreads();  // phase 2 is done with X and the Q/dO tiles

    if (more) {
      // each wave stores exactly its own 16 rows (16w..16w+15) of the next
      // Q/dO tile, so it reads its fragments back without a barrier (LDS
      // accesses of one wave complete in order)
      tile_store_direct(qn, Qt, tid);
      tile_store_direct(on, Ot, tid);
      qf[0] = dt_row8(Qt, 16 * w + c, g);
      qf[1] = dt_row8(Qt, 16 * w + c, 4 + g);
      gf[0] = dt_row8(Ot, 16 * w + c, g);
      gf[1] = dt_row8(Ot, 16 * w + c, 4 + g);
    }
  }
  // the last block of the sequence has no halo step: it is complete after
  // its own step (no query tile follows it)
  if (tE == tB - 1) {
    const uint32_t tk = (uint32_t)((tB - 1) * kTile + 16 * w + c);
    STORE_ROWS(sdk, tk, dk_old, inv_scale);
    STORE_ROWS(sdv, tk, dv_old, 1.f);
  }
#undef STORE_ROWS
}

template <int NORM, bool BIAS, bool DTAU, bool FAST>
static void go(const BandParams& p, hipStream_t st, unsigned nwg) {
  hipLaunchKernelGGL((mfma_bwd_fused<NORM, BIAS, DTAU, FAST>), dim3(nwg), dim3(kThreads), 0, st, p);
}

template <int NORM>
static void go_n(const BandParams& p, hipStream_t st, unsigned nwg, bool bias, bool dtau) {
  if (bias) {
    if (dtau) go<NORM, true, true, false>(p, st, nwg); else go<NORM, true, false, false>(p, st, nwg);
  } else if (dtau) {
    go<NORM, false, true, false>(p, st, nwg);
  } else if (p.win == kTile && p.T % kTile == 0) {
    go<NORM, false, false, true>(p, st, nwg);
  } else {
    go<NORM, false, false, false>(p, st, nwg);
  }
}

// p.chunk = runs per (b, h); grid = B * H * p.chunk
void launch_mfma_bwd_fused(const BandParams& p, hipStream_t st, unsigned nwg, int norm) {
  const bool bias = p.bias.p != nullptr, dtau = p.dtau.p != nullptr;
  switch (norm) {
    case NORM_MASS_: go_n<NORM_MASS_>(p, st, nwg, bias, dtau); break;
    case NORM_COUNT_: go_n<NORM_COUNT_>(p, st, nwg, bias, dtau); break;
    default: go_n<NORM_RAW>(p, st, nwg, bias, dtau); break;
  }
}

}  // namespace tension
