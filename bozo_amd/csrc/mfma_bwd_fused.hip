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
// Runs alternate direction: even runs step t = tA .. tB-1 and then the halo
// tB; odd runs start with the halo tB and step down to tA.  Two runs that
// share a boundary then reach it at the same time -- at their ends (an even
// run's halo, the next odd run's last step) or at their starts (an odd run's
// halo, the next even run's first step) -- so the boundary tiles and blocks
// the halo re-reads are read by both workgroups within one step (the runs
// of one (b, h) sit on one XCD, xcd_swizzle) and the second read is an L2
// hit instead of a second HBM read.  Ascending, the block a step completes
// is t-1 and block t is carried to the next step; descending, block t
// completes (it received tile t+1's part one step earlier) and block t-1 is
// carried down.
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

// Wave priority (s_setprio): 2 raises it over the whole of phase 1 (the
// step's longest dependent chain), so where the two workgroups of a CU are
// in different phases the phase-1 waves issue first and the other
// workgroup's phase-2 MFMAs fill their gaps (measured 0.3-0.7 us faster at
// config 2); 1 raises it over each group of MFMAs only (no gain); 0 off.
#ifndef TENSION_BWD_PRIO
#define TENSION_BWD_PRIO 2
#endif
#define BWD_PRIO(lvl, v)                                                   \
  do {                                                                     \
    if constexpr (TENSION_BWD_PRIO == (lvl)) __builtin_amdgcn_s_setprio(v); \
  } while (0)

// Alternating run directions (see above); 0 runs every run ascending.
#ifndef TENSION_BWD_ALTERNATE
#define TENSION_BWD_ALTERNATE 1
#endif

// FAST (W = 64, T a multiple of 64; a bias, or else dTau in bf16 rows): the band of every
// 16-query group is the same five key groups -- slot 0 the old block's
// diagonal group (key >= query - 64, i.e. 4g + r >= c within the group),
// slots 1..3 entirely valid, slot 4 the new block's diagonal group (key <=
// query - 1, i.e. 4g + r < c) -- so the masks are two per-lane constants and
// no per-element index arithmetic is needed.  With dTau, the step's dTau
// rows wait in each wave's G exchange sub-tiles until phase 1 reads them.
template <int NORM, bool BIAS, bool DTAU, bool FAST>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(TENSION_BWD_WAVES_PER_EU, TENSION_BWD_WAVES_PER_EU)))
void mfma_bwd_fused(BandArgs args) {
  static_assert(!FAST || !(BIAS && DTAU), "the fast path takes a bias or dTau, not both");
  touch_args(args);
  const BandParams p = band_params(args);
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
  const int tA = run_bound(run, p.ntiles, nch);
  const int tB = run_bound(run + 1, p.ntiles, nch);
  const int tE = tB < p.ntiles ? tB : tB - 1;  // the halo step when tB < ntiles, else tB - 1
  // the run's direction (uniform): odd runs step down from tE to tA
  const bool desc = TENSION_BWD_ALTERNATE && (run & 1) != 0;
  const int t0 = desc ? tE : tA;  // first step

  // per-sequence buffer views: rows >= T load as zeros, stores past T drop
  const SeqBuf sq = seq_view(p.q, b, h, T), sk = seq_view(p.k, b, h, T);
  const SeqBuf sv = seq_view(p.v, b, h, T), so = seq_view(p.dout, b, h, T);
  const SeqBuf sdq = seq_view(p.dq, b, h, T), sdk = seq_view(p.dk, b, h, T);
  const SeqBuf sdv = seq_view(p.dv, b, h, T);
  constexpr bool FDT = FAST && DTAU;  // dTau rows staged in the exchange tiles
  // thread tid moves 16 bytes of two staged tile rows (staged_row).  With
  // dTau the offsets are formed where they are used, from an opaque copy of
  // the thread index: as five loop-invariant registers they would push the
  // full register file into scratch.
  auto loff = [&](const SeqBuf& sb, uint32_t pre) -> uint32_t {
    if constexpr (FDT) {
      int x;
      asm volatile("v_mov_b32 %0, %1" : "=v"(x) : "v"(tid));
      return seq_lane_off(sb, x);
    } else {
      return pre;
    }
  };
  const uint32_t lq0 = FDT ? 0u : seq_lane_off(sq, tid), lk0 = FDT ? 0u : seq_lane_off(sk, tid);
  const uint32_t lv0 = FDT ? 0u : seq_lane_off(sv, tid), lo0 = FDT ? 0u : seq_lane_off(so, tid);
  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;
  SeqBuf sdt;
  if constexpr (FDT) sdt = seq_view(p.dtau, b, h, T);
  // FAST dTau: this wave's 16 dTau rows wait in its own G exchange sub-tiles
  // (free from the end of the previous phase 2 until this wave's phase 1
  // writes G there), row c shifted by c: slot s of query c sits at position
  // p = s + c of an 80-position row, position p in sub-tile p >> 4, column
  // p & 15.  Lane (g, c) then finds the dTau of its pairs (slots 16 sl + 4 g
  // + r - c) at sub-tile sl, row c, columns 4g..4g+3 -- exactly where it
  // writes their G afterwards, so no other lane touches them in between.
  auto dt_stage = [&](const TileRegs& x) {
    const int ra = (lane >> 3) & 7, ch = lane & 7;
    bf16* const base = XG + w * (kXSlots * kXSub);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int row = ra + 8 * hf;
      const bf16x8 v = __builtin_bit_cast(bf16x8, hf ? x.b : x.a);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int pos = 8 * ch + e + row;
        const int col = pos & 15;
        base[(pos >> 4) * kXSub + row * 16 + 4 * ((col >> 2) ^ xsw(row)) + (col & 3)] = v[e];
      }
    }
  };
  // the four dTau values of slot group sl of this lane's pairs, read just
  // before their use: the empty asm keeps the compiler from hoisting all
  // five reads (ten live registers) into the register-bound phase 1
  auto dt_at = [&](int sl) -> bf16x4 {
    asm volatile("" ::: "memory");
    return __builtin_bit_cast(bf16x4, *(const u16x4*)(XG + (w * kXSlots + sl) * kXSub + c * 16 + 4 * (g ^ xsw(c))));
  };

  // ---- prologue: blocks t0-1 (if any) and t0, tile t0
  {
    const uint32_t r0 = (uint32_t)(t0 * kTile);
    TileRegs k0 = seq_tile_load(sk, r0 * sk.rs2, loff(sk, lk0));
    TileRegs v0 = seq_tile_load(sv, r0 * sv.rs2, loff(sv, lv0));
    TileRegs q0 = seq_tile_load(sq, r0 * sq.rs2, loff(sq, lq0));
    TileRegs o0 = seq_tile_load(so, r0 * so.rs2, loff(so, lo0));
    if (t0 >= 1) {
      const uint32_t rm = r0 - kTile;
      TileRegs km = seq_tile_load(sk, rm * sk.rs2, loff(sk, lk0));
      TileRegs vm = seq_tile_load(sv, rm * sv.rs2, loff(sv, lv0));
      tile_store_direct(km, Kt[(t0 - 1) & 1], tid);
      tile_store_direct(vm, Vt[(t0 - 1) & 1], tid);
    }
    tile_store_direct(k0, Kt[t0 & 1], tid);
    tile_store_direct(v0, Vt[t0 & 1], tid);
    tile_store_direct(q0, Qt, tid);
    tile_store_direct(o0, Ot, tid);
    if constexpr (FDT) dt_stage(seq_tile_load(sdt, r0 * sdt.rs2, loff(sdt, 0)));
  }
  __syncthreads();
  // this wave's Q/dO fragments (query 16w + c, features 8g.., 32+8g..)
  bf16x8 qf[2], gf[2];
  qf[0] = dt_row8(Qt, 16 * w + c, g);
  qf[1] = dt_row8(Qt, 16 * w + c, 4 + g);
  gf[0] = dt_row8(Ot, 16 * w + c, g);
  gf[1] = dt_row8(Ot, 16 * w + c, 4 + g);

  // dK/dV (key group w) of the block the current step completes: carried
  // in from the previous step (ascending block t-1, descending block t)
  f32x4 dk_old[4] = {}, dv_old[4] = {};

  TileRegs dnext;  // FAST dTau: the next step's rows
  // FAST: diagonal-group masks (1 valid, 0 not) for keys 4g + r of query c
  // (lane conditions: the compiler keeps them as scalar lane masks)
  bool mo[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) mo[r] = 4 * g + r >= c;  // slot 0 keeps these; slot 4 the rest

  // FAST phase 1 with all five slots live (steps t >= 1; the halo only with
  // tau-mass normalisation): slot sl is key group w + sl of blocks t-1, t;
  // slot 0 is the old block's diagonal group, slot 4 the new block's
  // the step's bias (band_tile_bias, groups in slot order: j = (w + sl) & 3,
  // so slot sl reads bcur[sl & 3]; slots 0 and 4 share one element).  It
  // enters as the initial accumulator of the score product, scaled by
  // `scale` (sigma(S / scale + bias) = sigma((S + scale bias) / scale)), so
  // its registers are free once the product is issued.
  float bcur[BIAS ? 4 : 1][4];
  const float bsc = (float)p.scale;
  auto s_init = [&](int sl) -> f32x4 {
    if constexpr (BIAS && !DTAU) {
      const float* x = bcur[sl & 3];
      return f32x4{x[0] * bsc, x[1] * bsc, x[2] * bsc, x[3] * bsc};
    } else {
      return f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  auto phase1_live = [&](int t, auto dq_tag) {
    constexpr bool DQ = decltype(dq_tag)::value;
    const bf16* Kold = Kt[(t + 1) & 1];
    const bf16* Vold = Vt[(t + 1) & 1];
    const bf16* Knew = Kt[t & 1];
    const bf16* Vnew = Vt[t & 1];
    f32x4 sv[kXSlots], dv[kXSlots];
    BWD_PRIO(2, 1);
    BWD_PRIO(1, 1);
#pragma unroll
    for (int sl = 0; sl < kXSlots; ++sl) {
      const int gg = w + sl;
      const bf16* Ks = (gg >> 2) ? Knew : Kold;
      const bf16* Vs = (gg >> 2) ? Vnew : Vold;
      const int row = 16 * (gg & 3) + c;
      f32x4 a = s_init(sl), d = {};
      a = mfma(dt_row8(Ks, row, g), qf[0], a);
      a = mfma(dt_row8(Ks, row, 4 + g), qf[1], a);
      d = mfma(dt_row8(Vs, row, g), gf[0], d);
      d = mfma(dt_row8(Vs, row, 4 + g), gf[1], d);
      sv[sl] = a;
      dv[sl] = d;
    }
    BWD_PRIO(1, 0);
    float pv[kXSlots][4];
    float ms[kXSlots], ds[kXSlots];
#pragma unroll
    for (int sl = 0; sl < kXSlots; ++sl) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = sigmoid_scaled(sv[sl][r], k2, 0.f);
        if (sl == 0) x = mo[r] ? x : 0.f;
        if (sl == kXSlots - 1) x = mo[r] ? 0.f : x;
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
      bf16x4 dtv;
      if constexpr (FDT) dtv = dt_at(sl);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = pv[sl][r];
        float dt = fmaf(dv[sl][r], ca, -cc);
        if constexpr (FDT) {
          // positions outside the row (masked pairs, P = 0) hold stale bits
          const float d = (float)dtv[r];
          dt += (sl == 0 && !mo[r]) || (sl == kXSlots - 1 && mo[r]) ? 0.f : d;
        }
        gq[r] = dt * fmaf(-x, x, x);
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
      BWD_PRIO(1, 1);
      if ((w & 1) == 0) {
        dq_pair(w >> 1, gb[0], gb[1]);
        dq_pair((w >> 1) + 1, gb[2], gb[3]);
        dq_pair((w >> 1) + 2, gb[4], z);
      } else {
        dq_pair(w >> 1, z, gb[0]);
        dq_pair((w >> 1) + 1, gb[1], gb[2]);
        dq_pair((w >> 1) + 2, gb[3], gb[4]);
      }
      BWD_PRIO(1, 0);
      STORE_ROWS(sdq, (uint32_t)tq, acc, inv_scale);
    }
    BWD_PRIO(2, 0);
  };

  for (int t = t0; desc ? t >= tA : t <= tE; t += desc ? -1 : 1) {
    const bool halo = t >= tB;
    const bool more = desc ? t > tA : t < tE;
    const int tn = desc ? t - 1 : t + 1;  // the next step's tile
    // the K/V block the next step adds, into the slot of the block it no
    // longer needs: t+1 ascending (replacing t-1), t-2 descending (replacing
    // t; at t = 1 block 0 is stored again over itself)
    const int bn = desc ? (t >= 2 ? t - 2 : 0) : t + 1;
    // ---- prefetch of step t+1 into registers
    // the step's bias (band_tile_bias, groups in slot order: j = (w + sl) & 3)
    // goes out ahead of the next step's loads, and with a bias every step
    // issues those (the last step its own rows again, unused): on every path
    // the same loads are younger than the bias, so its first use in phase 1
    // waits for it alone, not for them
    // (With dTau as well that would spill: there the bias is loaded where
    // phase 1 starts.)
    constexpr bool BEARLY = BIAS && !DTAU;
    if constexpr (BEARLY) {
      band_tile_bias(p, b, t * kTile, w, g, c, w, bcur);
      asm volatile("" ::: "memory");
    }
    TileRegs kn, vn, qn, on;
    if (more || BEARLY) {
      const uint32_t rb = (uint32_t)((more ? bn : t) * kTile);
      kn = seq_tile_load(sk, rb * sk.rs2, loff(sk, lk0));
      vn = seq_tile_load(sv, rb * sv.rs2, loff(sv, lv0));
      if constexpr (!FAST) {  // fast path: issued at the start of phase 2
        const uint32_t r0 = (uint32_t)((more ? tn : t) * kTile);
        qn = seq_tile_load(sq, r0 * sq.rs2, loff(sq, lq0));
        on = seq_tile_load(so, r0 * so.rs2, loff(so, lo0));
      }
    }

    // ---- phase 1: queries 16w..16w+15 of tile t
    if (FAST && !BIAS && t >= 1 && (!halo || NORM == NORM_MASS_)) {
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
    // with dTau as well (BEARLY off): the band's bias, loaded ahead of the
    // products (pairs off the band read the batch's first element)
    float b2v[BIAS && !BEARLY ? kXSlots : 1][4];
    if constexpr (BIAS && !BEARLY) {
#pragma unroll
      for (int sl = 0; sl < kXSlots; ++sl) {
        const int gg = w + sl;
        const int key0 = (t - 1 + (gg >> 2)) * kTile + 16 * (gg & 3) + 4 * g;
        if (rowok && p.bias.s2 == 1 && sub_kind(wb, key0 - 4 * g) == 2) {
          // every key of the group is in the row's band: its four columns
          // are consecutive (one 16-byte load)
          const float* src = (const float*)p.bias.p + bias_off(p, b, tq, key0);
          float x[4];
          __builtin_memcpy(x, src, 16);
#pragma unroll
          for (int r = 0; r < 4; ++r) b2v[sl][r] = -kLog2e * x[r];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = key0 + r;
            const bool ok = (key >= lo) & (key <= hi);
            const float x = ld<float>(p.bias, ok ? bias_off(p, b, tq, key) : (int64_t)b * p.bias.s0);
            b2v[sl][r] = ok ? -kLog2e * x : 0.f;
          }
        }
      }
    }
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
      f32x4 s = s_init(sl), d = {};
      s = mfma(dt_row8(Ks, 16 * j + c, g), qf[0], s);
      s = mfma(dt_row8(Ks, 16 * j + c, 4 + g), qf[1], s);
      d = mfma(dt_row8(Vs, 16 * j + c, g), gf[0], d);
      d = mfma(dt_row8(Vs, 16 * j + c, 4 + g), gf[1], d);
      if (FAST) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = sigmoid_scaled(s[r], k2, 0.f);
          if (sl == 0) x = mo[r] ? x : 0.f;
          if (sl == kXSlots - 1) x = mo[r] ? 0.f : x;
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
        // computed on every lane (finite inputs) and selected: a conditional
        // sigmoid becomes a branch per element
        const float sg = sigmoid_scaled(s[r], k2, BIAS && DTAU ? b2v[sl][r] : 0.f);
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
        bf16x4 dtv;
        if constexpr (FDT) dtv = dt_at(sl);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = pv[sl][r];
          float dt = fmaf(dpv[sl][r], ca, -cc);
          if constexpr (FDT) {
            const float d = (float)dtv[r];
            dt += (sl == 0 && !mo[r]) || (sl == kXSlots - 1 && mo[r]) ? 0.f : d;
          }
          gq[r] = dt * fmaf(-x, x, x);
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

    if (more) {  // block bn replaces block t-1 (ascending) or t (descending)
      tile_store_direct(kn, Kt[bn & 1], tid);
      tile_store_direct(vn, Vt[bn & 1], tid);
      if constexpr (FAST) {
        // the next Q / dO tiles (and dTau rows): loaded here rather than with
        // K / V at the step's start, which leaves phase 1 16 more registers
        const uint32_t r1 = (uint32_t)(tn * kTile);
        qn = seq_tile_load(sq, r1 * sq.rs2, loff(sq, lq0));
        on = seq_tile_load(so, r1 * so.rs2, loff(so, lo0));
        if constexpr (FDT) dnext = seq_tile_load(sdt, r1 * sdt.rs2, loff(sdt, 0));
      }
    }

    // ---- phase 2: keys 16w..16w+15 of block t-1 (key group w) and of
    // block t (key group 4+w).  Query group j covers key groups j..j+4.
    // Block t-1 is this run's when t-1 >= tA, block t when t < tB.  The
    // accumulators hold the block the step completes (dk_old, dv_old: t-1
    // ascending, t descending) and the block carried to the next step
    // (dk_new, dv_new); only the exchange sub-tiles they read and the
    // conditions depend on the direction.
    const bool own_old = t > tA;
    const bool own_new = !halo;
    const bool own_done = desc ? own_new : own_old, own_next = desc ? own_old : own_new;
    f32x4 dk_new[4] = {}, dv_new[4] = {};
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int j0 = 2 * kk;
      // sub-tiles of block t-1 (key group w) and of block t (key group 4+w)
      // for query groups j0, j0+1 (x_pair arguments)
      const int o0 = w - j0, o1 = w - j0 - 1;
      const bool oq0 = true, oq1 = w >= j0 + 1;
      const int n0 = 4 + w - j0, n1 = 3 + w - j0;
      const bool nq0 = j0 >= w, nq1 = true;
      const bool need_old = j0 <= w, need_new = j0 + 1 >= w;
      const bool need_done = own_done && (desc ? need_new : need_old);
      const bool need_next = own_next && (desc ? need_old : need_new);
      if (!need_done && !need_next) continue;
      bf16x8 aq[4], ao[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        aq[m] = dt_tr8(Qt, m, 32 * kk, g, c);
        ao[m] = dt_tr8(Ot, m, 32 * kk, g, c);
      }
      if (need_done) {
        const int s0 = desc ? n0 : o0, s1 = desc ? n1 : o1;
        const bool q0 = desc ? nq0 : oq0, q1 = desc ? nq1 : oq1;
        const bf16x8 bp = x_pair(XP, j0, s0, q0, s1, q1, g, c);
        const bf16x8 bg = x_pair(XG, j0, s0, q0, s1, q1, g, c);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          dv_old[m] = mfma(ao[m], bp, dv_old[m]);
          dk_old[m] = mfma(aq[m], bg, dk_old[m]);
        }
      }
      if (need_next) {
        const int s0 = desc ? o0 : n0, s1 = desc ? o1 : n1;
        const bool q0 = desc ? oq0 : nq0, q1 = desc ? oq1 : nq1;
        const bf16x8 bp = x_pair(XP, j0, s0, q0, s1, q1, g, c);
        const bf16x8 bg = x_pair(XG, j0, s0, q0, s1, q1, g, c);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          dv_new[m] = mfma(ao[m], bp, dv_new[m]);
          dk_new[m] = mfma(aq[m], bg, dk_new[m]);
        }
      }
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
      // the next step's dTau rows (loaded during phase 2) into this wave's G
      // exchange sub-tiles, which phase 2 has finished reading; here, ahead
      // of the stores below, their wait does not include the stores
      if constexpr (FDT) {
        dt_stage(dnext);
        asm volatile("" ::: "memory");
      }
    }
    // the completed block's rows go out only now: on gfx9 stores count in
    // vmcnt, and issued before the next tile's rows were waited for above
    // (a store on some paths only, so the wait takes the stricter count)
    // they made every step wait for its stores' completion
    if (own_done) {
      const uint32_t tk = (uint32_t)((desc ? t : t - 1) * kTile + 16 * w + c);
      STORE_ROWS(sdk, tk, dk_old, inv_scale);
      STORE_ROWS(sdv, tk, dv_old, 1.f);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      dk_old[m] = dk_new[m];
      dv_old[m] = dv_new[m];
    }
  }
  // ascending, the last block of the sequence has no halo step: it is
  // complete after its own step (no query tile follows it)
  if (!desc && tE == tB - 1) {
    const uint32_t tk = (uint32_t)((tB - 1) * kTile + 16 * w + c);
    STORE_ROWS(sdk, tk, dk_old, inv_scale);
    STORE_ROWS(sdv, tk, dv_old, 1.f);
  }
#undef STORE_ROWS
}

template <int NORM, bool BIAS, bool DTAU, bool FAST>
static void go(const BandParams& p, hipStream_t st, unsigned nwg) {
  BandArgs a;
  if (!band_args(p, &a)) return;  // the host takes this kernel only with 32-bit strides
  hipLaunchKernelGGL((mfma_bwd_fused<NORM, BIAS, DTAU, FAST>), dim3(nwg), dim3(kThreads), 0, st, a);
}

template <int NORM>
static void go_n(const BandParams& p, hipStream_t st, unsigned nwg, bool bias, bool dtau) {
  if (bias) {
    if (dtau)
      go<NORM, true, true, false>(p, st, nwg);
    else if (p.win == kTile && p.T % kTile == 0)
      go<NORM, true, false, true>(p, st, nwg);
    else
      go<NORM, true, false, false>(p, st, nwg);
  } else if (dtau) {
    // bf16 dTau rows of 64 slots, 16-byte aligned: staged by the fast path
    const Buf& d = p.dtau;
    const bool rows16 = d.dt == TENSION_BF16 && ((d.s0 | d.s1 | d.s2) & 7) == 0 && ((uintptr_t)d.p & 15) == 0 &&
                        rows_fit_view((int64_t)p.T + 2 * kTile, d.s1);
    if (p.win == kTile && p.T % kTile == 0 && rows16)
      go<NORM, false, true, true>(p, st, nwg);
    else
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
