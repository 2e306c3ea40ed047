// bf16 MFMA forward of the global block (full causal, diagonal included,
// tau-mass normalised; model.py:217-238), head dim 64, no bias / tau_local.
//
// The block is MFMA-shaped (T x T causal) and its per-score VALU work (the
// sigmoid: one multiply, exp2, add, rcp, bf16 pack) outweighs the MFMA work,
// so the kernel is laid out to keep both units fed:
//   * a workgroup owns a 64-query tile and streams the key blocks 0 .. tile
//     through a two-deep LDS ring (global_load_lds);
//   * wave w takes query half qh = w & 1 (32 queries, two 16-row MFMA tiles)
//     against key half kh = w >> 1 (32 keys) of every 64-key block, so every
//     K and V^T fragment read from LDS feeds two MFMAs;
//   * only the diagonal block is masked (key <= query); every earlier block
//     lies wholly inside every query's band;
//   * the tau mass comes from the P.V product (an all-ones A operand), i.e.
//     it sums exactly the bf16 P the output is built from;
//   * the two key halves of a query half meet once, through LDS, at the end.
// Workgroups go out heaviest tile first; blockIdx -> (b, h) keeps every tile
// of one (b, h) on one XCD (round-robin dispatch, B*H a multiple of 8), so its
// 512 KB of K/V stays in that XCD's L2, and groups the heads of a sequence on
// as few XCDs as it can (gl_slot).
#include <type_traits>

#include "mfma_common.h"

namespace tension {

// Optional operands of the global block, per (query, key) pair of one lane:
// the pre-sigmoid bias [B, T, T] (head-agnostic; float32, host-checked), and
// the column of the down-sampled tau_local / dtau_local [B, T, H, Wl] (slot
// j = key T-1-j, model.py:235-236), -1 when the pair has no slot there.
__device__ __forceinline__ bool gl_bias_rows4(const BandParams& p) {
  return p.bias.s2 == 1 && (p.bias.s1 & 3) == 0 && (p.bias.s0 & 3) == 0 && ((uintptr_t)p.bias.p & 15) == 0;
}

// A lane's raw bias of one key block (queries t0 + 32 qh + 16 i + c, keys
// blk * 64 + 32 kh + 16 j + 4 g + r): four 16-byte loads when the block lies
// inside [0, T) and the rows allow it (rows4: unit column stride, 16-byte
// aligned rows), else sixteen element loads; rows and keys past T read T-1
// (those pairs are masked).  Nothing is computed from the values here: the
// callers start their score accumulators with them (times the scale), and
// the empty asm statements keep the loads of the two forms apart (merged,
// every address became a per-lane product).
__device__ __forceinline__ void gl_bias_block(const BandParams& p, int b, int t0, int blk, int qh, int kh, int g,
                                              int c, bool rows4, float (*b2)[2][4]) {
  const float* bb = (const float*)p.bias.p + b * p.bias.s0;
  const int kbase = blk * kTile + 32 * kh + 4 * g;
  asm volatile("" ::: "memory");
  if (rows4 && (blk + 1) * kTile <= p.T) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = t0 + 32 * qh + 16 * i + c;
      const float* row = bb + (int64_t)(q < p.T ? q : p.T - 1) * p.bias.s1 + kbase;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x4 x = *(const f32x4*)(row + 16 * j);
#pragma unroll
        for (int r = 0; r < 4; ++r) b2[i][j][r] = x[r];
      }
    }
    asm volatile("" ::: "memory");
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = t0 + 32 * qh + 16 * i + c;
      const float* row = bb + (int64_t)(q < p.T ? q : p.T - 1) * p.bias.s1;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int k = kbase + 16 * j + r;
          b2[i][j][r] = row[(int64_t)(k < p.T ? k : p.T - 1) * p.bias.s2];
        }
    }
    asm volatile("" ::: "memory");
  }
}

// blockIdx -> (tile rank, b * H + h).  Dispatch is round-robin over the 8
// XCDs (id % 8).  With B H a multiple of 8, XCD x takes the B H / 8
// consecutive (b, h) pairs from x B H / 8 on, rank by rank: every tile of one
// (b, h) runs on one XCD (its K / V or Q / dO stays in that XCD's L2), and the
// heads of one sequence share as few XCDs as the count allows (they read the
// same head-agnostic bias rows).  Otherwise (b, h) = id % (B H).
struct GlSlot {
  int rank, bh;
};
__device__ __forceinline__ GlSlot gl_slot(int BH, int id) {
  if ((BH & 7) == 0) {
    const int per = BH >> 3, n = id >> 3;
    return {n / per, (id & 7) * per + n % per};
  }
  return {id / BH, id % BH};
}

__device__ __forceinline__ int gl_tau_col(const BandParams& p, int q, int k) {
  const int j = p.T - 1 - k;
  return (q < p.T && k < p.T && j < p.Wtau) ? j : -1;
}

#ifndef TENSION_GL_FWD_WPE
#define TENSION_GL_FWD_WPE 3
#endif
// with a bias or tau_local the per-pair operands need more registers: two
// waves per SIMD instead of spilling
#ifndef TENSION_GL_FWD_WPE_OPT
#define TENSION_GL_FWD_WPE_OPT 2
#endif

// One 64-query tile of the forward, on the calling workgroup's LDS `lds`
// (two ring slots: K in lds[s], V in lds[2 + s]; reused for the key-half
// merge and the output staging).
template <bool BIAS, bool TAU>
__device__ __forceinline__ void gl_fwd_tile(const BandParams& p, int tile, int b, int h, bf16 (*lds)[kDTile]) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int qh = wave & 1, kh = wave >> 1;
  const int T = p.T;
  const int t0 = tile * kTile;
  const int nblk = tile + 1;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;

  // Q^T fragments of this wave's two query tiles (rows past T read row T-1)
  bf16x8 qf[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) load_qfrag(qb_, p.q.s1, t0 + 32 * qh + 16 * i + c, T, g, qf[i]);
  if (TAU) {
    // tau_local slots of keys past this tile (j < T - 64 (tile + 1)) hold no
    // pair of its queries: zero them; the visited blocks write every other
    // slot, pair by pair, so no slot is written twice
    const int ez = min(p.Wtau, max(0, T - (tile + 1) * kTile));
    const bool vec = p.tau.dt == TENSION_BF16 && (ez & 7) == 0 && ((p.tau.s0 | p.tau.s1 | p.tau.s2) & 7) == 0 &&
                     ((uintptr_t)p.tau.p & 15) == 0;
    if (vec) {  // 16-byte pieces of zeros
      const int n8 = ez >> 3;
      const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int i = tid; i < kTile * n8; i += kThreads) {
        const int tq = t0 + i / n8;
        if (tq < T) *(u16x8*)((bf16*)p.tau.p + tau_off(p.tau, b, tq, h, 8 * (i % n8))) = zero;
      }
    } else {
      for (int i = tid; i < kTile * ez; i += kThreads) {
        const int tq = t0 + i / ez;
        if (tq < T) st<float>(p.tau, tau_off(p.tau, b, tq, h, i % ez), 0.f);
      }
    }
  }
  // Copies: every block before the diagonal one lies inside [0, T) and is
  // read at a uniform base plus this lane's fixed offsets; the diagonal block
  // (the last) has rows past T when T is ragged, and those are clamped.  A
  // copy past the last block is clamped to it: it fills a free slot nothing
  // reads, which keeps every copy unconditional.
  const TileLane kl = tile_lane(p.k.s1, wave, lane), vl = tile_lane(p.v.s1, wave, lane);
  const int64_t kstep = (int64_t)kTile * p.k.s1, vstep = (int64_t)kTile * p.v.s1;
  const bool ragged = (T % kTile) != 0;
  auto copy = [&](int blk, auto slot_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(slot_tag)::value;
    blk = blk < nblk ? blk : nblk - 1;
    if (ragged && blk == nblk - 1) {
      tile_async(kb_, p.k.s1, blk * kTile, T, lds[S], wave, lane);
      tile_async(vb_, p.v.s1, blk * kTile, T, lds[2 + S], wave, lane);
    } else {
      tile_dma(kb_ + blk * kstep, kl, lds[S], wave);
      tile_dma(vb_ + blk * vstep, vl, lds[2 + S], wave);
    }
  };
  // this lane's LDS fragment offsets within a tile (loop-invariant; the ring
  // slot is an immediate offset)
  uint32_t ko[2][2], vlo[4], vhi[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    ko[j][0] = dt_row_off(32 * kh + 16 * j + c, g);
    ko[j][1] = dt_row_off(32 * kh + 16 * j + c, 4 + g);
  }
  const uint32_t lbase = lds_addr(&lds[0][0]);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    dt_tr_off(m, 32 * kh, g, c, &vlo[m], &vhi[m]);
    vlo[m] += lbase;
    vhi[m] += lbase;
  }
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  // bias (gl_bias_block): it starts the score accumulators, sigma(S / scale
  // + bias) = sigma((S + scale bias) / scale).  With tau_local (BPRE) block
  // 0's goes out before the first copies, and each block loads the next
  // one's once its score products have taken its own, ahead of that block's
  // ring copy, so the wait for the copy before it also covers the bias, whose
  // latency runs under the rest of the block (the last block loads its own
  // again, unused).  Without tau_local each block loads its own at its start:
  // the one-ahead form needs more registers there, and at two waves per SIMD
  // instead of three it measured slower (74 -> 90 us, B4 H12 T2048 with a bias).
  constexpr bool BPRE = BIAS && TAU;
  const bool rows4 = BIAS && gl_bias_rows4(p);  // 16-byte bias loads
  const float bsc = (float)p.scale;
  float b2v[BIAS ? 2 : 1][2][4];
  if constexpr (BPRE) gl_bias_block(p, b, t0, 0, qh, kh, g, c, rows4, b2v);
  copy(0, S0{});
  copy(1, S1{});
  const float k2 = -kLog2e * (float)(1.0 / p.scale);
  const bf16x8 ones = ones_bf16x8();
  f32x4 acc[2][4] = {};
  f32x4 macc[2] = {};

  // one 64-key block in ring slot S: S, P, O += P V, mass += P 1 (diag: the
  // last block, masked key <= query; TB: the block holds tau_local columns)
  auto block = [&](int blk, auto slot_tag, auto diag_tag, auto tau_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(slot_tag)::value;
    constexpr bool diag = decltype(diag_tag)::value;
    constexpr bool TB = TAU && decltype(tau_tag)::value;
    constexpr uint32_t KO = S * kDTile * 2, VO = (2 + S) * kDTile * 2;
    if constexpr (BIAS && !BPRE) gl_bias_block(p, b, t0, blk, qh, kh, g, c, rows4, b2v);
    // S^T = K Q^T for keys 32 kh + 16 j + (4 g + r), queries 16 i + c (plus
    // scale times the bias)
    f32x4 s[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bf16x8 a0 = lds_row8<KO>(&lds[0][0], ko[j][0]);
      const bf16x8 a1 = lds_row8<KO>(&lds[0][0], ko[j][1]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f32x4 z = {};
        if constexpr (BIAS) {
#pragma unroll
          for (int r = 0; r < 4; ++r) z[r] = b2v[i][j][r] * bsc;
        }
        z = mfma(a0, qf[i][0], z);
        s[i][j] = mfma(a1, qf[i][1], z);
      }
    }
    if constexpr (BPRE) gl_bias_block(p, b, t0, blk + 1 < nblk ? blk + 1 : blk, qh, kh, g, c, rows4, b2v);
    TrRead vr[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) vr[m] = tr8_issue_at<VO>(vlo[m], vhi[m]);
    bf16x8 vt[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float pr[2][4];
      const int dq = 32 * qh + 16 * i + c;  // query - t0 (= query - kb0 on the diagonal block)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = blk * kTile + 32 * kh + 16 * j + 4 * g + r, query = t0 + dq;
          const float pv = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(s[i][j][r] * k2));
          pr[j][r] = (diag && 32 * kh + 16 * j + 4 * g + r > dq) ? 0.f : pv;
          if (TB) {
            const int col = gl_tau_col(p, query, key);
            if (col >= 0) st<float>(p.tau, tau_off(p.tau, b, query, h, col), pr[j][r]);
          }
        }
      const bf16x8 pb = pack_b(pr[0], pr[1]);
      if (i == 0) {
        tr_wait4(vr);
#pragma unroll
        for (int m = 0; m < 4; ++m) vt[m] = tr_join(vr[m]);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[i][m] = mfma(vt[m], pb, acc[i][m]);
      macc[i] = mfma(ones, pb, macc[i]);
    }
  };
  // tau_local columns are keys T - Wtau .. T - 1: only the blocks that hold
  // one run the per-pair column code
  auto visit = [&](int blk, auto slot_tag, auto diag_tag) __attribute__((always_inline)) {
    if constexpr (TAU) {
      if ((blk + 1) * kTile > T - p.Wtau) {
        block(blk, slot_tag, diag_tag, std::true_type{});
        return;
      }
    }
    block(blk, slot_tag, diag_tag, std::false_type{});
  };
  // Two-slot ring, two blocks per trip (slot 0 then slot 1), both before
  // the diagonal block.  Each wait leaves exactly the next block's copy (4
  // instructions) in flight: the loop only continues when block blk + 3
  // exists, and its copy was issued in the previous trip or the prologue.
  int blk = 0;
  for (; blk + 2 < nblk; blk += 2) {
    wait_vm<4>();
    lds_barrier();
    visit(blk, S0{}, std::false_type{});
    lds_barrier();  // every wave is done with slot 0
    copy(blk + 2, S0{});
    wait_vm<4>();
    lds_barrier();
    visit(blk + 1, S1{}, std::false_type{});
    lds_barrier();
    copy(blk + 3, S1{});
  }
  if (blk + 2 == nblk) {  // an off-diagonal block in slot 0, the diagonal in slot 1
    wait_vm<4>();
    lds_barrier();
    visit(blk, S0{}, std::false_type{});
    wait_vm<0>();
    lds_barrier();
    visit(blk + 1, S1{}, std::true_type{});
  } else {  // the diagonal block in slot 0
    wait_vm<0>();
    lds_barrier();
    visit(blk, S0{}, std::true_type{});
  }

  // Key halves meet: wave (qh, kh) keeps query tile i = kh and hands its
  // partial of tile 1 - kh to its partner (qh, 1 - kh) through LDS:
  // red[slot][e][lane], slot = 2 qh + kh, 17 floats (16 of O^T, 1 mass).
  wait_vm<0>();     // a copy past the last block may still be in flight
  __syncthreads();  // the ring slots are free
  float* red = (float*)&lds[0][0];  // 4 x 17 x 64 floats = 17 KB of the 32 KB
  auto give = [&](const f32x4* a, const f32x4& mm) {
    float* dst = red + (2 * qh + kh) * 17 * 64 + lane;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[(4 * m + r) * 64] = a[m][r];
    dst[16 * 64] = mm[0];
  };
  if (kh == 0) give(acc[1], macc[1]); else give(acc[0], macc[0]);
  __syncthreads();
  f32x4 o[4];
  float m;
  if (kh == 0) {
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) o[mm] = acc[0][mm];
    m = macc[0][0];
  } else {
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) o[mm] = acc[1][mm];
    m = macc[1][0];
  }
  {
    const float* src = red + (2 * qh + (1 - kh)) * 17 * 64 + lane;
    m += src[16 * 64];
#pragma unroll
    for (int mm = 0; mm < 4; ++mm)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[mm][r] += src[(4 * mm + r) * 64];
  }
  // rows out through the wave's 2 KB of LDS as whole lines (the merge reads
  // are done past the barrier)
  const int r0 = t0 + 32 * qh + 16 * kh;  // the wave's first row
  __syncthreads();
  store_rows_staged((bf16*)p.out.p + b * p.out.s0 + (int64_t)r0 * p.out.s1 + h * p.out.s2, p.out.s1, T - r0, o,
                    1.f / (m > kMassEps ? m : kMassEps), g, c, lane, &lds[0][0] + wave * (16 * kTile));
  const int tq = r0 + c;
  if (tq < T && p.mass.p && g == 0) st<float>(p.mass, b * p.mass.s0 + (int64_t)tq * p.mass.s1 + h * p.mass.s2, m);
}

// A workgroup owns one 64-query tile of one (b, h); workgroups go out
// heaviest tile first, and blockIdx -> (b, h) (gl_slot) keeps the tiles of
// one (b, h) on one XCD (round-robin dispatch).  (Pairing a heavy and a light
// tile per workgroup, one round of equal workgroups, measured slower.)
template <bool BIAS, bool TAU>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(BIAS || TAU ? TENSION_GL_FWD_WPE_OPT : TENSION_GL_FWD_WPE, 8)))
void gl_fwd(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  __shared__ __attribute__((aligned(16))) bf16 lds[4][kDTile];
  const GlSlot sl = gl_slot(p.B * p.H, (int)blockIdx.x);
  gl_fwd_tile<BIAS, TAU>(p, p.ntiles - 1 - sl.rank, sl.bh / p.H, sl.bh % p.H, lds);
}

// ---------------------------------------------------------------- backward
//
// The dQ kernel forms the per-query tau-mass coefficients a_t = 1/m_t and
// c_t = dO_t.out_t / m_t of its tile from the forward's saved rows and
// writes them to the workspace, where the dK/dV kernel (launched after it)
// reads them, so
//   dtau = a_t dP - c_t,   G = dtau * P (1 - P)   (P recomputed in fp32),
// and use the forward's 2 x 2 wave split (32 queries x 32 keys per wave per
// 64 x 64 block): every fragment read from LDS feeds two MFMAs, and the two
// partial sums of an output row meet once, through LDS, at the end.

#ifndef TENSION_GL_DQ_WPE
#define TENSION_GL_DQ_WPE 2
#endif
#ifndef TENSION_GL_DKV_WPE
#define TENSION_GL_DKV_WPE 2
#endif

// dQ: query-centric like the forward.  Wave (qh = w & 1, kh = w >> 1):
//   S^T = K Q^T, dP^T = V dO^T      (A = K / V rows from LDS)
//   dQ^T += K^T G^T                  (A = K^T read transposed)
template <bool BIAS, bool DTAU>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(TENSION_GL_DQ_WPE, 8)))
void gl_dq(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  __shared__ __attribute__((aligned(16))) bf16 lds[4][kDTile];
  bf16(*Kb)[kDTile] = lds;
  bf16(*Vb)[kDTile] = lds + 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int qh = wave & 1, kh = wave >> 1;
  const GlSlot sl = gl_slot(p.B * p.H, (int)blockIdx.x);
  const int tile = p.ntiles - 1 - sl.rank;  // heaviest first
  const int bh = sl.bh;
  const int b = bh / p.H, h = bh % p.H, T = p.T;
  const int t0 = tile * kTile;
  const int nblk = tile + 1;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const bf16* gb_ = (const bf16*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;

  const bf16* ob_ = (const bf16*)p.out.p + b * p.out.s0 + h * p.out.s2;

  // The tau-mass coefficients of this tile's queries, from the forward's
  // saved rows: a_t = 1 / max(m_t, eps), c_t = (dO_t . out_t) a_t (0 when
  // m_t < eps); each lane holds 16 of a row's 64 features of dO and out, the
  // four lanes of a row add their parts.  They go to the workspace for the
  // dK/dV kernel (written once, by the waves of key half 0).
  bf16x8 qf[2][2], gf[2][2];
  float ca[2], cc[2];
  const int64_t nws = (int64_t)p.B * p.T * p.H;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int tq = t0 + 32 * qh + 16 * i + c;
    load_qfrag(qb_, p.q.s1, tq, T, g, qf[i]);
    load_qfrag(gb_, p.dout.s1, tq, T, g, gf[i]);
    bf16x8 of[2];
    load_qfrag(ob_, p.out.s1, tq, T, g, of);
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dot = fmaf((float)of[0][e], (float)gf[i][0][e], dot);
      dot = fmaf((float)of[1][e], (float)gf[i][1][e], dot);
    }
    dot = wave_sum_g(dot);
    const int tr = tq < T ? tq : T - 1;
    const float m = ld<float>(p.mass, b * p.mass.s0 + (int64_t)tr * p.mass.s1 + h * p.mass.s2);
    ca[i] = 1.f / (m > kMassEps ? m : kMassEps);
    cc[i] = m >= kMassEps ? dot * ca[i] : 0.f;
    if (kh == 0 && g == 0 && tq < T) {
      const int64_t wi = ((int64_t)b * p.T + tq) * p.H + h;
      ((float*)p.ws)[wi] = ca[i];
      ((float*)p.ws)[nws + wi] = cc[i];
    }
  }
  const TileSrc ksrc = tile_src(kb_, p.k.s1, T, wave, lane), vsrc = tile_src(vb_, p.v.s1, T, wave, lane);
  // bias as in the forward (gl_bias_block, one block ahead, starting the
  // score accumulators); with a bias every block issues a ring copy (past
  // the last block, a copy of it into the free slot), so that the bias
  // loads have the same younger loads on every path
  const bool rows4 = BIAS && gl_bias_rows4(p);  // 16-byte bias loads
  const float bsc = (float)p.scale;
  float b2v[BIAS ? 2 : 1][2][4];
  if constexpr (BIAS) gl_bias_block(p, b, t0, 0, qh, kh, g, c, rows4, b2v);
  tile_async_src(ksrc, 0, Kb[0], wave);
  tile_async_src(vsrc, 0, Vb[0], wave);
  if (nblk > 1) {
    tile_async_src(ksrc, kTile, Kb[1], wave);
    tile_async_src(vsrc, kTile, Vb[1], wave);
  }
  const float k2 = -kLog2e * (float)(1.0 / p.scale);
  f32x4 acc[2][4] = {};

  auto block = [&](int blk, auto diag_tag, auto tau_tag) __attribute__((always_inline)) {
    constexpr bool diag = decltype(diag_tag)::value;
    constexpr bool TB = DTAU && decltype(tau_tag)::value;  // the block holds dtau_local columns
    const bf16* Ks = Kb[blk & 1];
    const bf16* Vs = Vb[blk & 1];
    f32x4 s[2][2], dp[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 32 * kh + 16 * j + c;
      const bf16x8 k0 = dt_row8(Ks, row, g), k1 = dt_row8(Ks, row, 4 + g);
      const bf16x8 v0 = dt_row8(Vs, row, g), v1 = dt_row8(Vs, row, 4 + g);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f32x4 z = {};
        if constexpr (BIAS) {
#pragma unroll
          for (int r = 0; r < 4; ++r) z[r] = b2v[i][j][r] * bsc;
        }
        z = mfma(k0, qf[i][0], z);
        s[i][j] = mfma(k1, qf[i][1], z);
        f32x4 y = {};
        y = mfma(v0, gf[i][0], y);
        dp[i][j] = mfma(v1, gf[i][1], y);
      }
    }
    if constexpr (BIAS) gl_bias_block(p, b, t0, blk + 1 < nblk ? blk + 1 : blk, qh, kh, g, c, rows4, b2v);
    TrRead kr[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) kr[m] = dt_tr8_issue(Ks, m, 32 * kh, g, c);
    bf16x8 kt[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float gd[2][4];
      const int dq = 32 * qh + 16 * i + c;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = blk * kTile + 32 * kh + 16 * j + 4 * g + r, query = t0 + dq;
          const float x = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(s[i][j][r] * k2));
          float dt = dp[i][j][r] * ca[i] - cc[i];
          if (TB) {
            const int col = gl_tau_col(p, query, key);
            if (col >= 0) dt += ld<float>(p.dtau, tau_off(p.dtau, b, query, h, col));
          }
          const float gv = dt * (x - x * x);
          gd[j][r] = (diag && 32 * kh + 16 * j + 4 * g + r > dq) ? 0.f : gv;
        }
      const bf16x8 pb = pack_b(gd[0], gd[1]);
      if (i == 0) {
        tr_wait4(kr);
#pragma unroll
        for (int m = 0; m < 4; ++m) kt[m] = tr_join(kr[m]);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[i][m] = mfma(kt[m], pb, acc[i][m]);
    }
  };
  auto visit = [&](int blk, auto diag_tag) __attribute__((always_inline)) {  // as in the forward
    if constexpr (DTAU) {
      if ((blk + 1) * kTile > T - p.Wtau) {
        block(blk, diag_tag, std::true_type{});
        return;
      }
    }
    block(blk, diag_tag, std::false_type{});
  };
  for (int blk = 0; blk + 1 < nblk; ++blk) {  // as in the forward
    wait_vm<4>();
    lds_barrier();
    visit(blk, std::false_type{});
    if (BIAS || blk + 2 < nblk) {
      const int nb = blk + 2 < nblk ? blk + 2 : nblk - 1;
      lds_barrier();
      tile_async_src(ksrc, nb * kTile, Kb[blk & 1], wave);
      tile_async_src(vsrc, nb * kTile, Vb[blk & 1], wave);
    }
  }
  // with a bias and nblk > 1 the last copy (of block nblk - 1 again, into
  // the other slot) may stay in flight until the merge below
  if (BIAS && nblk > 1) wait_vm<4>(); else wait_vm<0>();
  lds_barrier();
  visit(nblk - 1, std::true_type{});
  if constexpr (BIAS) wait_vm<0>();  // the merge reuses the ring's LDS

  // key halves meet (as in the forward): 16 floats per lane
  __syncthreads();
  float* red = (float*)&lds[0][0];
  auto give = [&](const f32x4* a) {
    float* dst = red + (2 * qh + kh) * 16 * 64 + lane;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[(4 * m + r) * 64] = a[m][r];
  };
  if (kh == 0) give(acc[1]); else give(acc[0]);
  __syncthreads();
  f32x4 o[4];
  if (kh == 0) {
#pragma unroll
    for (int m = 0; m < 4; ++m) o[m] = acc[0][m];
  } else {
#pragma unroll
    for (int m = 0; m < 4; ++m) o[m] = acc[1][m];
  }
  const float* src = red + (2 * qh + (1 - kh)) * 16 * 64 + lane;
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) o[m][r] += src[(4 * m + r) * 64];
  const int r0 = t0 + 32 * qh + 16 * kh;  // the wave's first row
  __syncthreads();
  store_rows_staged((bf16*)p.dq.p + b * p.dq.s0 + (int64_t)r0 * p.dq.s1 + h * p.dq.s2, p.dq.s1, T - r0, o,
                    (float)(1.0 / p.scale), g, c, lane, &lds[0][0] + wave * (16 * kTile));
}

// dK / dV: key-centric.  A workgroup owns a 64-key tile and streams the
// query blocks tile .. ntiles-1 (Q and dO through a two-deep LDS ring, the
// block's a_t / c_t through a small LDS ring).  Wave (kh = w & 1, qh = w >> 1):
//   S = Q K^T, dP = dO V^T            (A = Q / dO rows from LDS, B = this
//                                      wave's K / V fragments)
//   dV^T += dO^T (a P),  dK^T += Q^T G  (A = dO^T / Q^T read transposed)
// Query rows past T get a = c = 0, which zeroes their P and G.
template <bool BIAS, bool DTAU>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(TENSION_GL_DKV_WPE, 8)))
void gl_dkv(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  // one LDS object: the Q / dO ring (4 tiles) and, behind it, the
  // coefficient ring coef[slot][a, c][query] (with a second object the
  // compiler waits for every copy in flight before each ring read)
  __shared__ __attribute__((aligned(16))) bf16 lds[4 * kDTile + 8 * kTile];  // + 2 x 2 x 64 floats
  float(*coef)[2][kTile] = (float(*)[2][kTile])(lds + 4 * kDTile);
  static_assert(sizeof(lds) == 4 * kDTile * sizeof(bf16) + 2 * 2 * kTile * sizeof(float), "LDS layout");
  bf16(*Qb)[kDTile] = (bf16(*)[kDTile])lds;
  bf16(*Gb)[kDTile] = Qb + 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int kh = wave & 1, qh = wave >> 1;
  const GlSlot sl = gl_slot(p.B * p.H, (int)blockIdx.x);
  const int tile = sl.rank;  // key tile 0 sees every query block: heaviest first
  const int bh = sl.bh;
  const int b = bh / p.H, h = bh % p.H, T = p.T;
  const int k0 = tile * kTile;
  const int nblk = p.ntiles - tile;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const bf16* gb_ = (const bf16*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;
  const int64_t nws = (int64_t)p.B * p.T * p.H;
  const float* wsf = (const float*)p.ws;

  // K / V fragments (B operands) of this wave's two key tiles
  bf16x8 kf[2][2], vf[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int tk = k0 + 32 * kh + 16 * i + c;
    load_qfrag(kb_, p.k.s1, tk, T, g, kf[i]);
    load_qfrag(vb_, p.v.s1, tk, T, g, vf[i]);
  }
  // coefficient of query block qb for thread tid < 128 (a for tid < 64, c
  // for 64..127).  Every lane loads (rows past T clamped to T - 1; such
  // queries are zeroed where the coefficients are read) and nothing tests
  // the value until the next block: a load under a lane branch, or a select
  // right behind it, makes the compiler wait for every copy in flight.
  auto coef_load = [&](int qb) -> float {
    const int t = qb * kTile + (tid & 63);
    const int64_t wi = ((int64_t)b * p.T + (t < T ? t : T - 1)) * p.H + h;
    return wsf[((tid >> 6) & 1) * nws + wi];
  };
  const int q_first = tile;  // query blocks tile .. ntiles-1
  if (tid < 128) coef[0][tid >> 6][tid & 63] = coef_load(q_first);
  float cnext = nblk > 1 ? coef_load(q_first + 1) : 0.f;
  const TileSrc qsrc = tile_src(qb_, p.q.s1, T, wave, lane), gsrc = tile_src(gb_, p.dout.s1, T, wave, lane);
  // bias (float32, host-checked): the lane's two key columns (keys past T
  // read column T-1; those pairs are masked) from its first query row of a
  // block's half, 32 qh + 4 g
  const float* bcol[2] = {nullptr, nullptr};
  if constexpr (BIAS) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = k0 + 32 * kh + 16 * i + c;
      bcol[i] = (const float*)p.bias.p + b * p.bias.s0 + (int64_t)(key < T ? key : T - 1) * p.bias.s2 +
                (int64_t)(32 * qh + 4 * g) * p.bias.s1;
    }
  }
  // the bias of block blk's pairs (query 16 j + 4 g + r of the half, key
  // tile i) into b2n; rows past T (the last block of a ragged sequence) read
  // row T-1 (masked).  BPRE: block blk + 1's is loaded at the end of block
  // blk, ahead of the ring copy of block blk + 2, so the wait for that
  // copy's predecessor at the loop head also covers it.  With dtau_local
  // that would spill; there each block loads its own at its start, ahead of
  // its products.  (The empty asm statements keep the two paths' loads
  // apart: merged, every row offset became a per-lane 64-bit product.)
  constexpr bool BPRE = BIAS && !DTAU;
  float b2n[BIAS ? 2 : 1][2][4];
  auto bias_fetch = [&](int blk) __attribute__((always_inline)) {
    const int qf = (q_first + blk) * kTile;
    const int64_t s1 = p.bias.s1;
    asm volatile("" ::: "memory");
    if (qf + kTile <= T) {
      const int64_t o = (int64_t)qf * s1;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) b2n[i][j][r] = bcol[i][o + (16 * j + r) * s1];
      asm volatile("" ::: "memory");
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int q = qf + 32 * qh + 16 * j + 4 * g + r;
            b2n[i][j][r] = bcol[i][(int64_t)((q < T ? q : T - 1) - 32 * qh - 4 * g) * s1];
          }
      asm volatile("" ::: "memory");
    }
  };
  if constexpr (BPRE) bias_fetch(0);
  tile_async_src(qsrc, q_first * kTile, Qb[0], wave);
  tile_async_src(gsrc, q_first * kTile, Gb[0], wave);
  if (nblk > 1) {
    tile_async_src(qsrc, (q_first + 1) * kTile, Qb[1], wave);
    tile_async_src(gsrc, (q_first + 1) * kTile, Gb[1], wave);
  }
  const float k2 = -kLog2e * (float)(1.0 / p.scale);
  f32x4 dk[2][4] = {}, dv[2][4] = {};

  // one 64-query block (diag: the first, masked query >= key; TB: the key
  // tile holds dtau_local columns)
  auto block = [&](int blk, auto diag_tag, auto tau_tag) __attribute__((always_inline)) {
    constexpr bool diag = decltype(diag_tag)::value;
    constexpr bool TB = DTAU && decltype(tau_tag)::value;
    // slot (blk + 1) & 1 was last read in block blk - 1: free past the barrier
    if (blk + 1 < nblk && tid < 128) coef[(blk + 1) & 1][tid >> 6][tid & 63] = cnext;
    // unconditional (clamped to the last block) for the same reason
    cnext = coef_load(q_first + (blk + 2 < nblk ? blk + 2 : nblk - 1));
    const bf16* Qs = Qb[blk & 1];
    const bf16* Gs = Gb[blk & 1];
    if constexpr (BIAS && !BPRE) bias_fetch(blk);
    f32x4 s[2][2], dp[2][2];  // [query tile j][key tile i]
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 32 * qh + 16 * j + c;
      const bf16x8 q0 = dt_row8(Qs, row, g), q1 = dt_row8(Qs, row, 4 + g);
      const bf16x8 d0 = dt_row8(Gs, row, g), d1 = dt_row8(Gs, row, 4 + g);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f32x4 z = {};
        z = mfma(q0, kf[i][0], z);
        s[j][i] = mfma(q1, kf[i][1], z);
        f32x4 y = {};
        y = mfma(d0, vf[i][0], y);
        dp[j][i] = mfma(d1, vf[i][1], y);
      }
    }
    // a / c of queries 32 qh + 16 j + 4 g + r (0 past T)
    f32x4 a4[2], c4[2];
    const int qrow = (q_first + blk) * kTile + 32 * qh + 4 * g;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      a4[j] = *(const f32x4*)&coef[blk & 1][0][32 * qh + 16 * j + 4 * g];
      c4[j] = *(const f32x4*)&coef[blk & 1][1][32 * qh + 16 * j + 4 * g];
      if ((q_first + blk + 1) * kTile > T) {  // the last block of a ragged sequence
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool out = qrow + 16 * j + r >= T;
          a4[j][r] = out ? 0.f : a4[j][r];
          c4[j][r] = out ? 0.f : c4[j][r];
        }
      }
    }
    TrRead qr[4], gr[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      qr[m] = dt_tr8_issue(Qs, m, 32 * qh, g, c);
      gr[m] = dt_tr8_issue(Gs, m, 32 * qh, g, c);
    }
    bf16x8 qt[4], gt[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float pa[2][4], gd[2][4];
      const int dk_ = 32 * kh + 16 * i + c;  // key - k0 (= key - q0 on the diagonal block)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int query = (q_first + blk) * kTile + 32 * qh + 16 * j + 4 * g + r, key = k0 + dk_;
          const float b2 = BIAS ? -kLog2e * b2n[i][j][r] : 0.f;
          const float x = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(fmaf(s[j][i][r], k2, b2)));
          const bool off = diag && 32 * qh + 16 * j + 4 * g + r < dk_;  // query before key
          float dt = dp[j][i][r] * a4[j][r] - c4[j][r];
          if (TB) {
            const int col = gl_tau_col(p, query, key);
            if (col >= 0) dt += ld<float>(p.dtau, tau_off(p.dtau, b, query, h, col));
          }
          pa[j][r] = off ? 0.f : x * a4[j][r];
          gd[j][r] = off ? 0.f : dt * (x - x * x);
        }
      const bf16x8 pb = pack_b(pa[0], pa[1]);
      const bf16x8 gbv = pack_b(gd[0], gd[1]);
      if (i == 0) {
        tr_wait4(qr);
        tr_wait4(gr);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          qt[m] = tr_join(qr[m]);
          gt[m] = tr_join(gr[m]);
        }
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        dv[i][m] = mfma(gt[m], pb, dv[i][m]);
        dk[i][m] = mfma(qt[m], gbv, dk[i][m]);
      }
    }
    // unconditional (the last block loads its own again) for the same
    // reason as the ring copies
    if constexpr (BPRE) bias_fetch(blk + 1 < nblk ? blk + 1 : blk);
  };
  // Block blk's ring slot takes block blk + 2, or past the end a copy of the
  // last block that nothing reads: with every copy and coefficient load
  // unconditional, the compiler can tell which loads are in flight and does
  // not add a full wait of its own before the ring reads.
  auto refill = [&](int blk) {
    const int nb = blk + 2 < nblk ? blk + 2 : nblk - 1;
    lds_barrier();
    tile_async_src(qsrc, (q_first + nb) * kTile, Qb[blk & 1], wave);
    tile_async_src(gsrc, (q_first + nb) * kTile, Gb[blk & 1], wave);
  };
  // The diagonal block comes first; every block but the last has the next
  // block's copy (4 instructions) in flight.  The barriers also publish the
  // coefficient ring writes (lgkmcnt(0) before each).
  // dtau_local columns are keys T - Wtau .. T - 1: only key tiles that hold
  // one run the per-pair column code
  const bool kt_tau = DTAU && k0 + kTile > T - p.Wtau;
  auto visit = [&](int blk, auto diag_tag) __attribute__((always_inline)) {
    if constexpr (DTAU) {
      if (kt_tau) {
        block(blk, diag_tag, std::true_type{});
        return;
      }
    }
    block(blk, diag_tag, std::false_type{});
  };
  if (nblk == 1) {
    wait_vm<0>();
    lds_barrier();
    visit(0, std::true_type{});
  } else {
    wait_vm<4>();
    lds_barrier();
    visit(0, std::true_type{});
    refill(0);
    for (int blk = 1; blk + 1 < nblk; ++blk) {
      wait_vm<4>();
      lds_barrier();
      visit(blk, std::false_type{});
      refill(blk);
    }
    wait_vm<0>();
    lds_barrier();
    visit(nblk - 1, std::false_type{});
  }

  // query halves meet: wave (kh, qh) keeps key tile i = qh and hands tile
  // 1 - qh to its partner (kh, 1 - qh): 32 floats per lane (dK, dV)
  __syncthreads();
  float* red = (float*)lds;  // 4 x 32 x 64 floats = the 32 KB of the ring
  auto give = [&](const f32x4* a, const f32x4* v) {
    float* dst = red + (2 * kh + qh) * 32 * 64 + lane;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dst[(4 * m + r) * 64] = a[m][r];
        dst[(16 + 4 * m + r) * 64] = v[m][r];
      }
  };
  if (qh == 0) give(dk[1], dv[1]); else give(dk[0], dv[0]);
  __syncthreads();
  f32x4 ok_[4], ov[4];
  if (qh == 0) {
#pragma unroll
    for (int m = 0; m < 4; ++m) { ok_[m] = dk[0][m]; ov[m] = dv[0][m]; }
  } else {
#pragma unroll
    for (int m = 0; m < 4; ++m) { ok_[m] = dk[1][m]; ov[m] = dv[1][m]; }
  }
  const float* src = red + (2 * kh + (1 - qh)) * 32 * 64 + lane;
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ok_[m][r] += src[(4 * m + r) * 64];
      ov[m][r] += src[(16 + 4 * m + r) * 64];
    }
  const int r0 = k0 + 32 * kh + 16 * qh;  // the wave's first row
  __syncthreads();
  bf16* sb = lds + wave * (16 * kTile);
  store_rows_staged((bf16*)p.dk.p + b * p.dk.s0 + (int64_t)r0 * p.dk.s1 + h * p.dk.s2, p.dk.s1, T - r0, ok_,
                    (float)(1.0 / p.scale), g, c, lane, sb);
  store_rows_staged((bf16*)p.dv.p + b * p.dv.s0 + (int64_t)r0 * p.dv.s1 + h * p.dv.s2, p.dv.s1, T - r0, ov, 1.f,
                    g, c, lane, sb);
}

// the optional operands are template switches (BIAS: p.bias, TAU / DTAU:
// p.tau / p.dtau)
#define GL_LAUNCH(kernel, x, y)                                                            \
  do {                                                                                     \
    const unsigned n = (unsigned)((int64_t)p.B * p.H * p.ntiles);                          \
    const BandArgs a = to_args(p);                                                         \
    if (x) {                                                                               \
      if (y) hipLaunchKernelGGL((kernel<true, true>), dim3(n), dim3(kThreads), 0, st, a);   \
      else hipLaunchKernelGGL((kernel<true, false>), dim3(n), dim3(kThreads), 0, st, a);    \
    } else {                                                                               \
      if (y) hipLaunchKernelGGL((kernel<false, true>), dim3(n), dim3(kThreads), 0, st, a);  \
      else hipLaunchKernelGGL((kernel<false, false>), dim3(n), dim3(kThreads), 0, st, a);   \
    }                                                                                      \
  } while (0)

void launch_gl_dq(const BandParams& p, hipStream_t st) { GL_LAUNCH(gl_dq, p.bias.p, p.dtau.p); }

void launch_gl_dkv(const BandParams& p, hipStream_t st) { GL_LAUNCH(gl_dkv, p.bias.p, p.dtau.p); }

void launch_gl_fwd(const BandParams& p, hipStream_t st) { GL_LAUNCH(gl_fwd, p.bias.p, p.tau.p); }

#undef GL_LAUNCH

}  // namespace tension
