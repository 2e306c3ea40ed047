// MFMA band kernels for the reference's autocast dtype flow: float32 Q, K
// (rotated, model.py:75-81) with a bfloat16 V, float32 out / tau, and in the
// backward a float32 dOut (the gradient of the float32 output) -> float32
// dQ, dK, bfloat16 dV.  Local windows W <= 64, head dim 64.  The reference
// computes this call in float32 (kernel.py:71-98: every load upcast).
//
// Every float32 operand x is split on its way into registers or LDS into a
// bfloat16 pair x = hi + lo + r with hi = bf16(x), lo = bf16(x - hi) and
// |r| <= 2^-17 |x|, and a product of two such operands takes three bf16
// MFMAs (lo.hi + hi.lo + hi.hi, small terms first into the float32
// accumulator; lo.lo ~ 2^-16 is left out), a product with an exact bf16
// operand (V) two.  Sums therefore carry ~16 significant bits per term and
// float32 accumulation: results agree with a float32 evaluation to about
// 1e-6 relative.  The products are 2-3x the bf16 kernels' MFMA work, which
// these memory-bound kernels absorb.
//
// Three kernels, each one 64-row tile per workgroup, four waves:
//   mx_fwd: query tile t, key blocks t-1 and t (the whole band);
//   mx_dq:  query tile t: S, dP, the normalisation coefficients a_t, c_t
//           of its queries (written to the workspace), G, dQ;
//   mx_dkv: key block k, query tiles k and k+1: S, dP, G, dK, dV.
// Tiles live in unpadded direct LDS tiles (mfma_common.h), filled from
// registers, read as rows (dt_row8) or transposed (dt_tr8).
#include "mfma_common.h"

namespace tension {

namespace {

// 8 consecutive float32 values split into bf16 hi / lo bit patterns.
__device__ __forceinline__ void split8(const float* x, u16x8& hi, u16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bf16 h = (bf16)x[e];
    hi[e] = bf16_bits(h);
    lo[e] = bf16_bits((bf16)(x[e] - (float)h));
  }
}

// 8 float32 values at p (16-byte aligned), split.
__device__ __forceinline__ void load_split8(const float* p, u16x8& hi, u16x8& lo) {
  const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
  const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  split8(x, hi, lo);
}

struct SplitFrag {  // an A / B operand of a float32 tensor
  bf16x8 hi, lo;
};

// Operand fragment: features 8 chunk .. +7 of row `row` (zero past T).
__device__ __forceinline__ SplitFrag frag_f32(const float* base, int64_t rs, int row, int T, int chunk) {
  SplitFrag f;
  u16x8 h = {0, 0, 0, 0, 0, 0, 0, 0}, l = h;
  if (row < T) load_split8(base + (int64_t)row * rs + 8 * chunk, h, l);
  f.hi = __builtin_bit_cast(bf16x8, h);
  f.lo = __builtin_bit_cast(bf16x8, l);
  return f;
}

// A float32 tile's two staged rows (staged_row, +8) of this thread, split:
// rows outside [0, T) are zero.
struct SplitRegs {
  TileRegs hi, lo;
};

__device__ __forceinline__ SplitRegs tile_load_split(const float* base, int64_t rs, int r0, int T, int tid) {
  const int ch = tid & 7;
  const int ra = r0 + staged_row(tid), rb = ra + 8;
  SplitRegs x;
  const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
  x.hi.a = z; x.lo.a = z; x.hi.b = z; x.lo.b = z;
  if (ra >= 0 && ra < T) load_split8(base + (int64_t)ra * rs + 8 * ch, x.hi.a, x.lo.a);
  if (rb >= 0 && rb < T) load_split8(base + (int64_t)rb * rs + 8 * ch, x.hi.b, x.lo.b);
  return x;
}

// A float32 tile's two staged rows of this thread as loaded (zero outside
// [0, T)); split_rows turns them into tile_load_split's result later.
struct RawRows {
  f32x4 a0, a1, b0, b1;
};

__device__ __forceinline__ RawRows tile_load_raw(const float* base, int64_t rs, int r0, int T, int tid) {
  const int ch = tid & 7;
  const int ra = r0 + staged_row(tid), rb = ra + 8;
  RawRows x;
  x.a0 = x.a1 = x.b0 = x.b1 = f32x4{0.f, 0.f, 0.f, 0.f};
  if (ra >= 0 && ra < T) {
    x.a0 = *(const f32x4*)(base + (int64_t)ra * rs + 8 * ch);
    x.a1 = *(const f32x4*)(base + (int64_t)ra * rs + 8 * ch + 4);
  }
  if (rb >= 0 && rb < T) {
    x.b0 = *(const f32x4*)(base + (int64_t)rb * rs + 8 * ch);
    x.b1 = *(const f32x4*)(base + (int64_t)rb * rs + 8 * ch + 4);
  }
  return x;
}

__device__ __forceinline__ SplitRegs split_rows(const RawRows& r) {
  SplitRegs x;
  const float a[8] = {r.a0[0], r.a0[1], r.a0[2], r.a0[3], r.a1[0], r.a1[1], r.a1[2], r.a1[3]};
  const float b[8] = {r.b0[0], r.b0[1], r.b0[2], r.b0[3], r.b1[0], r.b1[1], r.b1[2], r.b1[3]};
  split8(a, x.hi.a, x.lo.a);
  split8(b, x.hi.b, x.lo.b);
  return x;
}

// A bf16 tile's two staged rows of this thread (zero outside [0, T)).
__device__ __forceinline__ TileRegs tile_load_staged(const bf16* base, int64_t rs, int r0, int T, int tid) {
  const int ch = tid & 7;
  const int ra = r0 + staged_row(tid), rb = ra + 8;
  TileRegs x;
  const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
  x.a = z;
  x.b = z;
  if (ra >= 0 && ra < T) x.a = *(const u16x8*)(base + (int64_t)ra * rs + 8 * ch);
  if (rb >= 0 && rb < T) x.b = *(const u16x8*)(base + (int64_t)rb * rs + 8 * ch);
  return x;
}

// C += A B for split A and B: lo.hi + hi.lo + hi.hi.
__device__ __forceinline__ f32x4 mm3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh, const bf16x8& bl,
                                     f32x4 c) {
  c = mfma(al, bh, c);
  c = mfma(ah, bl, c);
  return mfma(ah, bh, c);
}

// C += A B for an exact bf16 A and a split B (or the transpose).
__device__ __forceinline__ f32x4 mm2(const bf16x8& a, const bf16x8& bh, const bf16x8& bl, f32x4 c) {
  c = mfma(a, bl, c);
  return mfma(a, bh, c);
}

// B operand from two 16-row groups of float32 C-layout values, split.
__device__ __forceinline__ void pack_split(const float* lo4, const float* hi4, bf16x8& h, bf16x8& l) {
  const float x[8] = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
  u16x8 a, b;
  split8(x, a, b);
  h = __builtin_bit_cast(bf16x8, a);
  l = __builtin_bit_cast(bf16x8, b);
}

// Four float32 C-layout rows (features 16m + 4g .. +3) of one output row,
// scaled by f, as 16-byte stores.
__device__ __forceinline__ void store_row_f32(float* row, const f32x4* acc, float f, int g) {
#pragma unroll
  for (int m = 0; m < 4; ++m) *(f32x4*)(row + 16 * m + 4 * g) = acc[m] * f;
}

}  // namespace

// ---------------------------------------------------------------- forward

// Key blocks t-1 and t pass through one set of LDS tiles in turn (24 KB)
// rather than side by side; without bias, block t's rows are loaded into
// registers while block t-1 is worked on.
// Neighbouring tiles visit their shared block / tile in the same stage.
#ifndef TENSION_MX_ALTERNATE
#define TENSION_MX_ALTERNATE 1
#endif

#ifndef TENSION_MX_FWD_SLOTS
#define TENSION_MX_FWD_SLOTS 1
#endif
#ifndef TENSION_MX_FWD_PREFETCH
#define TENSION_MX_FWD_PREFETCH 1
#endif

template <int NORM, bool BIAS, bool TAU>
__global__ __launch_bounds__(kThreads) void mx_fwd(BandParams p) {
  // key block t-1+s in slot s % NS: K hi, K lo, V
  constexpr int NS = TENSION_MX_FWD_SLOTS;
  __shared__ __attribute__((aligned(16))) bf16 lds[3 * NS * kDTile];
  bf16* const Kh = lds;
  bf16* const Kl = lds + NS * kDTile;
  bf16* const Vs = lds + 2 * NS * kDTile;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, false);
  const int b = id.b, h = id.h, T = p.T;
  const int t0 = id.tile * kTile;
  const int tq = t0 + wave * 16 + c;
  const int lo = tq - p.win > 0 ? tq - p.win : 0;
  const int hi = tq < T ? tq - 1 : -1;  // hi < lo: no key for this row
  const WaveBand wb = wave_band(p, t0 + wave * 16);
  // odd tiles take block t first: the block two neighbouring tiles share is
  // then read by both in the same stage (the second read an L2 hit)
  const bool rev = TENSION_MX_ALTERNATE && (id.tile & 1) != 0;
  auto blk0 = [&](int s) { return t0 - kTile + (rev ? 1 - s : s) * kTile; };

  const float* qb_ = (const float*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const float* kb_ = (const float*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;

  // key block t-1+s into slot s % NS
  auto store_blk = [&](int s, const SplitRegs& kx, const TileRegs& vx) {
    const int sl = (s % NS) * kDTile;
    tile_store_direct(kx.hi, Kh + sl, tid);
    tile_store_direct(kx.lo, Kl + sl, tid);
    tile_store_direct(vx, Vs + sl, tid);
  };
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int kb0 = blk0(s);
    store_blk(s, tile_load_split(kb_, p.k.s1, kb0, T, tid), tile_load_staged(vb_, p.v.s1, kb0, T, tid));
  }
  // with one slot and no bias (whose per-pair loads need the registers):
  // block t's rows in flight during block t-1
  constexpr bool PF = NS == 1 && !BIAS && TENSION_MX_FWD_PREFETCH;
  RawRows kn{};
  TileRegs vn{};
  const SplitFrag q0 = frag_f32(qb_, p.q.s1, tq, T, g), q1 = frag_f32(qb_, p.q.s1, tq, T, 4 + g);
  __syncthreads();

  const float k2 = -kLog2e * (float)(1.0 / p.scale);
  f32x4 acc[4] = {};
  float msum = 0.f;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int kb0 = blk0(s);
    if (PF && s == 0) {
      kn = tile_load_raw(kb_, p.k.s1, blk0(1), T, tid);
      vn = tile_load_staged(vb_, p.v.s1, blk0(1), T, tid);
    }
    if (s >= NS) {  // the slot of block s - NS is free once every wave is past it
      __syncthreads();
      if constexpr (PF)
        store_blk(s, split_rows(kn), vn);
      else
        store_blk(s, tile_load_split(kb_, p.k.s1, kb0, T, tid), tile_load_staged(vb_, p.v.s1, kb0, T, tid));
      __syncthreads();
    }
    const bf16* kh = Kh + (s % NS) * kDTile;
    const bf16* kl = Kl + (s % NS) * kDTile;
    float pr[4][4];
    int kind[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kind[j] = kb0 + 16 * j + 15 < 0 ? 0 : sub_kind(wb, kb0 + 16 * j);
      if (kind[j] == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[j][r] = 0.f;
        continue;
      }
      // S^T = K Q^T: keys 16 j + 4 g + r (rows), query c (column)
      f32x4 sc = {};
      sc = mm3(dt_row8(kh, 16 * j + c, g), dt_row8(kl, 16 * j + c, g), q0.hi, q0.lo, sc);
      sc = mm3(dt_row8(kh, 16 * j + c, 4 + g), dt_row8(kl, 16 * j + c, 4 + g), q1.hi, q1.lo, sc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = (key >= lo) & (key <= hi);
        float b2 = 0.f;
        if (BIAS && ok) b2 = -kLog2e * ld<float>(p.bias, bias_off(p, b, tq, key));
        const float pv = ok ? sigmoid_scaled(sc[r], k2, b2) : 0.f;
        if (TAU && ok) {
          const int col = tau_col(p, tq, key);
          if (col >= 0) st<float>(p.tau, tau_off(p.tau, b, tq, h, col), pv);
        }
        msum += pv;
        pr[j][r] = pv;
      }
    }
    // O^T += V^T P^T over 32-key pairs (A = V^T read transposed)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if (kind[2 * kk] == 0 && kind[2 * kk + 1] == 0) continue;
      bf16x8 ph, pl;
      pack_split(pr[2 * kk], pr[2 * kk + 1], ph, pl);
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m] = mm2(dt_tr8(Vs + (s % NS) * kDTile, m, 32 * kk, g, c), ph, pl, acc[m]);
    }
  }
  msum = wave_sum_g(msum);
  if (tq >= T) return;
  float* orow = (float*)p.out.p + b * p.out.s0 + (int64_t)tq * p.out.s1 + h * p.out.s2;
  store_row_f32(orow, acc, out_factor<NORM>(msum, tq, p.W), g);
  if (p.mass.p && g == 0) st<float>(p.mass, b * p.mass.s0 + (int64_t)tq * p.mass.s1 + h * p.mass.s2, msum);
  if (TAU) {
    const int e = tau_empty_bound(p, tq);
    for (int col = g; col < e; col += 4) st<float>(p.tau, tau_off(p.tau, b, tq, h, col), 0.f);
  }
}

// ---------------------------------------------------------------- dQ

template <int NORM, bool BIAS, bool DTAU>
__global__ __launch_bounds__(kThreads) void mx_dq(BandParams p) {
  __shared__ __attribute__((aligned(16))) bf16 lds[6 * kDTile];
  bf16* const Kh = lds;
  bf16* const Kl = lds + 2 * kDTile;
  bf16* const Vs = lds + 4 * kDTile;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, false);
  const int b = id.b, h = id.h, T = p.T;
  const int t0 = id.tile * kTile;
  const int tq = t0 + wave * 16 + c;
  const bool qok = tq < T;
  const int lo = tq - p.win > 0 ? tq - p.win : 0;
  const int hi = qok ? tq - 1 : -1;
  const WaveBand wb = wave_band(p, t0 + wave * 16);

  const float* qb_ = (const float*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const float* kb_ = (const float*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const float* ob_ = (const float*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;

#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int kb0 = t0 - kTile + s * kTile;
    const SplitRegs kx = tile_load_split(kb_, p.k.s1, kb0, T, tid);
    const TileRegs vx = tile_load_staged(vb_, p.v.s1, kb0, T, tid);
    tile_store_direct(kx.hi, Kh + s * kDTile, tid);
    tile_store_direct(kx.lo, Kl + s * kDTile, tid);
    tile_store_direct(vx, Vs + s * kDTile, tid);
  }
  const SplitFrag q0 = frag_f32(qb_, p.q.s1, tq, T, g), q1 = frag_f32(qb_, p.q.s1, tq, T, 4 + g);
  const SplitFrag o0 = frag_f32(ob_, p.dout.s1, tq, T, g), o1 = frag_f32(ob_, p.dout.s1, tq, T, 4 + g);
  __syncthreads();

  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;
  // P and dP of the whole band (two blocks) stay in registers
  float P[2][4][4], D[2][4][4];
  int kind[2][4];
  float msum = 0.f, dsum = 0.f;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int kb0 = t0 - kTile + s * kTile;
    const bf16* kh = Kh + s * kDTile;
    const bf16* kl = Kl + s * kDTile;
    const bf16* vs = Vs + s * kDTile;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kind[s][j] = kb0 + 16 * j + 15 < 0 ? 0 : sub_kind(wb, kb0 + 16 * j);
      if (kind[s][j] == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) P[s][j][r] = D[s][j][r] = 0.f;
        continue;
      }
      f32x4 sc = {}, dp = {};
      sc = mm3(dt_row8(kh, 16 * j + c, g), dt_row8(kl, 16 * j + c, g), q0.hi, q0.lo, sc);
      sc = mm3(dt_row8(kh, 16 * j + c, 4 + g), dt_row8(kl, 16 * j + c, 4 + g), q1.hi, q1.lo, sc);
      dp = mm2(dt_row8(vs, 16 * j + c, g), o0.hi, o0.lo, dp);
      dp = mm2(dt_row8(vs, 16 * j + c, 4 + g), o1.hi, o1.lo, dp);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = (key >= lo) & (key <= hi);
        float b2 = 0.f;
        if (BIAS && ok) b2 = -kLog2e * ld<float>(p.bias, bias_off(p, b, tq, key));
        const float pv = ok ? sigmoid_scaled(sc[r], k2, b2) : 0.f;
        P[s][j][r] = pv;
        D[s][j][r] = ok ? dp[r] : 0.f;
        msum += pv;
        dsum = fmaf(pv, D[s][j][r], dsum);
      }
    }
  }
  // normalisation coefficients of this lane's query (the whole band is in
  // the wave): dtau = a dP - c (+ dTau)
  float ca = 1.f, cc = 0.f;
  if (NORM == NORM_MASS_) {
    msum = wave_sum_g(msum);
    dsum = wave_sum_g(dsum);
    const float m = msum > kMassEps ? msum : kMassEps;
    ca = 1.f / m;
    cc = msum >= kMassEps ? dsum * ca * ca : 0.f;
    if (p.ws && qok && g == 0) {
      const int64_t nws = (int64_t)p.B * p.T * p.H;
      const int64_t wi = ((int64_t)b * p.T + tq) * p.H + h;
      ((float*)p.ws)[wi] = ca;
      ((float*)p.ws)[nws + wi] = cc;
    }
  } else if (NORM == NORM_COUNT_) {
    const int cnt = tq < p.W ? tq : p.W;
    ca = 1.f / (float)(cnt > 1 ? cnt : 1);
  }
  f32x4 acc[4] = {};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int kb0 = t0 - kTile + s * kTile;
    float G[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = kind[s][j] != 0 && (key >= lo) & (key <= hi);
        float dt = fmaf(D[s][j][r], ca, -cc);
        if (DTAU && ok) {
          const int col = tau_col(p, tq, key);
          if (col >= 0) dt += ld<float>(p.dtau, tau_off(p.dtau, b, tq, h, col));
        }
        const float x = P[s][j][r];
        G[j][r] = ok ? dt * (x - x * x) : 0.f;
      }
    // dQ^T += K^T G^T over 32-key pairs (A = K^T read transposed)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if (kind[s][2 * kk] == 0 && kind[s][2 * kk + 1] == 0) continue;
      bf16x8 gh, gl;
      pack_split(G[2 * kk], G[2 * kk + 1], gh, gl);
#pragma unroll
      for (int m = 0; m < 4; ++m)
        acc[m] = mm3(dt_tr8(Kh + s * kDTile, m, 32 * kk, g, c), dt_tr8(Kl + s * kDTile, m, 32 * kk, g, c), gh, gl,
                     acc[m]);
    }
  }
  if (!qok) return;
  store_row_f32((float*)p.dq.p + b * p.dq.s0 + (int64_t)tq * p.dq.s1 + h * p.dq.s2, acc, inv_scale, g);
}

// ---------------------------------------------------------------- dK / dV

// Query tiles k and k + 1 pass through one set of LDS tiles in turn (33 KB:
// three workgroups per CU, register-limited) rather than side by side;
// without bias / dTau, tile k + 1's rows are loaded into registers while
// tile k is worked on.
#ifndef TENSION_MX_DKV_SLOTS
#define TENSION_MX_DKV_SLOTS 1
#endif

template <int NORM, bool BIAS, bool DTAU>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 8))) void mx_dkv(BandParams p) {
  // query tile k + s in slot s % NS: Q hi, Q lo, dO hi, dO lo
  constexpr int NS = TENSION_MX_DKV_SLOTS;
  __shared__ __attribute__((aligned(16))) bf16 lds[4 * NS * kDTile];
  __shared__ float sa[2 * kTile], sc[2 * kTile];
  bf16* const Qh = lds;
  bf16* const Ql = lds + NS * kDTile;
  bf16* const Oh = lds + 2 * NS * kDTile;
  bf16* const Ol = lds + 3 * NS * kDTile;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, false);
  const int b = id.b, h = id.h, T = p.T;
  const int k0 = id.tile * kTile;
  const int tk = k0 + wave * 16 + c;
  const bool kok = tk < T;
  // queries that see this lane's key: [tk + 1, min(tk + W, T - 1)]
  const int qlo = tk + 1;
  const int qhi = !kok ? -1 : (tk + p.win > T - 1 ? T - 1 : tk + p.win);
  // odd key tiles take query tile k + 1 first: the query tile two
  // neighbouring key tiles share is then read by both in the same stage
  const bool rev = TENSION_MX_ALTERNATE && (id.tile & 1) != 0;
  auto qs = [&](int s) { return rev ? 1 - s : s; };

  const float* qb_ = (const float*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const float* kb_ = (const float*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const float* ob_ = (const float*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;

  // query tile k + s into slot s % NS
  auto store_tile = [&](int s, const SplitRegs& qx, const SplitRegs& ox) {
    const int sl = (s % NS) * kDTile;
    tile_store_direct(qx.hi, Qh + sl, tid);
    tile_store_direct(qx.lo, Ql + sl, tid);
    tile_store_direct(ox.hi, Oh + sl, tid);
    tile_store_direct(ox.lo, Ol + sl, tid);
  };
#pragma unroll
  for (int s = 0; s < NS; ++s)
    store_tile(s, tile_load_split(qb_, p.q.s1, k0 + qs(s) * kTile, T, tid),
               tile_load_split(ob_, p.dout.s1, k0 + qs(s) * kTile, T, tid));
  // with one slot and no bias / dTau (whose per-pair loads need the
  // registers): tile k + 1's rows in flight during tile k
  constexpr bool PF = NS == 1 && !BIAS && !DTAU;
  RawRows qn{}, on{};
  if (tid < 2 * kTile) {
    const int t = k0 + tid;
    float a = 1.f, cv = 0.f;
    if (t < T) {
      if (NORM == NORM_MASS_) {
        const int64_t nws = (int64_t)p.B * p.T * p.H;
        const int64_t wi = ((int64_t)b * p.T + t) * p.H + h;
        a = ((const float*)p.ws)[wi];
        cv = ((const float*)p.ws)[nws + wi];
      } else if (NORM == NORM_COUNT_) {
        const int cnt = t < p.W ? t : p.W;
        a = 1.f / (float)(cnt > 1 ? cnt : 1);
      }
    }
    sa[tid] = a;
    sc[tid] = cv;
  }
  // this lane's key row as B operands: K split, V exact
  const SplitFrag kf0 = frag_f32(kb_, p.k.s1, tk, T, g), kf1 = frag_f32(kb_, p.k.s1, tk, T, 4 + g);
  bf16x8 vf0 = {}, vf1 = {};
  if (kok) {
    vf0 = load8(vb_ + (int64_t)tk * p.v.s1 + 8 * g);
    vf1 = load8(vb_ + (int64_t)tk * p.v.s1 + 32 + 8 * g);
  }
  __syncthreads();

  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;
  f32x4 dk[4] = {}, dv[4] = {};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (PF && s == 0) {
      qn = tile_load_raw(qb_, p.q.s1, k0 + qs(1) * kTile, T, tid);
      on = tile_load_raw(ob_, p.dout.s1, k0 + qs(1) * kTile, T, tid);
    }
    if (s >= NS) {  // the slot of tile s - NS is free once every wave is past it
      __syncthreads();
      if constexpr (PF)
        store_tile(s, split_rows(qn), split_rows(on));
      else
        store_tile(s, tile_load_split(qb_, p.q.s1, k0 + qs(s) * kTile, T, tid),
                   tile_load_split(ob_, p.dout.s1, k0 + qs(s) * kTile, T, tid));
      __syncthreads();
    }
    const bf16* qh = Qh + (s % NS) * kDTile;
    const bf16* ql = Ql + (s % NS) * kDTile;
    const bf16* oh = Oh + (s % NS) * kDTile;
    const bf16* ol = Ol + (s % NS) * kDTile;
    float Pa[4][4], G[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // S = Q K^T, dP = dO V^T: queries 16 j + 4 g + r (rows), key c (column)
      f32x4 sv = {}, dp = {};
      sv = mm3(dt_row8(qh, 16 * j + c, g), dt_row8(ql, 16 * j + c, g), kf0.hi, kf0.lo, sv);
      sv = mm3(dt_row8(qh, 16 * j + c, 4 + g), dt_row8(ql, 16 * j + c, 4 + g), kf1.hi, kf1.lo, sv);
      dp = mfma(dt_row8(ol, 16 * j + c, g), vf0, dp);
      dp = mfma(dt_row8(oh, 16 * j + c, g), vf0, dp);
      dp = mfma(dt_row8(ol, 16 * j + c, 4 + g), vf1, dp);
      dp = mfma(dt_row8(oh, 16 * j + c, 4 + g), vf1, dp);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ql_ = qs(s) * kTile + 16 * j + 4 * g + r;  // query - k0
        const int t = k0 + ql_;
        const bool ok = t >= qlo && t <= qhi;
        float b2 = 0.f;
        if (BIAS && ok) b2 = -kLog2e * ld<float>(p.bias, bias_off(p, b, t, tk));
        const float pv = sigmoid_scaled(sv[r], k2, b2);
        const float a = sa[ql_];
        float dt = fmaf(dp[r], a, -sc[ql_]);
        if (DTAU && ok) {
          const int col = tau_col(p, t, tk);
          if (col >= 0) dt += ld<float>(p.dtau, tau_off(p.dtau, b, t, h, col));
        }
        Pa[j][r] = ok ? pv * a : 0.f;
        G[j][r] = ok ? dt * (pv - pv * pv) : 0.f;
      }
    }
    // dV^T += dO^T (a P),  dK^T += Q^T G over 32-query pairs
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 ph, pl, gh, gl;
      pack_split(Pa[2 * kk], Pa[2 * kk + 1], ph, pl);
      pack_split(G[2 * kk], G[2 * kk + 1], gh, gl);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        dv[m] = mm3(dt_tr8(oh, m, 32 * kk, g, c), dt_tr8(ol, m, 32 * kk, g, c), ph, pl, dv[m]);
        dk[m] = mm3(dt_tr8(qh, m, 32 * kk, g, c), dt_tr8(ql, m, 32 * kk, g, c), gh, gl, dk[m]);
      }
    }
  }
  if (!kok) return;
  store_row_f32((float*)p.dk.p + b * p.dk.s0 + (int64_t)tk * p.dk.s1 + h * p.dk.s2, dk, inv_scale, g);
  store_row4x4((bf16*)p.dv.p + b * p.dv.s0 + (int64_t)tk * p.dv.s1 + h * p.dv.s2, dv, 1.f, g);
}

// ---------------------------------------------------------------- launch

#define MX_LAUNCH(kernel, nrm, x, y)                                                            \
  do {                                                                                          \
    if (x) {                                                                                    \
      if (y) hipLaunchKernelGGL((kernel<nrm, true, true>), dim3(n), dim3(kThreads), 0, st, p);  \
      else hipLaunchKernelGGL((kernel<nrm, true, false>), dim3(n), dim3(kThreads), 0, st, p);   \
    } else {                                                                                    \
      if (y) hipLaunchKernelGGL((kernel<nrm, false, true>), dim3(n), dim3(kThreads), 0, st, p); \
      else hipLaunchKernelGGL((kernel<nrm, false, false>), dim3(n), dim3(kThreads), 0, st, p);  \
    }                                                                                           \
  } while (0)

#define MX_NORMS(kernel, x, y)                                  \
  do {                                                          \
    if (p.flags & TENSION_NORM_MASS) MX_LAUNCH(kernel, NORM_MASS_, x, y);  \
    else if (p.flags & TENSION_NORM_COUNT) MX_LAUNCH(kernel, NORM_COUNT_, x, y); \
    else MX_LAUNCH(kernel, NORM_RAW, x, y);                     \
  } while (0)

// phase 0: forward, 1: dQ (+ coefficients), 2: dK / dV
int launch_mixed(int phase, const BandParams& p_in, hipStream_t st, hipError_t* err) {
  BandParams p = p_in;
  p.ntiles = (p.T + kTile - 1) / kTile;
  const int64_t nwg = (int64_t)p.B * p.H * p.ntiles;
  if (nwg <= 0 || nwg > 0x7fffffff) return -1;
  const unsigned n = (unsigned)nwg;
  const bool bias = p.bias.p != nullptr;
  switch (phase) {
    case 0: MX_NORMS(mx_fwd, bias, p.tau.p != nullptr); break;
    case 1: MX_NORMS(mx_dq, bias, p.dtau.p != nullptr); break;
    case 2: MX_NORMS(mx_dkv, bias, p.dtau.p != nullptr); break;
    default: return -1;
  }
  *err = hipGetLastError();
  return 0;
}

#undef MX_NORMS
#undef MX_LAUNCH

}  // namespace tension
