// bf16 MFMA band kernels for gfx950, head dim 64.
//
// Work unit: a 64-row tile of one (b, h) pair, 256 threads = 4 wave64s.
// Matrix products use v_mfma_f32_16x16x32_bf16 (A 16x32, B 32x16, C 16x16
// fp32).  Operand layout for lane l, g = l/16, c = l%16:
//   A: row c,  k = 8g..8g+7        B: column c, k = 8g..8g+7
//   C: rows 4g..4g+3, column c
// (a permutation of k that is the same for A and B does not change the
// product, which the P.V-type products below rely on).
//
// Scores are computed "transposed" where the next product contracts over
// keys: S^T = K Q^T leaves lane (g, c) holding keys 4g+r of query c, which is
// exactly a B operand (query = column c) for O^T = V^T P^T once the 8 keys
// {4g..4g+3, 16+4g..16+4g+3} of two 16-key groups are packed -- the A
// operand V^T then reads the same 8 keys from a transposed LDS copy.
//
//   forward   (query tile, waves split queries):  S^T = K Q^T, P = sigma(.)
//             O^T += V^T P^T                      LDS: K rows, V^T
//   dq        (query tile, waves split queries):  S^T, dP^T = V dO^T,
//             G = dtau*P*(1-P), dQ^T += K^T G^T    LDS: K rows, V rows, K^T
//   dkv       (key tile, waves split keys):       S = Q K^T, dP = dO V^T,
//             dV^T += dO^T (a.P), dK^T += Q^T G    LDS: Q, dO rows, Q^T, dO^T
// dK/dV are owned by exactly one workgroup each: no atomics, deterministic.
#include "kernels.h"

namespace tension {

constexpr int kTile = 64;
constexpr int kThreads = 256;
constexpr int kPitch = 72;  // LDS row pitch in bf16 elements (64 + 8 pad)

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 load8(const bf16* p) {
  return __builtin_bit_cast(bf16x8, *(const u16x8*)p);
}

__device__ __forceinline__ bf16x8 lds8(const bf16* p) {
  return __builtin_bit_cast(bf16x8, *(const u16x8*)p);
}

// A operand from a transposed LDS tile: row `row`, keys {4g..4g+3} and
// {16+4g..16+4g+3} of the 32-key group starting at k0.
__device__ __forceinline__ bf16x8 lds_tr8(const bf16* base, int row, int k0, int g) {
  const u16x4 lo = *(const u16x4*)(base + row * kPitch + k0 + 4 * g);
  const u16x4 hi = *(const u16x4*)(base + row * kPitch + k0 + 16 + 4 * g);
  u16x8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return __builtin_bit_cast(bf16x8, r);
}

// B operand from two 16-key groups of fp32 C-layout values.
__device__ __forceinline__ bf16x8 pack_b(const float* lo4, const float* hi4) {
  bf16x8 r;
  r[0] = (bf16)lo4[0]; r[1] = (bf16)lo4[1]; r[2] = (bf16)lo4[2]; r[3] = (bf16)lo4[3];
  r[4] = (bf16)hi4[0]; r[5] = (bf16)hi4[1]; r[6] = (bf16)hi4[2]; r[7] = (bf16)hi4[3];
  return r;
}

// Stage rows [r0, r0+64) of a [.., T, .., 64] bf16 tensor (row r at
// base + r*rs) into LDS: row-major into `rm` and/or transposed (rt[d][row])
// into `rt`.  Rows outside [0, T) read as zero.  Thread tid loads 16 bytes
// of rows r0+2p and r0+2p+1 (p = tid/8, d-chunk tid%8), so eight lanes cover
// one 128-byte row and every global load instruction is fully coalesced.
__device__ __forceinline__ void stage_tile(const bf16* base, int64_t rs, int r0, int T,
                                           bf16* rm, bf16* rt, int tid) {
  const int pr = tid >> 3, ch = tid & 7;
  const int ra = r0 + 2 * pr, rb = ra + 1;
  u16x8 xa = {0, 0, 0, 0, 0, 0, 0, 0}, xb = {0, 0, 0, 0, 0, 0, 0, 0};
  if (ra >= 0 && ra < T) xa = *(const u16x8*)(base + (int64_t)ra * rs + 8 * ch);
  if (rb >= 0 && rb < T) xb = *(const u16x8*)(base + (int64_t)rb * rs + 8 * ch);
  if (rm) {
    *(u16x8*)(rm + (2 * pr) * kPitch + 8 * ch) = xa;
    *(u16x8*)(rm + (2 * pr + 1) * kPitch + 8 * ch) = xb;
  }
  if (rt) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t w = (uint32_t)xa[e] | ((uint32_t)xb[e] << 16);
      *(uint32_t*)(rt + (8 * ch + e) * kPitch + 2 * pr) = w;
    }
  }
}

__device__ __forceinline__ float wave_sum_g(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

struct TileId {
  int b, h, tile;
};

__device__ __forceinline__ TileId tile_id(const BandParams& p, bool heavy_first) {
  const int id = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);
  TileId r;
  const int bh = id / p.ntiles;
  int tile = id % p.ntiles;
  if (heavy_first) tile = p.ntiles - 1 - tile;
  r.b = bh / p.H;
  r.h = bh % p.H;
  r.tile = tile;
  return r;
}

// ------------------------------------------------------------------ forward

__global__ __launch_bounds__(kThreads) void mfma_fwd(BandParams p) {
  __shared__ __attribute__((aligned(16))) bf16 Ks[kTile * kPitch];
  __shared__ __attribute__((aligned(16))) bf16 Vt[kTile * kPitch];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, p.glob != 0);
  const int b = id.b, h = id.h, T = p.T;
  const int t0 = id.tile * kTile;
  const int tq = t0 + wave * 16 + c;
  const bool qok = tq < T;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;

  bf16x8 qf[2];
  {
    const int tr = qok ? tq : T - 1;
    qf[0] = load8(qb_ + (int64_t)tr * p.q.s1 + 8 * g);
    qf[1] = load8(qb_ + (int64_t)tr * p.q.s1 + 32 + 8 * g);
    if (!qok) { qf[0] = bf16x8{}; qf[1] = bf16x8{}; }
  }
  const float inv_scale = (float)(1.0 / p.scale);
  f32x4 acc[4] = {};
  float msum = 0.f;

  int s_lo = t0 - p.win;
  if (s_lo < 0) s_lo = 0;
  int s_hi = t0 + kTile - 2 + p.diag;
  if (s_hi > T - 1) s_hi = T - 1;
  for (int kb0 = s_lo & ~(kTile - 1); kb0 <= s_hi; kb0 += kTile) {
    __syncthreads();
    stage_tile(kb_, p.k.s1, kb0, T, Ks, nullptr, tid);
    stage_tile(vb_, p.v.s1, kb0, T, nullptr, Vt, tid);
    __syncthreads();
    float pr[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 s = {};
      s = mfma(lds8(Ks + (16 * j + c) * kPitch + 8 * g), qf[0], s);
      s = mfma(lds8(Ks + (16 * j + c) * kPitch + 32 + 8 * g), qf[1], s);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = qok && band_valid(p, tq, key);
        float x = s[r] * inv_scale;
        if (ok && p.bias.p) x += ld<float>(p.bias, bias_off(p, b, tq, key));
        const float pv = ok ? sigmoid_fast(x) : 0.f;
        if (ok && p.tau.p) {
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
      for (int m = 0; m < 4; ++m) acc[m] = mfma(lds_tr8(Vt, 16 * m + c, 32 * kk, g), pb, acc[m]);
    }
  }
  msum = wave_sum_g(msum);
  if (!qok) return;
  float inv = 1.f;
  if (p.flags & TENSION_NORM_MASS) inv = 1.f / (msum > kMassEps ? msum : kMassEps);
  if (p.flags & TENSION_NORM_COUNT) {
    const int cnt = tq < p.W ? tq : p.W;
    inv = 1.f / (float)(cnt > 1 ? cnt : 1);
  }
  bf16* orow = (bf16*)p.out.p + b * p.out.s0 + (int64_t)tq * p.out.s1 + h * p.out.s2;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    u16x4 o;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = bf16_bits((bf16)(acc[m][r] * inv));
    *(u16x4*)(orow + 16 * m + 4 * g) = o;
  }
  if (p.mass.p && g == 0)
    st<float>(p.mass, b * p.mass.s0 + (int64_t)tq * p.mass.s1 + h * p.mass.s2, msum);
  if (p.tau.p) {
    const int e = tau_empty_bound(p, tq);
    for (int col = g; col < e; col += 4) st<float>(p.tau, tau_off(p.tau, b, tq, h, col), 0.f);
  }
}

// ------------------------------------------------------------------ dQ

// S^T and dP^T of one 64-key block for this wave's 16 queries (C layout:
// lane (g, c) holds keys 16j + 4g + r of query c).
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

__global__ __launch_bounds__(kThreads) void mfma_bwd_dq(BandParams p) {
  __shared__ __attribute__((aligned(16))) bf16 Ks[kTile * kPitch];
  __shared__ __attribute__((aligned(16))) bf16 Vs[kTile * kPitch];
  __shared__ __attribute__((aligned(16))) bf16 Kt[kTile * kPitch];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, p.glob != 0);
  const int b = id.b, h = id.h, T = p.T;
  const int t0 = id.tile * kTile;
  const int tq = t0 + wave * 16 + c;
  const bool qok = tq < T;
  const int tr = qok ? tq : T - 1;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const bf16* gb_ = (const bf16*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;

  bf16x8 qf[2], gf[2];
  qf[0] = load8(qb_ + (int64_t)tr * p.q.s1 + 8 * g);
  qf[1] = load8(qb_ + (int64_t)tr * p.q.s1 + 32 + 8 * g);
  gf[0] = load8(gb_ + (int64_t)tr * p.dout.s1 + 8 * g);
  gf[1] = load8(gb_ + (int64_t)tr * p.dout.s1 + 32 + 8 * g);
  if (!qok) { qf[0] = bf16x8{}; qf[1] = bf16x8{}; gf[0] = bf16x8{}; gf[1] = bf16x8{}; }

  const float inv_scale = (float)(1.0 / p.scale);
  int s_lo = t0 - p.win;
  if (s_lo < 0) s_lo = 0;
  int s_hi = t0 + kTile - 2 + p.diag;
  if (s_hi > T - 1) s_hi = T - 1;
  const int kb_first = s_lo & ~(kTile - 1);

  // Per-query coefficients (dtau = a * dP - c + dTau).  Tau-mass: a = 1/m,
  // c = sum_s tau dP / m^2, both from a first pass over the band in fp32 (no
  // use of the bf16 forward output, whose rounding would not cancel in
  // dP - c when one key dominates a query).
  float ca = 1.f, cc = 0.f;
  if (p.flags & TENSION_NORM_MASS) {
    float msum = 0.f, dsum = 0.f;
    for (int kb0 = kb_first; kb0 <= s_hi; kb0 += kTile) {
      __syncthreads();
      stage_tile(kb_, p.k.s1, kb0, T, Ks, nullptr, tid);
      stage_tile(vb_, p.v.s1, kb0, T, Vs, nullptr, tid);
      __syncthreads();
      f32x4 s[4], dp[4];
      scores_block(Ks, Vs, qf, gf, g, c, s, dp);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kb0 + 16 * j + 4 * g + r;
          const bool ok = qok && band_valid(p, tq, key);
          float x = s[j][r] * inv_scale;
          if (ok && p.bias.p) x += ld<float>(p.bias, bias_off(p, b, tq, key));
          const float pv = ok ? sigmoid_fast(x) : 0.f;
          msum += pv;
          dsum += pv * dp[j][r];
        }
      }
    }
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
  } else if (p.flags & TENSION_NORM_COUNT) {
    const int cnt = tq < p.W ? tq : p.W;
    ca = 1.f / (float)(cnt > 1 ? cnt : 1);
  }

  f32x4 acc[4] = {};
  for (int kb0 = kb_first; kb0 <= s_hi; kb0 += kTile) {
    __syncthreads();
    stage_tile(kb_, p.k.s1, kb0, T, Ks, Kt, tid);
    stage_tile(vb_, p.v.s1, kb0, T, Vs, nullptr, tid);
    __syncthreads();
    f32x4 s[4], dp[4];
    scores_block(Ks, Vs, qf, gf, g, c, s, dp);
    float gd[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = qok && band_valid(p, tq, key);
        float x = s[j][r] * inv_scale;
        if (ok && p.bias.p) x += ld<float>(p.bias, bias_off(p, b, tq, key));
        const float pv = sigmoid_fast(x);
        float dt = dp[j][r] * ca - cc;
        if (ok && p.dtau.p) {
          const int col = tau_col(p, tq, key);
          if (col >= 0) dt += ld<float>(p.dtau, tau_off(p.dtau, b, tq, h, col));
        }
        gd[j][r] = ok ? dt * pv * (1.f - pv) : 0.f;
      }
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const bf16x8 pb = pack_b(gd[2 * kk], gd[2 * kk + 1]);
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m] = mfma(lds_tr8(Kt, 16 * m + c, 32 * kk, g), pb, acc[m]);
    }
  }
  if (!qok) return;
  bf16* drow = (bf16*)p.dq.p + b * p.dq.s0 + (int64_t)tq * p.dq.s1 + h * p.dq.s2;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    u16x4 o;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = bf16_bits((bf16)(acc[m][r] * inv_scale));
    *(u16x4*)(drow + 16 * m + 4 * g) = o;
  }
}

// ------------------------------------------------------------------ dK / dV

__global__ __launch_bounds__(kThreads) void mfma_bwd_dkv(BandParams p) {
  __shared__ __attribute__((aligned(16))) bf16 Qs[kTile * kPitch];
  __shared__ __attribute__((aligned(16))) bf16 Gs[kTile * kPitch];
  __shared__ __attribute__((aligned(16))) bf16 Qt[kTile * kPitch];
  __shared__ __attribute__((aligned(16))) bf16 Gt[kTile * kPitch];
  __shared__ float sa[kTile], sc[kTile];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  // light tiles (late keys see few queries in the global band) last
  const TileId id = tile_id(p, false);
  const int b = id.b, h = id.h, T = p.T;
  const int k0 = id.tile * kTile;
  const int tk = k0 + wave * 16 + c;
  const bool kok = tk < T;
  const int kr = kok ? tk : T - 1;

  const bf16* qb_ = (const bf16*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const bf16* kb_ = (const bf16*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const bf16* vb_ = (const bf16*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const bf16* gb_ = (const bf16*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;

  bf16x8 kf[2], vf[2];
  kf[0] = load8(kb_ + (int64_t)kr * p.k.s1 + 8 * g);
  kf[1] = load8(kb_ + (int64_t)kr * p.k.s1 + 32 + 8 * g);
  vf[0] = load8(vb_ + (int64_t)kr * p.v.s1 + 8 * g);
  vf[1] = load8(vb_ + (int64_t)kr * p.v.s1 + 32 + 8 * g);
  if (!kok) { kf[0] = bf16x8{}; kf[1] = bf16x8{}; vf[0] = bf16x8{}; vf[1] = bf16x8{}; }

  const float inv_scale = (float)(1.0 / p.scale);
  const int64_t nws = (int64_t)p.B * p.T * p.H;
  f32x4 dk[4] = {}, dv[4] = {};
  // queries that see keys [k0, k0+64): t in [k0 + 1 - diag, k0 + 63 + win]
  const int t_lo = k0 + 1 - p.diag;
  int64_t t_hi64 = (int64_t)k0 + kTile - 1 + p.win;
  const int t_hi = t_hi64 > T - 1 ? T - 1 : (int)t_hi64;
  for (int q0 = t_lo & ~(kTile - 1); q0 <= t_hi; q0 += kTile) {
    __syncthreads();
    stage_tile(qb_, p.q.s1, q0, T, Qs, Qt, tid);
    stage_tile(gb_, p.dout.s1, q0, T, Gs, Gt, tid);
    if (tid < kTile) {
      const int t = q0 + tid;
      float a = 1.f, cc = 0.f;
      if (t < T) {
        if (p.flags & TENSION_NORM_MASS) {
          const int64_t wi = ((int64_t)b * p.T + t) * p.H + h;
          a = ((const float*)p.ws)[wi];
          cc = ((const float*)p.ws)[nws + wi];
        } else if (p.flags & TENSION_NORM_COUNT) {
          const int cnt = t < p.W ? t : p.W;
          a = 1.f / (float)(cnt > 1 ? cnt : 1);
        }
      }
      sa[tid] = a;
      sc[tid] = cc;
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
        const bool ok = kok && t < T && band_valid(p, t, tk);
        float x = s[r] * inv_scale;
        if (ok && p.bias.p) x += ld<float>(p.bias, bias_off(p, b, t, tk));
        const float pv = sigmoid_fast(x);
        const float a = sa[ql];
        float dt = dp[r] * a - sc[ql];
        if (ok && p.dtau.p) {
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
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    u16x4 ok_, ov;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ok_[r] = bf16_bits((bf16)(dk[m][r] * inv_scale));
      ov[r] = bf16_bits((bf16)dv[m][r]);
    }
    *(u16x4*)(dkrow + 16 * m + 4 * g) = ok_;
    *(u16x4*)(dvrow + 16 * m + 4 * g) = ov;
  }
}

// ------------------------------------------------------------------ launch

int launch_mfma(int phase, const BandParams& p_in, hipStream_t st, hipError_t* err) {
  BandParams p = p_in;
  p.ntiles = (p.T + kTile - 1) / kTile;
  const int64_t nwg = (int64_t)p.B * p.H * p.ntiles;
  if (nwg <= 0 || nwg > 0x7fffffff) return -1;
  switch (phase) {
    case 0: hipLaunchKernelGGL(mfma_fwd, dim3((unsigned)nwg), dim3(kThreads), 0, st, p); break;
    case 1: hipLaunchKernelGGL(mfma_bwd_dq, dim3((unsigned)nwg), dim3(kThreads), 0, st, p); break;
    case 2: hipLaunchKernelGGL(mfma_bwd_dkv, dim3((unsigned)nwg), dim3(kThreads), 0, st, p); break;
    default: return -1;
  }
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
