// Split-operand MFMA band kernels (gfx950): every operand enters
// v_mfma_f32_16x16x32_bf16 as a sum of NT bf16 terms.
//
//   NT = 1  bf16 tensors, taken as stored;
//   NT = 2  float16 tensors, split as x = t0 + t1 with t0 = bf16(x),
//           t1 = bf16(x - t0): exact (11 significant bits in two terms of
//           8, the exponent range of bf16 covers float16's);
//   NT = 3  float32 tensors, split on their way into registers or LDS as
//           x = t0 + t1 + t2 + r with t0 = bf16(x), t1 = bf16(x - t0),
//           t2 = bf16(x - t0 - t1) (both differences are exact in float32)
//           and |r| <= 2^-24 |x|, the size of float32 rounding itself.
//
// A product of two split operands keeps the terms t_i u_j with i + j <= L,
// smallest first into the float32 accumulator: L = 2 (six MFMAs for
// NT = 3) where the result is float32, L = 1 (three) where it is rounded to
// bf16 (dV); a product with the exact bf16 V takes the three t_i v.  The
// dropped terms are below 3 * 2^-24 of each product term, so sums agree
// with a float32 evaluation to its own rounding level.  The float32 flow is
// the reference's autocast one: RoPE hands the op float32 Q / K
// (model.py:75-81), V stays bf16, and the Triton kernel computes the call in
// float32 (kernel.py:71-98); out, tau, dOut, dQ, dK are float32, dV bf16.
// With NT = 1 the same kernels are the bf16 MFMA path of the head dims and
// windows the dedicated bf16 kernels do not take.
//
// NV: the terms of V (and the element of dV), 1 for a bf16 V as above, 3
// for a float32 V (the reference's float32 flow, no autocast: every input
// and gradient float32), 2 for a float16 V (float16 throughout).  Products
// with V then keep t_i v_j with i + j <= 2, and so does dV.  With NT = 2
// every product of two float16 operands is exact (all four terms); the
// fp32 P, P' and G fed to the second products go in as two terms
// (residual <= 2^-18 relative, below float16's own rounding).
//
// Head dim D = 32 or 64: LDS tiles are 64 rows x 64 bf16 (direct tiles,
// mfma_common.h); D = 32 fills the first four 16-byte chunks of each row
// and runs half the feature chunks.  Any band (local window of any width,
// or the global block): the forward and dQ kernels stream the key blocks
// of one 64-query tile's band through LDS, the dK / dV kernel the query
// tiles that see one 64-key tile.  Each kernel: 256 threads (4 waves), a
// wave owns 16 rows of the tile.
#pragma once

#include <type_traits>

#include "mfma_common.h"

namespace tension {
namespace split {

template <int NT>
using Elem = typename std::conditional<NT == 1, bf16, typename std::conditional<NT == 2, f16, float>::type>::type;

__device__ __forceinline__ unsigned short f16_bits(f16 x) { return __builtin_bit_cast(unsigned short, x); }

// 8 float16 values (as stored) as float32 (whole-vector bit cast)
__device__ __forceinline__ void f16x8_to_f32(const u16x8& u, float* x) {
  const f16x8 h = __builtin_bit_cast(f16x8, u);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)h[e];
}

// ----------------------------------------------------------------- terms

// 8 float32 values -> NT bf16 bit patterns per value.
template <int NT>
__device__ __forceinline__ void split8(const float* x, u16x8* t) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bf16 h = (bf16)x[e];
    t[0][e] = bf16_bits(h);
    if constexpr (NT >= 2) {
      const float r = x[e] - (float)h;
      const bf16 m = (bf16)r;
      t[1][e] = bf16_bits(m);
      if constexpr (NT == 3) t[2][e] = bf16_bits((bf16)(r - (float)m));
    }
  }
}

// C += sum of A_i B_j over i < NA, j < NB, i + j <= L, largest i + j first.
template <int NA, int NB, int L>
__device__ __forceinline__ f32x4 mmx(const bf16x8* a, const bf16x8* b, f32x4 c) {
#pragma unroll
  for (int s = L; s >= 0; --s)
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int j = s - i;
      if (j >= 0 && j < NB) c = mfma(a[i], b[j], c);
    }
  return c;
}

// The same sum for an accumulator that runs over many products (a band's
// key or query pairs): with SEP the terms of this product gather in a
// zero-started accumulator that joins C in one add, so C -- the largest
// value -- takes one rounding per product instead of one per term (the
// float32-V flow, where a product has six terms).
template <int NA, int NB, int L, bool SEP>
__device__ __forceinline__ f32x4 mmx_run(const bf16x8* a, const bf16x8* b, f32x4 c) {
  if constexpr (SEP) {
    const f32x4 z = mmx<NA, NB, L>(a, b, f32x4{0.f, 0.f, 0.f, 0.f});
    return c + z;
  } else {
    return mmx<NA, NB, L>(a, b, c);
  }
}

// B operand of a product over 32 tile rows from two 16-row groups of
// float32 C-layout values (the pairing dt_tr8 uses), as NT terms.
template <int NT>
__device__ __forceinline__ void pack_terms(const float* lo4, const float* hi4, bf16x8* t) {
  const float x[8] = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
  u16x8 u[NT];
  split8<NT>(x, u);
#pragma unroll
  for (int i = 0; i < NT; ++i) t[i] = __builtin_bit_cast(bf16x8, u[i]);
}

// Operand fragment from global memory: features 8 chunk .. +7 of row `row`
// of a tensor of Elem<NT> (zero outside [0, T)), loaded as stored
// (frag_load) and then as NT terms (frag_terms), so a load can run ahead of
// its use; frag_row does both.
template <int NT>
struct RawFrag;
template <>
struct RawFrag<1> {
  u16x8 a;
};
template <>
struct RawFrag<2> {
  u16x8 a;
};
template <>
struct RawFrag<3> {
  f32x4 a, b;
};

template <int NT>
__device__ __forceinline__ RawFrag<NT> frag_load(const Elem<NT>* base, int64_t rs, int row, int T, int chunk) {
  RawFrag<NT> x;
  const bool ok = row >= 0 && row < T;
  const Elem<NT>* src = base + (int64_t)row * rs + 8 * chunk;
  if constexpr (NT != 3) {
    x.a = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    if (ok) x.a = *(const u16x8*)src;
  } else {
    x.a = x.b = f32x4{0.f, 0.f, 0.f, 0.f};
    if (ok) {
      x.a = *(const f32x4*)src;
      x.b = *(const f32x4*)(src + 4);
    }
  }
  return x;
}

template <int NT>
__device__ __forceinline__ void frag_terms(const RawFrag<NT>& x, bf16x8* t) {
  if constexpr (NT == 1) {
    t[0] = __builtin_bit_cast(bf16x8, x.a);
  } else {
    float v[8];
    if constexpr (NT == 2) {
      f16x8_to_f32(x.a, v);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = x.a[e];
        v[4 + e] = x.b[e];
      }
    }
    u16x8 u[NT];
    split8<NT>(v, u);
#pragma unroll
    for (int i = 0; i < NT; ++i) t[i] = __builtin_bit_cast(bf16x8, u[i]);
  }
}

template <int NT>
__device__ __forceinline__ void frag_row(const Elem<NT>* base, int64_t rs, int row, int T, int chunk,
                                         bf16x8* t) {
  frag_terms<NT>(frag_load<NT>(base, rs, row, T, chunk), t);
}

// ----------------------------------------------------------------- staging

// A thread's two staged rows (staged_row(tid), +8; chunk tid % 8) of a
// 64-row tile as loaded: bf16 (NT = 1), float16 (NT = 2) or float32 (NT = 3).
template <int NT>
struct Raw;
template <>
struct Raw<1> {
  u16x8 a, b;
};
template <>
struct Raw<2> {
  u16x8 a, b;
};
template <>
struct Raw<3> {
  f32x4 a0, a1, b0, b1;
};

// Rows outside [0, T) and chunks past the head dim read as zero.
template <int NT, int D>
__device__ __forceinline__ Raw<NT> load_raw(const Elem<NT>* base, int64_t rs, int r0, int T, int tid) {
  const int ch = tid & 7;
  const int ra = r0 + staged_row(tid), rb = ra + 8;
  const bool okc = ch < D / 8;
  const bool oka = okc && ra >= 0 && ra < T, okb = okc && rb >= 0 && rb < T;
  Raw<NT> x;
  if constexpr (NT != 3) {
    x.a = x.b = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    if (oka) x.a = *(const u16x8*)(base + (int64_t)ra * rs + 8 * ch);
    if (okb) x.b = *(const u16x8*)(base + (int64_t)rb * rs + 8 * ch);
  } else {
    x.a0 = x.a1 = x.b0 = x.b1 = f32x4{0.f, 0.f, 0.f, 0.f};
    if (oka) {
      x.a0 = *(const f32x4*)(base + (int64_t)ra * rs + 8 * ch);
      x.a1 = *(const f32x4*)(base + (int64_t)ra * rs + 8 * ch + 4);
    }
    if (okb) {
      x.b0 = *(const f32x4*)(base + (int64_t)rb * rs + 8 * ch);
      x.b1 = *(const f32x4*)(base + (int64_t)rb * rs + 8 * ch + 4);
    }
  }
  return x;
}

// The rows into NT consecutive direct tiles (term i at tile0 + i kDTile).
template <int NT>
__device__ __forceinline__ void store_raw(const Raw<NT>& x, bf16* tile0, int tid) {
  if constexpr (NT == 1) {
    tile_store_direct(TileRegs{x.a, x.b}, tile0, tid);
  } else {
    float a[8], b[8];
    if constexpr (NT == 2) {
      f16x8_to_f32(x.a, a);
      f16x8_to_f32(x.b, b);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[e] = x.a0[e];
        a[4 + e] = x.a1[e];
        b[e] = x.b0[e];
        b[4 + e] = x.b1[e];
      }
    }
    u16x8 ta[NT], tb[NT];
    split8<NT>(a, ta);
    split8<NT>(b, tb);
#pragma unroll
    for (int i = 0; i < NT; ++i) tile_store_direct(TileRegs{ta[i], tb[i]}, tile0 + i * kDTile, tid);
  }
}

// One output row's C-layout values (features 16 m + 4 g .. +3), times f.
template <typename O, int D>
__device__ __forceinline__ void store_acc(O* row, const f32x4* acc, float f, int g) {
#pragma unroll
  for (int m = 0; m < D / 16; ++m) {
    if constexpr (std::is_same<O, float>::value) {
      *(f32x4*)(row + 16 * m + 4 * g) = acc[m] * f;
    } else {
      u16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (std::is_same<O, f16>::value) o[r] = f16_bits((f16)(acc[m][r] * f));
        else o[r] = bf16_bits((bf16)(acc[m][r] * f));
      }
      *(u16x4*)(row + 16 * m + 4 * g) = o;
    }
  }
}

// --------------------------------------------------------------- geometry

// The key blocks of a query tile's band: [kb_first, kb_first + 64 nblk).
struct Blocks {
  int first, n;
};

__device__ __forceinline__ Blocks band_blocks(const BandParams& p, int t0) {
  int s_lo = t0 - p.win;
  if (s_lo < 0) s_lo = 0;
  int s_hi = t0 + kTile - 2 + p.diag;
  if (s_hi > p.T - 1) s_hi = p.T - 1;
  Blocks r;
  r.first = s_lo & ~(kTile - 1);
  r.n = s_hi < r.first ? 0 : (s_hi - r.first) / kTile + 1;
  return r;
}

// Keys go through LDS: buffer `buf` holds block terms K_0 .. K_{NT-1},
// V_0 .. V_{NV-1}.
template <int NT, int NV>
__device__ __forceinline__ bf16* key_buf(bf16* lds, int buf) {
  return lds + buf * (NT + NV) * kDTile;
}

// Stream the key blocks of a band through NBUF LDS buffers: block i is
// staged (from registers loaded during block i - 1) while the waves work on
// block i - 1 (NBUF = 2) or after they leave it (NBUF = 1);
// body(tiles, first key) runs once per block with its buffer filled.
template <int NT, int NV, int D, int NBUF, typename Body>
__device__ __forceinline__ void stream_keys(bf16* lds, const Elem<NT>* kb_, int64_t ks, const Elem<NV>* vb_,
                                            int64_t vs, const Blocks& bl, int T, int tid, Body body) {
  if (bl.n <= 0) return;
  store_raw<NT>(load_raw<NT, D>(kb_, ks, bl.first, T, tid), key_buf<NT, NV>(lds, 0), tid);
  store_raw<NV>(load_raw<NV, D>(vb_, vs, bl.first, T, tid), key_buf<NT, NV>(lds, 0) + NT * kDTile, tid);
  __syncthreads();
  for (int i = 0; i < bl.n; ++i) {
    const int kb0 = bl.first + i * kTile;
    const int buf = NBUF == 2 ? (i & 1) : 0;
    const bool more = i + 1 < bl.n;
    Raw<NT> kn;
    Raw<NV> vn;
    if (more) {
      kn = load_raw<NT, D>(kb_, ks, kb0 + kTile, T, tid);
      vn = load_raw<NV, D>(vb_, vs, kb0 + kTile, T, tid);
    }
    body((const bf16*)key_buf<NT, NV>(lds, buf), kb0);
    if (more) {
      if (NBUF == 1) __syncthreads();  // every wave is done with the buffer
      bf16* nb = key_buf<NT, NV>(lds, NBUF == 2 ? (buf ^ 1) : 0);
      store_raw<NT>(kn, nb, tid);
      store_raw<NV>(vn, nb + NT * kDTile, tid);
    }
    __syncthreads();
  }
}

// S^T (keys 16 j + 4 g + r, query c) of one 16-key group against this
// lane's query fragments.
template <int NT, int D>
__device__ __forceinline__ f32x4 scores_t(const bf16* kt, const bf16x8 (*qf)[NT], int j, int g, int c) {
  f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ch = 0; ch < D / 32; ++ch) {
    bf16x8 ka[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) ka[i] = dt_row8(kt + i * kDTile, 16 * j + c, 4 * ch + g);
    sc = mmx<NT, NT, 2>(ka, qf[ch], sc);
  }
  return sc;
}

// ----------------------------------------------------------- tau staging
// tau / dTau cross the kernels as whole row segments: a wave's 16 query rows
// x 64 keys of one key block sit in LDS, and each row's segment moves
// between LDS and memory as one coalesced 64-lane access (column =
// key - t + W, local; T - 1 - key, global).  Rows of 64 elements; the
// 4-element chunk k of row r sits at chunk k ^ (r & 15), so the C-layout
// accesses (16 rows at one chunk) and the row accesses (one row, 64 lanes)
// both spread over distinct banks.
constexpr int kStageRows = 16 * 64;  // elements per wave

__device__ __forceinline__ int stage_at(int row, int col) {
  return row * 64 + ((((col >> 2) ^ (row & 15))) << 2) + (col & 3);
}

// This lane's four C-layout values (keys 16 j + 4 g .. +3, query c) <-> LDS.
template <typename E>
__device__ __forceinline__ void stage_put4(E* st, int c, int j, int g, const float* v) {
  E* at = st + stage_at(c, 16 * j + 4 * g);
  if constexpr (std::is_same<E, float>::value) {
    *(f32x4*)at = f32x4{v[0], v[1], v[2], v[3]};
  } else {
    u16x4 o;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (std::is_same<E, f16>::value) o[r] = f16_bits((f16)v[r]);
      else o[r] = bf16_bits((bf16)v[r]);
    }
    *(u16x4*)at = o;
  }
}

template <typename E>
__device__ __forceinline__ void stage_get4(const E* st, int c, int j, int g, float* v) {
  const E* at = st + stage_at(c, 16 * j + 4 * g);
  if constexpr (std::is_same<E, float>::value) {
    const f32x4 x = *(const f32x4*)at;
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
  } else if constexpr (std::is_same<E, f16>::value) {
    const f16x4 x = __builtin_bit_cast(f16x4, *(const u16x4*)at);
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = (float)x[r];
  } else {
    // bit-cast the whole vector (a bit_cast of one subscripted element has
    // compiled to element 0 for every index on this toolchain)
    const bf16x4 x = __builtin_bit_cast(bf16x4, *(const u16x4*)at);
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = (float)x[r];
  }
}

// Column of key `key` in query row t's tau, or -1 outside its band / slots.
__device__ __forceinline__ int band_tau_col(const BandParams& p, int t, int key) {
  const int lo = t - p.win > 0 ? t - p.win : 0;
  if (key < lo || key > t - 1 + p.diag) return -1;
  return tau_col(p, t, key);
}

// The raw pre-sigmoid bias of a lane's 16 pairs of one key block (query tq,
// row `brow` of the bias; keys kb0 + 16 j + 4 g + r): loaded together ahead
// of the block's products, so the loads' latency runs under them (a pair off
// the band [lo, hi] reads the row's first element and is masked where the
// bias is used).  The -log2(e) factor is applied at the use: nothing waits
// for the loads right behind them.
__device__ __forceinline__ void bias_block(const BandParams& p, const float* brow, int tq, int kb0, int g, int lo,
                                           int hi, float (*b2)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kb0 + 16 * j + 4 * g + r;
      const bool ok = (key >= lo) & (key <= hi);
      b2[j][r] = brow[ok ? bias_col(p, tq, key) : 0];
    }
}

// Rows t0w .. t0w + 15 (the wave's queries) of a [B,T,H,Wtau] tau / dTau of
// this (b, h): lane l moves key kb0 + l of each row.
template <typename E>
__device__ __forceinline__ void tau_rows_store(const BandParams& p, E* base, const E* st, int t0w, int kb0,
                                               int lane) {
#pragma unroll 4
  for (int rr = 0; rr < 16; ++rr) {
    const int t = t0w + rr;
    if (t >= p.T) break;
    const int col = band_tau_col(p, t, kb0 + lane);
    if (col >= 0) base[(int64_t)t * p.tau.s1 + col] = st[stage_at(rr, lane)];
  }
}

template <typename E>
__device__ __forceinline__ void dtau_rows_load(const BandParams& p, const E* base, E* v, int t0w, int kb0,
                                               int lane) {
#pragma unroll
  for (int rr = 0; rr < 16; ++rr) {
    const int t = t0w + rr;
    const int col = t < p.T ? band_tau_col(p, t, kb0 + lane) : -1;
    v[rr] = col >= 0 ? base[(int64_t)t * p.dtau.s1 + col] : (E)0.f;
  }
}

template <typename E>
__device__ __forceinline__ void dtau_rows_put(E* st, const E* v, int lane) {
#pragma unroll
  for (int rr = 0; rr < 16; ++rr) st[stage_at(rr, lane)] = v[rr];
}

// ----------------------------------------------------------------- forward

// One 64-query tile's lane state in the forward kernels: the lane's query
// row as B operands (Q as NT terms), its band, its O^T accumulators and
// tau mass, its rows of tau (dtype of Q, host-checked) and of the bias
// (float32, unit column stride); rows past T are never written.
template <int NT, int NV, int D, int NORM, bool BIAS, bool TAU>
struct FwdTile {
  using E = Elem<NT>;
  int b, h, g, c, lane, wave, t0, tq, lo, hi;
  WaveBand wb;
  float k2, msum;
  bf16x8 qf[D / 32][NT];
  f32x4 acc[D / 16];
  E* tbh;  // tau of this (b, h)
  E* trow;
  E* tst;  // this wave's tau staging rows
  const float* brow;
  float braw[BIAS ? 4 : 1][4];  // the raw bias of the block being visited

  __device__ __forceinline__ void init(const BandParams& p, int b_, int h_, int lane_, int wave_, E* tstage) {
    b = b_;
    h = h_;
    lane = lane_;
    wave = wave_;
    g = lane >> 4;
    c = lane & 15;
    k2 = -kLog2e * (float)(1.0 / p.scale);
    tbh = TAU ? (E*)p.tau.p + b * p.tau.s0 + h * p.tau.s2 : nullptr;
    tst = tstage + (TAU ? wave * kStageRows : 0);
  }

  // the tile at t0_: band, tau and bias rows, cleared sums (the query
  // fragments are set apart)
  __device__ __forceinline__ void at(const BandParams& p, int t0_) {
    const int T = p.T;
    t0 = t0_;
    tq = t0 + wave * 16 + c;
    lo = tq - p.win > 0 ? tq - p.win : 0;
    hi = tq < T ? tq - 1 + p.diag : -1;  // hi < lo: no key for this row
    wb = wave_band(p, t0 + wave * 16);
    const int tr = tq < T ? tq : T - 1;
    trow = TAU ? tbh + (int64_t)tr * p.tau.s1 : nullptr;
    brow = BIAS ? (const float*)p.bias.p + b * p.bias.s0 + (int64_t)tr * p.bias.s1 : nullptr;
#pragma unroll
    for (int m = 0; m < D / 16; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    msum = 0.f;
  }

  // the raw bias of key block kb0 (nothing without a bias)
  __device__ __forceinline__ void bias_load(const BandParams& p, int kb0) {
    if constexpr (BIAS) bias_block(p, brow, tq, kb0, g, lo, hi, braw);
  }

  // one key block (tiles K_0 .. K_{NT-1}, V_0 .. at kt; first key kb0); LOADED:
  // its bias is in braw already (bias_load), else it is loaded here
  template <bool LOADED = false>
  __device__ __forceinline__ void visit(const BandParams& p, const bf16* kt, int kb0) {
    float pr[4][4];
    int kind[4];
    if constexpr (!LOADED) bias_load(p, kb0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kind[j] = sub_kind(wb, kb0 + 16 * j);
      if (kind[j] == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[j][r] = 0.f;
        continue;
      }
      const f32x4 sc = scores_t<NT, D>(kt, qf, j, g, c);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = (key >= lo) & (key <= hi);
        const float b2 = BIAS ? -kLog2e * braw[j][r] : 0.f;
        // computed on every lane and selected (the bias of a pair off the
        // band is some element of the row, finite): written as a
        // conditional, the sigmoid with a bias became a branch per element
        const float sg = sigmoid_scaled(sc[r], k2, b2);
        const float pv = ok ? sg : 0.f;
        msum += pv;
        pr[j][r] = pv;
      }
    }
    // whole row segments out (keys outside each row's band are not stored;
    // a global block holds tau_local keys only from T - Wtau on)
    if (TAU && !(p.glob && kb0 + kTile <= p.T - p.Wtau)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) stage_put4(tst, c, j, g, pr[j]);
      tau_rows_store(p, tbh, tst, t0 + wave * 16, kb0, lane);
    }
    // O^T += V^T P^T over 32-key pairs (A = V^T read transposed)
    const bf16* vt = kt + NT * kDTile;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if (kind[2 * kk] == 0 && kind[2 * kk + 1] == 0) continue;
      bf16x8 ps[NT];
      pack_terms<NT>(pr[2 * kk], pr[2 * kk + 1], ps);
#pragma unroll
      for (int m = 0; m < D / 16; ++m) {
        bf16x8 va[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) va[i] = dt_tr8(vt + i * kDTile, m, 32 * kk, g, c);
        acc[m] = mmx_run<NV, NT, 2, NV == 3>(va, ps, acc[m]);
      }
    }
  }

  // the tile's output rows, mass and empty tau slots
  __device__ __forceinline__ void finish(const BandParams& p) {
    msum = wave_sum_g(msum);
    if (tq >= p.T) return;
    store_acc<E, D>((E*)p.out.p + b * p.out.s0 + (int64_t)tq * p.out.s1 + h * p.out.s2, acc,
                    out_factor<NORM>(msum, tq, p.W), g);
    if (p.mass.p && g == 0) st<float>(p.mass, b * p.mass.s0 + (int64_t)tq * p.mass.s1 + h * p.mass.s2, msum);
    if (TAU) {
      const int e = tau_empty_bound(p, tq);
      for (int col = g; col < e; col += 4) trow[col] = (E)0.f;
    }
  }
};

template <int NT, int NV, int D, int NORM, bool BIAS, bool TAU>
__global__ __launch_bounds__(kThreads) void xb_fwd(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  constexpr int NBUF = NT == 1 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) bf16 lds[NBUF * (NT + NV) * kDTile];
  __shared__ __attribute__((aligned(16))) Elem<NT> tstage[TAU ? 4 * kStageRows : 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const TileId id = tile_id(p, p.glob != 0);
  const int T = p.T;
  FwdTile<NT, NV, D, NORM, BIAS, TAU> st;
  st.init(p, id.b, id.h, lane, wave, tstage);
  st.at(p, id.tile * kTile);
  const Blocks bl = band_blocks(p, st.t0);

  using E = Elem<NT>;
  const E* qb_ = (const E*)p.q.p + st.b * p.q.s0 + st.h * p.q.s2;
  const E* kb_ = (const E*)p.k.p + st.b * p.k.s0 + st.h * p.k.s2;
  const Elem<NV>* vb_ = (const Elem<NV>*)p.v.p + st.b * p.v.s0 + st.h * p.v.s2;
#pragma unroll
  for (int ch = 0; ch < D / 32; ++ch) frag_row<NT>(qb_, p.q.s1, st.tq, T, 4 * ch + st.g, st.qf[ch]);
  stream_keys<NT, NV, D, NBUF>(lds, kb_, p.k.s1, vb_, p.v.s1, bl, T, tid,
                           [&](const bf16* kt, int kb0) { st.visit(p, kt, kb0); });
  st.finish(p);
}

// Runs of query tiles for local windows W <= 64, where tile t's band is key
// blocks t-1 and t: a workgroup owns tiles [tA, tB) of one (b, h) (p.chunk
// runs per (b, h)) and keeps one key block in LDS -- block t, which tile t
// visits last, is the block tile t + 1 visits first -- loading block t + 1
// into registers while tile t + 1 visits block t, and tile t + 1's query
// rows while tile t visits block t.  Per tile one block staged instead of
// two, and about three workgroups per CU in one round.
template <int NT, int NV, int D, int NORM, bool BIAS, bool TAU>
__global__ __launch_bounds__(kThreads) void xb_fwd_run(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  __shared__ __attribute__((aligned(16))) bf16 lds[(NT + NV) * kDTile];
  __shared__ __attribute__((aligned(16))) Elem<NT> tstage[TAU ? 4 * kStageRows : 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nr = p.chunk;
  const int id = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);
  const int bh = id / nr, run = id % nr;
  const int b = bh / p.H, h = bh % p.H, T = p.T;
  const int tA = run_bound(run, p.ntiles, nr);
  const int tB = run_bound(run + 1, p.ntiles, nr);
  if (tA >= tB) return;

  using E = Elem<NT>;
  const E* qb_ = (const E*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const E* kb_ = (const E*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const Elem<NV>* vb_ = (const Elem<NV>*)p.v.p + b * p.v.s0 + h * p.v.s2;
  FwdTile<NT, NV, D, NORM, BIAS, TAU> st;
  st.init(p, b, h, lane, wave, tstage);
  st.at(p, tA * kTile);
#pragma unroll
  for (int ch = 0; ch < D / 32; ++ch) frag_row<NT>(qb_, p.q.s1, st.tq, T, 4 * ch + st.g, st.qf[ch]);
  // the first block in LDS: block tA - 1 (block 0 for tA = 0, which tile 0
  // visits as its only block)
  {
    const int r0 = (tA > 0 ? tA - 1 : 0) * kTile;
    store_raw<NT>(load_raw<NT, D>(kb_, p.k.s1, r0, T, tid), lds, tid);
    store_raw<NV>(load_raw<NV, D>(vb_, p.v.s1, r0, T, tid), lds + NT * kDTile, tid);
  }
  __syncthreads();
  // With a bias, each visit's bias loads go out ahead of the loads issued
  // for what comes next (block t, tile t + 1's rows), which every tile then
  // issues (the last its own rows again, unused), so that the wait for the
  // bias does not include them.
  for (int t = tA; t < tB; ++t) {
    if (t >= 1) {  // block t - 1, in LDS, while block t arrives
      if constexpr (BIAS) {
        st.bias_load(p, (t - 1) * kTile);
        asm volatile("" ::: "memory");
      }
      const Raw<NT> kn = load_raw<NT, D>(kb_, p.k.s1, t * kTile, T, tid);
      const Raw<NV> vn = load_raw<NV, D>(vb_, p.v.s1, t * kTile, T, tid);
      st.template visit<BIAS>(p, lds, (t - 1) * kTile);
      __syncthreads();  // every wave is done with block t - 1
      store_raw<NT>(kn, lds, tid);
      store_raw<NV>(vn, lds + NT * kDTile, tid);
      __syncthreads();
    }
    // block t, while tile t + 1's query rows arrive
    const bool more = t + 1 < tB;
    if constexpr (BIAS) {
      st.bias_load(p, t * kTile);
      asm volatile("" ::: "memory");
    }
    RawFrag<NT> qn[D / 32];
    if (more || BIAS) {
      const int tq1 = BIAS && !more ? st.tq : st.tq + kTile;
#pragma unroll
      for (int ch = 0; ch < D / 32; ++ch) qn[ch] = frag_load<NT>(qb_, p.q.s1, tq1, T, 4 * ch + st.g);
      if constexpr (BIAS) asm volatile("" ::: "memory");
    }
    st.template visit<BIAS>(p, lds, t * kTile);
    st.finish(p);
    if (more) {
      st.at(p, (t + 1) * kTile);
#pragma unroll
      for (int ch = 0; ch < D / 32; ++ch) frag_terms<NT>(qn[ch], st.qf[ch]);
    }
  }
}

// ---------------------------------------------------------------------- dQ

// MODE 0: raw / valid-count (the coefficients are known): one pass.
// MODE 1: tau-mass with the band within two key blocks (W <= 64): P and dP
//         of the band stay in registers while the coefficients form.
// MODE 2: tau-mass over a wider band: a first pass forms the coefficients,
//         a second recomputes S and dP.
// MODE 3: tau-mass with the forward's output rows and tau mass (p.out,
//         p.mass): a = 1 / max(m, 1e-6), c = (dO . out) a (zero where
//         m < 1e-6, the clamp branch), then one pass.  out = msg a, so
//         c = (dO . msg) a^2 = sum_s P dP / m^2.  The host passes the rows
//         for float32 out (NT = 3: dO . out does not cancel the way a bf16
//         out does).
// The tau-mass coefficients of each query (dtau = a dP - c + dTau,
// a = 1 / m, c = sum_s P dP / m^2, model.py:257-258 differentiated) go to
// the workspace for the dK / dV kernel.

// One query tile's lane state in the dQ kernels -- the lane's query row
// (Q and dOut as terms), its band, the coefficients a = ca, c = cc, the dQ
// accumulators -- and the pieces the MODE passes are made of.  dbh / dst:
// dTau of this (b, h) and the wave's staging rows.
template <int NT, int NV, int D, int NORM, bool BIAS, bool DTAU>
struct DqTile {
  using E = Elem<NT>;
  int b, h, g, c, lane;
  int t0, t0w, tq, lo, hi;
  bool qok;
  WaveBand wb;
  Blocks bl;
  const float* brow;
  const E* dbh;
  E* dst;
  float k2, ca, cc, msum, dsum;
  bf16x8 qf[D / 32][NT], of[D / 32][NT];
  f32x4 acc[D / 16];

  // the tile at t0 for wave `wave`: band, bias row, count coefficient,
  // cleared sums and accumulators (the fragments are set apart)
  __device__ __forceinline__ void at(const BandParams& p, int t0_, int wave) {
    const int T = p.T;
    t0 = t0_;
    t0w = t0 + wave * 16;
    tq = t0w + c;
    qok = tq < T;
    lo = tq - p.win > 0 ? tq - p.win : 0;
    hi = qok ? tq - 1 + p.diag : -1;
    wb = wave_band(p, t0w);
    bl = band_blocks(p, t0);
    const int tr = qok ? tq : T - 1;
    brow = BIAS ? (const float*)p.bias.p + b * p.bias.s0 + (int64_t)tr * p.bias.s1 : nullptr;
    ca = 1.f;
    cc = 0.f;
    if (NORM == NORM_COUNT_) {
      const int cnt = tq < p.W ? tq : p.W;
      ca = 1.f / (float)(cnt > 1 ? cnt : 1);
    }
    msum = dsum = 0.f;
#pragma unroll
    for (int m = 0; m < D / 16; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // S^T and dP^T (keys 16 j + 4 g + r, query c) of one 16-key group
  __device__ __forceinline__ void sdp(const bf16* kt, int j, f32x4& sc, f32x4& dp) const {
    sc = scores_t<NT, D>(kt, qf, j, g, c);
    dp = f32x4{0.f, 0.f, 0.f, 0.f};
    const bf16* vt = kt + NT * kDTile;
#pragma unroll
    for (int ch = 0; ch < D / 32; ++ch) {
      bf16x8 va[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) va[i] = dt_row8(vt + i * kDTile, 16 * j + c, 4 * ch + g);
      dp = mmx<NV, NT, 2>(va, of[ch], dp);
    }
  }

  // tau (masked) of one element; b2: its raw bias_block value
  __device__ __forceinline__ float tau_of(float s, float b2, bool ok) const {
    return ok ? sigmoid_scaled(s, k2, BIAS ? -kLog2e * b2 : 0.f) : 0.f;
  }

  // bias_block of key block kb0 for this lane (nothing without a bias)
  __device__ __forceinline__ void bias_of(const BandParams& p, int kb0, float (*b2)[4]) const {
    if constexpr (BIAS) bias_block(p, brow, tq, kb0, g, lo, hi, b2);
  }

  // G = tau (1 - tau) (a dP - c + dTau), zero off the band (dtv: the staged
  // dTau of the pair, zero where it has no slot)
  __device__ __forceinline__ float g_of(float pv, float dpv, float dtv, bool ok) const {
    const float dt = fmaf(dpv, ca, -cc) + dtv;
    return ok ? dt * (pv - pv * pv) : 0.f;
  }

  // dQ^T += K^T G^T over 32-key pairs (A = K^T read transposed)
  __device__ __forceinline__ void dq_product(const bf16* kt, const int* kind, float (*G)[4]) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if (kind[2 * kk] == 0 && kind[2 * kk + 1] == 0) continue;
      bf16x8 gs[NT];
      pack_terms<NT>(G[2 * kk], G[2 * kk + 1], gs);
#pragma unroll
      for (int m = 0; m < D / 16; ++m) {
        bf16x8 ka[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) ka[i] = dt_tr8(kt + i * kDTile, m, 32 * kk, g, c);
        acc[m] = mmx_run<NT, NT, 2, NV == 3>(ka, gs, acc[m]);
      }
    }
  }

  // one block's S, dP -> G -> dQ with the coefficients known; with dTau its
  // rows are loaded before the products and staged through LDS after them
  __device__ __forceinline__ void g_pass(const BandParams& p, const bf16* kt, int kb0) {
    E dv[DTAU ? 16 : 1];
    if constexpr (DTAU) dtau_rows_load(p, dbh, dv, t0w, kb0, lane);
    float b2v[BIAS ? 4 : 1][4];
    bias_of(p, kb0, b2v);
    f32x4 sc[4], dp[4];
    int kind[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kind[j] = sub_kind(wb, kb0 + 16 * j);
      if (kind[j] != 0) sdp(kt, j, sc[j], dp[j]);
    }
    if constexpr (DTAU) dtau_rows_put(dst, dv, lane);
    float G[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float dtv[4] = {0.f, 0.f, 0.f, 0.f};
      if (DTAU && kind[j] != 0) stage_get4(dst, c, j, g, dtv);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = kind[j] != 0 && (key >= lo) & (key <= hi);
        G[j][r] = kind[j] != 0 ? g_of(tau_of(sc[j][r], BIAS ? b2v[j][r] : 0.f, ok), dp[j][r], dtv[r], ok) : 0.f;
      }
    }
    dq_product(kt, kind, G);
  }

  // a, c from the band sums (msum = sum P, dsum = sum P dP over the row)
  __device__ __forceinline__ void coefficients(const BandParams& p) {
    msum = wave_sum_g(msum);
    dsum = wave_sum_g(dsum);
    const float m = msum > kMassEps ? msum : kMassEps;
    ca = 1.f / m;
    cc = msum >= kMassEps ? dsum * ca * ca : 0.f;
    put_coefficients(p);
  }

  __device__ __forceinline__ void put_coefficients(const BandParams& p) const {
    if (p.ws && qok && g == 0) {
      const int64_t nws = (int64_t)p.B * p.T * p.H;
      const int64_t wi = ((int64_t)b * p.T + tq) * p.H + h;
      ((float*)p.ws)[wi] = ca;
      ((float*)p.ws)[nws + wi] = cc;
    }
  }

  // MODE 1: the band's blocks (bl.n <= 2) sit in LDS buffers u0, u1
  __device__ __forceinline__ void mode1(const BandParams& p, const bf16* lds, int u0, int u1) {
    const bf16* kts[2] = {key_buf<NT, NV>((bf16*)lds, u0), key_buf<NT, NV>((bf16*)lds, u1)};
    float P[2][4][4], Dp[2][4][4];
    E dv[2][DTAU ? 16 : 1];
    if constexpr (DTAU) {
      dtau_rows_load(p, dbh, dv[0], t0w, bl.first, lane);
      dtau_rows_load(p, dbh, dv[1], t0w, bl.first + kTile, lane);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) P[s][j][r] = Dp[s][j][r] = 0.f;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (s >= bl.n) break;
      const int kb0 = bl.first + s * kTile;
      float b2v[BIAS ? 4 : 1][4];
      bias_of(p, kb0, b2v);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (sub_kind(wb, kb0 + 16 * j) == 0) continue;
        f32x4 sc, dp;
        sdp(kts[s], j, sc, dp);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kb0 + 16 * j + 4 * g + r;
          const bool ok = (key >= lo) & (key <= hi);
          const float pv = tau_of(sc[r], BIAS ? b2v[j][r] : 0.f, ok);
          P[s][j][r] = pv;
          Dp[s][j][r] = ok ? dp[r] : 0.f;
          msum += pv;
          dsum = fmaf(pv, Dp[s][j][r], dsum);
        }
      }
    }
    coefficients(p);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (s >= bl.n) break;
      const int kb0 = bl.first + s * kTile;
      if constexpr (DTAU) dtau_rows_put(dst, dv[s], lane);
      float G[4][4];
      int kind[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kind[j] = sub_kind(wb, kb0 + 16 * j);
        float dtv[4] = {0.f, 0.f, 0.f, 0.f};
        if (DTAU && kind[j] != 0) stage_get4(dst, c, j, g, dtv);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kb0 + 16 * j + 4 * g + r;
          const bool ok = kind[j] != 0 && (key >= lo) & (key <= hi);
          G[j][r] = g_of(P[s][j][r], Dp[s][j][r], dtv[r], ok);
        }
      }
      dq_product(kts[s], kind, G);
    }
  }

  // MODE 2 first pass: the band sums of one block
  __device__ __forceinline__ void sums_pass(const BandParams& p, const bf16* kt, int kb0) {
    float b2v[BIAS ? 4 : 1][4];
    bias_of(p, kb0, b2v);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (sub_kind(wb, kb0 + 16 * j) == 0) continue;
      f32x4 sc, dp;
      sdp(kt, j, sc, dp);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * j + 4 * g + r;
        const bool ok = (key >= lo) & (key <= hi);
        const float pv = tau_of(sc[r], BIAS ? b2v[j][r] : 0.f, ok);
        msum += pv;
        dsum = fmaf(pv, ok ? dp[r] : 0.f, dsum);
      }
    }
  }

  // MODE 3: a, c from the saved output row and tau mass: dO . out over this
  // lane's features (its dO terms summed back to the float32 value: t0 + t1
  // + t2 is exact in float32), then over the row
  __device__ __forceinline__ void saved_coefficients(const BandParams& p) {
    float dot = 0.f;
    if (qok) {
      const E* orow = (const E*)p.out.p + b * p.out.s0 + (int64_t)tq * p.out.s1 + h * p.out.s2;
#pragma unroll
      for (int ch = 0; ch < D / 32; ++ch) {
        bf16x8 ot[NT];
        frag_row<NT>(orow, 0, 0, 1, 4 * ch + g, ot);  // the row's features 8 (4 ch + g) ..
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float ov = 0.f, dv_ = 0.f;
#pragma unroll
          for (int i = 0; i < NT; ++i) {
            ov += (float)ot[i][e];
            dv_ += (float)of[ch][i][e];
          }
          dot = fmaf(dv_, ov, dot);
        }
      }
    }
    dot = wave_sum_g(dot);
    const float m = qok ? ld<float>(p.mass, b * p.mass.s0 + (int64_t)tq * p.mass.s1 + h * p.mass.s2) : 1.f;
    ca = 1.f / (m > kMassEps ? m : kMassEps);
    cc = m >= kMassEps ? dot * ca : 0.f;
    put_coefficients(p);
  }

  __device__ __forceinline__ void store(const BandParams& p, float inv_scale) const {
    if (!qok) return;
    store_acc<E, D>((E*)p.dq.p + b * p.dq.s0 + (int64_t)tq * p.dq.s1 + h * p.dq.s2, acc, inv_scale, g);
  }
};

// The lane's query-row fragments (Q, dOut) as loaded, for a load ahead of use.
template <int NT, int D>
struct QueryRaw {
  RawFrag<NT> q[D / 32], o[D / 32];
};

template <int NT, int NV, int D, int NORM, bool BIAS, bool DTAU>
__device__ __forceinline__ DqTile<NT, NV, D, NORM, BIAS, DTAU> dq_tile_base(const BandParams& p, int b, int h,
                                                                            int lane, Elem<NT>* dst) {
  DqTile<NT, NV, D, NORM, BIAS, DTAU> q;
  q.b = b;
  q.h = h;
  q.lane = lane;
  q.g = lane >> 4;
  q.c = lane & 15;
  q.k2 = -kLog2e * (float)(1.0 / p.scale);
  q.dbh = DTAU ? (const Elem<NT>*)p.dtau.p + b * p.dtau.s0 + h * p.dtau.s2 : nullptr;
  q.dst = dst;
  return q;
}

template <int NT, int NV, int D, int NORM, bool BIAS, bool DTAU, int MODE>
__global__ __launch_bounds__(kThreads) void xb_dq(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  constexpr int NBUF = (NT == 1 || MODE == 1) ? 2 : 1;
  __shared__ __attribute__((aligned(16))) bf16 lds[NBUF * (NT + NV) * kDTile];
  __shared__ __attribute__((aligned(16))) Elem<NT> dstage[DTAU ? 4 * kStageRows : 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const TileId id = tile_id(p, p.glob != 0);
  const int b = id.b, h = id.h, T = p.T;

  using E = Elem<NT>;
  const E* qb_ = (const E*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const E* kb_ = (const E*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const Elem<NV>* vb_ = (const Elem<NV>*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const E* ob_ = (const E*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;
  DqTile<NT, NV, D, NORM, BIAS, DTAU> st =
      dq_tile_base<NT, NV, D, NORM, BIAS, DTAU>(p, b, h, lane, dstage + (DTAU ? wave * kStageRows : 0));
  st.at(p, id.tile * kTile, wave);
#pragma unroll
  for (int ch = 0; ch < D / 32; ++ch) {
    frag_row<NT>(qb_, p.q.s1, st.tq, T, 4 * ch + st.g, st.qf[ch]);
    frag_row<NT>(ob_, p.dout.s1, st.tq, T, 4 * ch + st.g, st.of[ch]);
  }
  const Blocks bl = st.bl;
  auto g_pass = [&](const bf16* kt, int kb0) { st.g_pass(p, kt, kb0); };

  if constexpr (MODE == 0) {
    stream_keys<NT, NV, D, NBUF>(lds, kb_, p.k.s1, vb_, p.v.s1, bl, T, tid, g_pass);
  } else if constexpr (MODE == 3) {
    st.saved_coefficients(p);
    stream_keys<NT, NV, D, NBUF>(lds, kb_, p.k.s1, vb_, p.v.s1, bl, T, tid, g_pass);
  } else if constexpr (MODE == 1) {
    // both blocks stay resident (buffers 0 and 1)
    if (bl.n > 0) {
      store_raw<NT>(load_raw<NT, D>(kb_, p.k.s1, bl.first, T, tid), key_buf<NT, NV>(lds, 0), tid);
      store_raw<NV>(load_raw<NV, D>(vb_, p.v.s1, bl.first, T, tid), key_buf<NT, NV>(lds, 0) + NT * kDTile, tid);
    }
    if (bl.n > 1) {
      store_raw<NT>(load_raw<NT, D>(kb_, p.k.s1, bl.first + kTile, T, tid), key_buf<NT, NV>(lds, 1), tid);
      store_raw<NV>(load_raw<NV, D>(vb_, p.v.s1, bl.first + kTile, T, tid),
                    key_buf<NT, NV>(lds, 1) + NT * kDTile, tid);
    }
    __syncthreads();
    st.mode1(p, lds, 0, 1);
  } else {
    stream_keys<NT, NV, D, NBUF>(lds, kb_, p.k.s1, vb_, p.v.s1, bl, T, tid,
                             [&](const bf16* kt, int kb0) { st.sums_pass(p, kt, kb0); });
    st.coefficients(p);
    stream_keys<NT, NV, D, NBUF>(lds, kb_, p.k.s1, vb_, p.v.s1, bl, T, tid, g_pass);
  }
  st.store(p, (float)(1.0 / p.scale));
}

// Runs of query tiles for local windows W <= 64 (MODE 0 or 1), where query
// tile t sees key blocks t - 1 and t only: a workgroup owns query tiles
// [tA, tB) of one (b, h) (p.chunk runs per (b, h)); key block j sits in LDS
// buffer j & 1, so tile t + 1 finds block t where tile t left it, and block
// t + 1 and the next tile's query rows load into registers while tile t
// computes.
template <int NT, int NV, int D, int NORM, bool BIAS, bool DTAU, int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) void xb_dq_run(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  static_assert(MODE == 0 || MODE == 1, "runs take the one-pass and register tau-mass modes");
  __shared__ __attribute__((aligned(16))) bf16 lds[2 * (NT + NV) * kDTile];
  __shared__ __attribute__((aligned(16))) Elem<NT> dstage[DTAU ? 4 * kStageRows : 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nr = p.chunk;
  const int id = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);
  const int bh = id / nr, run = id % nr;
  const int b = bh / p.H, h = bh % p.H, T = p.T;
  const int tA = run_bound(run, p.ntiles, nr);
  const int tB = run_bound(run + 1, p.ntiles, nr);
  if (tA >= tB) return;

  using E = Elem<NT>;
  const E* qb_ = (const E*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const E* kb_ = (const E*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const Elem<NV>* vb_ = (const Elem<NV>*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const E* ob_ = (const E*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;
  const float inv_scale = (float)(1.0 / p.scale);
  DqTile<NT, NV, D, NORM, BIAS, DTAU> st =
      dq_tile_base<NT, NV, D, NORM, BIAS, DTAU>(p, b, h, lane, dstage + (DTAU ? wave * kStageRows : 0));
  st.at(p, tA * kTile, wave);
#pragma unroll
  for (int ch = 0; ch < D / 32; ++ch) {
    frag_row<NT>(qb_, p.q.s1, st.tq, T, 4 * ch + st.g, st.qf[ch]);
    frag_row<NT>(ob_, p.dout.s1, st.tq, T, 4 * ch + st.g, st.of[ch]);
  }
  // blocks tA - 1 (when tA > 0) and tA
  for (int j = tA > 0 ? tA - 1 : 0; j <= tA; ++j) {
    bf16* kbuf = key_buf<NT, NV>(lds, j & 1);
    store_raw<NT>(load_raw<NT, D>(kb_, p.k.s1, j * kTile, T, tid), kbuf, tid);
    store_raw<NV>(load_raw<NV, D>(vb_, p.v.s1, j * kTile, T, tid), kbuf + NT * kDTile, tid);
  }
  __syncthreads();
  for (int t = tA; t < tB; ++t) {
    const bool more = t + 1 < tB;
    Raw<NT> kn;
    Raw<NV> vn;
    QueryRaw<NT, D> qn;
    if (more) {
      kn = load_raw<NT, D>(kb_, p.k.s1, (t + 1) * kTile, T, tid);
      vn = load_raw<NV, D>(vb_, p.v.s1, (t + 1) * kTile, T, tid);
      const int tq1 = st.tq + kTile;
#pragma unroll
      for (int ch = 0; ch < D / 32; ++ch) {
        qn.q[ch] = frag_load<NT>(qb_, p.q.s1, tq1, T, 4 * ch + st.g);
        qn.o[ch] = frag_load<NT>(ob_, p.dout.s1, tq1, T, 4 * ch + st.g);
      }
    }
    // the band of tile t: blocks bl.first (t - 1, or 0 for t = 0) and on
    const int j0 = st.bl.first / kTile;
    if constexpr (MODE == 1) {
      st.mode1(p, lds, j0 & 1, (j0 + 1) & 1);
    } else {
      for (int s = 0; s < st.bl.n; ++s) st.g_pass(p, key_buf<NT, NV>(lds, (j0 + s) & 1), (j0 + s) * kTile);
    }
    st.store(p, inv_scale);
    if (more) {
      __syncthreads();  // every wave is done with block t - 1's buffer
      bf16* kbuf = key_buf<NT, NV>(lds, (t + 1) & 1);
      store_raw<NT>(kn, kbuf, tid);
      store_raw<NV>(vn, kbuf + NT * kDTile, tid);
      st.at(p, (t + 1) * kTile, wave);
#pragma unroll
      for (int ch = 0; ch < D / 32; ++ch) {
        frag_terms<NT>(qn.q[ch], st.qf[ch]);
        frag_terms<NT>(qn.o[ch], st.of[ch]);
      }
      __syncthreads();
    }
  }
}

// ----------------------------------------------------------------- dK / dV

// One key tile's lane state in the dK / dV kernels: the lane's key row as B
// operands (K and V as terms), the queries that see it, its dK / dV
// accumulators, and the number of query tiles whose band reaches the tile.
template <int NT, int NV, int D>
struct KeyTile {
  bf16x8 kf[D / 32][NT], vf[D / 32][NV];
  f32x4 dk[D / 16], dv[D / 16];
  int tk, qlo, qhi, wq_lo, wq_hi, nqt;
};

// Key tile k0's geometry for lane (wave, c); accumulators cleared.
template <int NT, int NV, int D>
__device__ __forceinline__ void key_tile_init(const BandParams& p, int k0, int wave, int c,
                                              KeyTile<NT, NV, D>& kt) {
  const int T = p.T;
  kt.tk = k0 + wave * 16 + c;
  // queries that see this lane's key: [tk + 1 - diag, min(tk + win, T - 1)]
  kt.qlo = kt.tk + 1 - p.diag;
  kt.qhi = kt.tk >= T ? -1 : (kt.tk > T - 1 - p.win ? T - 1 : kt.tk + p.win);
  // queries that see any key of this wave (a 16-query group outside is skipped)
  const int ka = k0 + wave * 16;
  const int kz = ka + 15 < T - 1 ? ka + 15 : T - 1;
  kt.wq_lo = ka + 1 - p.diag;
  kt.wq_hi = kz < ka ? -1 : (kz > T - 1 - p.win ? T - 1 : kz + p.win);
  // query tiles k .. k + nqt - 1
  const int last_q = k0 + kTile - 1 > T - 1 - p.win ? T - 1 : k0 + kTile - 1 + p.win;
  kt.nqt = last_q < k0 ? 0 : (last_q >> 6) - (k0 >> 6) + 1;
#pragma unroll
  for (int m = 0; m < D / 16; ++m) kt.dk[m] = kt.dv[m] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// The lane's key row (features 8 (4 ch + g) .. +7 of K and V) as loaded.
template <int NT, int NV, int D>
struct KeyRaw {
  RawFrag<NT> k[D / 32];
  RawFrag<NV> v[D / 32];
};

template <int NT, int NV, int D>
__device__ __forceinline__ KeyRaw<NT, NV, D> key_raw_load(const Elem<NT>* kb_, int64_t ks, const Elem<NV>* vb_,
                                                          int64_t vs, int tk, int T, int g) {
  KeyRaw<NT, NV, D> r;
#pragma unroll
  for (int ch = 0; ch < D / 32; ++ch) {
    r.k[ch] = frag_load<NT>(kb_, ks, tk, T, 4 * ch + g);
    r.v[ch] = frag_load<NV>(vb_, vs, tk, T, 4 * ch + g);
  }
  return r;
}

template <int NT, int NV, int D>
__device__ __forceinline__ void key_raw_terms(const KeyRaw<NT, NV, D>& r, KeyTile<NT, NV, D>& kt) {
#pragma unroll
  for (int ch = 0; ch < D / 32; ++ch) {
    frag_terms<NT>(r.k[ch], kt.kf[ch]);
    frag_terms<NV>(r.v[ch], kt.vf[ch]);
  }
}

// Query tile q0 into LDS: Q terms at base, dOut terms after them, and its
// rows' coefficients a, c (tau mass: from the workspace the dQ kernel wrote;
// valid count: 1 / count; raw: 1, 0).
template <int NT, int D, int NORM>
__device__ __forceinline__ void dkv_stage(const BandParams& p, bf16* base, float* sa_, float* scf_, int q0,
                                          const Raw<NT>& qx, const Raw<NT>& ox, int b, int h, int tid) {
  store_raw<NT>(qx, base, tid);
  store_raw<NT>(ox, base + NT * kDTile, tid);
  if (tid < kTile) {
    const int t = q0 + tid;
    float a = 1.f, cv = 0.f;
    if (t < p.T) {
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
    sa_[tid] = a;
    scf_[tid] = cv;
  }
}

// One query tile q0 (terms in LDS at qt, coefficient rows sa_ / scf_)
// against key tile kt:  dV^T += dO^T (a P),  dK^T += Q^T G.  dtb / bb: dTau
// and bias of this (b, h) (dtype of Q / float32).
template <int NT, int NV, int D, bool BIAS, bool DTAU>
__device__ __forceinline__ void dkv_visit(const BandParams& p, const bf16* qt, const float* sa_, const float* scf_,
                                          int q0, KeyTile<NT, NV, D>& kt, const Elem<NT>* dtb, const float* bb,
                                          float k2, int g, int c) {
  const bf16* ot = qt + NT * kDTile;
  float Pa[4][4], G[4][4];
  bool live[4];
  // dTau of the visit's pairs, loaded before the products so its latency
  // runs under them: every load is issued (a pair without a slot reads the
  // (b, h)'s first element) and masked afterwards
  float dtv[DTAU ? 4 : 1][4], b2v[BIAS ? 4 : 1][4];
  if constexpr (BIAS) {  // the bias of the same pairs, likewise
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = q0 + 16 * j + 4 * g + r;
        const bool ok = t >= kt.qlo && t <= kt.qhi;
        b2v[j][r] = bb[ok ? (int64_t)t * p.bias.s1 + bias_col(p, t, kt.tk) : 0];  // raw; masked below
      }
  }
  if constexpr (DTAU) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = q0 + 16 * j + 4 * g + r;
        const bool ok = t >= kt.qlo && t <= kt.qhi;
        const int col = ok ? tau_col(p, t, kt.tk) : -1;
        const float x = (float)dtb[col >= 0 ? (int64_t)t * p.dtau.s1 + col : 0];
        dtv[j][r] = col >= 0 ? x : 0.f;
      }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int qa = q0 + 16 * j;
    live[j] = qa + 15 >= kt.wq_lo && qa <= kt.wq_hi;
    if (!live[j]) {
#pragma unroll
      for (int r = 0; r < 4; ++r) Pa[j][r] = G[j][r] = 0.f;
      continue;
    }
    // S = Q K^T, dP = dO V^T: queries 16 j + 4 g + r (rows), key c (column)
    f32x4 sv = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ch = 0; ch < D / 32; ++ch) {
      bf16x8 qa_[NT], oa_[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        qa_[t] = dt_row8(qt + t * kDTile, 16 * j + c, 4 * ch + g);
        oa_[t] = dt_row8(ot + t * kDTile, 16 * j + c, 4 * ch + g);
      }
      sv = mmx<NT, NT, 2>(qa_, kt.kf[ch], sv);
      dp = mmx<NT, NV, 2>(oa_, kt.vf[ch], dp);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ql = 16 * j + 4 * g + r;  // query - q0
      const int t = q0 + ql;
      const bool ok = t >= kt.qlo && t <= kt.qhi;
      const float pv = sigmoid_scaled(sv[r], k2, BIAS ? -kLog2e * b2v[j][r] : 0.f);
      const float a = sa_[ql];
      float dt = fmaf(dp[r], a, -scf_[ql]);
      if constexpr (DTAU) dt += dtv[j][r];
      Pa[j][r] = ok ? pv * a : 0.f;
      G[j][r] = ok ? dt * (pv - pv * pv) : 0.f;
    }
  }
  // dV^T += dO^T (a P),  dK^T += Q^T G over 32-query pairs
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    if (!live[2 * kk] && !live[2 * kk + 1]) continue;
    bf16x8 ps[NT], gs[NT];
    pack_terms<NT>(Pa[2 * kk], Pa[2 * kk + 1], ps);
    pack_terms<NT>(G[2 * kk], G[2 * kk + 1], gs);
#pragma unroll
    for (int m = 0; m < D / 16; ++m) {
      bf16x8 oa_[NT], qa_[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        oa_[t] = dt_tr8(ot + t * kDTile, m, 32 * kk, g, c);
        qa_[t] = dt_tr8(qt + t * kDTile, m, 32 * kk, g, c);
      }
      kt.dv[m] = mmx_run<NT, NT, NV == 1 ? 1 : 2, NV == 3>(oa_, ps, kt.dv[m]);
      kt.dk[m] = mmx_run<NT, NT, 2, NV == 3>(qa_, gs, kt.dk[m]);
    }
  }
}

// The lane's dK row (dtype of Q; times 1 / scale) and dV row (dtype of V).
template <int NT, int NV, int D>
__device__ __forceinline__ void dkv_store(const BandParams& p, const KeyTile<NT, NV, D>& kt, int b, int h,
                                          float inv_scale, int g) {
  if (kt.tk >= p.T) return;
  using E = Elem<NT>;
  using EV = Elem<NV>;
  store_acc<E, D>((E*)p.dk.p + b * p.dk.s0 + (int64_t)kt.tk * p.dk.s1 + h * p.dk.s2, kt.dk, inv_scale, g);
  store_acc<EV, D>((EV*)p.dv.p + b * p.dv.s0 + (int64_t)kt.tk * p.dv.s1 + h * p.dv.s2, kt.dv, 1.f, g);
}

// Key tile k: the query tiles whose band reaches it pass through LDS in
// turn (Q and dOut as NT terms each, plus their rows' coefficients a, c).
template <int NT, int NV, int D, int NORM, bool BIAS, bool DTAU>
__global__ __launch_bounds__(kThreads) void xb_dkv(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  constexpr int NBUF = NT == 1 ? 2 : 1;
  constexpr int TPB = 2 * NT;  // tiles per buffer: Q terms, then dOut terms
  __shared__ __attribute__((aligned(16))) bf16 lds[NBUF * TPB * kDTile];
  __shared__ float sa[NBUF][kTile], scf[NBUF][kTile];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const TileId id = tile_id(p, false);
  const int b = id.b, h = id.h, T = p.T;
  const int k0 = id.tile * kTile;

  using E = Elem<NT>;
  const E* qb_ = (const E*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const E* kb_ = (const E*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const Elem<NV>* vb_ = (const Elem<NV>*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const E* ob_ = (const E*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;

  KeyTile<NT, NV, D> kt;
  key_tile_init<NT, NV, D>(p, k0, wave, c, kt);
  key_raw_terms<NT, NV, D>(key_raw_load<NT, NV, D>(kb_, p.k.s1, vb_, p.v.s1, kt.tk, T, g), kt);

  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;
  // dTau (dtype of Q, host-checked) and bias (float32) of this (b, h)
  const E* const dtb = DTAU ? (const E*)p.dtau.p + b * p.dtau.s0 + h * p.dtau.s2 : nullptr;
  const float* const bb = BIAS ? (const float*)p.bias.p + b * p.bias.s0 : nullptr;

  const int nqt = kt.nqt;
  if (nqt > 0) {
    dkv_stage<NT, D, NORM>(p, lds, sa[0], scf[0], k0, load_raw<NT, D>(qb_, p.q.s1, k0, T, tid),
                           load_raw<NT, D>(ob_, p.dout.s1, k0, T, tid), b, h, tid);
    __syncthreads();
  }
  for (int i = 0; i < nqt; ++i) {
    const int q0 = k0 + i * kTile;
    const int buf = NBUF == 2 ? (i & 1) : 0;
    const bool more = i + 1 < nqt;
    Raw<NT> qn, on;
    if (more) {
      qn = load_raw<NT, D>(qb_, p.q.s1, q0 + kTile, T, tid);
      on = load_raw<NT, D>(ob_, p.dout.s1, q0 + kTile, T, tid);
    }
    dkv_visit<NT, NV, D, BIAS, DTAU>(p, lds + buf * TPB * kDTile, sa[buf], scf[buf], q0, kt, dtb, bb, k2, g, c);
    if (more) {
      if (NBUF == 1) __syncthreads();  // every wave is done with the buffer
      const int nb = NBUF == 2 ? (buf ^ 1) : 0;
      dkv_stage<NT, D, NORM>(p, lds + nb * TPB * kDTile, sa[nb], scf[nb], q0 + kTile, qn, on, b, h, tid);
      __syncthreads();
    }
  }
  dkv_store<NT, NV, D>(p, kt, b, h, inv_scale, g);
}

// Runs of key tiles for local windows W <= 64, where key tile k is seen by
// query tiles k and k + 1 only: a workgroup owns key tiles [kA, kB) of one
// (b, h) (p.chunk runs per (b, h)) and walks query tiles kA .. kB once --
// consecutive key tiles share a query tile, which stays in the LDS buffer
// from the last visit of one to the first visit of the next -- with the
// next query tile loading into registers during a key tile's first visit
// and the next key rows during its second.  Odd runs walk down (key tile k
// visits query tile k + 1, then k): two runs that share a boundary query
// tile then read it at the same time (both at their ends or both at their
// starts), and the second read is an L2 hit.
template <int NT, int NV, int D, int NORM, bool BIAS, bool DTAU>
__global__ __launch_bounds__(kThreads) void xb_dkv_run(BandArgs args) {
  touch_args(args);
  const BandParams p = band_params(args);
  constexpr int TPB = 2 * NT;
  __shared__ __attribute__((aligned(16))) bf16 lds[TPB * kDTile];
  __shared__ float sa[kTile], scf[kTile];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int nr = p.chunk;
  const int id = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);
  const int bh = id / nr, run = id % nr;
  const int b = bh / p.H, h = bh % p.H, T = p.T;
  const int kA = run_bound(run, p.ntiles, nr);
  const int kB = run_bound(run + 1, p.ntiles, nr);
  const bool desc = (run & 1) != 0;

  using E = Elem<NT>;
  const E* qb_ = (const E*)p.q.p + b * p.q.s0 + h * p.q.s2;
  const E* kb_ = (const E*)p.k.p + b * p.k.s0 + h * p.k.s2;
  const Elem<NV>* vb_ = (const Elem<NV>*)p.v.p + b * p.v.s0 + h * p.v.s2;
  const E* ob_ = (const E*)p.dout.p + b * p.dout.s0 + h * p.dout.s2;
  const float inv_scale = (float)(1.0 / p.scale);
  const float k2 = -kLog2e * inv_scale;
  const E* const dtb = DTAU ? (const E*)p.dtau.p + b * p.dtau.s0 + h * p.dtau.s2 : nullptr;
  const float* const bb = BIAS ? (const float*)p.bias.p + b * p.bias.s0 : nullptr;
  const int n = kB - kA;
  if (n <= 0) return;

  const int kfirst = desc ? kB - 1 : kA;
  KeyTile<NT, NV, D> kt;
  key_tile_init<NT, NV, D>(p, kfirst * kTile, wave, c, kt);
  key_raw_terms<NT, NV, D>(key_raw_load<NT, NV, D>(kb_, p.k.s1, vb_, p.v.s1, kt.tk, T, g), kt);
  {
    // a key tile's first visit: query tile k (up), k + 1 when it sees the
    // tile (down); the trip before left that tile in LDS
    const int q0 = (desc && kt.nqt > 1 ? kfirst + 1 : kfirst) * kTile;
    dkv_stage<NT, D, NORM>(p, lds, sa, scf, q0, load_raw<NT, D>(qb_, p.q.s1, q0, T, tid),
                           load_raw<NT, D>(ob_, p.dout.s1, q0, T, tid), b, h, tid);
  }
  __syncthreads();
  for (int i = 0; i < n; ++i) {
    const int k = desc ? kB - 1 - i : kA + i;
    const bool two = kt.nqt > 1;  // query tile k + 1 sees this key tile
    const int q1 = (desc && two ? k + 1 : k) * kTile;  // in LDS
    const int q2 = (desc ? k : k + 1) * kTile;         // the second visit, when two
    Raw<NT> qn, on;
    if (two) {
      qn = load_raw<NT, D>(qb_, p.q.s1, q2, T, tid);
      on = load_raw<NT, D>(ob_, p.dout.s1, q2, T, tid);
    }
    dkv_visit<NT, NV, D, BIAS, DTAU>(p, lds, sa, scf, q1, kt, dtb, bb, k2, g, c);
    if (two) {
      __syncthreads();  // every wave is done with the first visit's tile
      dkv_stage<NT, D, NORM>(p, lds, sa, scf, q2, qn, on, b, h, tid);
      __syncthreads();
    }
    const bool next = i + 1 < n;
    const int kn0 = (desc ? k - 1 : k + 1) * kTile;
    KeyRaw<NT, NV, D> kr;
    if (next) kr = key_raw_load<NT, NV, D>(kb_, p.k.s1, vb_, p.v.s1, kn0 + wave * 16 + c, T, g);
    if (two) dkv_visit<NT, NV, D, BIAS, DTAU>(p, lds, sa, scf, q2, kt, dtb, bb, k2, g, c);
    dkv_store<NT, NV, D>(p, kt, b, h, inv_scale, g);
    if (next) {
      key_tile_init<NT, NV, D>(p, kn0, wave, c, kt);
      key_raw_terms<NT, NV, D>(kr, kt);
    }
  }
}

// ----------------------------------------------------------------- launch

template <int NT, int NV, int D, int NORM, int PHASE>
void launch_norm(const BandParams& p, hipStream_t st, unsigned n) {
  const bool bias = p.bias.p != nullptr;
  const dim3 grid(n), block(kThreads);
  const BandArgs a = to_args(p);
#define XB_BT(K, ...)                                                                           \
  do {                                                                                          \
    if (bias) {                                                                                 \
      if (opt) hipLaunchKernelGGL((K<NT, NV, D, NORM, true, true __VA_ARGS__>), grid, block, 0, st, a);  \
      else hipLaunchKernelGGL((K<NT, NV, D, NORM, true, false __VA_ARGS__>), grid, block, 0, st, a);     \
    } else {                                                                                    \
      if (opt) hipLaunchKernelGGL((K<NT, NV, D, NORM, false, true __VA_ARGS__>), grid, block, 0, st, a); \
      else hipLaunchKernelGGL((K<NT, NV, D, NORM, false, false __VA_ARGS__>), grid, block, 0, st, a);    \
    }                                                                                           \
  } while (0)
  if constexpr (PHASE == 0) {
    const bool opt = p.tau.p != nullptr;
    if (p.chunk > 0) XB_BT(xb_fwd_run);
    else XB_BT(xb_fwd);
  } else if constexpr (PHASE == 1) {
    const bool opt = p.dtau.p != nullptr;
    // runs of tiles (a local window W <= 64): float32 Q / K at head dim 32
    // without dTau, where they measured faster (B32 H4 T1024 W32 tau-mass
    // step 82.8 -> 76.5 us); at head dim 64 the run kernel's registers
    // (246 VGPRs, and spills with dTau) cost what the shared blocks save;
    // with a float32 V two resident key blocks of six terms each would
    // take 96 KB of LDS
    constexpr bool kRuns = NT == 3 && NV == 1 && D == 32;
    if constexpr (kRuns) {
      if (p.chunk > 0 && !opt) {
        constexpr int M = NORM == NORM_MASS_ ? 1 : 0;
        if (bias) hipLaunchKernelGGL((xb_dq_run<NT, NV, D, NORM, true, false, M>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((xb_dq_run<NT, NV, D, NORM, false, false, M>), grid, block, 0, st, a);
        return;
      }
    }
    if constexpr (NORM != NORM_MASS_) {
      XB_BT(xb_dq, , 0);
    } else if constexpr (NV == 3) {
      // float32 V: the register tau-mass mode would keep two blocks of six
      // terms in LDS (96 KB); the saved rows (one pass) or two passes
      if (p.coef_pre) XB_BT(xb_dq, , 3);
      else XB_BT(xb_dq, , 2);
    } else if constexpr (NT == 3) {
      // a band within two blocks keeps P and dP in registers (faster than
      // one pass from saved rows at W = 64: 42 against 48 us at config 2)
      if (!p.glob && p.win <= kTile) XB_BT(xb_dq, , 1);
      else if (p.coef_pre) XB_BT(xb_dq, , 3);
      else XB_BT(xb_dq, , 2);
    } else {  // bf16 / fp16 rows: the coefficients from the band (a 16-bit out would cancel)
      if (!p.glob && p.win <= kTile) XB_BT(xb_dq, , 1);
      else XB_BT(xb_dq, , 2);
    }
  } else {
    const bool opt = p.dtau.p != nullptr;
    if (p.chunk > 0) XB_BT(xb_dkv_run);
    else XB_BT(xb_dkv);
  }
#undef XB_BT
}

// PHASE 0: forward, 1: dQ (+ coefficients), 2: dK / dV; one workgroup per
// 64-row tile (n of them)
template <int NT, int NV, int PHASE>
void launch(const BandParams& p, hipStream_t st, unsigned n) {
  const int norm = (p.flags & TENSION_NORM_MASS)    ? NORM_MASS_
                   : (p.flags & TENSION_NORM_COUNT) ? NORM_COUNT_
                                                    : NORM_RAW;
  if (p.D == 32) {
    if (norm == NORM_MASS_) launch_norm<NT, NV, 32, NORM_MASS_, PHASE>(p, st, n);
    else if (norm == NORM_COUNT_) launch_norm<NT, NV, 32, NORM_COUNT_, PHASE>(p, st, n);
    else launch_norm<NT, NV, 32, NORM_RAW, PHASE>(p, st, n);
  } else {
    if (norm == NORM_MASS_) launch_norm<NT, NV, 64, NORM_MASS_, PHASE>(p, st, n);
    else if (norm == NORM_COUNT_) launch_norm<NT, NV, 64, NORM_COUNT_, PHASE>(p, st, n);
    else launch_norm<NT, NV, 64, NORM_RAW, PHASE>(p, st, n);
  }
}

}  // namespace split
}  // namespace tension
