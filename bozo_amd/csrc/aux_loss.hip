// The model's tau regularisers (model.py:498-611) in two passes over the
// materialised tau of every layer: the forward accumulates per-layer sums,
// the backward writes dTau from per-layer coefficients.
//
// Per row (b, t, h) of a layer, tau[0..W) (w = 0 oldest), all in fp32, each
// workgroup writing its four sums to its slot of the partials buffer:
//   diversity : S = sum tau, p = tau / (S + 1e-8),
//               ent = -sum p log(p + 1e-8)             (acc 0: sum of ent)
//   consistency (rows r with terms; n = min(W - 2, 4), T_out = T - n - 1):
//               for w1 = 1..n with w1 + 1 <= r <= w1 + T_out:
//               relu(tau[r, w1-1] * tau[r-1, 0] - tau[r, w1])  (acc 1)
//   entropy   : m = mean tau, relu(0.05 - m) (acc 2), relu(m - 0.8) (acc 3)
// Eight lanes share a row: lane ch holds the 8-slot chunks ch, ch + 8, ..
// (NCH = ceil(W / 64) of them, W <= 256), so a wave load instruction reads
// eight whole 128-byte row pieces (bf16); row sums fold through DPP.  A
// workgroup walks 1024 consecutive rows of one layer, 4 / NCH rows per lane
// in flight at a time, and (forward) reduces its sums once at the end.
//
// Backward, with per-layer coefficients k = (k_div, k_cons, k_ent):
//   dTau[w]  = k_div (e_w - sum_v e_v p_v) / (S + 1e-8),  e = -(log(p + 1e-8) + p / (p + 1e-8))
//            + k_ent ([m > 0.8] - [m < 0.05]) / W
//            + k_cons (terms of row t: b for slot w1-1, -1 for slot w1, where
//              the term is active; terms of row t+1: its slot w1-1 value
//              for slot 0)
// so every row's gradient is written by the eight lanes that own it (no
// atomics).
#include "kernels.h"

namespace tension {

namespace {

constexpr float kDivEps = 1e-8f;  // model.py:527-528
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kThreadsAux = 256;
constexpr int kRowsPerPass = kThreadsAux / 8;  // one row per 8 lanes
constexpr int kUnrollVals = 4;                 // row chunks per lane whose loads are in flight together

// the eight values of lane chunk ch of a row (0 past W).  VEC (bf16, W and
// the strides multiples of 8, 16-byte aligned base): one 16-byte load, issued
// for every lane (chunks past W read chunk 0 and are zeroed), so a pass's
// loads carry no branch; otherwise element loads.
// VEC: 0 element loads of any dtype, 1 one 16-byte load of bf16, 2 two of
// float32 (vec_kind)
template <int VEC, bool FULL = false>
__device__ __forceinline__ void row8(const Buf& b, int64_t off, int ch, int W, float* v) {
  if constexpr (VEC == 1) {
    const bool in = FULL || 8 * ch < W;
    const bf16x8 x = __builtin_bit_cast(bf16x8, *(const u16x8*)((const bf16*)b.p + off + (in ? 8 * ch : 0)));
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = in ? (float)x[e] : 0.f;
  } else if constexpr (VEC == 2) {
    const bool in = FULL || 8 * ch < W;
    const float* q = (const float*)b.p + off + (in ? 8 * ch : 0);
    const f32x4 x0 = *(const f32x4*)q, x1 = *(const f32x4*)(q + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = in ? x0[e] : 0.f;
      v[4 + e] = in ? x1[e] : 0.f;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int w = 8 * ch + e;
      v[e] = w < W ? ld<float>(b, off + w) : 0.f;
    }
  }
}

// store counterpart of row8
template <int VEC, bool FULL = false>
__device__ __forceinline__ void row8_store(const Buf& b, int64_t off, int ch, int W, const float* v) {
  if constexpr (VEC == 1) {
    if (FULL || 8 * ch < W) {
      bf16x8 x;
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (bf16)v[e];
      *(u16x8*)((bf16*)b.p + off + 8 * ch) = __builtin_bit_cast(u16x8, x);
    }
  } else if constexpr (VEC == 2) {
    if (FULL || 8 * ch < W) {
      float* q = (float*)b.p + off + 8 * ch;
      *(f32x4*)q = f32x4{v[0], v[1], v[2], v[3]};
      *(f32x4*)(q + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (8 * ch + e < W) st<float>(b, off + 8 * ch + e, v[e]);
  }
}

// The NCH chunks ch + 8 k of a row (slots 8 (ch + 8 k) .. +7) into v[8 k ..].
template <int VEC, bool FULL, int NCH>
__device__ __forceinline__ void rowN(const Buf& b, int64_t off, int ch, int W, float* v) {
#pragma unroll
  for (int k = 0; k < NCH; ++k) row8<VEC, FULL>(b, off, ch + 8 * k, W, v + 8 * k);
}

template <int VEC, bool FULL, int NCH>
__device__ __forceinline__ void rowN_store(const Buf& b, int64_t off, int ch, int W, const float* v) {
#pragma unroll
  for (int k = 0; k < NCH; ++k) row8_store<VEC, FULL>(b, off, ch + 8 * k, W, v + 8 * k);
}

// 1: bf16 rows read 16 bytes (8 slots) at a time, 2: float32 rows read 32
// bytes at a time (W a multiple of 8, 16-byte aligned slots), 0: neither
__device__ __forceinline__ int vec_kind(const Buf& b, int W) {
  if ((W & 7) != 0 || ((uintptr_t)b.p & 15) != 0) return 0;
  if (b.dt == TENSION_BF16 && ((b.s0 | b.s1 | b.s2) & 7) == 0) return 1;
  if (b.dt == TENSION_F32 && ((b.s0 | b.s1 | b.s2) & 3) == 0) return 2;
  return 0;
}

__device__ __forceinline__ float at(const Buf& b, int64_t off) { return ld<float>(b, off); }

// number of consistency terms n and the row range of term w1
__device__ __forceinline__ int cons_n(int W, int T) {
  if (W < 3 || T < 3) return 0;
  const int n = W - 2 < 4 ? W - 2 : 4;
  return T - (n + 1) > 0 ? n : 0;
}

// Walks one lane's rows row0, row0 + 32, ... of a [B, T, H, W] tensor (flat
// row b T H + t H + h) with its element offset in two stride sets (tau,
// dtau), updated incrementally: the divisions happen once per workgroup.
struct RowWalk {
  int64_t row, off, doff;
  int t, h;
  int dq, dr;                       // kRowsPerPass = dq H + dr
  int64_t step, dstep;              // offset change of dq rows of t, dr of h
  int64_t hwrap, dhwrap, twrap, dtwrap;  // on h >= H / t >= T

  __device__ __forceinline__ void init(int64_t r, int T, int H, const Buf& a, const Buf& d) {
    row = r;
    h = (int)(r % H);
    const int64_t bt = r / H;
    t = (int)(bt % T);
    const int64_t b = bt / T;
    off = b * a.s0 + (int64_t)t * a.s1 + (int64_t)h * a.s2;
    doff = b * d.s0 + (int64_t)t * d.s1 + (int64_t)h * d.s2;
    dq = kRowsPerPass / H;
    dr = kRowsPerPass % H;
    step = (int64_t)dq * a.s1 + (int64_t)dr * a.s2;
    dstep = (int64_t)dq * d.s1 + (int64_t)dr * d.s2;
    hwrap = a.s1 - (int64_t)H * a.s2;
    dhwrap = d.s1 - (int64_t)H * d.s2;
    twrap = a.s0 - (int64_t)T * a.s1;
    dtwrap = d.s0 - (int64_t)T * d.s1;
  }
  __device__ __forceinline__ void next(int T, int H) {
    row += kRowsPerPass;
    off += step;
    doff += dstep;
    h += dr;
    t += dq;
    if (h >= H) {
      h -= H;
      ++t;
      off += hwrap;
      doff += dhwrap;
    }
    while (t >= T) {  // once at most when T > kRowsPerPass
      t -= T;
      off += twrap;
      doff += dtwrap;
    }
  }
};

// Forward over this workgroup's kAuxRowsPerBlock rows of one layer: the four
// sums accumulate per lane (one lane per row contributes) and meet once at
// the end.
template <int VEC, bool FULL, int NCH>
__device__ __forceinline__ void fwd_rows(const AuxLossParams& p, const Buf& tb, float* sums) {
  constexpr int kUnroll = kUnrollVals / NCH, NV = 8 * NCH;
  const int ch = threadIdx.x & 7;
  const int64_t nrow = (int64_t)p.B * p.T * p.H;
  const int n = cons_n(p.W, p.T), T_out = p.T - (n + 1);
  RowWalk rw;
  rw.init((int64_t)blockIdx.x * kAuxRowsPerBlock + (threadIdx.x >> 3), p.T, p.H, tb, tb);
  for (int it = 0; it < kAuxRowsPerBlock / kRowsPerPass; it += kUnroll) {
    float v[kUnroll][NV], prev0[kUnroll];
    int ts[kUnroll];
    bool live[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (u) rw.next(p.T, p.H);
      // rows past the end read row 0 of the layer and contribute nothing
      live[u] = rw.row < nrow;
      ts[u] = rw.t;
      const int64_t off = live[u] ? rw.off : 0;
      rowN<VEC, FULL, NCH>(tb, off, ch, p.W, v[u]);
      // tau[t-1, 0] (a clamped row for t = 0); slots 0..4 of row t are in
      // lane 0's v[]
      prev0[u] = at(tb, live[u] && rw.t >= 1 ? off - tb.s1 : off);
    }
    rw.next(p.T, p.H);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < NV; ++e) s += v[u][e];
      s = row_sum8(s);
      const float inv = __builtin_amdgcn_rcpf(s + kDivEps);
      // -sum p ln(p + eps) = -(inv ln 2) sum tau log2(tau inv + eps); slots
      // past W hold tau = 0 and add nothing
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < NV; ++e) acc = fmaf(v[u][e], __builtin_amdgcn_logf(fmaf(v[u][e], inv, kDivEps)), acc);
      const float ent = -kLn2 * inv * row_sum8(acc);
      const float m = s / (float)p.W;
      float cons = 0.f;
      const int t = ts[u];
      if (n > 0 && t >= 1) {
#pragma unroll
        for (int w1 = 1; w1 <= 4; ++w1) {  // n <= 4
          if (w1 > n || t < w1 + 1 || t > w1 + T_out) continue;
          const float x = v[u][w1 - 1] * prev0[u] - v[u][w1];
          cons += x > 0.f ? x : 0.f;
        }
      }
      if (ch == 0 && live[u]) {
        sums[0] += ent;
        sums[1] += cons;
        sums[2] += m < 0.05f ? 0.05f - m : 0.f;
        sums[3] += m > 0.8f ? m - 0.8f : 0.f;
      }
    }
  }
}

template <int VEC, bool FULL, int NCH>
__device__ __forceinline__ void bwd_rows(const AuxLossParams& p, int l, const Buf& tb, const Buf& db) {
  constexpr int kUnroll = kUnrollVals / NCH, NV = 8 * NCH;
  const int ch = threadIdx.x & 7;
  const int64_t nrow = (int64_t)p.B * p.T * p.H;
  const int n = cons_n(p.W, p.T), T_out = p.T - (n + 1);
  const float kdiv = p.coef[3 * l], kcons = p.coef[3 * l + 1], kent = p.coef[3 * l + 2];
  RowWalk rw;
  rw.init((int64_t)blockIdx.x * kAuxRowsPerBlock + (threadIdx.x >> 3), p.T, p.H, tb, db);
  for (int it = 0; it < kAuxRowsPerBlock / kRowsPerPass; it += kUnroll) {
    float v[kUnroll][NV], vn[kUnroll][8], bprev[kUnroll];
    int ts[kUnroll];
    bool live[kUnroll];
    int64_t doffs[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (u) rw.next(p.T, p.H);
      live[u] = rw.row < nrow;
      ts[u] = rw.t;
      doffs[u] = rw.doff;
      const int64_t off = live[u] ? rw.off : 0;
      const int t = live[u] ? rw.t : 0;
      rowN<VEC, FULL, NCH>(tb, off, ch, p.W, v[u]);
      // the consistency neighbours (clamped rows at the ends): tau[t-1, 0]
      // and slots 0..7 of row t+1
      bprev[u] = at(tb, t >= 1 ? off - tb.s1 : off);
      row8<VEC>(tb, t + 1 < p.T ? off + tb.s1 : off, 0, p.W, vn[u]);
    }
    rw.next(p.T, p.H);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < NV; ++e) s += v[u][e];
      s = row_sum8(s);
      const float inv = __builtin_amdgcn_rcpf(s + kDivEps);
      // e_w = -(ln(p + eps) + p / (p + eps)); slots past W hold p = 0, so
      // they add nothing to sum e p
      float ee[NV], dot = 0.f;
#pragma unroll
      for (int e = 0; e < NV; ++e) {
        const float pe = v[u][e] * inv, x = pe + kDivEps;
        ee[e] = -fmaf(__builtin_amdgcn_logf(x), kLn2, pe * __builtin_amdgcn_rcpf(x));
        dot = fmaf(ee[e], pe, dot);
      }
      dot = row_sum8(dot);
      const float m = s / (float)p.W;
      const float gent = kent * ((m > 0.8f ? 1.f : 0.f) - (m < 0.05f ? 1.f : 0.f)) / (float)p.W;
      // g = k_div (e - dot) / (S + eps) + gent = kd e + (gent - kd dot)
      const float kd = kdiv * inv, g0 = fmaf(-kd, dot, gent);
      float g[NV];
#pragma unroll
      for (int e = 0; e < NV; ++e) g[e] = fmaf(kd, ee[e], g0);
      // consistency: slots 0..n live in lane chunk 0 (n <= 4 < 8)
      const int t = ts[u];
      if (ch == 0 && n > 0 && kcons != 0.f) {
        if (t >= 1) {  // terms of row t: a = tau[t, w1-1], b = tau[t-1, 0], c = tau[t, w1]
#pragma unroll
          for (int w1 = 1; w1 <= 4; ++w1) {
            if (w1 > n || t < w1 + 1 || t > w1 + T_out) continue;
            if (v[u][w1 - 1] * bprev[u] - v[u][w1] > 0.f) {
              g[w1 - 1] += kcons * bprev[u];
              g[w1] -= kcons;
            }
          }
        }
        if (t + 1 < p.T) {  // terms of row t+1 use tau[t, 0] as b
#pragma unroll
          for (int w1 = 1; w1 <= 4; ++w1) {
            if (w1 > n || t + 1 < w1 + 1 || t + 1 > w1 + T_out) continue;
            const float a = vn[u][w1 - 1];
            if (a * v[u][0] - vn[u][w1] > 0.f) g[0] += kcons * a;
          }
        }
      }
      if (live[u]) rowN_store<VEC, FULL, NCH>(db, doffs[u], ch, p.W, g);
    }
  }
}

}  // namespace

__global__ __launch_bounds__(kThreadsAux) void aux_loss_fwd_kernel(AuxLossParams p) {
  const int l = blockIdx.y;
  const Buf tb = p.tau[l];
  float sums[4] = {0.f, 0.f, 0.f, 0.f};
  // W = 64 NCH (e.g. the model's 64): every lane's chunks are in the row
  const int vk = vec_kind(tb, p.W);
  const int nch = p.W <= 64 ? 1 : p.W <= 128 ? 2 : 4;
  const bool full = p.W == 64 * nch;
#define AUX_FWD(N)                                             \
  if (vk == 1 && full) fwd_rows<1, true, N>(p, tb, sums);      \
  else if (vk == 1) fwd_rows<1, false, N>(p, tb, sums);        \
  else if (vk == 2 && full) fwd_rows<2, true, N>(p, tb, sums); \
  else if (vk == 2) fwd_rows<2, false, N>(p, tb, sums);        \
  else fwd_rows<0, false, N>(p, tb, sums);
  if (nch == 1) {
    AUX_FWD(1)
  } else if (nch == 2) {
    AUX_FWD(2)
  } else {
    AUX_FWD(4)
  }
#undef AUX_FWD
  // the block's sums go to its own slot of the partials buffer (summed by
  // the caller: deterministic, no atomics)
  __shared__ double red[4][kRowsPerPass];
  const int slot = threadIdx.x >> 3;
  if ((threadIdx.x & 7) == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) red[k][slot] = (double)sums[k];
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    double a = 0.0;
    for (int i = 0; i < kRowsPerPass; ++i) a += red[threadIdx.x][i];
    p.acc[((int64_t)l * gridDim.x + blockIdx.x) * 4 + threadIdx.x] = a;
  }
}

__global__ __launch_bounds__(kThreadsAux) void aux_loss_bwd_kernel(AuxLossParams p) {
  const int l = blockIdx.y;
  const Buf tb = p.tau[l], db = p.dtau[l];
  const int vt = vec_kind(tb, p.W), vk = vt == vec_kind(db, p.W) ? vt : 0;
  const int nch = p.W <= 64 ? 1 : p.W <= 128 ? 2 : 4;
  const bool full = p.W == 64 * nch;
#define AUX_BWD(N)                                                   \
  if (vk == 1 && full) bwd_rows<1, true, N>(p, l, tb, db);           \
  else if (vk == 1) bwd_rows<1, false, N>(p, l, tb, db);             \
  else if (vk == 2 && full) bwd_rows<2, true, N>(p, l, tb, db);      \
  else if (vk == 2) bwd_rows<2, false, N>(p, l, tb, db);             \
  else bwd_rows<0, false, N>(p, l, tb, db);
  if (nch == 1) {
    AUX_BWD(1)
  } else if (nch == 2) {
    AUX_BWD(2)
  } else {
    AUX_BWD(4)
  }
#undef AUX_BWD
}

int launch_aux_loss(bool bwd, const AuxLossParams& p, hipStream_t st, hipError_t* err) {
  const dim3 grid((unsigned)aux_loss_blocks((int64_t)p.B * p.T * p.H), (unsigned)p.L);
  if (bwd)
    hipLaunchKernelGGL(aux_loss_bwd_kernel, grid, dim3(kThreadsAux), 0, st, p);
  else
    hipLaunchKernelGGL(aux_loss_fwd_kernel, grid, dim3(kThreadsAux), 0, st, p);
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
