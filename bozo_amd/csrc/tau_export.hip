// Reductions over materialised tau for the graph exporter: per-(layer, head)
// profile statistics and the head-masked aggregate tau[t, w].
//
// Both read tau [B, T, H, W] of up to kMaxLayers local layers (any float
// dtype, strided, w innermost), averaged over the batch as it is read.  They
// are HBM/L2 streams with a few flops per element, so the kernels only aim
// at reading each row once per pass with whole-row accesses.
#include "kernels.h"

namespace tension {

namespace {

constexpr int kStatThreads = 512;  // one workgroup per (layer, head): 8 waves stream it

// Batch mean of tau[:, t, h, w] (0 for a masked cell), in float.
__device__ __forceinline__ float tau_at(const Buf& b, int B, int t, int h, int w, int W, bool valid_only) {
  if (valid_only && t + w < W) return 0.f;
  const int64_t off = (int64_t)t * b.s1 + (int64_t)h * b.s2 + w;
  float s = 0.f;
  for (int i = 0; i < B; ++i) s += ld<float>(b, off + (int64_t)i * b.s0);
  return B == 1 ? s : s / (float)B;
}

__device__ __forceinline__ double block_sum(double x, double* red) {
  for (int o = 32; o > 0; o >>= 1) x += __shfl_down(x, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = x;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < kStatThreads / 64; ++i) s += red[i];
  return s;
}

constexpr int kStatVals = 128;  // values per thread of the register-resident select (T W <= 65536)

// The next order statistic after xk (xk again when more than k + 1 values
// are <= xk, else the smallest value above it: le / gt are this thread's
// counts), the interpolated quantile and the head's four statistics.
__device__ void head_quantile_out(const TauStatParams& p, int l, int h, int64_t n, float g, int64_t k, float xk,
                                  double le, float gt, double sum, double rmax, double rarg, int T, double* red) {
  const int tid = threadIdx.x;
  le = block_sum(le, red);
  for (int o = 32; o > 0; o >>= 1) gt = fminf(gt, __shfl_down(gt, o, 64));
  __shared__ float gred[kStatThreads / 64];
  if ((tid & 63) == 0) gred[tid >> 6] = gt;
  __syncthreads();
  if (tid == 0) {
    float gm = gred[0];
    for (int i = 1; i < kStatThreads / 64; ++i) gm = fminf(gm, gred[i]);
    const float xk1 = (k + 1 >= n || le >= (double)(k + 2)) ? xk : gm;
    // numpy's linear interpolation in the values' dtype (float32), each step
    // rounded on its own: a + (b - a) t, or b - (b - a) (1 - t) for t >= 0.5
    const float t = __fsub_rn(g, (float)k);
    const float d = __fsub_rn(xk1, xk);
    float* o = p.stats + ((int64_t)l * p.H + h) * 4;
    o[0] = (float)(sum / (double)n);
    o[1] = t >= 0.5f ? __fsub_rn(xk1, __fmul_rn(d, __fsub_rn(1.f, t))) : __fadd_rn(xk, __fmul_rn(d, t));
    o[2] = (float)(rarg / (double)T);
    o[3] = (float)(rmax / (double)T);
  }
}

}  // namespace

// One workgroup per (layer, head): mean of tau over (t, w), mean over t of
// the row maximum and of its first arg-max over w, and the 0.99 quantile of
// all T*W values with linear interpolation between order statistics k and
// k+1 (k = floor(0.99 (n - 1)), in float32 as numpy computes it).  The order statistics come from a radix
// select over the float bit patterns (tau >= 0, so they order as unsigned
// integers): four 8-bit passes with an LDS histogram, then one pass for the
// next value up.
__global__ __launch_bounds__(kStatThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void tau_head_stats_kernel(TauStatParams p) {
  const int l = blockIdx.x / p.H, h = blockIdx.x % p.H;
  const Buf tb = p.tau[l];
  const int T = p.T, W = p.W, B = p.B;
  const bool vo = p.valid_only != 0;
  const int tid = threadIdx.x;
  __shared__ double red[kStatThreads / 64];
  __shared__ unsigned hist[256];
  __shared__ unsigned sel[2];  // prefix bits, rank left within the prefix

  double sum = 0.0, rmax = 0.0, rarg = 0.0;
  const int64_t n = (int64_t)T * W;
  // The reference takes np.quantile(vals, 0.99) of float32 values
  // (head_filter.py:108-113).  numpy >= 2 keeps a Python-float q in the
  // array's dtype, so q, the rank (n - 1) q and the interpolation weight are
  // float32: the rank is 2034.45007 for n = 2056, not 2034.45.
  const float g = __fmul_rn((float)(n - 1), 0.99f);
  const int64_t k = (int64_t)g;
  if (tid == 0) {
    sel[0] = 0u;
    sel[1] = (unsigned)k;
  }
  if (B == 1 && W <= 64 && kStatThreads % W == 0 && n <= (int64_t)kStatThreads * kStatVals &&
      (tb.dt == TENSION_BF16 || tb.dt == TENSION_F32)) {
    // the head's values stay in registers for every radix pass: thread tid
    // holds slot w0 = tid % W of rows t0 + (512 / W) j, i.e. flat values
    // tid + 512 j; per-wave histograms keep the LDS atomics of clustered
    // values (a few top bytes) from serialising on one address
    const int nn = (int)n;
    const int w0 = tid % W, t0 = tid / W, rstep = kStatThreads / W;
    float v[kStatVals];
    auto load_all = [&](auto tag) {
      using E = decltype(tag);
      const E* base = (const E*)tb.p + (int64_t)h * tb.s2 + w0;
#pragma unroll
      for (int j = 0; j < kStatVals; ++j) {
        const int t = t0 + rstep * j;
        const bool in = t < T && !(vo && t + w0 < W);
        v[j] = in ? (float)base[(int64_t)t * tb.s1] : 0.f;
      }
    };
    if (tb.dt == TENSION_BF16)
      load_all(bf16{});
    else
      load_all(float{});
    // row sum, maximum and first arg-max: a row is W adjacent lanes (one
    // per slot), reduced by xor shuffles inside the W-lane segment
#pragma unroll
    for (int j = 0; j < kStatVals; ++j) {
      float rs = v[j], m = v[j];
      int am = w0;
      for (int o = 1; o < W; o <<= 1) {
        rs += __shfl_xor(rs, o, 64);
        const float m2 = __shfl_xor(m, o, 64);
        const int a2 = __shfl_xor(am, o, 64);
        if (m2 > m || (m2 == m && a2 < am)) {
          m = m2;
          am = a2;
        }
      }
      if (w0 == 0 && t0 + rstep * j < T) {
        sum += rs;
        rmax += m;
        rarg += am;
      }
    }
    sum = block_sum(sum, red);
    rmax = block_sum(rmax, red);
    rarg = block_sum(rarg, red);
    __shared__ unsigned whist[kStatThreads / 64][256 + 1];  // +1: the waves' copies of a bin in different banks
    __shared__ unsigned tot[256];
    unsigned* const my = whist[tid >> 6];
    // batch-mean-free bf16 input has zero low 16 bits: two passes decide it
    const bool exact16 = B == 1 && tb.dt == TENSION_BF16;
    unsigned msk = 0u;
    for (int shift = 24; shift >= (exact16 ? 16 : 0); shift -= 8) {
      for (int i = tid; i < (kStatThreads / 64) * 257; i += kStatThreads) (&whist[0][0])[i] = 0u;
      __syncthreads();
      const unsigned prefix = sel[0];
      {
#pragma unroll
        for (int j = 0; j < kStatVals; ++j) {
          const unsigned bits = __float_as_uint(v[j]);
          if (tid + kStatThreads * j < nn && (bits & msk) == prefix) atomicAdd(&my[(bits >> shift) & 255u], 1u);
        }
      }
      __syncthreads();
      if (tid < 256) {
        unsigned c = 0u;
#pragma unroll
        for (int wv = 0; wv < kStatThreads / 64; ++wv) c += whist[wv][tid];
        tot[tid] = c;
      }
      __syncthreads();
      if (tid < 64) {
        // wave 0 finds the bin holding rank r: lane L owns bins 4L..4L+3;
        // an inclusive scan of the lanes' counts brackets r in one lane
        const unsigned r = sel[1];
        unsigned c4[4], own = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          c4[q] = tot[4 * tid + q];
          own += c4[q];
        }
        unsigned inc = own;
        for (int o = 1; o < 64; o <<= 1) {
          const unsigned up = __shfl_up(inc, o, 64);
          if (tid >= o) inc += up;
        }
        unsigned c = inc - own;
        if (c <= r && r < inc) {
          int bin = 4 * tid;
#pragma unroll
          for (int q = 0; q < 3; ++q) {
            if (c + c4[q] > r) break;
            c += c4[q];
            ++bin;
          }
          sel[0] = prefix | ((unsigned)bin << shift);
          sel[1] = r - c;
        }
      }
      __syncthreads();
      msk |= 255u << shift;
    }
    const float xk = __uint_as_float(sel[0]);
    double le = 0.0;
    float gt = 3.0e38f;
#pragma unroll
    for (int j = 0; j < kStatVals; ++j) {
      if (tid + kStatThreads * j < nn) {
        if (v[j] <= xk) le += 1.0;
        else gt = fminf(gt, v[j]);
      }
    }
    head_quantile_out(p, l, h, n, g, k, xk, le, gt, sum, rmax, rarg, T, red);
    return;
  }
  for (int t = tid; t < T; t += kStatThreads) {
    float m = -1.f, s = 0.f;
    int am = 0;
    for (int w = 0; w < W; ++w) {
      const float v = tau_at(tb, B, t, h, w, W, vo);
      s += v;
      if (v > m) {
        m = v;
        am = w;
      }
    }
    sum += s;
    rmax += m;
    rarg += am;
  }
  sum = block_sum(sum, red);
  rmax = block_sum(rmax, red);
  rarg = block_sum(rarg, red);

  unsigned mask = 0u;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += kStatThreads) hist[i] = 0u;
    __syncthreads();
    const unsigned prefix = sel[0];
    for (int64_t i = tid; i < n; i += kStatThreads) {
      const int t = (int)(i / W), w = (int)(i % W);
      const unsigned bits = __float_as_uint(tau_at(tb, B, t, h, w, W, vo));
      if ((bits & mask) == prefix) atomicAdd(&hist[(bits >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      unsigned r = sel[1], c = 0u;
      int bin = 0;
      for (; bin < 255; ++bin) {
        if (c + hist[bin] > r) break;
        c += hist[bin];
      }
      sel[0] = prefix | ((unsigned)bin << shift);
      sel[1] = r - c;
    }
    __syncthreads();
    mask |= 255u << shift;
  }
  const float xk = __uint_as_float(sel[0]);
  // the next order statistic: xk again if more than k + 1 values are <= xk,
  // else the smallest value above it
  double le = 0.0;
  float gt = 3.0e38f;
  for (int64_t i = tid; i < n; i += kStatThreads) {
    const int t = (int)(i / W), w = (int)(i % W);
    const float v = tau_at(tb, B, t, h, w, W, vo);
    if (v <= xk) le += 1.0;
    else gt = fminf(gt, v);
  }
  head_quantile_out(p, l, h, n, g, k, xk, le, gt, sum, rmax, rarg, T, red);
}

// aggregated[t, w] = mean over the selected (layer, head) pairs of the batch
// mean of tau[l][:, t, h, w] (all pairs when none is selected).  One thread
// per (t, w), consecutive threads along w (whole rows per wave load).  Wave 0
// first compacts the selection into a list in LDS (ballot + popcount per
// 64-entry chunk), so the sum loop has no branch and its loads can be
// issued back to back.
__global__ __launch_bounds__(256) void tau_aggregate_kernel(TauAggParams p) {
  __shared__ short sel[kMaxLayers * 64];
  __shared__ int nsel;
  const int LH = p.L * p.H;
  const int tid = threadIdx.x;
  if (tid < 64) {
    int n = 0;
    for (int base = 0; base < LH; base += 64) {
      const int i = base + tid;
      const bool on = i < LH && p.mask[i] != 0;
      const unsigned long long bal = __ballot(on);
      if (on) sel[n + __popcll(bal & ((1ull << tid) - 1ull))] = (short)i;
      n += __popcll(bal);
    }
    if (n == 0)  // no selection: every pair
      for (int i = tid; i < LH; i += 64) sel[i] = (short)i;
    if (tid == 0) nsel = n ? n : LH;
  }
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + tid;
  if (i >= (int64_t)p.T * p.W) return;
  const int t = (int)(i / p.W), w = (int)(i % p.W);
  const int n = nsel;
  double s = 0.0;
#pragma unroll 4
  for (int j = 0; j < n; ++j) {
    const int lh = sel[j];
    const int l = lh / p.H, h = lh - l * p.H;
    s += tau_at(p.tau[l], p.B, t, h, w, p.W, false);
  }
  p.agg[i] = (float)(s / (double)n);
}

int launch_tau_stats(const TauStatParams& p, hipStream_t st, hipError_t* err) {
  hipLaunchKernelGGL(tau_head_stats_kernel, dim3((unsigned)(p.L * p.H)), dim3(kStatThreads), 0, st, p);
  *err = hipGetLastError();
  return 0;
}

int launch_tau_aggregate(const TauAggParams& p, hipStream_t st, hipError_t* err) {
  const int64_t n = (int64_t)p.T * p.W;
  hipLaunchKernelGGL(tau_aggregate_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p);
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
