// Streaming decode step over a ring K/V cache, and the RoPE rotation.
//
// Decode is a pure HBM stream: every step reads the whole cache of each
// (sequence, head) once (2 * W * D * 2 bytes) and does 4*D flops per slot.
// One workgroup owns one (n, h); eight lanes cover one 128-byte cache row so
// each wave load instruction reads 1 KB of contiguous cache, all loads of a
// workgroup are issued before any arithmetic, and the sums are folded with
// cross-lane shuffles and one LDS pass.
#include "kernels.h"

namespace tension {

// Window slot w (0 = oldest) of ring slot `slot` when `pos` tokens are cached.
__device__ __forceinline__ int ring_w(int slot, int pos, int W) {
  int w = (slot - pos) % W;
  return w < 0 ? w + W : w;
}

// Cache rows are read once per step: non-temporal loads keep them from
// displacing reusable lines in L2.
__device__ __forceinline__ u16x8 cache_load(const bf16* p) {
#ifdef TENSION_DECODE_TEMPORAL
  return *(const u16x8*)p;
#else
  return __builtin_nontemporal_load((const u16x8*)p);
#endif
}

// Fast path: bf16 q / cache / out, D = 64, W % 32 == 0, W <= 512.
constexpr int kDecThreads = 256;
constexpr int kDecMaxPasses = 16;  // W <= 16 * 32

__global__ __launch_bounds__(kDecThreads) void decode_bf16_d64(DecodeParams p) {
  __shared__ float red[4][64 + 1];
  __shared__ float mred[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ch = lane & 7, rw = lane >> 3;  // d-chunk, row within a pass
  const int n = blockIdx.x / p.H, h = blockIdx.x % p.H;
  const int pos = p.pos_in[n] > 0 ? p.pos_in[n] : 0;
  const int W = p.W;
  const int npass = W >> 5;

  const bf16* qrow = (const bf16*)p.q.p + n * p.q.s0 + h * p.q.s1;
  // Whole-vector bit casts only: a bit cast of one subscripted vector
  // element (bit_cast<bf16>(v[i])) compiles to element 0 for every i.
  const bf16x8 qv = __builtin_bit_cast(bf16x8, *(const u16x8*)(qrow + 8 * ch));
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = (float)qv[i];

  const bf16* kbase = (const bf16*)p.kc.p + n * p.kc.s0 + h * p.kc.s1;
  const bf16* vbase = (const bf16*)p.vc.p + n * p.vc.s0 + h * p.vc.s1;
  bf16x8 kr[kDecMaxPasses], vr[kDecMaxPasses];
#pragma unroll
  for (int i = 0; i < kDecMaxPasses; ++i) {
    if (i < npass) {
      const int slot = i * 32 + wave * 8 + rw;
      kr[i] = __builtin_bit_cast(bf16x8, cache_load(kbase + (int64_t)slot * p.kc.s2 + 8 * ch));
    }
  }
#pragma unroll
  for (int i = 0; i < kDecMaxPasses; ++i) {
    if (i < npass) {
      const int slot = i * 32 + wave * 8 + rw;
      vr[i] = __builtin_bit_cast(bf16x8, cache_load(vbase + (int64_t)slot * p.vc.s2 + 8 * ch));
    }
  }
  const float inv_scale = (float)(1.0 / p.scale);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float msum = 0.f;
#pragma unroll
  for (int i = 0; i < kDecMaxPasses; ++i) {
    if (i < npass) {
      const int slot = i * 32 + wave * 8 + rw;
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) part += q[e] * (float)kr[i][e];
      part += __shfl_xor(part, 1);
      part += __shfl_xor(part, 2);
      part += __shfl_xor(part, 4);
      const bool ok = pos >= W || slot < pos;
      const float tau = ok ? sigmoid_fast(part * inv_scale) : 0.f;
      if (p.tau.p && ch == 0)
        st<float>(p.tau, n * p.tau.s0 + h * p.tau.s1 + ring_w(slot, pos, W), tau);
      msum += tau;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += tau * (float)vr[i][e];
    }
  }
  // fold rows within the wave (lanes with equal ch)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[e] += __shfl_xor(acc[e], 8);
    acc[e] += __shfl_xor(acc[e], 16);
    acc[e] += __shfl_xor(acc[e], 32);
  }
  msum += __shfl_xor(msum, 8);
  msum += __shfl_xor(msum, 16);
  msum += __shfl_xor(msum, 32);
  if (rw == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[wave][8 * ch + e] = acc[e];
    if (ch == 0) mred[wave] = msum;
  }
  __syncthreads();  // every cache read of this (n, h) is complete past here
  if (tid < 64) {
    const float o = red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid];
    const float m = mred[0] + mred[1] + mred[2] + mred[3];
    float inv = 1.f;
    if (p.flags & TENSION_NORM_MASS) inv = 1.f / (m > kMassEps ? m : kMassEps);
    bf16* orow = (bf16*)p.out.p + n * p.out.s0 + h * p.out.s1;
    orow[tid] = (bf16)(o * inv);
  } else if (tid < 64 + 16) {
    // append k_new / v_new at slot pos % W (8 lanes x 16 bytes each)
    const int i = tid - 64;
    const int slot = pos % W;
    if (i < 8) {
      const bf16* src = (const bf16*)p.kn.p + n * p.kn.s0 + h * p.kn.s1;
      bf16* dst = (bf16*)p.kc.p + n * p.kc.s0 + h * p.kc.s1 + (int64_t)slot * p.kc.s2;
      *(u16x8*)(dst + 8 * i) = *(const u16x8*)(src + 8 * i);
    } else {
      const int j = i - 8;
      const bf16* src = (const bf16*)p.vn.p + n * p.vn.s0 + h * p.vn.s1;
      bf16* dst = (bf16*)p.vc.p + n * p.vc.s0 + h * p.vc.s1 + (int64_t)slot * p.vc.s2;
      *(u16x8*)(dst + 8 * j) = *(const u16x8*)(src + 8 * j);
    }
  } else if (tid == 64 + 16 && h == 0 && p.pos_out) {
    p.pos_out[n] = pos + 1;
  }
}

// Exact path: any dtype, any D <= 256, any W; one thread per (n, h).  The
// thread reads every slot before it overwrites slot pos % W, so the
// read-before-write order holds within the thread.
template <typename A>
__global__ __launch_bounds__(64) void decode_exact(DecodeParams p) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.N * p.H) return;
  const int n = idx / p.H, h = idx % p.H;
  const int pos = p.pos_in[n] > 0 ? p.pos_in[n] : 0;
  const int W = p.W, D = p.D;
  const A scale = (A)p.scale;
  A acc[256];
  for (int d = 0; d < D; ++d) acc[d] = A(0);
  A msum = A(0);
  const int64_t qo = n * p.q.s0 + h * p.q.s1;
  for (int slot = 0; slot < W; ++slot) {
    const bool ok = pos >= W || slot < pos;
    A tau = A(0);
    if (ok) {
      const int64_t ko = n * p.kc.s0 + h * p.kc.s1 + (int64_t)slot * p.kc.s2;
      const int64_t vo = n * p.vc.s0 + h * p.vc.s1 + (int64_t)slot * p.vc.s2;
      A dot = A(0);
      for (int d = 0; d < D; ++d) dot += ld<A>(p.q, qo + d) * ld<A>(p.kc, ko + d);
      tau = sigmoid_exact(dot / scale);
      for (int d = 0; d < D; ++d) acc[d] += tau * ld<A>(p.vc, vo + d);
    }
    msum += tau;
    if (p.tau.p) st<A>(p.tau, n * p.tau.s0 + h * p.tau.s1 + ring_w(slot, pos, W), tau);
  }
  A inv = A(1);
  if (p.flags & TENSION_NORM_MASS) inv = A(1) / (msum > A(kMassEps) ? msum : A(kMassEps));
  const int64_t oo = n * p.out.s0 + h * p.out.s1;
  for (int d = 0; d < D; ++d) st<A>(p.out, oo + d, acc[d] * inv);
  const int slot = pos % W;
  const int64_t ko = n * p.kc.s0 + h * p.kc.s1 + (int64_t)slot * p.kc.s2;
  const int64_t vo = n * p.vc.s0 + h * p.vc.s1 + (int64_t)slot * p.vc.s2;
  const int64_t no = n * p.kn.s0 + h * p.kn.s1;
  const int64_t nvo = n * p.vn.s0 + h * p.vn.s1;
  for (int d = 0; d < D; ++d) {
    st<A>(p.kc, ko + d, ld<A>(p.kn, no + d));
    st<A>(p.vc, vo + d, ld<A>(p.vn, nvo + d));
  }
  if (h == 0 && p.pos_out) p.pos_out[n] = pos + 1;
}

int launch_decode(bool fast, bool f64, const DecodeParams& p, hipStream_t st, hipError_t* err) {
  if (fast) {
    hipLaunchKernelGGL(decode_bf16_d64, dim3((unsigned)(p.N * p.H)), dim3(kDecThreads), 0, st, p);
  } else {
    const unsigned grid = (unsigned)((p.N * p.H + 63) / 64);
    if (f64)
      hipLaunchKernelGGL(decode_exact<double>, dim3(grid), dim3(64), 0, st, p);
    else
      hipLaunchKernelGGL(decode_exact<float>, dim3(grid), dim3(64), 0, st, p);
  }
  *err = hipGetLastError();
  return 0;
}

// ------------------------------------------------------------------ RoPE

// y[i]      = x[i] cos - x[i+half] sin      (model.py:81)
// y[i+half] = x[i] sin + x[i+half] cos
// inverse: the transpose (rotation by -theta).  One thread per (row, i<half);
// each thread reads both halves before writing, so y may alias x.
template <typename A>
__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
  const int half = p.D >> 1;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.T * p.H * half;
  if (idx >= total) return;
  const int i = (int)(idx % half);
  int64_t r = idx / half;
  const int h = (int)(r % p.H);
  r /= p.H;
  const int t = (int)(r % p.T);
  const int b = (int)(r / p.T);
  const int64_t xo = b * p.x.s0 + (int64_t)t * p.x.s1 + h * p.x.s2;
  const int64_t yo = b * p.y.s0 + (int64_t)t * p.y.s1 + h * p.y.s2;
  const int64_t to = (p.pos_offset + t) * half + i;
  const A c = (A)p.cos[to], s = p.inverse ? -(A)p.sin[to] : (A)p.sin[to];
  const A x1 = ld<A>(p.x, xo + i), x2 = ld<A>(p.x, xo + i + half);
  st<A>(p.y, yo + i, x1 * c - x2 * s);
  st<A>(p.y, yo + i + half, x1 * s + x2 * c);
}

int launch_rope(bool f64, const RopeParams& p, hipStream_t st, hipError_t* err) {
  const int64_t total = (int64_t)p.B * p.T * p.H * (p.D / 2);
  const unsigned grid = (unsigned)((total + 255) / 256);
  if (f64)
    hipLaunchKernelGGL(rope_kernel<double>, dim3(grid), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(rope_kernel<float>, dim3(grid), dim3(256), 0, st, p);
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
