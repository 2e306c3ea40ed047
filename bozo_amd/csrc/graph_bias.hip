// Graph-bias builder: the [B, T, W] (window) or [B, T, T] (global) additive
// pre-sigmoid bias alpha * weight(content[s] -> content[t]) from a
// content-pair -> weight map, looked up on the device.
//
// The map is an open-addressing hash table in device memory: 64-bit keys
// (src content id << 32 | dst content id), double weights, a power-of-two
// capacity at most half full, Fibonacci hashing (key * 2^64/phi, top bits)
// and linear probing.  Insertion claims a slot with a 64-bit compare-and-swap.
// Every bias element is written (zeros included), so the output needs no
// clearing; the statistics (hits, weight sum, weight max) are accumulated
// with atomics into a caller-zeroed buffer.
#include "kernels.h"

namespace tension {

namespace {

constexpr unsigned long long kEmptyKey = ~0ull;

__device__ __forceinline__ unsigned long long slot_of(unsigned long long key, int log2cap) {
  return (key * 0x9E3779B97F4A7C15ull) >> (64 - log2cap);
}

}  // namespace

__global__ __launch_bounds__(256) void bias_table_insert(BiasTableParams p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.n) return;
  const unsigned long long key = p.in_keys[i];
  const unsigned long long mask = (1ull << p.log2cap) - 1ull;
  unsigned long long s = slot_of(key, p.log2cap);
  // the host sizes the table to at least twice the key count, so a free or
  // matching slot exists and the probe ends within cap steps
  for (int64_t step = 0; step < ((int64_t)1 << p.log2cap); ++step) {
    const unsigned long long prev = atomicCAS(&p.keys[s], kEmptyKey, key);
    if (prev == kEmptyKey || prev == key) {
      p.vals[s] = p.in_vals[i];
      return;
    }
    s = (s + 1ull) & mask;
  }
}

template <typename OUT>
__global__ __launch_bounds__(256) void bias_build(BiasBuildParams p) {
  const int64_t n = (int64_t)p.T * p.K;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int t = (int)(i / p.K), j = (int)(i % p.K);
  // window: key s = t - (W - j); global: s = j, keys s < t
  const int s = p.global ? j : t - (p.K - j);
  double wgt = 0.0;
  if (s >= 0 && s < t) {
    const int src = p.ids[s], dst = p.ids[t];
    if (src >= 0 && dst >= 0) {
      const unsigned long long key = ((unsigned long long)(unsigned)src << 32) | (unsigned)dst;
      const unsigned long long mask = (1ull << p.log2cap) - 1ull;
      unsigned long long sl = slot_of(key, p.log2cap);
      for (int64_t step = 0; step < ((int64_t)1 << p.log2cap); ++step) {
        const unsigned long long k = p.keys[sl];
        if (k == key) {
          wgt = p.vals[sl];
          break;
        }
        if (k == kEmptyKey) break;
        sl = (sl + 1ull) & mask;
      }
    }
  }
  const bool hit = wgt > 0.0;
  const double boost = hit ? p.alpha * wgt : 0.0;
  // narrower outputs round through float, as a float scalar written into a
  // half-precision tensor does
  const OUT v = sizeof(OUT) == 8 ? (OUT)boost : (OUT)(float)boost;
  OUT* out = (OUT*)p.out;
  for (int b = 0; b < p.B; ++b) out[(int64_t)b * p.os0 + (int64_t)t * p.os1 + j] = v;
  if (p.stats && hit) {
    atomicAdd(&p.stats[0], 1.0);
    atomicAdd(&p.stats[1], wgt);
    // weights are positive here, so their bit patterns order as integers
    atomicMax((unsigned long long*)&p.stats[2], (unsigned long long)__double_as_longlong(wgt));
  }
}

int launch_bias_insert(const BiasTableParams& p, hipStream_t st, hipError_t* err) {
  hipLaunchKernelGGL(bias_table_insert, dim3((unsigned)((p.n + 255) / 256)), dim3(256), 0, st, p);
  *err = hipGetLastError();
  return 0;
}

int launch_bias_build(int out_dtype, const BiasBuildParams& p, hipStream_t st, hipError_t* err) {
  const int64_t n = (int64_t)p.T * p.K;
  const dim3 grid((unsigned)((n + 255) / 256));
  switch (out_dtype) {
    case TENSION_F32: hipLaunchKernelGGL(bias_build<float>, grid, dim3(256), 0, st, p); break;
    case TENSION_BF16: hipLaunchKernelGGL(bias_build<bf16>, grid, dim3(256), 0, st, p); break;
    case TENSION_F16: hipLaunchKernelGGL(bias_build<f16>, grid, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL(bias_build<double>, grid, dim3(256), 0, st, p); break;
  }
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
