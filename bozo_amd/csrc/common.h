// Shared device helpers for the gfx950 sigmoid-tension kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tension_hip.h"

namespace tension {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kMassEps = 1e-6f;      // model.py:227,257,281 clamp(min=1e-6)
constexpr float kLog2e = 1.4426950408889634f;

// Device view of a tension_buf: pointer, dtype and element strides.
struct Buf {
  const void* p;
  int dt;
  int64_t s0, s1, s2, s3;
};

// Host-side size arithmetic on caller-supplied int64 values: a * b when both
// are non-negative and the product is at most `lim`, else -1 (an overflowing
// product counts as too large, never as a wrapped small value).
inline int64_t mul_cap(int64_t a, int64_t b, int64_t lim) {
  int64_t r;
  if (a < 0 || b < 0 || __builtin_mul_overflow(a, b, &r) || r > lim) return -1;
  return r;
}

// Every byte offset of `rows` rows at a row stride of `s1` two-byte elements
// fits a 32-bit buffer view (rows * s1 * 2 < 2^32).
inline bool rows_fit_view(int64_t rows, int64_t s1) {
  return s1 > 0 && mul_cap(rows, s1, ((int64_t)1 << 31) - 1) >= 0;
}

inline Buf make_buf(const tension_buf* b) {
  Buf r;
  r.p = b ? b->ptr : nullptr;
  r.dt = b ? b->dtype : 0;
  r.s0 = b ? b->s[0] : 0;
  r.s1 = b ? b->s[1] : 0;
  r.s2 = b ? b->s[2] : 0;
  r.s3 = b ? b->s[3] : 0;
  return r;
}

// Scalar load / store with the dtype chosen at run time.  The switch is
// wave-uniform (one dtype per buffer), so it costs a few scalar
// instructions, not divergence.  Used by the exact kernels and for the
// sparse operands (bias, tau, dtau) of the MFMA kernels.
template <typename A>
__device__ __forceinline__ A ld(const Buf& b, int64_t off) {
  switch (b.dt) {
    case TENSION_F32: return (A)((const float*)b.p)[off];
    case TENSION_BF16: return (A)(float)((const bf16*)b.p)[off];
    case TENSION_F16: return (A)(float)((const f16*)b.p)[off];
    default: return (A)((const double*)b.p)[off];
  }
}

template <typename A>
__device__ __forceinline__ void st(const Buf& b, int64_t off, A x) {
  switch (b.dt) {
    case TENSION_F32: ((float*)b.p)[off] = (float)x; break;
    case TENSION_BF16: ((bf16*)b.p)[off] = (bf16)(float)x; break;
    case TENSION_F16: ((f16*)b.p)[off] = (f16)(float)x; break;
    default: ((double*)b.p)[off] = (double)x; break;
  }
}

// Eight consecutive elements: one dtype switch per chunk keeps the unrolled
// row loops of the exact kernels small.
template <typename A>
__device__ __forceinline__ void ld8(const Buf& b, int64_t off, A* o) {
  switch (b.dt) {
    case TENSION_F32: {
      const float* s = (const float*)b.p + off;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (A)s[i];
    } break;
    case TENSION_BF16: {
      const bf16* s = (const bf16*)b.p + off;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (A)(float)s[i];
    } break;
    case TENSION_F16: {
      const f16* s = (const f16*)b.p + off;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (A)(float)s[i];
    } break;
    default: {
      const double* s = (const double*)b.p + off;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (A)s[i];
    } break;
  }
}

template <typename A>
__device__ __forceinline__ void st8(const Buf& b, int64_t off, const A* x) {
  switch (b.dt) {
    case TENSION_F32: {
      float* d = (float*)b.p + off;
#pragma unroll
      for (int i = 0; i < 8; ++i) d[i] = (float)x[i];
    } break;
    case TENSION_BF16: {
      bf16* d = (bf16*)b.p + off;
#pragma unroll
      for (int i = 0; i < 8; ++i) d[i] = (bf16)(float)x[i];
    } break;
    case TENSION_F16: {
      f16* d = (f16*)b.p + off;
#pragma unroll
      for (int i = 0; i < 8; ++i) d[i] = (f16)(float)x[i];
    } break;
    default: {
      double* d = (double*)b.p + off;
#pragma unroll
      for (int i = 0; i < 8; ++i) d[i] = (double)x[i];
    } break;
  }
}

// Accurate logistic function (exact kernels): libm exp and IEEE division.
__device__ __forceinline__ float sigmoid_exact(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ double sigmoid_exact(double x) { return 1.0 / (1.0 + exp(-x)); }

// Fast logistic function (MFMA kernels): sigma(x) = 1 / (1 + 2^(-x log2 e))
// on the hardware v_exp_f32 / v_rcp_f32 (about 1 ulp each).  Saturates
// correctly: 2^(+big) = inf -> rcp = 0, 2^(-big) = 0 -> rcp(1) = 1.
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// Lane move within a DPP row (bound_ctrl: every source lane of the controls
// used here exists, so no lane reads the zero fill).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over an aligned group of 8 lanes (all 8 must be active).
__device__ __forceinline__ float row_sum8(float x) {
  x += dpp_move<0xB1>(x);   // quad_perm [1,0,3,2]: lane ^ 1
  x += dpp_move<0x4E>(x);   // quad_perm [2,3,0,1]: lane ^ 2
  x += dpp_move<0x141>(x);  // row_half_mirror: lane i <-> 7 - i of its 8-lane half-row
  return x;
}

__device__ __forceinline__ unsigned short bf16_bits(bf16 x) {
  return __builtin_bit_cast(unsigned short, x);
}

// Map a linear workgroup id so that consecutive logical tiles land on the
// same XCD (gfx950 dispatches workgroups round-robin over its 8 XCDs, each
// with a private L2): neighbouring tiles share K/V rows, so keeping them on
// one XCD turns the re-reads into L2 hits.
__device__ __forceinline__ int xcd_swizzle(int id, int n) {
  if ((n & 7) != 0) return id;
  return (id & 7) * (n >> 3) + (id >> 3);
}

}  // namespace tension
